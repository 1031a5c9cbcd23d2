"""GPU parity at the BASELINE configurations (C1, C3, C4, C5; C2 is covered
in test_gpu_attn.py and bench.py).  Each runs the configuration's own flow at
its real shape on one layer or two (C5: the full 64-layer, ~137 GB pool),
checks sampled rows against the CPU oracle within 2e-3 (over the sequence
gathered through the product's gather kernel), and checks the size-
independent properties the flow offers bit-exactly: batch == solo, forked
sequences equal their source, pages after eviction are reused, rollback
keeps the kept prefix."""

import math
import random

import numpy as np
import pytest

import oracle
from gpu_util import fill_layer_random, fragment, make_pool, oracle_layer, oracle_seq, say, scattered_alloc

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _spec(rows, nq, hd, m, window=0, softcap=0.0, row_off=0):
    from flint_amd import ops

    return ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None,
                        args=rows, row_off=row_off, softcap=softcap)


def _check_rows(torch, pool, layer, y, q, rows_idx, positions, seqs, nq, hd, label, window=0, softcap=0.0,
                scale=None):
    """Oracle over each sampled row's own sequence (gathered)."""
    scale = scale or 1.0 / math.sqrt(hd)
    worst = 0.0
    by_seq = {}
    for r in rows_idx:
        by_seq.setdefault(seqs[r], []).append(r)
    for s, rs in by_seq.items():
        n = max(positions[r] for r in rs) + 1
        ref = oracle_seq(torch, pool, layer, s, n)
        qs = q[rs].float().cpu().numpy()
        want = ref.attn(qs, oracle.row_meta([positions[r] for r in rs], [0] * len(rs)), len(rs), nq, scale,
                        window=window, softcap=softcap)
        got = y[rs].float().cpu().numpy()
        err = float(np.max(np.abs(got - want)))
        worst = max(worst, err)
        assert np.all(np.isfinite(got)), (label, s)
    say(label, "max abs err", worst)
    assert worst <= TOL, (label, worst)


def test_c1_qwen2_small_decode_steps(torch_cuda):
    """C1: 14 q / 2 KV heads, hd 64, f16 KV, page 16, B=4, ctx U[128,512],
    tables scattered over a 256-page pool; 8 steps of append 1 token + decode
    (f32 K/V/Q sources as the reference's forward pass produces them).  Every
    step is checked against the oracle and the pool stays bit-exact against
    the oracle's own appends."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    rng = random.Random(1001)
    nq, nkv, hd, P, steps = 14, 2, 64, 16, 8
    ctx = [rng.randint(128, 512) for _ in range(4)]
    budget = [c + steps for c in ctx]
    pool = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16",
                     extra_pages=256 - sum(-(-b // P) for b in budget))
    assert pool.arena.pages() == 256
    scattered_alloc(pool, budget, rng, P)
    fill_layer_random(torch, pool, 0, seed=1001)
    ref = oracle_layer(torch, pool)
    rows = RowMeta(8)
    g = torch.Generator(device="cuda")
    g.manual_seed(1001)
    for step in range(steps):
        pos = [c + step for c in ctx]
        rows.write(pos, [0, 1, 2, 3], 4)
        k = torch.randn(4, nkv, hd, device="cuda", generator=g)
        v = torch.randn(4, nkv, hd, device="cuda", generator=g)
        q = torch.randn(4, nq, hd, device="cuda", generator=g)
        y = torch.empty_like(q)
        ops.kv_store_attn(k, v, q, pool, 0, y, _spec(rows, nq, hd, 4))
        torch.cuda.synchronize()
        meta = oracle.row_meta(pos, [0, 1, 2, 3])
        ref.kv_store(k.cpu().numpy(), v.cpu().numpy(), meta, 4, oracle.SRC_F32)
        want = ref.attn(q.cpu().numpy(), meta, 4, nq, 1.0 / math.sqrt(hd))
        err = float(np.max(np.abs(y.cpu().numpy() - want)))
        say("C1 step", step, "max abs err", err)
        assert err <= TOL
    got = oracle_layer(torch, pool)
    assert np.array_equal(got.k, ref.k) and np.array_equal(got.v, ref.v)
    pool.close()


def test_c3_qwen3_ragged_continuous_batch(torch_cuda):
    """C3: 32 q / 8 KV, hd 128, f16, page 16.  64 decode sequences with
    log-normal contexts clipped to [256, 32768] (median 2048) and 8 new
    sequences chunk-prefilling 512 causal tokens, all in ONE call, in a pool
    60% pre-occupied at random (fragmented free list)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    rng = random.Random(1003)
    nprng = np.random.default_rng(1003)
    nq, nkv, hd, P = 32, 8, 128, 16
    ctx = np.clip(np.round(nprng.lognormal(math.log(2048), 1.0, 64)), 256, 32768).astype(int).tolist()
    ctx[0] = 32768  # make sure the longest case is present
    pre = 512
    need = sum(-(-(c + 1) // P) for c in ctx) + 8 * (pre // P)
    pages = int(need / 0.4) + 64
    n_fill = 256
    fill_budget = -(-pages // n_fill) * 4 * P
    budgets = [fill_budget] * n_fill + [c + 1 for c in ctx] + [pre] * 8
    pool = make_pool([], kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16", seq_lens=budgets,
                     extra_pages=pages - sum(-(-b // P) for b in budgets))
    assert pool.arena.pages() == pages
    fragment(pool, list(range(n_fill)), 0.6, rng)
    say("C3 pool pages", pages, "used by filler", pool.arena.used())
    dec = list(range(n_fill, n_fill + 64))
    pf = list(range(n_fill + 64, n_fill + 72))
    for s, c in zip(dec, ctx):
        pool.alloc(s, 0, c + 1)
    for s in pf:
        pool.alloc(s, 0, pre)
    fill_layer_random(torch, pool, 0, seed=1003)
    positions = [c for c in ctx] + [p for _ in pf for p in range(pre)]
    seqs = dec + [s for s in pf for _ in range(pre)]
    m = len(seqs)
    rows = RowMeta(m)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(1003)
    k = torch.randn(m, nkv, hd, device="cuda", generator=g).half()
    v = torch.randn(m, nkv, hd, device="cuda", generator=g).half()
    q = torch.randn(m, nq, hd, device="cuda", generator=g).half()
    y = torch.empty_like(q)
    ops.kv_store_attn(k, v, q, pool, 0, y, _spec(rows, nq, hd, m))
    torch.cuda.synchronize()
    sample_dec = [0, 1, int(np.argmax(ctx[1:])) + 1, 63]
    sample_pf = [64 + i * pre + r for i in (0, 7) for r in (0, 1, 255, 511)]
    _check_rows(torch, pool, 0, y, q, sample_dec + sample_pf, positions, seqs, nq, hd, "C3 batch")
    # batch == solo: one decode row and one prefill chunk on their own
    rows_solo = RowMeta(pre)
    for idx in ([0], list(range(64 + 3 * pre, 64 + 4 * pre))):
        rows_solo.write([positions[i] for i in idx], [seqs[i] for i in idx], len(idx))
        ys = torch.empty(len(idx), nq, hd, device="cuda", dtype=torch.float16)
        ops.attn(q[idx].contiguous(), pool, 0, ys, _spec(rows_solo, nq, hd, len(idx)))
        torch.cuda.synchronize()
        assert torch.equal(ys, y[idx]), "batch == solo"
    pool.close()


def test_c4_gemma2_window_softcap_speculative(torch_cuda):
    """C4: 16 q / 8 KV, hd 256, f16, page 16; layer 0 sliding window 4096,
    layer 1 global; logit soft-cap 50; B=16 at context 8192.  Speculative
    step: append 4 draft tokens per sequence and verify them with a 4-row
    causal decode (fused launch), roll back a seeded U{0..4} rejected tokens
    by block-table truncation, then append the corrected token and decode.
    A fork of sequence 0 taken mid-page exercises the copy-on-write of the
    partial block; its outputs equal its source's bit-exactly."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    rng = random.Random(1004)
    nq, nkv, hd, P, B, ctx, cap = 16, 8, 256, 16, 16, 8192, 50.0
    budget = [ctx + 8] * (B + 1)
    pool = make_pool([], kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16", layers=2, seq_lens=budget,
                     extra_pages=4)
    scattered_alloc(pool, [ctx - 3] * B, rng, P)  # contexts end mid-page
    for layer in range(2):
        fill_layer_random(torch, pool, layer, seed=1004 + layer, scale=3.0)
    base = ctx - 3
    pool.fork(0, B, base)  # shares full pages, copies the partial page
    for s in range(B + 1):
        pool.alloc(s, base, 4)
    seqs = [s for s in range(B + 1) for _ in range(4)]
    positions = [base + i for _ in range(B + 1) for i in range(4)]
    m = len(seqs)
    rows = RowMeta(m)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(1004)
    k = torch.randn(m, nkv, hd, device="cuda", generator=g)
    v = torch.randn(m, nkv, hd, device="cuda", generator=g)
    q = torch.randn(m, nq, hd, device="cuda", generator=g) * 2
    # the fork drafts the same tokens and queries as sequence 0
    k[4 * B:] = k[:4]
    v[4 * B:] = v[:4]
    q[4 * B:] = q[:4]
    scale = 1.0 / 16
    for layer, window in ((0, 4096), (1, 0)):
        y = torch.empty_like(q)
        spec = _spec(rows, nq, hd, m, window=window, softcap=cap)
        spec.scale = scale
        ops.kv_store_attn(k[:, :, :], v, q, pool, layer, y, spec)
        torch.cuda.synchronize()
        assert torch.equal(y[4 * B:], y[:4]), "fork == source"
        _check_rows(torch, pool, layer, y, q, [0, 1, 2, 3, 4 * 7 + 2, 4 * 15 + 3], positions, seqs, nq, hd,
                    f"C4 verify layer {layer}", window=window, softcap=cap, scale=scale)
    # roll back U{0..4} rejected drafts, then append the corrected token
    keep = [base + 4 - rng.randint(0, 4) for _ in range(B + 1)]
    keep[B] = keep[0]
    checked = (1, 5, B)
    before = {(layer, s): oracle_seq(torch, pool, layer, s, base + 4).gather(0, 0, base + 4)
              for layer in range(2) for s in checked}
    for s in range(B + 1):
        pool.truncate(s, keep[s])
        pool.alloc(s, keep[s], 1)
    rows.write(keep, list(range(B + 1)), B + 1)
    k1 = torch.randn(B + 1, nkv, hd, device="cuda", generator=g)
    v1 = torch.randn(B + 1, nkv, hd, device="cuda", generator=g)
    q1 = torch.randn(B + 1, nq, hd, device="cuda", generator=g) * 2
    k1[B], v1[B], q1[B] = k1[0], v1[0], q1[0]
    for layer, window in ((0, 4096), (1, 0)):
        y1 = torch.empty_like(q1)
        spec = _spec(rows, nq, hd, B + 1, window=window, softcap=cap)
        spec.scale = scale
        ops.kv_store_attn(k1, v1, q1, pool, layer, y1, spec)
        torch.cuda.synchronize()
        assert torch.equal(y1[B], y1[0]), "fork == source after rollback"
        _check_rows(torch, pool, layer, y1, q1, list(range(0, B + 1, 3)), keep, list(range(B + 1)), nq, hd,
                    f"C4 after rollback layer {layer}", window=window, softcap=cap, scale=scale)
        # the kept prefix of every sequence is untouched by the rollback
        for s in checked:
            kk, vv = oracle_seq(torch, pool, layer, s, keep[s]).gather(0, 0, keep[s])
            bk, bv = before[(layer, s)]
            assert np.array_equal(kk, bk[:, :keep[s]]) and np.array_equal(vv, bv[:, :keep[s]])
    pool.close()


def test_c5_qwen25_32b_capacity_fork_evict(torch_cuda):
    """C5: 64 layers, 40 q / 8 KV, hd 128, f16, page 16, 4 sequences at
    context 131072 in one ~148 GB arena (137 GB of KV).  Every sequence is
    forked (full pages shared, the partial last page copied); a random 25%
    of the 8 sequences is evicted and their freed pages go to 2 new
    sequences; then one decode step (append + attention) runs on layers 0
    and 63.  Forks decode bit-identically to their source; sampled sequences
    match the oracle."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    torch.cuda.empty_cache()
    rng = random.Random(1005)
    L, nq, nkv, hd, P = 64, 40, 8, 128, 16
    ctx = 131072 - 5
    new_ctx = 20000
    budgets = [131072 + 8] * 8 + [new_ctx + 8] * 2
    pages = 4 * (131072 // P) + 4 + 2 * (-(-(new_ctx + 1) // P)) + 64
    pool = make_pool([], kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16", layers=L, seq_lens=budgets,
                     extra_pages=pages - sum(-(-b // P) for b in budgets))
    base, nbytes = pool.memory()
    say("C5 arena bytes", nbytes)
    assert nbytes >= 137 * 10 ** 9
    scattered_alloc(pool, [ctx] * 4, rng, P)
    for layer in (0, L - 1):
        fill_layer_random(torch, pool, layer, seed=1005 + layer)
    for s in range(4):
        pool.fork(s, 4 + s, ctx)
        assert pool.arena.table_of(4 + s)[:-1] == pool.arena.table_of(s)[:-1]
        assert pool.arena.table_of(4 + s)[-1] != pool.arena.table_of(s)[-1]
    evict = rng.sample(range(8), 2)
    survivors = [s for s in range(8) if s not in evict]
    held = {p for s in survivors for p in pool.arena.table_of(s)}
    expect = {p for s in evict for p in pool.arena.table_of(s)} - held
    free_before = pool.arena.pages() - pool.arena.used()
    for s in evict:
        pool.free_seq(s)
    freed = pool.arena.pages() - pool.arena.used() - free_before
    say("C5 evicted", evict, "freed pages", freed)
    assert freed == len(expect)  # shared pages stay with the surviving holder
    live = survivors + [8, 9]
    for s in (8, 9):
        pool.alloc(s, 0, new_ctx)
    reused = set(pool.arena.table_of(8)) | set(pool.arena.table_of(9))
    assert expect <= reused or len(expect) > len(reused), "freed pages are handed out first (LIFO)"
    pos = {s: (ctx if s < 8 else new_ctx) for s in live}
    for s in live:
        pool.alloc(s, pos[s], 1)
    rows = RowMeta(len(live))
    rows.write([pos[s] for s in live], live, len(live))
    g = torch.Generator(device="cuda")
    g.manual_seed(1005)
    m = len(live)
    k = torch.randn(m, nkv, hd, device="cuda", generator=g).half()
    v = torch.randn(m, nkv, hd, device="cuda", generator=g).half()
    q = torch.randn(m, nq, hd, device="cuda", generator=g).half()
    # a surviving fork pair gets identical new tokens and queries
    pair = next(((live.index(s), live.index(s + 4)) for s in range(4) if s in live and s + 4 in live), None)
    if pair:
        k[pair[1]], v[pair[1]], q[pair[1]] = k[pair[0]], v[pair[0]], q[pair[0]]
    for layer in (0, L - 1):
        y = torch.empty_like(q)
        ops.kv_store_attn(k, v, q, pool, layer, y, _spec(rows, nq, hd, m))
        torch.cuda.synchronize()
        if pair:
            assert torch.equal(y[pair[0]], y[pair[1]]), "fork == source"
        sample = [0, live.index(8)]
        _check_rows(torch, pool, layer, y, q, sample, [pos[s] for s in live], live, nq, hd, f"C5 layer {layer}")
    pool.close()
