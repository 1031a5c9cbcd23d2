"""GPU parity of the device-side page allocator (free stack, reference counts,
page counts and block table in HBM) against oracle/arena.py, which restates
KvArena (reference crates/thuban_model/src/pool.rs:11-118, pinned by the
reference's tests/pool.rs) and the engine's per-plan alloc loop
(thuban_generate/src/engine.rs:197-200).  After every operation the device
state read back from HBM, the host mirror and the oracle must agree exactly:
free-stack order, reference counts and the flattened block table."""

import math
import random

import numpy as np
import pytest

from gpu_util import fill, make_pool, say, scattered_alloc
from oracle.arena import ArenaError, KvArena

pytestmark = pytest.mark.gpu


def _same_state(pool, orc, label):
    free, refs, table = pool.read_state()
    assert free == orc.free, (label, "device free stack")
    assert refs == orc.refs, (label, "device reference counts")
    assert table == orc.table(), (label, "device block table")
    assert pool.arena.free_list() == orc.free, (label, "mirror free stack")
    assert pool.arena.refs() == orc.refs, (label, "mirror reference counts")
    assert pool.arena.table() == orc.table(), (label, "mirror block table")


def _apply(label, fn_pool, fn_orc):
    """Runs one op on the product and on the oracle; both must fail with the
    same message or both succeed."""
    from flint_amd import ThubanError

    err_p = err_o = None
    try:
        fn_orc()
    except ArenaError as e:
        err_o = str(e)
    try:
        fn_pool()
    except ThubanError as e:
        err_p = str(e)
    assert err_p == err_o, (label, err_p, err_o)
    return err_o


@pytest.mark.parametrize("page_len", [16, 32])
def test_random_page_ops_match_oracle(torch_cuda, page_len):
    """300 random alloc (host API), alloc_rows (device), free, truncate and
    fork calls on a pool a little smaller than its budgets, so that the
    arena runs out now and then; every state is compared."""
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    rng = random.Random(100 + page_len)
    n_seq = 12
    lens = [rng.randrange(40, 320) for _ in range(n_seq)]
    pages = int(0.6 * sum(-(-n // page_len) for n in lens))
    pool = KvPool(ArenaSpec(lens, pages), 2, 64, layers=2, page_len=page_len, kv_dtype="f16")
    orc = KvArena(lens, pages=pages, page_len=page_len)
    rows = RowMeta(64)
    pos = [0] * n_seq  # tokens each sequence holds
    kinds = ["alloc", "rows", "rows", "rows", "free", "truncate", "fork"]
    counts = {k: 0 for k in kinds}
    errors = 0
    for it in range(300):
        kind = rng.choice(kinds)
        label = f"op {it} {kind}"
        if kind == "alloc":
            s = rng.randrange(n_seq)
            n = rng.randrange(0, 40)
            err = _apply(label, lambda: pool.alloc(s, pos[s], n), lambda: orc.alloc(s, pos[s], n))
            if err is None:
                pos[s] += n
        elif kind == "rows":
            chosen = rng.sample(range(n_seq), rng.randrange(1, 6))
            positions, seqs = [], []
            for s in chosen:
                k = rng.choice([1, 1, 1, 2, 4, 17])
                positions += list(range(pos[s], pos[s] + k))
                seqs += [s] * k
            rows.write(positions, seqs, len(seqs))
            err = _apply(label, lambda: pool.alloc_rows(rows, len(seqs)), lambda: orc.alloc_rows(positions, seqs))
            for s in chosen:  # runs before a failure keep their pages
                pos[s] = min(len(orc.tables[s]) * page_len, pos[s] + seqs.count(s)) if err else pos[s] + seqs.count(s)
        elif kind == "free":
            s = rng.randrange(n_seq)
            _apply(label, lambda: pool.free_seq(s), lambda: orc.free_seq(s))
            pos[s] = 0
        elif kind == "truncate":
            s = rng.randrange(n_seq)
            keep = rng.randrange(0, pos[s] + 1)
            _apply(label, lambda: pool.truncate(s, keep), lambda: orc.truncate(s, keep))
            pos[s] = min(pos[s], keep)
        else:
            src = rng.randrange(n_seq)
            empty = [s for s in range(n_seq) if not orc.tables[s] and s != src]
            if not empty or pos[src] == 0:
                continue
            dst = rng.choice(empty)
            t = rng.randrange(1, pos[src] + 1)
            err = _apply(label, lambda: pool.fork(src, dst, t), lambda: orc.fork(src, dst, t))
            if err is None:
                pos[dst] = t
        counts[kind] += 1
        errors += err is not None
        orc.copies.clear()
        _same_state(pool, orc, label)
        orc.check_invariants()
    say("page ops", counts, "errors", errors)
    assert errors > 0 and all(counts[k] > 0 for k in kinds)


def test_alloc_rows_failure_status_and_pull(torch_cuda):
    """A call that runs out of pages: the runs before the failing one keep
    their pages (engine.rs's `?`), the message is the reference's, the
    device records the same failure (thb_pool_status), and reloading the
    mirror from the device changes nothing."""
    from flint_amd import ThubanError
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    lens = [64, 64, 64, 64]
    pool = KvPool(ArenaSpec(lens, 4), 2, 64, page_len=16, kv_dtype="f16")
    orc = KvArena(lens, pages=4, page_len=16)
    rows = RowMeta(64)
    positions = list(range(0, 20)) + list(range(0, 33)) + list(range(0, 5))
    seqs = [2] * 20 + [0] * 33 + [3] * 5
    rows.write(positions, seqs, len(seqs))
    with pytest.raises(ArenaError) as eo:
        orc.alloc_rows(positions, seqs)
    with pytest.raises(ThubanError) as ep:
        pool.alloc_rows(rows, len(seqs))
    assert str(ep.value) == str(eo.value) == "KV arena exhausted: 3 pages requested, 2 free"
    assert ep.value.kind == "Model"
    with pytest.raises(ThubanError) as es:
        pool.status()
    assert str(es.value) == str(eo.value)
    pool.status()  # cleared
    _same_state(pool, orc, "after failure")
    before = (pool.arena.free_list(), pool.arena.refs(), pool.arena.table())
    pool.pull()
    assert (pool.arena.free_list(), pool.arena.refs(), pool.arena.table()) == before
    # the context limit, on the device too
    rows.write([60, 61, 62, 63, 64], [1] * 5, 5)
    with pytest.raises(ThubanError) as ep:
        pool.alloc_rows(rows, 5)
    assert str(ep.value) == "context limit 64 reached"
    with pytest.raises(ThubanError) as es:
        pool.status()
    assert str(es.value) == "context limit 64 reached"
    # one run per sequence
    rows.write([0, 0, 1], [1, 3, 1], 3)
    with pytest.raises(ThubanError) as ep:
        pool.alloc_rows(rows, 3)
    assert ep.value.kind == "Invalid"


def test_copy_on_write_through_alloc_rows(torch_cuda):
    """fork shares full pages; after a truncate back into a shared page,
    alloc_rows copies it (copy-on-write of the slots below the write) before
    the append, so the fork's prefix equals its source's and the source is
    untouched by the fork's new tokens."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    lens = [96, 96]
    pool = KvPool(ArenaSpec(lens, 16), 2, 64, layers=2, page_len=16, kv_dtype="f16")
    rows = RowMeta(128)
    pool.alloc(0, 0, 48)
    fill(torch, pool, rows, [48, 0], layer=0, seed=3)
    fill(torch, pool, rows, [48, 0], layer=1, seed=4)
    pool.fork(0, 1, 48)  # three shared full pages
    pool.truncate(1, 20)  # seq 1 keeps two pages, the second shared with seq 0
    shared = pool.arena.table_of(1)[1]
    assert pool.arena.refs()[shared] == 2
    rows.write([20, 21], [1, 1], 2)
    pool.alloc_rows(rows, 2)
    t1 = pool.arena.table_of(1)
    assert t1[1] != shared and pool.arena.refs()[shared] == 1
    orc = KvArena(lens, pages=16, page_len=16)
    orc.alloc(0, 0, 48)
    orc.fork(0, 1, 48)
    orc.truncate(1, 20)
    orc.alloc_rows([20, 21], [1, 1])
    assert orc.copies == [(shared, t1[1], 4)]
    orc.copies.clear()
    _same_state(pool, orc, "copy-on-write")
    for layer in range(2):
        k = torch.randn(2, 2, 64, device="cuda").half()
        ops.kv_store(k, k, pool, layer, 2, rows)
        kd = torch.empty(1, 2, 48, 64, dtype=torch.int16, device="cuda")
        vd = torch.empty_like(kd)
        ops.kv_gather(pool, layer, 0, 0, 48, kd[0], vd[0])
        k1 = torch.empty(2, 22, 64, dtype=torch.int16, device="cuda")
        v1 = torch.empty_like(k1)
        ops.kv_gather(pool, layer, 1, 0, 22, k1, v1)
        torch.cuda.synchronize()
        assert torch.equal(k1[:, :20], kd[0, :, :20]) and torch.equal(v1[:, :20], vd[0, :, :20])
        assert torch.equal(k1[:, 20:22], k.view(torch.int16).transpose(0, 1))
        assert not torch.equal(kd[0, :, 20:22], k1[:, 20:22])


def test_decode_steps_with_device_alloc_bit_identical(torch_cuda):
    """Llama-3-8B heads, 8 sequences crossing page boundaries: twenty steps
    of (alloc_rows on the device + fused append + attention) give outputs,
    tables and pool contents bit-identical to (host page API + the same
    call)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    B, nq, nkv, hd, P, T = 8, 32, 8, 128, 16, 20
    rng = random.Random(77)
    ctx = [rng.randrange(100, 400) for _ in range(B)]
    budget = [c + T for c in ctx]
    pools = []
    for _ in range(2):
        pool = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16", extra_pages=8)
        scattered_alloc(pool, ctx, random.Random(5), P)
        pools.append(pool)
    rows = [RowMeta(B), RowMeta(B)]
    fill_rows = RowMeta(256)
    for pool in pools:
        fill(torch, pool, fill_rows, ctx, seed=21)
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    pos = list(ctx)
    for step in range(T):
        k = torch.randn(B, nkv, hd, device="cuda", generator=g).half()
        v = torch.randn(B, nkv, hd, device="cuda", generator=g).half()
        q = torch.randn(B, nq, hd, device="cuda", generator=g).half()
        ys = []
        for i, pool in enumerate(pools):
            rows[i].write(pos, list(range(B)), B)
            if i == 0:
                for s in range(B):
                    pool.alloc(s, pos[s], 1)
            else:
                pool.alloc_rows(rows[i], B)
            y = torch.empty_like(q)
            spec = ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=B, causal=True, seq=None,
                                args=rows[i])
            ops.kv_store_attn(k, v, q, pool, 0, y, spec)
            ys.append(y)
        torch.cuda.synchronize()
        assert torch.equal(ys[0], ys[1]), step
        assert pools[0].arena.table() == pools[1].arena.table() == pools[1].read_state()[2], step
        pos = [p + 1 for p in pos]
    ka, va = pools[0].read_layer(0)
    kb, vb = pools[1].read_layer(0)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    say("device-alloc decode steps", T, "pages used", pools[1].arena.used())


def test_scatter_refuses_shared_pages_and_copy_fans_out(torch_cuda):
    """kv_scatter writes in place, so a page another sequence holds (a fork's
    shared prefix) is refused; block_copy may read one source page into
    several destinations."""
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    pool = KvPool(ArenaSpec([64, 64, 64], 12), 2, 64, page_len=16, kv_dtype="f16")
    rows = RowMeta(64)
    pool.alloc(0, 0, 40)
    fill(torch, pool, rows, [40, 0, 0], seed=6)
    pool.fork(0, 1, 32)
    buf = torch.zeros(2, 8, 64, dtype=torch.int16, device="cuda")
    with pytest.raises(ThubanError) as e:
        ops.kv_scatter(pool, 0, 1, 8, 8, buf, buf)
    assert "shared" in str(e.value) and e.value.kind == "Model"
    pool.alloc(2, 0, 48)
    pool.sync()
    src = pool.arena.table_of(0)[0]
    d1, d2 = pool.arena.table_of(2)[1], pool.arena.table_of(2)[2]
    ops.block_copy(pool, [(src, d1, 16), (src, d2, 16)])
    with pytest.raises(ThubanError):
        ops.block_copy(pool, [(src, d1, 16), (d1, d2, 16)])  # d1 read and written
    with pytest.raises(ThubanError):
        ops.block_copy(pool, [(src, d1, 16), (d2, d1, 16)])  # d1 written twice
    k = torch.empty(2, 48, 64, dtype=torch.int16, device="cuda")
    v = torch.empty_like(k)
    ops.kv_gather(pool, 0, 2, 0, 48, k, v)
    k0 = torch.empty(2, 16, 64, dtype=torch.int16, device="cuda")
    v0 = torch.empty_like(k0)
    ops.kv_gather(pool, 0, 0, 0, 16, k0, v0)
    torch.cuda.synchronize()
    for j in (1, 2):
        assert torch.equal(k[:, 16 * j:16 * j + 16], k0) and torch.equal(v[:, 16 * j:16 * j + 16], v0)
