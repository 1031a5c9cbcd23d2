"""Seeded random decode / verify calls over the attention paths at once: for
each case a random pool geometry (head_dim 64/128/256, page 16/32, f16 or
bf16 KV, a short split-K partition length so that groups span many
partitions), random contexts, 1-4 rows per sequence, a random window and
soft-cap.  Checked against the CPU oracle (exact softmax in double, the
reference's kv_len / window / causal rules of attn.wgsl:78-88,169), and
bit for bit between the paths that must agree: the fused append
(thb_attn_append) against kv_store followed by attn, the device-planned
append (thb_attn_append_dplan) against both in outputs and pool bytes, the
device-planned calls (thb_dplan_*: the fixed grid and the work list) and the
no-allocation call
(thb_attn_noalloc, whose split groups are combined by the merge kernel after
the launch) against thb_attn (combined inside the launch).  A second set of
seeded calls mixes decode rows with prefill chunks (random sizes and
prefixes) and checks the work-list plan against the oracle and thb_attn."""

import ctypes
import math
import random

import numpy as np
import pytest

import oracle
from gpu_util import fill, make_pool, oracle_layer, say, scattered_alloc

pytestmark = pytest.mark.gpu

TOL = 2e-3
TIGHT = 1e-4
N_CASES = 12


def _case(seed):
    rng = random.Random(seed)
    hd = rng.choice([64, 128, 128, 256])
    nkv = rng.choice([1, 2, 4, 8])
    g = rng.choice([1, 2, 4, 7, 8])
    rps = rng.choice([1, 1, 2, 3, 4])
    if g * rps > 16:  # one query group per sequence, so the append can fuse
        rps = max(1, 16 // g)
    pl = rng.choice([16, 32])
    part_len = rng.choice([2 * pl, 128, 256, 512])
    lens = [rng.randint(rps + 1, 1500) for _ in range(rng.randint(1, 5))]
    window = rng.choice([0, 0, rng.randint(1, 600)])
    cap = rng.choice([0.0, 0.0, 30.0])
    kv = rng.choice(["f16", "bf16"])
    return dict(hd=hd, nkv=nkv, nq=g * nkv, rps=rps, pl=pl, part_len=part_len, lens=lens, window=window, cap=cap,
                kv=kv)


def _noalloc(pool, q, y, spec):
    from flint_amd import _lib, ops
    from flint_amd.pool import _stream_ptr

    c = ops._spec_c(spec, q, y)
    return _lib.lib().thb_attn_noalloc(pool.handle, 0, q.data_ptr(), y.data_ptr(), ctypes.byref(c),
                                       spec.args.handle, _stream_ptr(None))


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_calls_agree(torch_cuda, seed):
    torch = torch_cuda
    from flint_amd import _lib, ops
    from flint_amd.pool import RowMeta

    c = _case(1000 + seed)
    say("random call", seed, c)
    hd, nkv, nq, rps, pl = c["hd"], c["nkv"], c["nq"], c["rps"], c["pl"]
    budget = [n + rps for n in c["lens"]]
    pools = []
    for _ in range(3):
        P = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=pl, kv_dtype=c["kv"], extra_pages=3,
                      part_len=c["part_len"])
        scattered_alloc(P, budget, random.Random(seed), pl)
        pools.append(P)
    rows = RowMeta(256)
    for P in pools:
        fill(torch, P, rows, c["lens"], seed=seed)
    positions, seqs = [], []
    for s, n in enumerate(c["lens"]):
        positions += list(range(n, n + rps))
        seqs += [s] * rps
    m = len(seqs)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    k_new = torch.randn(m, nkv, hd, device="cuda", generator=gen).half()
    v_new = torch.randn(m, nkv, hd, device="cuda", generator=gen).half()
    q = torch.randn(m, nq, hd, device="cuda", generator=gen)
    rows.write(positions, seqs, m)
    spec = ops.AttnSpec(q_heads=nq, window=c["window"], scale=1 / math.sqrt(hd), m=m, causal=True, seq=None,
                        args=rows, softcap=c["cap"])
    ya, yb = torch.empty_like(q), torch.empty_like(q)
    ops.kv_store(k_new, v_new, pools[0], 0, m, rows)
    ops.attn(q, pools[0], 0, ya, spec)
    ops.kv_store_attn(k_new, v_new, q, pools[1], 0, yb, spec)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb), (seed, "fused append", float((ya - yb).abs().max()))
    ka, va = pools[0].read_layer(0)
    kb, vb = pools[1].read_layer(0)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb), (seed, "appended pages")
    # the same step over a device plan with the append inside the launch (one
    # group per sequence, so the plan's checks pass)
    ye = torch.full_like(q, 7.0)
    aplan = ops.DevicePlan(pools[2], max_m=m, q_heads=nq, append=True)
    aplan.build(spec, q, ye)
    aplan.attn_append(0, k_new, v_new, q, ye)
    torch.cuda.synchronize()
    aplan.close()
    pools[2].status()
    assert torch.equal(ye, ya), (seed, "device-planned append", float((ye - ya).abs().max()))
    kc, vc = pools[2].read_layer(0)
    assert np.array_equal(ka, kc) and np.array_equal(va, vc), (seed, "device-planned appended pages")

    want = oracle_layer(torch, pools[0]).attn(q.cpu().numpy(), oracle.row_meta(positions, seqs), m, nq,
                                              1 / math.sqrt(hd), window=c["window"], softcap=c["cap"])
    got = ya.cpu().numpy()
    finite = np.isfinite(want)
    assert np.array_equal(finite, np.isfinite(got)), (seed, "NaN rows differ from the oracle")
    err = float(np.max(np.abs(got[finite] - want[finite]))) if finite.any() else 0.0
    say("random call", seed, "max abs err", err)
    assert err <= TIGHT, (seed, err)

    for prefill in (False, True):  # the fixed grid and the work list
        yc = torch.full_like(q, 7.0)
        plan = ops.DevicePlan(pools[0], max_m=m, q_heads=nq, prefill=prefill)
        plan.build(spec, q, yc)
        plan.attn(0, q, yc)
        torch.cuda.synchronize()
        plan.close()
        assert torch.equal(yc, ya), (seed, "device plan", prefill, float((yc - ya).abs().max()))

    yd = torch.full_like(q, 7.0)
    rc = _noalloc(pools[0], q, yd, spec)
    if rc != 0:  # partials beyond the fixed array: refused, as documented
        msg = _lib.lib().thb_last_error().decode()
        assert rc == _lib.THB_ERR_INVALID and "scratch" in msg, (rc, msg)
        return
    torch.cuda.synchronize()
    assert torch.equal(yd, ya), (seed, "no-allocation call", float((yd - ya).abs().max()))


N_MIXED = 10


def _mixed_case(seed):
    rng = random.Random(seed)
    hd = rng.choice([64, 128, 128, 256])
    nkv = rng.choice([1, 2, 4, 8])
    g = rng.choice([1, 2, 4, 7, 8])
    pl = rng.choice([16, 32])
    part_len = rng.choice([128, 512, 1024, 2048])
    dlens = [rng.randint(2, 1500) for _ in range(rng.randint(0, 4))]
    chunks = [(rng.randint(0, 1200), rng.randint(4, 200)) for _ in range(rng.randint(1, 2))]  # (prefix, rows)
    window = rng.choice([0, 0, rng.randint(64, 900)])
    cap = rng.choice([0.0, 0.0, 30.0])
    return dict(hd=hd, nkv=nkv, nq=g * nkv, pl=pl, part_len=part_len, dlens=dlens, chunks=chunks, window=window,
                cap=cap, kv=rng.choice(["f16", "bf16"]), q16=rng.choice([True, False]))


@pytest.mark.parametrize("seed", range(N_MIXED))
def test_random_mixed_calls_list_plan(torch_cuda, seed):
    """Seeded random calls of decode rows and prefill chunks (random head_dim,
    grouping, page and partition lengths, window, soft-cap, KV type, f16 or
    f32 queries, chunk sizes and prefixes): the work-list device plan against
    the oracle (1e-4) and against thb_attn, bit for bit when every chunk's
    keys fit one partition (its blocks then run on the prefill kernel in
    both), else within 1e-5 (a block spanning partitions runs as decode
    groups in the list)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    c = _mixed_case(2000 + seed)
    say("random mixed call", seed, c)
    hd, nkv, nq, pl, PL, window = c["hd"], c["nkv"], c["nq"], c["pl"], c["part_len"], c["window"]
    lens = c["dlens"] + [p + n for p, n in c["chunks"]]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=pl, kv_dtype=c["kv"], extra_pages=3, part_len=PL)
    scattered_alloc(pool, lens, random.Random(seed), pl)
    fill(torch, pool, RowMeta(256), lens, seed=seed)
    positions = [n - 1 for n in c["dlens"]]
    seqs = list(range(len(c["dlens"])))
    exact = True
    align = max(pl, 16)
    for i, (p, n) in enumerate(c["chunks"]):
        positions += list(range(p, p + n))
        seqs += [len(c["dlens"]) + i] * n
        lo = max(0, p + 1 - window) if window else 0
        exact = exact and (p + n) - (lo - lo % align) <= PL
    m = len(seqs)
    rows = RowMeta(m)
    rows.write(positions, seqs, m)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    q = torch.randn(m, nq, hd, device="cuda", generator=gen)
    if c["q16"]:
        q = q.half()
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=1 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=c["cap"])
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    ops.attn(q, pool, 0, want, spec)
    plan = ops.DevicePlan(pool, max_m=m, q_heads=nq, prefill=True)
    plan.build(spec, q, got)
    plan.attn(0, q, got)
    torch.cuda.synchronize()
    plan.close()
    ref = oracle_layer(torch, pool).attn(q.float().cpu().numpy(), oracle.row_meta(positions, seqs), m, nq,
                                         1 / math.sqrt(hd), window=window, softcap=c["cap"])
    g_np = got.cpu().numpy()
    finite = np.isfinite(ref)
    assert np.array_equal(finite, np.isfinite(g_np)), (seed, "NaN rows differ from the oracle")
    err = float(np.max(np.abs(g_np[finite] - ref[finite]))) if finite.any() else 0.0
    say("random mixed call", seed, "exact" if exact else "split blocks", "max abs err vs oracle", err)
    assert err <= TIGHT, (seed, err)
    if exact:
        assert torch.equal(got, want), (seed, float((got - want).abs().max()))
    else:
        assert float((got - want).abs().max()) <= 1e-5, seed
