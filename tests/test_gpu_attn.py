"""GPU parity of paged attention against the CPU oracle (exact softmax in
double): within 2e-3 max abs (the north-star tolerance for f16 outputs of
an fp32-accumulating reference), plus bit-exact invariants (paged ==
contiguous, batch == solo, repeatability) from the reference's
tests/batch.rs:163-347."""

import math
import random
import zlib

import numpy as np
import pytest

import oracle
from gpu_util import fill, make_pool, oracle_layer, say, scattered_alloc

pytestmark = pytest.mark.gpu

TOL = 2e-3
# The kernels multiply with both f16 (bf16) halves of the query and of the
# probabilities, so their products are f32-grade: with f32 outputs they stay
# within 1e-4 of the exact softmax (measured 3e-7 .. 1.1e-5).  The reference
# contract is TOL; TIGHT catches a lost low half or a lossy rescaling.
TIGHT = 1e-4


def run_attn(torch, pool, rows, q, positions, seqs, spec_seq=None, window=0, causal=True, softcap=0.0,
             scale=None, y_dtype=None, layer=0, row_off=0):
    from flint_amd import ops

    m, nq, hd = q.shape
    rows.write(positions, seqs, len(positions))
    y = torch.empty(m, nq, hd, device="cuda", dtype=y_dtype or torch.float32)
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=scale or 1.0 / math.sqrt(hd), m=m, causal=causal,
                        seq=spec_seq, args=rows, row_off=row_off, softcap=softcap)
    ops.attn(q, pool, layer, y, spec)
    torch.cuda.synchronize()
    return y


def check_parity(torch, pool, rows, q, positions, seqs, label, **kw):
    y = run_attn(torch, pool, rows, q, positions, seqs, **kw)
    ref = oracle_layer(torch, pool, kw.get("layer", 0))
    m, nq, hd = q.shape
    want = ref.attn(q.float().cpu().numpy(), oracle.row_meta(positions, seqs), m, nq,
                    kw.get("scale") or 1.0 / math.sqrt(hd), window=kw.get("window", 0),
                    causal=kw.get("causal", True), seq=kw.get("spec_seq"), softcap=kw.get("softcap", 0.0))
    got = y.float().cpu().numpy()
    err = float(np.max(np.abs(got - want)))
    say(label, "max abs err", err)
    assert np.all(np.isfinite(got)), label
    assert err <= TOL, (label, err)
    if y.dtype == torch.float32:
        assert err <= TIGHT, (label, "precision regression", err)
    return y


CASES = [
    # name, nq, nkv, hd, page_len, kv, lens
    ("qwen2-0.5b", 14, 2, 64, 16, "bf16", [128, 512, 300, 201]),
    ("qwen2-0.5b-p32", 14, 2, 64, 32, "f16", [130, 420, 511, 256]),
    ("llama3-8b", 32, 8, 128, 16, "f16", [1500, 513, 2048, 77]),
    ("llama3-8b-bf16", 32, 8, 128, 16, "bf16", [900, 1025]),
    ("qwen2.5-32b", 40, 8, 128, 16, "f16", [1200, 700]),
    ("gemma2-9b", 16, 8, 256, 16, "f16", [1300, 600]),
    ("hd80", 8, 2, 80, 16, "f16", [333, 40]),
    ("hd512", 8, 2, 512, 16, "f16", [700, 100]),
    ("mqa-g16", 16, 1, 128, 32, "f16", [640, 50]),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_batched_parity(torch_cuda, case):
    torch = torch_cuda
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, pl, kv, lens = case
    say("decode", name)
    rng = random.Random(zlib.crc32(name.encode()))
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=pl, kv_dtype=kv, extra_pages=7)
    scattered_alloc(pool, lens, rng, pl)
    rows = RowMeta(256)
    fill(torch, pool, rows, lens, seed=1)
    B = len(lens)
    q = torch.randn(B, nq, hd, device="cuda")
    positions = [n - 1 for n in lens]
    check_parity(torch, pool, rows, q, positions, list(range(B)), name)
    # f16 in / f16 out
    check_parity(torch, pool, rows, q.half(), positions, list(range(B)), name + "-f16io", y_dtype=torch.float16)


def test_window_and_softcap_gemma(torch_cuda):
    torch = torch_cuda
    from flint_amd.pool import RowMeta

    lens = [1500, 900]
    pool = make_pool(lens, kv_heads=8, head_dim=256, page_len=16, kv_dtype="f16", extra_pages=4)
    scattered_alloc(pool, lens, random.Random(2), 16)
    rows = RowMeta(64)
    fill(torch, pool, rows, lens, seed=2, scale=3.0)
    q = torch.randn(2, 16, 256, device="cuda") * 2
    for window in (0, 64, 700, 4096):
        check_parity(torch, pool, rows, q, [1499, 899], [0, 1], f"gemma window={window}", window=window,
                     softcap=50.0, scale=1.0 / 16)


def test_speculative_verify_rows(torch_cuda):
    """4 causal query rows per sequence (draft verify), batched."""
    torch = torch_cuda
    from flint_amd.pool import RowMeta

    lens = [700, 1031, 64]
    pool = make_pool(lens, kv_heads=8, head_dim=256, page_len=16, kv_dtype="f16", extra_pages=2)
    scattered_alloc(pool, lens, random.Random(3), 16)
    rows = RowMeta(64)
    fill(torch, pool, rows, lens, seed=3)
    positions, seqs = [], []
    for s, n in enumerate(lens):
        positions += [n - 4 + i for i in range(4)]
        seqs += [s] * 4
    q = torch.randn(len(seqs), 16, 256, device="cuda")
    check_parity(torch, pool, rows, q, positions, seqs, "verify m=4", window=512)


@pytest.mark.parametrize("causal", [True, False])
def test_reference_mode_chunk(torch_cuda, causal):
    """AttnSpec.seq fixed (one dispatch per sequence chunk, forward.rs:316-336):
    a 40-row prefill chunk with the reference's 8-row kv_len rule."""
    torch = torch_cuda
    from flint_amd.pool import RowMeta

    lens = [300, 520]
    pool = make_pool(lens, kv_heads=2, head_dim=64, page_len=32, kv_dtype="bf16")
    scattered_alloc(pool, lens, random.Random(4), 32)
    rows = RowMeta(128)
    fill(torch, pool, rows, lens, seed=4)
    m = 40
    positions = list(range(520 - m, 520))
    q = torch.randn(m, 14, 64, device="cuda")
    # the call's rows sit at row_off 5 of the row meta (forward.rs:332)
    from flint_amd import ops

    rows.write([0] * 5 + positions, [0] * 5 + [1] * m, 5 + m)
    y = torch.empty_like(q)
    ops.attn(q, pool, 0, y, ops.AttnSpec(q_heads=14, window=0, scale=0.125, m=m, causal=causal, seq=1,
                                          args=rows, row_off=5))
    torch.cuda.synchronize()
    want = oracle_layer(torch, pool).attn(q.cpu().numpy(), oracle.row_meta(positions, [1] * m), m, 14, 0.125,
                                          causal=causal, seq=1)
    err = float(np.max(np.abs(y.cpu().numpy() - want)))
    say("reference-mode chunk causal", causal, err)
    assert err <= TOL
    if y.dtype == torch.float32:
        assert err <= TIGHT, ("reference-mode chunk", "precision regression", err)


def test_empty_key_range_is_nan(torch_cuda):
    """A row with no valid key: reference mode, causal, window 5, a chunk
    whose second row (position 10) sets the 8-row block's kv_len to 11 while
    the first row (position 100) starts its window at 96.  attn.wgsl divides
    0 by 0 there (NaN); the other row stays finite and matches the oracle."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    lens = [128]
    pool = make_pool(lens, kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16")
    scattered_alloc(pool, lens, random.Random(9), 16)
    rows = RowMeta(8)
    fill(torch, pool, rows, lens, seed=9)
    positions, seqs = [100, 10], [0, 0]
    q = torch.randn(2, 4, 64, device="cuda")
    rows.write(positions, seqs, 2)
    y = torch.empty_like(q)
    ops.attn(q, pool, 0, y, ops.AttnSpec(q_heads=4, window=5, scale=0.125, m=2, causal=True, seq=0, args=rows))
    torch.cuda.synchronize()
    want = oracle_layer(torch, pool).attn(q.cpu().numpy(), oracle.row_meta(positions, seqs), 2, 4, 0.125,
                                          window=5, causal=True, seq=0)
    got = y.cpu().numpy()
    say("empty key range", got[0, 0, :2], want[0, 0, :2])
    assert np.isnan(want[0]).all() and np.isnan(got[0]).all()
    assert np.isfinite(got[1]).all()
    assert float(np.max(np.abs(got[1] - want[1]))) <= TIGHT


def test_reference_anchor_through_gpu(torch_cuda, golden):
    """anchor_attn_causal_and_window (kernels.rs:1439-1481) embedded in the
    first two dims of a head_dim-64 pool: [2, 3] full, [3, 4] window 1."""
    torch = torch_cuda
    from flint_amd.pool import RowMeta

    for case in golden("attn_cases.json"):
        pool = make_pool([2], kv_heads=1, head_dim=64, page_len=16, kv_dtype="bf16")
        pool.alloc(0, 0, 2)
        rows = RowMeta(4)
        rows.write([0, 1], [0, 0], 2)
        k = torch.zeros(2, 1, 64, device="cuda")
        v = torch.zeros(2, 1, 64, device="cuda")
        k[:, 0, :2] = torch.tensor(case["k"]).view(2, 2)
        v[:, 0, :2] = torch.tensor(case["v"]).view(2, 2)
        from flint_amd import ops

        ops.kv_store(k, v, pool, 0, 2, rows)
        q = torch.zeros(1, 1, 64, device="cuda")
        q[0, 0, :2] = torch.tensor(case["q"])
        y = run_attn(torch, pool, rows, q, [case["pos"]], [0], window=case["window"], scale=1 / math.sqrt(2))
        got = y[0, 0, :2].cpu().numpy()
        say("anchor", case["name"], got)
        assert np.allclose(got, case["expect"], atol=1e-6)


def test_invariants_bit_exact(torch_cuda):
    """paged == contiguous, batch == solo, identical sequences give identical
    outputs, repeat runs are identical (batch.rs:163-347)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    lens = [1800, 1800, 650]
    rng = random.Random(9)
    # pool A: scattered pages; pool B: same data, pages in a different order
    A = make_pool(lens, kv_heads=8, head_dim=128, page_len=16, kv_dtype="f16", extra_pages=9)
    B = make_pool(lens, kv_heads=8, head_dim=128, page_len=16, kv_dtype="f16", extra_pages=9)
    scattered_alloc(A, lens, rng, 16)
    B.alloc(2, 0, 650)  # different order, different physical pages
    B.alloc(1, 0, 1800)
    B.alloc(0, 0, 1800)
    rows = RowMeta(256)
    fill(torch, A, rows, [1800, 0, 650], seed=5)
    fill(torch, B, rows, [1800, 0, 650], seed=5)
    # seq 1 := copy of seq 0 (identical sequence), through gather/scatter
    kd = torch.empty(8, 1800, 128, dtype=torch.int16, device="cuda")
    vd = torch.empty_like(kd)
    for P in (A, B):
        ops.kv_gather(P, 0, 0, 0, 1800, kd, vd)
        ops.kv_scatter(P, 0, 1, 0, 1800, kd, vd)
    q = torch.randn(3, 32, 128, device="cuda")
    q[1] = q[0]
    pos, seqs = [1799, 1799, 649], [0, 1, 2]
    ya = run_attn(torch, A, rows, q, pos, seqs)
    yb = run_attn(torch, B, rows, q, pos, seqs)
    assert torch.equal(ya, yb), "paged == contiguous"
    assert torch.equal(ya[0], ya[1]), "identical sequences"
    solo = run_attn(torch, A, rows, q[2:3].contiguous(), [649], [2])
    assert torch.equal(solo[0], ya[2]), "batch == solo"
    again = run_attn(torch, A, rows, q, pos, seqs)
    assert torch.equal(again, ya), "repeatable"


SPLIT_CASES = [
    # name, nq, nkv, hd, kv, lens, part_len, window, softcap
    ("hd128-32-partitions", 32, 8, 128, "f16", [1100, 700, 64, 300], 64, 0, 0.0),
    ("hd256-window-softcap", 16, 8, 256, "f16", [2100, 900], 256, 1000, 50.0),
    ("hd512-tree-merge", 8, 2, 512, "f16", [900, 400], 128, 0, 0.0),
    ("g32-head-split-bf16", 32, 1, 128, "bf16", [800, 333], 128, 0, 0.0),
    # spans a few keys over 2 and 4 pieces of 1024 (2 and 4 longer partitions) and one key past
    # that tolerance (4 partitions)
    ("hd128-span-tolerance", 32, 8, 128, "f16", [2050, 2081, 2080, 4100], 1024, 0, 0.0),
]


def _attn_noalloc(torch, pool, q, y, spec):
    import ctypes

    from flint_amd import _lib, ops
    from flint_amd.pool import _stream_ptr

    c = ops._spec_c(spec, q, y)
    rc = _lib.lib().thb_attn_noalloc(pool.handle, 0, q.data_ptr(), y.data_ptr(), ctypes.byref(c), spec.args.handle,
                                     _stream_ptr(None))
    assert rc == 0, _lib.lib().thb_last_error().decode()
    torch.cuda.synchronize()


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_split_groups_combined_in_launch(torch_cuda, case):
    """Decode groups split over many partitions are combined by the
    workgroup of each group's last partition (thb_attn): parity with the
    oracle, and bit-identical to the combination by the merge kernel after
    the launch (thb_attn_noalloc), over calls of different shapes in a row
    (the arrival counters are left at zero for the next call)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, kv, lens, part_len, window, cap = case
    say("split groups", name)
    rng = random.Random(zlib.crc32(name.encode()))
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=7, part_len=part_len)
    scattered_alloc(pool, lens, rng, 16)
    rows = RowMeta(256)
    fill(torch, pool, rows, lens, seed=41)
    g = torch.Generator(device="cuda")
    g.manual_seed(41)
    n = len(lens)
    calls = [(list(range(n)), [x - 1 for x in lens]),
             ([0, 0, 0, 0], [lens[0] - 4 + i for i in range(4)]),  # a 4-row verify chunk
             ([n - 1, 0], [lens[-1] // 2, lens[0] - 1]),
             (list(range(n)), [x - 1 for x in lens])]
    for i, (seqs, positions) in enumerate(calls):
        m = len(seqs)
        q = torch.randn(m, nq, hd, device="cuda", generator=g)
        y = check_parity(torch, pool, rows, q, positions, seqs, f"{name} call {i}", window=window, softcap=cap)
        spec = ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None,
                            args=rows, softcap=cap)
        y2 = torch.full_like(y, float("nan"))
        _attn_noalloc(torch, pool, q, y2, spec)
        assert torch.equal(y, y2), (name, i, float((y - y2).abs().max()))


def test_llama3_full_shape(torch_cuda):
    """BASELINE config 2 at full size (B=32, ctx 4096, 32q/8kv/hd128, f16 KV,
    scattered block tables): the oracle checks all 32 sequences in full, and
    every output is a convex combination of V (|y| <= max |V|)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    B, ctx = 32, 4096
    lens = [ctx] * B
    pool = make_pool(lens, kv_heads=8, head_dim=128, page_len=16, kv_dtype="f16")
    scattered_alloc(pool, lens, random.Random(10), 16)
    k, v = pool.layer_tensors(0)
    g = torch.Generator(device="cuda")
    g.manual_seed(10)
    k.view(torch.float16).copy_(torch.randn(k.shape, device="cuda", generator=g).half())
    v.view(torch.float16).copy_(torch.randn(v.shape, device="cuda", generator=g).half())
    rows = RowMeta(64)
    q = torch.randn(B, 32, 128, device="cuda")
    say("llama3 full shape")
    y = run_attn(torch, pool, rows, q, [ctx - 1] * B, list(range(B)))
    assert float(y.abs().max()) <= float(v.view(torch.float16).abs().max()) + 1e-3
    ref = oracle_layer(torch, pool)
    want = ref.attn(q.cpu().numpy(), oracle.row_meta([ctx - 1] * B, list(range(B))), B, 32, 1 / math.sqrt(128))
    errs = np.max(np.abs(y.cpu().numpy() - want).reshape(B, -1), axis=1)
    say("llama3 full shape: max |gpu - oracle| per sequence", float(errs.min()), "...", float(errs.max()))
    assert float(errs.max()) <= TOL
    if y.dtype == torch.float32:
        assert float(errs.max()) <= TIGHT, ("llama3 full shape", "precision regression", float(errs.max()))


def test_attn_errors(torch_cuda):
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    pool = make_pool([100], kv_heads=2, head_dim=64, page_len=16)
    pool.alloc(0, 0, 40)
    rows = RowMeta(4)
    q = torch.zeros(1, 4, 64, device="cuda")
    y = torch.empty_like(q)
    rows.write([60], [0], 1)
    with pytest.raises(ThubanError) as e:
        ops.attn(q, pool, 0, y, ops.AttnSpec(4, 0, 0.125, 1, True, None, rows))
    assert "pages must cover" in str(e.value)
    with pytest.raises(ThubanError):
        ops.attn(q, pool, 0, y, ops.AttnSpec(3, 0, 0.125, 1, True, None, rows))  # 3 % 2 != 0
    rows.write([39], [0], 1)
    ops.attn(q, pool, 0, y, ops.AttnSpec(4, 0, 0.125, 1, True, None, rows))
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()


FUSE_CASES = [
    # name, nq, nkv, hd, kv, src dtype, rows per sequence, fused in one launch
    ("decode-llama3-f16", 32, 8, 128, "f16", "f16", 1, True),
    ("decode-qwen2-bf16-f32src", 14, 2, 64, "bf16", "f32", 1, True),
    ("verify4-gemma2", 16, 8, 256, "f16", "f32", 4, True),
    # 32 query heads per KV head: each row is two query groups in two
    # workgroups, and both store the row's token (the same bytes)
    ("decode-mqa32-two-groups", 32, 1, 128, "f16", "f16", 1, True),
    ("prefill40-fallback", 8, 2, 128, "f16", "bf16", 40, False),
    # verify chunks of 8 rows (two groups of 4 query heads per row), and of
    # 16 rows at head_dim 256: 1024 append items per group, more than the
    # first pass over the wave's lanes takes
    ("verify8-g2-f32src", 16, 8, 128, "f16", "f32", 8, True, [704, 1496, 41]),
    ("verify16-hd256", 8, 8, 256, "f16", "f16", 16, True, [512, 1200, 47]),
]


@pytest.mark.parametrize("case", FUSE_CASES, ids=[c[0] for c in FUSE_CASES])
def test_fused_append_matches_separate_calls(torch_cuda, case):
    """kv_store_attn (thb_attn_append) gives bit-identical outputs and pool
    contents to kv_store followed by attn, whether it fuses or falls back."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, kv, src, rps, _ = case[:8]
    say("fused append", name)
    lens = case[8] if len(case) > 8 else [700, 1500, 33]  # tokens already in the cache
    budget = [n + rps for n in lens]
    pools = []
    for _ in range(2):
        P = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=3)
        scattered_alloc(P, budget, random.Random(zlib.crc32(name.encode())), 16)
        pools.append(P)
    rows = RowMeta(256)
    for P in pools:
        fill(torch, P, rows, lens, seed=7)
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[src]
    positions, seqs = [], []
    for s, n in enumerate(lens):
        positions += list(range(n, n + rps))
        seqs += [s] * rps
    m = len(seqs)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    k_new = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    v_new = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    q = torch.randn(m, nq, hd, device="cuda", generator=g)
    rows.write(positions, seqs, m)
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows)
    ya = torch.empty_like(q)
    yb = torch.empty_like(q)
    ops.kv_store(k_new, v_new, pools[0], 0, m, rows)
    ops.attn(q, pools[0], 0, ya, spec)
    ops.kv_store_attn(k_new, v_new, q, pools[1], 0, yb, spec)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)
    ka, va = pools[0].read_layer(0)
    kb, vb = pools[1].read_layer(0)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # and the output is right: oracle over the appended cache
    want = oracle_layer(torch, pools[1]).attn(q.cpu().numpy(), oracle.row_meta(positions, seqs), m, nq,
                                              1 / math.sqrt(hd))
    err = float(np.max(np.abs(yb.cpu().numpy() - want)))
    say("fused append", name, "max abs err", err)
    assert err <= TOL
    if yb.dtype == torch.float32:
        assert err <= TIGHT, (name, "precision regression", err)


@pytest.mark.parametrize("hd,nq,nkv", [(128, 32, 8), (64, 14, 2), (256, 16, 8)])
def test_prefill_f16_query_bit_identical_to_f32(torch_cuda, hd, nq, nkv):
    """An f16 query against f16 keys takes the prefill kernels that skip the
    products of the query's low half (exactly zero after the split).  The
    output must equal, bit for bit, the same call with the query widened to
    f32 (the kernels that compute those products): a call mixing decode rows
    with a prefill chunk (one launch), and the chunk alone."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    say("f16 query == f32 query", hd)
    rng = random.Random(hd)
    lens = [1400, 777, 2100]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", extra_pages=3)
    scattered_alloc(pool, lens, rng, 16)
    rows = RowMeta(256)
    fill(torch, pool, rows, lens, seed=hd)
    ref = oracle_layer(torch, pool)
    positions = list(range(1200, 1400)) + [776, 2099]
    seqs = [0] * 200 + [1, 2]
    g = torch.Generator(device="cuda")
    g.manual_seed(hd)
    q16 = torch.randn(len(seqs), nq, hd, device="cuda", generator=g).half()
    scale = 1.0 / math.sqrt(hd)
    for m in (len(seqs), 200):  # mixed call, then the chunk alone
        rows.write(positions[:m], seqs[:m], m)
        spec = ops.AttnSpec(q_heads=nq, window=0, scale=scale, m=m, causal=True, seq=None, args=rows)
        y16 = torch.empty(m, nq, hd, device="cuda")
        y32 = torch.empty_like(y16)
        ops.attn(q16[:m].contiguous(), pool, 0, y16, spec)
        ops.attn(q16[:m].float().contiguous(), pool, 0, y32, spec)
        torch.cuda.synchronize()
        assert torch.equal(y16, y32), (hd, m)
        want = ref.attn(q16[:m].float().cpu().numpy(), oracle.row_meta(positions[:m], seqs[:m]), m, nq, scale)
        sample = [0, 1, 63, 64, 150, 199] + list(range(200, m))
        err = float(np.max(np.abs(y16.cpu().numpy()[sample] - want[sample])))
        say("f16 query", hd, m, "max abs err", err)
        assert err <= TIGHT


PREFILL_CASES = [
    # name, nq, nkv, hd, page_len, kv, prefix tokens, chunk rows, window, softcap
    ("llama-long-prefix", 32, 8, 128, 16, "f16", 9000, 300, 0, 0.0),
    ("gemma-window-softcap", 16, 8, 256, 16, "f16", 5000, 200, 4096, 50.0),
    ("qwen2-page8-bf16", 14, 2, 64, 8, "bf16", 100, 150, 0, 0.0),
    ("hd512-page32", 8, 2, 512, 32, "f16", 333, 70, 0, 0.0),
    ("mqa32-head-split", 32, 1, 128, 32, "f16", 700, 64, 0, 0.0),
    # the head_dim <= 128 kernel with soft-cap and a window, and with bf16 probabilities split in two
    ("hd128-window-softcap", 32, 8, 128, 16, "f16", 3000, 200, 1024, 30.0),
    ("hd64-bf16-softcap-split", 8, 2, 64, 16, "bf16", 6000, 130, 0, 20.0),
    # a score scale above 1 / log2(e): the query carries it times 2^-1
    ("hd128-scale-above-one", 32, 8, 128, 16, "f16", 500, 100, 0, 0.0, 1.0),
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_chunked_prefill_parity(torch_cuda, case):
    """A causal chunk of rows appended after a prefix (chunked prefill),
    batched with a decode row of another sequence: sampled rows against the
    oracle; the chunk alone is bit-identical to the batch."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, pl, kv, prefix, chunk, window, cap = case[:10]
    say("prefill", name)
    rng = random.Random(zlib.crc32(name.encode()))
    lens = [prefix + chunk, 777]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=pl, kv_dtype=kv, extra_pages=5)
    scattered_alloc(pool, lens, rng, pl)
    rows = RowMeta(max(chunk + 1, 256))
    fill(torch, pool, rows, [prefix, 776], seed=21, scale=2.0 if cap else 1.0)
    positions = list(range(prefix, prefix + chunk)) + [776]
    seqs = [0] * chunk + [1]
    m = len(seqs)
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    k = torch.randn(m, nkv, hd, device="cuda", generator=g)
    v = torch.randn(m, nkv, hd, device="cuda", generator=g)
    q = torch.randn(m, nq, hd, device="cuda", generator=g) * (2.0 if cap else 1.0)
    scale = case[10] if len(case) > 10 else 1.0 / math.sqrt(hd)
    rows.write(positions, seqs, m)
    y = torch.empty_like(q)
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=scale, m=m, causal=True, seq=None, args=rows,
                        softcap=cap)
    ops.kv_store_attn(k, v, q, pool, 0, y, spec)
    torch.cuda.synchronize()
    ref = oracle_layer(torch, pool)
    sample = sorted(set([0, 1, 2, 7, 8, 15, 16, chunk // 2, chunk - 2, chunk - 1, chunk] +
                        rng.sample(range(chunk), min(8, chunk))))
    meta = oracle.row_meta(positions, seqs)
    want = ref.attn(q.cpu().numpy(), meta, m, nq, scale, window=window, softcap=cap)
    got = y.cpu().numpy()
    err = float(np.max(np.abs(got[sample] - want[sample])))
    say("prefill", name, "max abs err", err)
    assert np.all(np.isfinite(got)) and err <= TOL
    assert err <= TIGHT, (name, "precision regression")
    # the chunk alone (rows already appended) is bit-identical
    rows.write(positions[:chunk], seqs[:chunk], chunk)
    ys = torch.empty(chunk, nq, hd, device="cuda")
    ops.attn(q[:chunk].contiguous(), pool, 0, ys, ops.AttnSpec(q_heads=nq, window=window, scale=scale, m=chunk,
                                                              causal=True, seq=None, args=rows, softcap=cap))
    torch.cuda.synchronize()
    assert torch.equal(ys, y[:chunk]), "batch == solo"


def test_gemma2_prefill_chunks(torch_cuda):
    """Gemma-2-9B geometry (16q/8kv/hd256, window 4096, soft-cap 50): eight
    fresh 512-token causal chunks in one call, the head_dim-256 path of
    attn_prefill_wide (pairs of 64-row blocks, 16x16x32 products).  Three
    chunks in full against the oracle; one chunk called alone is
    bit-identical to the batch."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd, n, pre = 16, 8, 256, 8, 512
    lens = [pre] * n
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16")
    scattered_alloc(pool, lens, random.Random(2024), 16)
    rows = RowMeta(n * pre)
    fill(torch, pool, RowMeta(256), lens, seed=2024, scale=2.0)
    positions = [p for _ in range(n) for p in range(pre)]
    seqs = [s for s in range(n) for _ in range(pre)]
    m = len(seqs)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(2024)
    q = (torch.randn(m, nq, hd, device="cuda", generator=g) * 2.0).half()
    y = torch.empty(m, nq, hd, device="cuda")
    spec = ops.AttnSpec(q_heads=nq, window=4096, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=50.0)
    ops.attn(q, pool, 0, y, spec)
    torch.cuda.synchronize()
    ref = oracle_layer(torch, pool)
    qn, got_all = q.float().cpu().numpy(), y.cpu().numpy()
    assert np.all(np.isfinite(got_all))
    for c in (0, 5, 7):  # whole chunks: the oracle derives each row's keys from its chunk's rows
        r = slice(c * pre, (c + 1) * pre)
        want = ref.attn(qn[r], oracle.row_meta(positions[r], seqs[r]), pre, nq, 1.0 / math.sqrt(hd), window=4096,
                        softcap=50.0)
        err = float(np.max(np.abs(got_all[r] - want)))
        say("gemma2 prefill chunk", c, "max abs err", err)
        assert err <= TIGHT, (c, err)
    rows1 = RowMeta(pre)
    rows1.write(positions[3 * pre:4 * pre], seqs[3 * pre:4 * pre], pre)
    y1 = torch.empty(pre, nq, hd, device="cuda")
    ops.attn(q[3 * pre:4 * pre].contiguous(), pool, 0, y1,
             ops.AttnSpec(q_heads=nq, window=4096, scale=1.0 / math.sqrt(hd), m=pre, causal=True, seq=None,
                          args=rows1, softcap=50.0))
    torch.cuda.synchronize()
    assert torch.equal(y1, y[3 * pre:4 * pre]), "batch == solo"
