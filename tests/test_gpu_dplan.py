"""Device-planned decode calls (thb_dplan_build + thb_attn_dplan, no
reference counterpart): the plan made on the device from the row meta gives
the outputs of thb_attn (ops::attn, crates/thuban_model/src/ops/attn.rs:18-51)
bit for bit, also when the two launches are captured in a graph and replayed
while the rows' positions move; a row its pages do not cover reads nothing
and is reported by the allocator's status."""

import math
import random
import zlib

import numpy as np
import pytest

import oracle
from gpu_util import fill, make_pool, oracle_layer, say, scattered_alloc

pytestmark = pytest.mark.gpu

# name, nq, nkv, hd, kv, lens, rows per sequence, part_len, window, softcap, q dtype
CASES = [
    ("decode-ragged-split", 32, 8, 128, "f16", [3000, 40, 1500, 777, 2049], 1, 512, 0, 0.0, "f16"),
    ("verify4-window-softcap-hd256", 16, 8, 256, "f16", [1300, 600, 900], 4, 512, 700, 50.0, "f32"),
    ("mqa32-head-split", 32, 1, 128, "f16", [640, 50, 1000], 1, 256, 0, 0.0, "f32"),
    ("qwen2-bf16", 14, 2, 64, "bf16", [128, 512, 300, 1], 1, 128, 0, 0.0, "f32"),
    ("verify3-g8", 16, 2, 128, "f16", [900, 2000], 3, 1024, 0, 0.0, "f16"),
]


def _rows_of(lens, rps):
    positions, seqs = [], []
    for s, n in enumerate(lens):
        positions += list(range(n - rps, n))
        seqs += [s] * rps
    return positions, seqs


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_device_plan_matches_attn(torch_cuda, case):
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, kv, lens, rps, part_len, window, softcap, qdt = case
    say("device plan", name)
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=5, part_len=part_len)
    scattered_alloc(pool, lens, random.Random(zlib.crc32(name.encode())), 16)
    rows = RowMeta(256)
    fill(torch, pool, rows, lens, seed=3)
    positions, seqs = _rows_of(lens, rps)
    m = len(seqs)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    q = torch.randn(m, nq, hd, device="cuda", generator=g).to(torch.float16 if qdt == "f16" else torch.float32)
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=softcap)
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    ops.attn(q, pool, 0, want, spec)
    plan = ops.DevicePlan(pool, max_m=m + 3, q_heads=nq)
    plan.build(spec, q, got)
    plan.attn(0, q, got)
    torch.cuda.synchronize()
    assert torch.isfinite(want).all(), name
    assert torch.equal(got, want), (name, float((got - want).abs().max()))
    plan.close()


@pytest.mark.parametrize("prefill", [False, True], ids=["grid", "list"])
def test_device_plan_fixed_sequence(torch_cuda, prefill):
    """Reference mode: spec.seq fixed, a 3-row chunk (one group of 4 heads x 3
    rows at G = 4), rows of the chunk reading different key counts; in both
    plan forms."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    lens = [300, 500]
    pool = make_pool(lens, kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16", part_len=128)
    scattered_alloc(pool, lens, random.Random(4), 16)
    rows = RowMeta(64)
    fill(torch, pool, rows, lens, seed=4)
    rows.write([200, 201, 499], [1, 1, 1], 3)
    q = torch.randn(3, 8, 64, device="cuda")
    spec = ops.AttnSpec(q_heads=8, window=0, scale=0.125, m=3, causal=True, seq=1, args=rows)
    want, got = torch.empty_like(q), torch.empty_like(q)
    ops.attn(q, pool, 0, want, spec)
    plan = ops.DevicePlan(pool, max_m=3, q_heads=8, prefill=prefill)
    plan.build(spec, q, got)
    plan.attn(0, q, got)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_list_plan_fixed_sequence_prefill_chunk(torch_cuda):
    """Reference mode in a work-list plan: a 40-row prefill chunk of one
    sequence with spec.seq fixed (the reference's one dispatch per chunk),
    causal and not, cut into prefill blocks; equal to thb_attn bit for bit."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    lens = [700, 300]
    pool = make_pool(lens, kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16", part_len=1024)
    scattered_alloc(pool, lens, random.Random(40), 16)
    rows = RowMeta(64)
    fill(torch, pool, rows, lens, seed=40)
    rows.write(list(range(600, 640)), [0] * 40, 40)
    q = torch.randn(40, 16, 64, device="cuda")
    plan = ops.DevicePlan(pool, max_m=40, q_heads=16, prefill=True)
    for causal in (True, False):
        spec = ops.AttnSpec(q_heads=16, window=0, scale=0.125, m=40, causal=causal, seq=0, args=rows)
        want, got = torch.empty_like(q), torch.full_like(q, 7.0)
        ops.attn(q, pool, 0, want, spec)
        plan.build(spec, q, got)
        plan.attn(0, q, got)
        torch.cuda.synchronize()
        say("list plan fixed-seq chunk, causal", causal)
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (causal, float((got - want).abs().max()))
    plan.close()


def test_graph_replay_with_moving_positions(torch_cuda):
    """The device plan and the attention launches captured once, replayed for
    six decode steps after the row meta moves one position per step (and
    one sequence crosses a partition boundary); every replay equals thb_attn
    at that step's positions, bit for bit."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd = 32, 8, 128
    start = [700, 1500, 333, 2045]  # 2045 + steps crosses 2048 = 4 partitions of 512
    budget = [n + 8 for n in start]
    pool = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", part_len=512)
    scattered_alloc(pool, budget, random.Random(12), 16)
    rows = RowMeta(256)
    fill(torch, pool, rows, budget, seed=12)
    B = len(start)
    seqs = list(range(B))
    rows.write([n - 1 for n in start], seqs, B)
    q = torch.randn(B, nq, hd, device="cuda").half()
    y = torch.empty(B, nq, hd, device="cuda")
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=B, causal=True, seq=None, args=rows)
    plan = ops.DevicePlan(pool, max_m=B, q_heads=nq)
    plan.build(spec, q, y)  # outside the capture first: nothing left to set up
    plan.attn(0, q, y)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            plan.build(spec, q, y)
            plan.attn(0, q, y)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = torch.empty_like(y)
    for step in range(6):
        positions = [n - 1 + step for n in start]
        rows.write(positions, seqs, B)
        torch.cuda.synchronize()
        y.fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ops.attn(q, pool, 0, want, spec)
        torch.cuda.synchronize()
        say("graph replay step", step, "positions", positions)
        assert torch.isfinite(want).all()
        assert torch.equal(y, want), (step, float((y - want).abs().max()))
    del graph
    plan.close()


@pytest.mark.parametrize("prefill", [False, True], ids=["grid", "list"])
def test_uncovered_row_reads_nothing_and_is_reported(torch_cuda, prefill):
    """A row past its sequence's pages: thb_attn refuses the call; the device
    plan (either form) gives that row NaN, the other rows their thb_attn
    values, and thb_pool_status reports the first uncovered row (then
    clears)."""
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    held = [100, 200]
    pool = make_pool(held, kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16", seq_lens=[400, 400])
    scattered_alloc(pool, held, random.Random(8), 16)
    rows = RowMeta(16)
    fill(torch, pool, rows, held, seed=8)
    rows.write([350, 150], [0, 1], 2)
    q = torch.randn(2, 4, 64, device="cuda")
    spec = ops.AttnSpec(q_heads=4, window=0, scale=0.125, m=2, causal=True, seq=None, args=rows)
    with pytest.raises(ThubanError) as e:
        ops.attn(q, pool, 0, torch.empty_like(q), spec)
    assert "pages must cover the chunk" in str(e.value)
    got = torch.empty_like(q)
    plan = ops.DevicePlan(pool, max_m=2, q_heads=4, prefill=prefill)
    plan.build(spec, q, got)
    plan.attn(0, q, got)
    torch.cuda.synchronize()
    assert torch.isnan(got[0]).all()
    want = torch.empty(1, 4, 64, device="cuda")
    ops.attn(q[1:].contiguous(), pool, 0, want,
             ops.AttnSpec(q_heads=4, window=0, scale=0.125, m=1, causal=True, seq=None, args=rows, row_off=1))
    torch.cuda.synchronize()
    assert torch.equal(got[1:], want)
    with pytest.raises(ThubanError) as e:
        pool.status()
    say("device plan status", str(e.value))
    assert str(e.value) == "pages must cover the chunk: sequence 0 holds 112 slots, a row reads 351"
    pool.status()  # cleared


def test_device_plan_errors(torch_cuda):
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    pool = make_pool([64], kv_heads=2, head_dim=64)
    with pytest.raises(ThubanError):
        ops.DevicePlan(pool, max_m=5000, q_heads=4)
    with pytest.raises(ThubanError):
        ops.DevicePlan(pool, max_m=4, q_heads=3)
    plan = ops.DevicePlan(pool, max_m=4, q_heads=4)
    q = torch.zeros(2, 4, 64, device="cuda")
    with pytest.raises(ThubanError):
        plan.attn(0, q, torch.empty_like(q))
    rows = RowMeta(8)
    rows.write([3, 4], [0, 0], 2)
    with pytest.raises(ThubanError) as e:
        plan.build(ops.AttnSpec(q_heads=8, window=0, scale=0.1, m=2, causal=True, seq=None, args=rows), q, q)
    assert "q_heads" in str(e.value)
    with pytest.raises(ThubanError) as e:
        plan.build(ops.AttnSpec(q_heads=4, window=0, scale=0.1, m=6, causal=True, seq=None, args=rows), q, q)
    assert "rows" in str(e.value)
    plan.close()
    np.testing.assert_equal(True, True)


# name, nq, nkv, hd, kv, decode lens, prefill chunks (seq len, chunk rows), part_len, window, softcap, exact.
# exact: every prefill block's keys fit one partition, so the list plan runs
# each block on the prefill kernel as thb_attn does (bit-identical); a block
# spanning partitions runs as decode groups (thb_attn: the prefill kernel plus
# the merge), a different summation order: within the oracle's bound.
LIST_CASES = [
    ("c3-like", 32, 8, 128, "f16", [3000, 40, 1500, 777, 2049, 9000], [(512, 512), (700, 300)], 4096, 0, 0.0, True),
    ("gemma-window-softcap", 16, 8, 256, "f16", [1300, 5000], [(600, 200), (4700, 130)], 4096, 4096, 50.0, False),
    ("long-prefix-split-blocks", 32, 8, 128, "f16", [900], [(6000, 256)], 2048, 0, 0.0, False),
    ("qwen2-bf16", 14, 2, 64, "bf16", [128, 512, 300], [(400, 100)], 512, 0, 0.0, True),
    ("gemma-one-partition", 16, 8, 256, "f16", [1300, 2000], [(600, 200), (512, 512)], 4096, 4096, 50.0, True),
    ("6k-rows", 32, 8, 128, "f16", [5000] * 5 + [90, 17000, 1], [(2048, 2048), (4096, 2048), (3000, 1999)], 4096, 0,
     0.0, True),
    ("g32-two-groups-per-row", 32, 1, 128, "f16", [700, 3000], [(600, 300), (5000, 77)], 2048, 0, 0.0, False),
    ("8192-rows", 32, 8, 128, "f16", [3000, 90], [(4096, 4094), (4096, 4096)], 4096, 0, 0.0, True),
]


@pytest.mark.parametrize("case", LIST_CASES, ids=[c[0] for c in LIST_CASES])
def test_list_plan_with_prefill_matches_attn(torch_cuda, case):
    """A work-list device plan (prefill=True): decode rows and prefill
    chunks in one call, the chunks' blocks on the prefill kernel (or, when a
    block spans several partitions, as decode groups).  Where every block
    fits one partition the outputs equal thb_attn's bit for bit; otherwise
    they are within 1e-4 of the oracle and 1e-5 of thb_attn."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, kv, dlens, chunks, part_len, window, softcap, exact = case
    say("list plan", name)
    lens = dlens + [n for n, _ in chunks]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=5, part_len=part_len)
    scattered_alloc(pool, lens, random.Random(zlib.crc32(name.encode())), 16)
    fill(torch, pool, RowMeta(256), lens, seed=11)
    positions = [n - 1 for n in dlens]
    seqs = list(range(len(dlens)))
    for i, (n, c) in enumerate(chunks):
        positions += list(range(n - c, n))
        seqs += [len(dlens) + i] * c
    m = len(seqs)
    rows = RowMeta(m)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(12)
    q = torch.randn(m, nq, hd, device="cuda", generator=g).half()
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=softcap)
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    ops.attn(q, pool, 0, want, spec)
    plan = ops.DevicePlan(pool, max_m=min(m + 5, 8192), q_heads=nq, prefill=True)
    plan.build(spec, q, got)
    plan.attn(0, q, got)
    plan.attn(0, q, got)  # a second launch: the claim counter was reset by the first
    torch.cuda.synchronize()
    assert torch.isfinite(want).all(), name
    if exact:
        assert torch.equal(got, want), (name, float((got - want).abs().max()))
    else:
        assert float((got - want).abs().max()) <= 1e-5, name
        ref = oracle_layer(torch, pool)
        oracle_y = ref.attn(q.float().cpu().numpy(), oracle.row_meta(positions, seqs), m, nq, 1.0 / math.sqrt(hd),
                            window=window, softcap=softcap)
        err = float(np.max(np.abs(got.cpu().numpy() - oracle_y)))
        say("list plan", name, "max abs err vs oracle", err)
        assert err <= 1e-4, (name, err)
    pool.status()
    plan.close()


def test_list_plan_graph_replay_chunked_prefill(torch_cuda):
    """A captured step of the list plan (build + attention over two layers)
    replayed while a 256-row prefill chunk advances through a 1024-token
    prompt beside four decode rows: every replay equals thb_attn at that
    step's positions, bit for bit."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd, L = 32, 8, 128, 2
    dlens = [2100, 700, 4500, 1300]
    budget = [n + 8 for n in dlens] + [1024]
    pool = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", layers=L, part_len=1024)
    scattered_alloc(pool, budget, random.Random(33), 16)
    for layer in range(L):
        fill(torch, pool, RowMeta(256), budget, layer=layer, seed=33 + layer)
    c = 256
    m = len(dlens) + c
    rows = RowMeta(m)
    g = torch.Generator(device="cuda")
    g.manual_seed(34)
    q = [torch.randn(m, nq, hd, device="cuda", generator=g).half() for _ in range(L)]
    y = [torch.empty(m, nq, hd, device="cuda") for _ in range(L)]
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows)
    plan = ops.DevicePlan(pool, max_m=m, q_heads=nq, prefill=True)
    seqs = list(range(len(dlens))) + [len(dlens)] * c

    def positions(step):
        return [n - 1 + step for n in dlens] + list(range(step * c, step * c + c))

    rows.write(positions(0), seqs, m)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            plan.build(spec, q[0], y[0])
            for layer in range(L):
                plan.attn(layer, q[layer], y[layer])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = torch.empty(m, nq, hd, device="cuda")
    for step in range(4):
        rows.write(positions(step), seqs, m)
        for t in y:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            ops.attn(q[layer], pool, layer, want, spec)
            torch.cuda.synchronize()
            say("list plan replay step", step, "layer", layer)
            assert torch.isfinite(want).all()
            assert torch.equal(y[layer], want), (step, layer, float((y[layer] - want).abs().max()))
    pool.status()
    del graph
    plan.close()
