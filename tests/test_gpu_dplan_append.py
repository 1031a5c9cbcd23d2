"""Device-planned decode steps with the append inside the attention launch
(thb_dplan_create_ex with THB_DPLAN_APPEND + thb_attn_append_dplan, no
reference counterpart): kv_store then attn (transformer/forward.rs:300-336)
in one launch over a plan made on the device.  Outputs and pool bytes equal
thb_attn_append's bit for bit (twin pools of identical pages and contents),
eagerly and replayed from a graph while positions move; a call whose append
cannot run inside the launch is planned empty (nothing appended, NaN
outputs) and reported by the allocator's status."""

import math
import random
import zlib

import pytest

from gpu_util import fill, make_pool, say, scattered_alloc

pytestmark = pytest.mark.gpu

# name, nq, nkv, hd, kv, lens, rows per sequence, part_len, window, softcap, q dtype, src dtype
CASES = [
    ("decode-ragged-split", 32, 8, 128, "f16", [3000, 40, 1500, 777, 2049], 1, 512, 0, 0.0, "f16", "f32"),
    ("verify4-window-softcap-hd256", 16, 8, 256, "f16", [1300, 600, 900], 4, 512, 700, 50.0, "f32", "f16"),
    ("mqa32-head-split", 32, 1, 128, "f16", [640, 50, 1000], 1, 256, 0, 0.0, "f32", "f32"),
    ("qwen2-bf16-first-token", 14, 2, 64, "bf16", [128, 512, 300, 1], 1, 128, 0, 0.0, "f32", "bf16"),
    ("verify2-g8", 16, 2, 128, "f16", [900, 2000], 2, 1024, 0, 0.0, "f16", "f32"),
]

_DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


def _twin_pools(torch, name, lens, nkv, hd, kv, part_len, seed):
    """Two pools with the same page tables and contents."""
    from flint_amd.pool import RowMeta

    pools = []
    for _ in range(2):
        pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=5,
                         part_len=part_len)
        scattered_alloc(pool, lens, random.Random(zlib.crc32(name.encode())), 16)
        fill(torch, pool, RowMeta(256), lens, seed=seed)
        pools.append(pool)
    return pools


def _same_bytes(torch, a, b, layer=0):
    return all(torch.equal(x, y) for x, y in zip(a.layer_tensors(layer), b.layer_tensors(layer)))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_append_plan_matches_attn_append(torch_cuda, case):
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, kv, lens, rps, part_len, window, softcap, qdt, sdt = case
    say("append plan", name)
    eager, planned = _twin_pools(torch, name, lens, nkv, hd, kv, part_len, seed=21)
    positions = [p for n in lens for p in range(n - rps, n)]
    seqs = [s for s, _ in enumerate(lens) for _ in range(rps)]
    m = len(seqs)
    rows = RowMeta(64)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(22)
    sdt_t = getattr(torch, _DT[sdt])
    k = torch.randn(m, nkv, hd, device="cuda", generator=g).to(sdt_t)
    v = torch.randn(m, nkv, hd, device="cuda", generator=g).to(sdt_t)
    q = torch.randn(m, nq, hd, device="cuda", generator=g).to(getattr(torch, _DT[qdt]))
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=softcap)
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    ops.kv_store_attn(k, v, q, eager, 0, want, spec)
    plan = ops.DevicePlan(planned, max_m=m + 3, q_heads=nq, append=True)
    plan.build(spec, q, got)
    plan.attn_append(0, k, v, q, got)
    torch.cuda.synchronize()
    assert torch.isfinite(want).all(), name
    assert torch.equal(got, want), (name, float((got - want).abs().max()))
    assert _same_bytes(torch, eager, planned), name
    planned.status()  # nothing reported
    # the plan also serves plain attention over the same call
    again = torch.empty_like(want)
    plan.attn(0, q, again)
    torch.cuda.synchronize()
    assert torch.equal(again, want)
    plan.close()


def _refused(torch, pool, rows, positions, seqs, nq, hd, seq=None):
    """Builds and runs an append plan over a call its launch cannot append;
    returns the status message after checking that nothing was appended and
    every output is NaN."""
    from flint_amd import ThubanError, ops

    m = len(seqs)
    rows.write(positions, seqs, m)
    before = [t.clone() for t in pool.layer_tensors(0)]
    k = torch.randn(m, pool.kv_heads, hd, device="cuda")
    v = torch.randn(m, pool.kv_heads, hd, device="cuda")
    q = torch.randn(m, nq, hd, device="cuda")
    y = torch.zeros(m, nq, hd, device="cuda")
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=seq, args=rows)
    plan = ops.DevicePlan(pool, max_m=8, q_heads=nq, append=True)
    plan.build(spec, q, y)
    plan.attn_append(0, k, v, q, y)
    torch.cuda.synchronize()
    assert torch.isnan(y).all()
    assert all(torch.equal(a, b) for a, b in zip(before, pool.layer_tensors(0)))
    with pytest.raises(ThubanError) as e:
        pool.status()
    pool.status()  # cleared
    plan.close()
    say("append plan refused:", str(e.value))
    return str(e.value)


def test_append_plan_refuses_calls_it_cannot_fuse(torch_cuda):
    torch = torch_cuda
    from flint_amd.pool import RowMeta

    lens = [300, 500, 200]
    pool = make_pool(lens, kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16", part_len=128)
    scattered_alloc(pool, lens, random.Random(5), 16)
    fill(torch, pool, RowMeta(256), lens, seed=5)
    rows = RowMeta(16)
    tail = "; nothing was appended"
    # G = 8: a group holds 2 rows of a chunk; a 3-row chunk does not fit
    msg = _refused(torch, pool, rows, [100, 101, 102], [1, 1, 1], 16, 64)
    assert msg == "the append cannot run inside the attention launch: row 0 (sequence 1): its chunk holds more " \
                  "rows than one group" + tail
    # a sequence heading two chunks (rows 0 and 2)
    msg = _refused(torch, pool, rows, [10, 20, 11], [0, 1, 0], 8, 64)
    assert msg == "the append cannot run inside the attention launch: row 2 (sequence 0): its sequence heads an " \
                  "earlier chunk of the call too" + tail
    # positions falling within a chunk: the chunk's keys end at its last
    # row's position, so row 1's keys stop short of its new token
    msg = _refused(torch, pool, rows, [50, 150, 149], [0, 1, 1], 8, 64)
    assert msg.startswith("the append cannot run inside the attention launch: row 1 (sequence 1): its keys do not "
                          "end at its new token")
    # a row whose own sequence is not the fixed one
    msg = _refused(torch, pool, rows, [40], [2], 8, 64, seq=0)
    assert msg == "the append cannot run inside the attention launch: row 0 (sequence 2): its sequence is not " \
                  "the call's fixed sequence" + tail
    # a row its pages do not cover: the cover failure is reported first
    msg = _refused(torch, pool, rows, [10, 250], [0, 2], 8, 64)
    assert msg == "pages must cover the chunk: sequence 2 holds 208 slots, a row reads 251"


def test_append_plan_argument_errors(torch_cuda):
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    pool = make_pool([64], kv_heads=2, head_dim=64)
    pool.alloc(0, 0, 64)
    rows = RowMeta(8)
    rows.write([3], [0], 1)
    q = torch.zeros(1, 4, 64, device="cuda")
    k = torch.zeros(1, 2, 64, device="cuda")
    with pytest.raises(ThubanError) as e:
        ops.DevicePlan(pool, max_m=4, q_heads=4, prefill=True, append=True)
    assert "THB_DPLAN_APPEND" in str(e.value)
    plain = ops.DevicePlan(pool, max_m=4, q_heads=4)
    plain.build(ops.AttnSpec(q_heads=4, window=0, scale=0.1, m=1, causal=True, seq=None, args=rows), q, q)
    with pytest.raises(ThubanError) as e:
        plain.attn_append(0, k, k, q, torch.empty_like(q))
    assert "THB_DPLAN_APPEND" in str(e.value)
    plain.close()
    plan = ops.DevicePlan(pool, max_m=4, q_heads=4, append=True)
    with pytest.raises(ThubanError) as e:
        plan.build(ops.AttnSpec(q_heads=4, window=0, scale=0.1, m=1, causal=False, seq=None, args=rows), q, q)
    assert "causal" in str(e.value)
    plan.close()
    pool.status()


def test_captured_append_plan_replays_like_attn_append(torch_cuda):
    """thb_dplan_build + thb_attn_append_dplan over two layers captured once
    and replayed for eight decode steps, new K/V each step, one sequence
    crossing a page and a partition boundary; after every replay the outputs
    and both layers' bytes equal an eager kv_store_attn twin's."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd, L = 32, 8, 128, 2
    start = [700, 1500, 333, 2044]  # 2044 + steps crosses 2048 = 4 partitions of 512
    budget = [n + 8 for n in start]
    pools = []
    for _ in range(2):
        pool = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", layers=L, part_len=512)
        scattered_alloc(pool, budget, random.Random(19), 16)
        for layer in range(L):
            fill(torch, pool, RowMeta(256), start, layer=layer, seed=19 + layer)
        pools.append(pool)
    eager, planned = pools
    B = len(start)
    seqs = list(range(B))
    rows = RowMeta(B)
    rows.write(start, seqs, B)
    g = torch.Generator(device="cuda")
    g.manual_seed(20)
    k = [torch.empty(B, nkv, hd, device="cuda") for _ in range(L)]
    v = [torch.empty(B, nkv, hd, device="cuda") for _ in range(L)]
    q = [torch.empty(B, nq, hd, device="cuda").half() for _ in range(L)]
    y = [torch.empty(B, nq, hd, device="cuda") for _ in range(L)]
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=B, causal=True, seq=None, args=rows)
    plan = ops.DevicePlan(planned, max_m=B, q_heads=nq, append=True)
    plan.build(spec, q[0], y[0])  # outside the capture first: nothing left to set up
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            plan.build(spec, q[0], y[0])
            for layer in range(L):
                plan.attn_append(layer, k[layer], v[layer], q[layer], y[layer])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = torch.empty(B, nq, hd, device="cuda")
    for step in range(8):
        positions = [n + step for n in start]
        rows.write(positions, seqs, B)
        for layer in range(L):
            k[layer].normal_(generator=g)
            v[layer].normal_(generator=g)
            q[layer].copy_(torch.randn(B, nq, hd, device="cuda", generator=g))
            y[layer].fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            ops.kv_store_attn(k[layer], v[layer], q[layer], eager, layer, want, spec)
            torch.cuda.synchronize()
            say("append plan replay step", step, "layer", layer, "positions", positions)
            assert torch.isfinite(want).all()
            assert torch.equal(y[layer], want), (step, layer, float((y[layer] - want).abs().max()))
            assert _same_bytes(torch, eager, planned, layer), (step, layer)
    planned.status()
    del graph
    plan.close()


N_RANDOM = 24


def _random_case(seed):
    rng = random.Random(seed)
    hd = rng.choice([64, 128, 256])
    nkv = rng.choice([1, 2, 4, 8])
    g = rng.choice([1, 2, 4, 7, 8, 16, 32])
    rg = 16 // g if g <= 16 else 1  # rows of one chunk that one group holds
    lens = [rng.randint(24, 1200) for _ in range(rng.randint(1, 5))]
    rps = [rng.randint(1, min(rg, 4)) for _ in lens]
    if rng.random() < 0.25:  # one chunk a row longer than a group holds
        rps[rng.randrange(len(rps))] = rg + 1
    # the rows of each sequence, in order; sometimes one sequence comes back as a second chunk
    chunks = [(s, list(range(n - r, n))) for s, (n, r) in enumerate(zip(lens, rps))]
    if len(chunks) > 1 and rng.random() < 0.25:
        s, pos = chunks[0]
        if len(pos) > 1:
            chunks[0] = (s, pos[:-1])
            chunks.append((s, pos[-1:]))
        else:
            chunks.append((s, [pos[0] - 1]))
    return dict(hd=hd, nkv=nkv, nq=g * nkv, g=g, lens=lens, chunks=chunks, part_len=rng.choice([128, 512, 4096]),
                window=rng.choice([0, 0, rng.randint(1, 700)]), cap=rng.choice([0.0, 30.0]),
                src=rng.choice(["f32", "f16", "bf16"]))


@pytest.mark.parametrize("seed", range(N_RANDOM))
def test_random_append_plan_calls(torch_cuda, seed):
    """Seeded random decode / verify calls (head_dim, grouping up to 32 query
    heads per KV head, 1-5 rows per sequence, sometimes a sequence heading
    two chunks, window, soft-cap, source type) through the append plan, on
    twin pools.  Where build_plan's rule lets the append run inside the
    launch (every chunk fits one group, no sequence in two chunks) the
    outputs and pool bytes equal thb_attn_append's; otherwise the call is
    planned empty: every output NaN, the pool untouched, the status names
    the first failing row's reason."""
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    c = _random_case(5000 + seed)
    say("random append plan", seed, {k: v for k, v in c.items() if k != "chunks"}, [len(p) for _, p in c["chunks"]])
    eager, planned = _twin_pools(torch, f"rnd{seed}", c["lens"], c["nkv"], c["hd"], "f16", c["part_len"], seed=seed)
    positions = [p for _, pos in c["chunks"] for p in pos]
    seqs = [s for s, pos in c["chunks"] for _ in pos]
    m = len(seqs)
    rows = RowMeta(64)
    rows.write(positions, seqs, m)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    dt = getattr(torch, _DT[c["src"]])
    k = torch.randn(m, c["nkv"], c["hd"], device="cuda", generator=gen).to(dt)
    v = torch.randn(m, c["nkv"], c["hd"], device="cuda", generator=gen).to(dt)
    q = torch.randn(m, c["nq"], c["hd"], device="cuda", generator=gen)
    spec = ops.AttnSpec(q_heads=c["nq"], window=c["window"], scale=1.0 / math.sqrt(c["hd"]), m=m, causal=True,
                        seq=None, args=rows, softcap=c["cap"])
    rg = 16 // c["g"] if c["g"] <= 16 else 1
    heads = [s for s, _ in c["chunks"]]
    fits = all(len(pos) <= rg for _, pos in c["chunks"])
    fusable = fits and len(set(heads)) == len(heads)
    got = torch.full_like(q, 7.0)
    plan = ops.DevicePlan(planned, max_m=m, q_heads=c["nq"], append=True)
    plan.build(spec, q, got)
    plan.attn_append(0, k, v, q, got)
    torch.cuda.synchronize()
    plan.close()
    if fusable:
        want = torch.empty_like(q)
        ops.kv_store_attn(k, v, q, eager, 0, want, spec)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all(), seed
        assert torch.equal(got, want), (seed, float((got - want).abs().max()))
        assert _same_bytes(torch, eager, planned), seed
        planned.status()
        return
    assert torch.isnan(got).all(), seed
    assert _same_bytes(torch, eager, planned), (seed, "a refused call appended")
    with pytest.raises(ThubanError) as e:
        planned.status()
    msg = str(e.value)
    say("random append plan", seed, "refused:", msg)
    assert msg.startswith("the append cannot run inside the attention launch"), msg
    assert ("holds more rows than one group" in msg) if not fits else ("heads an earlier chunk" in msg), msg
