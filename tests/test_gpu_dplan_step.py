"""thb_attn_step over a device plan (thb_attn_step_dplan, no reference
counterpart): the thb_attn_io extensions (rotary embedding with q/k norm,
query stride, sigmoid gate, and the append inside the launch) on plans made
on the device, bit-identical to the host-planned thb_attn_step
(ops::attn + rope/norm_rope + kv_store, transformer/forward.rs:300-336,
qwen35/layers.rs:231-238) on twin pools, eagerly and replayed from a graph;
rows past the plan's position limit read nothing and are reported."""

import math
import random
import zlib

import numpy as np
import pytest

from gpu_util import fill, make_pool, say, scattered_alloc

pytestmark = pytest.mark.gpu


def _rope(hd, rot, norm, max_pos, seed=0):
    from flint_amd.rope import Rope, rope_tables

    cos, sin = rope_tables(max_pos, rot, rot, 5e5)
    rng = np.random.default_rng(seed)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    return Rope(cos, sin, rot, q_norm=qn, k_norm=kn, eps=1e-6)


def _twins(torch, name, lens, nkv, hd, part_len, layers=1, fill_lens=None):
    from flint_amd.pool import RowMeta

    pools = []
    for _ in range(2):
        pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", extra_pages=5,
                         part_len=part_len, layers=layers)
        scattered_alloc(pool, lens, random.Random(zlib.crc32(name.encode())), 16)
        for layer in range(layers):
            fill(torch, pool, RowMeta(256), fill_lens or lens, layer=layer, seed=31 + layer)
        pools.append(pool)
    return pools


def _same_bytes(torch, a, b, layer=0):
    return all(torch.equal(x, y) for x, y in zip(a.layer_tensors(layer), b.layer_tensors(layer)))


# name, nq, nkv, hd, rot, norm, lens, rows per sequence, part_len, window, softcap, src dtype, gate
CASES = [
    ("llama-rope-decode", 32, 8, 128, 128, False, [3000, 40, 1500, 2049], 1, 512, 0, 0.0, "f16", False),
    ("qwen3-norm-rope-gate", 32, 8, 128, 128, True, [700, 1300, 90], 1, 1024, 0, 0.0, "f32", True),
    ("gemma-verify4-rope-softcap", 16, 8, 256, 256, False, [1300, 600], 4, 512, 700, 50.0, "f32", False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_step_plan_with_append_matches_attn_step(torch_cuda, case):
    """Fixed-grid plan with THB_DPLAN_APPEND: rope (and q/k norm, a q|gate
    projection read with q_stride and the gate) with the append inside the
    launch, against thb_attn_step on a twin pool: outputs and pool bytes."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    name, nq, nkv, hd, rot, norm, lens, rps, part_len, window, softcap, sdt, gated = case
    say("step plan", name)
    eager, planned = _twins(torch, name, lens, nkv, hd, part_len)
    rope = _rope(hd, rot, norm, max_pos=4096, seed=3)
    positions = [p for n in lens for p in range(n - rps, n)]
    seqs = [s for s, _ in enumerate(lens) for _ in range(rps)]
    m = len(seqs)
    rows = RowMeta(64)
    rows.write(positions, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(32)
    dt = torch.float16 if sdt == "f16" else torch.float32
    k = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    v = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    if gated:  # a fused q|gate projection: each head's q then its gate
        qg = torch.randn(m, nq, 2 * hd, device="cuda", generator=g)
        q, gate, stride = qg[:, :, :hd], qg[:, :, hd:], 2 * hd
    else:
        q, gate, stride = torch.randn(m, nq, hd, device="cuda", generator=g), None, 0
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=softcap)
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    ops.attn_step(eager, 0, spec, q, want, q_stride=stride, gate=gate, gate_stride=stride, k_src=k, v_src=v,
                  rope=rope)
    plan = ops.DevicePlan(planned, max_m=m, q_heads=nq, append=True)
    plan.set_pos_limit(rope.max_pos)
    plan.build(spec, q, got)
    plan.step(0, q, got, q_stride=stride, gate=gate, gate_stride=stride, k_src=k, v_src=v, rope=rope)
    torch.cuda.synchronize()
    assert torch.isfinite(want).all(), name
    assert torch.equal(got, want), (name, float((got - want).abs().max()))
    assert _same_bytes(torch, eager, planned), name
    planned.status()
    plan.close()


def test_step_list_plan_with_rope_matches_attn_step(torch_cuda):
    """Work-list plan: decode rows and two prefill chunks with q/k norm and
    rotation of the queries in the launch (keys rotated by kv_store_rope
    before), bit-identical to thb_attn_step with the same rope."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd = 32, 8, 128
    dlens, chunks = [2100, 700, 4500], [(512, 512), (900, 200)]
    lens = dlens + [n for n, _ in chunks]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", part_len=4096)
    scattered_alloc(pool, lens, random.Random(41), 16)
    fill(torch, pool, RowMeta(256), lens, seed=41)
    rope = _rope(hd, hd, True, max_pos=8192, seed=4)
    positions = [n - 1 for n in dlens]
    seqs = list(range(len(dlens)))
    for i, (n, c) in enumerate(chunks):
        positions += list(range(n - c, n))
        seqs += [len(dlens) + i] * c
    m = len(seqs)
    rows = RowMeta(m)
    rows.write(positions, seqs, m)
    q = torch.randn(m, nq, hd, device="cuda")
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows)
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    ops.attn_step(pool, 0, spec, q, want, rope=rope)
    plan = ops.DevicePlan(pool, max_m=m, q_heads=nq, prefill=True)
    plan.set_pos_limit(rope.max_pos)
    plan.build(spec, q, got)
    plan.step(0, q, got, rope=rope)
    torch.cuda.synchronize()
    assert torch.isfinite(want).all()
    assert torch.equal(got, want), float((got - want).abs().max())
    pool.status()
    plan.close()


def test_step_plan_position_limit(torch_cuda):
    """A row at or past the plan's position limit reads nothing (NaN) and is
    reported with the host's message; the others equal thb_attn_step.  With
    THB_DPLAN_APPEND the whole call is planned empty and nothing is
    appended.  Launches without a fitting limit are refused."""
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    lens = [900, 400]
    pool = make_pool(lens, kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16", part_len=256)
    scattered_alloc(pool, lens, random.Random(9), 16)
    fill(torch, pool, RowMeta(256), lens, seed=9)
    rope = _rope(64, 64, False, max_pos=600, seed=9)
    rows = RowMeta(8)
    rows.write([700, 300], [0, 1], 2)
    q = torch.randn(2, 8, 64, device="cuda")
    spec = ops.AttnSpec(q_heads=8, window=0, scale=0.125, m=2, causal=True, seq=None, args=rows)
    plan = ops.DevicePlan(pool, max_m=2, q_heads=8)
    plan.build(spec, q, q)
    with pytest.raises(ThubanError) as e:  # no limit
        plan.step(0, q, torch.empty_like(q), rope=rope)
    assert "position limit" in str(e.value)
    plan.set_pos_limit(601)
    plan.build(spec, q, q)
    with pytest.raises(ThubanError) as e:  # a limit above the tables
        plan.step(0, q, torch.empty_like(q), rope=rope)
    assert "position limit" in str(e.value)
    with pytest.raises(ThubanError) as e:  # that build already reported row 0 against its limit
        pool.status()
    assert str(e.value) == "row position 700 outside the rope tables (601 positions)"
    plan.set_pos_limit(600)
    with pytest.raises(ThubanError):  # not built since the limit changed
        plan.step(0, q, torch.empty_like(q), rope=rope)
    got = torch.zeros_like(q)
    plan.build(spec, q, got)
    plan.step(0, q, got, rope=rope)
    torch.cuda.synchronize()
    assert torch.isnan(got[0]).all()
    want = torch.empty(1, 8, 64, device="cuda")
    ops.attn_step(pool, 0, ops.AttnSpec(q_heads=8, window=0, scale=0.125, m=1, causal=True, seq=None, args=rows,
                                        row_off=1), q[1:].contiguous(), want, rope=rope)
    torch.cuda.synchronize()
    assert torch.equal(got[1:], want)
    with pytest.raises(ThubanError) as e:
        pool.status()
    assert str(e.value) == "row position 700 outside the rope tables (600 positions)"
    plan.close()
    # with the append: nothing appended, every output NaN
    before = [t.clone() for t in pool.layer_tensors(0)]
    k = torch.randn(2, 2, 64, device="cuda")
    ap = ops.DevicePlan(pool, max_m=2, q_heads=8, append=True)
    ap.set_pos_limit(600)
    y = torch.zeros_like(q)
    ap.build(spec, q, y)
    ap.step(0, q, y, k_src=k, v_src=k, rope=rope)
    torch.cuda.synchronize()
    assert torch.isnan(y).all()
    assert all(torch.equal(a, b) for a, b in zip(before, pool.layer_tensors(0)))
    with pytest.raises(ThubanError) as e:
        pool.status()
    assert str(e.value) == "row position 700 outside the rope tables (600 positions)"
    plain = ops.DevicePlan(pool, max_m=2, q_heads=8)
    plain.build(spec, q, q)
    with pytest.raises(ThubanError) as e:  # the append needs THB_DPLAN_APPEND
        plain.step(0, q, torch.empty_like(q), k_src=k, v_src=k)
    assert "THB_DPLAN_APPEND" in str(e.value)
    pool.status()
    ap.close()
    plain.close()


def test_captured_rope_step_replays_like_attn_step(torch_cuda):
    """One build and, for two layers, q/k norm + rotation + append in one
    launch each, captured once and replayed for six decode steps with new
    K/V/Q each step and one sequence crossing a partition boundary; after
    every replay outputs and both layers' bytes equal an eager thb_attn_step
    twin's."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd, L = 32, 8, 128, 2
    start = [700, 1500, 1022]  # 1022 + steps crosses 1024 = 2 partitions of 512
    budget = [n + 8 for n in start]
    eager, planned = _twins(torch, "captured-rope", budget, nkv, hd, 512, layers=L, fill_lens=start)
    rope = _rope(hd, hd, True, max_pos=2048, seed=5)
    B = len(start)
    seqs = list(range(B))
    rows = RowMeta(B)
    rows.write(start, seqs, B)
    g = torch.Generator(device="cuda")
    g.manual_seed(44)
    k = [torch.empty(B, nkv, hd, device="cuda") for _ in range(L)]
    v = [torch.empty(B, nkv, hd, device="cuda") for _ in range(L)]
    q = [torch.empty(B, nq, hd, device="cuda") for _ in range(L)]
    y = [torch.empty(B, nq, hd, device="cuda") for _ in range(L)]
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=B, causal=True, seq=None, args=rows)
    plan = ops.DevicePlan(planned, max_m=B, q_heads=nq, append=True)
    plan.set_pos_limit(rope.max_pos)
    plan.build(spec, q[0], y[0])
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            plan.build(spec, q[0], y[0])
            for layer in range(L):
                plan.step(layer, q[layer], y[layer], k_src=k[layer], v_src=v[layer], rope=rope)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = torch.empty(B, nq, hd, device="cuda")
    for step in range(6):
        positions = [n + step for n in start]
        rows.write(positions, seqs, B)
        for layer in range(L):
            k[layer].normal_(generator=g)
            v[layer].normal_(generator=g)
            q[layer].normal_(generator=g)
            y[layer].fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            ops.attn_step(eager, layer, spec, q[layer], want, k_src=k[layer], v_src=v[layer], rope=rope)
            torch.cuda.synchronize()
            say("rope step replay", step, "layer", layer, "positions", positions)
            assert torch.isfinite(want).all()
            assert torch.equal(y[layer], want), (step, layer, float((y[layer] - want).abs().max()))
            assert _same_bytes(torch, eager, planned, layer), (step, layer)
    planned.status()
    del graph
    plan.close()


N_RANDOM = 16


@pytest.mark.parametrize("seed", range(N_RANDOM))
def test_random_step_plan_calls(torch_cuda, seed):
    """Seeded random calls of thb_attn_step_dplan against thb_attn_step on
    twin pools: head_dim 64/128/256, 1-8 query heads per KV head, one group
    of 1-4 rows per sequence, rotation of the whole head or its first half,
    q/k norm or not, a q|gate projection with the gate or not, window and
    soft-cap; the fixed-grid plan with the append inside the launch, or
    without the append on either plan form (the keys appended first by
    thb_kv_store_rope on both pools).  Outputs and pool bytes bit-identical."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta
    from flint_amd.rope import kv_store_rope

    rng = random.Random(7000 + seed)
    hd = rng.choice([64, 128, 256])
    nkv = rng.choice([1, 2, 4, 8])
    g = rng.choice([1, 2, 4, 8])
    nq = g * nkv
    rps = rng.randint(1, min(4, 16 // g))
    lens = [rng.randint(rps + 8, 1500) for _ in range(rng.randint(1, 4))]
    rot = rng.choice([hd, hd // 2]) if hd // 2 % 16 == 0 else hd
    norm, gated = rng.random() < 0.5, rng.random() < 0.4
    window, cap = rng.choice([0, 0, rng.randint(1, 600)]), rng.choice([0.0, 0.0, 30.0])
    form = rng.choice(["append", "grid", "list"])
    part_len = rng.choice([128, 512, 4096])
    say("random step plan", seed, dict(hd=hd, nkv=nkv, g=g, rps=rps, lens=lens, rot=rot, norm=norm, gated=gated,
                                       window=window, cap=cap, form=form, part_len=part_len))
    eager, planned = _twins(torch, f"step{seed}", [n + rps for n in lens], nkv, hd, part_len, fill_lens=lens)
    rope = _rope(hd, rot, norm, max_pos=2048, seed=seed)
    positions = [p for n in lens for p in range(n, n + rps)]
    seqs = [s for s, _ in enumerate(lens) for _ in range(rps)]
    m = len(seqs)
    rows = RowMeta(64)
    rows.write(positions, seqs, m)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    k = torch.randn(m, nkv, hd, device="cuda", generator=gen)
    v = torch.randn(m, nkv, hd, device="cuda", generator=gen)
    if gated:
        qg = torch.randn(m, nq, 2 * hd, device="cuda", generator=gen)
        q, gate, stride = qg[:, :, :hd], qg[:, :, hd:], 2 * hd
    else:
        q, gate, stride = torch.randn(m, nq, hd, device="cuda", generator=gen), None, 0
    spec = ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows,
                        softcap=cap)
    append = form == "append"
    if not append:  # the keys go in first, rotated, on both pools
        for P in (eager, planned):
            kv_store_rope(k, v, P, 0, m, rows, rope)
    want = torch.empty(m, nq, hd, device="cuda")
    got = torch.full_like(want, 7.0)
    src = dict(k_src=k, v_src=v) if append else {}
    ops.attn_step(eager, 0, spec, q, want, q_stride=stride, gate=gate, gate_stride=stride, rope=rope, **src)
    plan = ops.DevicePlan(planned, max_m=m, q_heads=nq, prefill=form == "list", append=append)
    plan.set_pos_limit(rope.max_pos)
    plan.build(spec, q, got)
    plan.step(0, q, got, q_stride=stride, gate=gate, gate_stride=stride, rope=rope, **src)
    torch.cuda.synchronize()
    plan.close()
    planned.status()
    assert torch.isfinite(want).all(), seed
    assert torch.equal(got, want), (seed, float((got - want).abs().max()))
    assert _same_bytes(torch, eager, planned), seed
