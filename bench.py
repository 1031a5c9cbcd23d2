#!/usr/bin/env python3
"""Benchmark of the MI355X paged KV-cache path (one GPU).

Workload (Llama-3-8B-shaped decode): 32 layers, 32 query
heads, 8 KV heads, head_dim 128, f16 KV in pages of 16 tokens, batch 32 at
context 4096 with block tables randomly scattered over the pool.  One step =
for every layer: append 1 token per sequence (kv_store) + paged decode
attention over the 4096 keys.  Inputs are synthetic N(0,1) and resident in
HBM before the timed region.

Prints one JSON line.  value = achieved HBM GB/s of the whole step
(algorithmic bytes: every K/V byte once + Q, O, block table, appended rows)
/ step time.  roofline = the attention kernel: HIP events on the launch
stream around the run of layers 1..L-1 of every timed step, divided by L-1
(layer 0 also carries the step's row-meta plan upload, which the step time
includes; two events per step keep the instrumentation out of the step
time).  The standalone append kernel is timed from a captured HIP graph of
back-to-back launches (Python cannot enqueue 5-us kernels fast enough to
keep the GPU busy).  traffic = HBM bytes per launch from the committed rocprofv3
counter summary.  cpu_baseline = the CPU oracle (restatement of the
reference's f32 online-softmax algorithm) on layer 0 of the same step.
gather / scatter / block_copy = the page-move kernels at the same shape
(secondary fields of the same line).  hbm_ceiling = the device's achievable
linear read and copy rates (thb_hbm_stream over 1 GiB), against which every
fraction is also stated.  c1_* / c3_* / c4_* / c5_* = the other BASELINE
configurations measured in the same run (C1 with its CPU baseline).

--config selects one of the other BASELINE configurations instead (C1
qwen2-0.5b, C3 qwen3-8b, C4 gemma2-9b, C5 qwen2.5-32b).  Those are parity-
test shapes; their lines are secondary measurements of the same kernels and
carry no cpu_baseline.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import random
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0

CONFIGS = {
    "llama3-8b": dict(layers=32, batch=32, ctx=4096, q_heads=32, kv_heads=8, head_dim=128, page_len=16),
}
SECONDARY = ("qwen2-0.5b", "qwen3-8b", "gemma2-9b", "qwen2.5-32b")


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def scattered_alloc(pool, lens, rng, page_len):
    need = [-(-n // page_len) for n in lens]
    have = [0] * len(lens)
    order = [s for s in range(len(lens)) for _ in range(need[s])]
    rng.shuffle(order)
    for s in order:
        n = min(page_len, lens[s] - have[s] * page_len)
        pool.alloc(s, have[s] * page_len, n)
        have[s] += 1


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def time_append_graph(torch, ops, pool, rows, k, v, layer, m, launches=50, replays=5):
    """Average duration of the standalone append kernel (ops.kv_store), from
    a HIP graph of back-to-back launches replayed with events around it.
    Returns None if the graph cannot be captured."""
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            ops.kv_store(k, v, pool, layer, m, rows)  # warm: nothing left to upload
            side.synchronize()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(launches):
                    ops.kv_store(k, v, pool, layer, m, rows)
        torch.cuda.current_stream().wait_stream(side)
        graph.replay()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(replays):
            graph.replay()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / (replays * launches) * 1e3
    except Exception as exc:  # capture refused: report no figure rather than a host-bound one
        log(f"append graph timing unavailable: {exc}")
        return None


def time_decode_graph(torch, ops, pool, spec, q, k_new, v_new, y_eager, L, B, nq, replays):
    """The headline step as a serving loop replays it: one thb_dplan_build,
    then for each layer thb_attn_append_dplan (append + decode in one launch
    over the device plan), captured once in a HIP graph.  Returns (us per
    layer over the replays, outputs bit-identical to the eager step's)."""
    plan = ops.DevicePlan(pool, max_m=B, q_heads=nq, append=True)
    yg = torch.empty_like(y_eager)

    def body():
        plan.build(spec, q[0], yg[0])
        for layer in range(L):
            plan.attn_append(layer, k_new[layer], v_new[layer], q[layer], yg[layer])

    body()  # outside the capture first: nothing left to set up
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            body()
    torch.cuda.current_stream().wait_stream(side)
    yg.fill_(float("nan"))
    us = _time_steps(torch, graph.replay, replays, 2) / L
    same = bool(torch.equal(yg, y_eager))
    pool.status()  # the plan's checks passed on every replay
    del graph
    plan.close()
    return us, same


def time_reference_mode(torch, ops, dev, B, ctx, nq, nkv, hd, layers=4, steps=5):
    """The headline shape in the reference's compatibility mode: KV stored
    as bf16 by truncation (kv_store.wgsl:20-22) in pages of 32 tokens, f32
    queries, outputs and appended rows.  Two dispatch patterns per layer:
    one batched call (the rows of every sequence, seq taken per row) and the
    reference's own pattern, kv_store for all rows then one attn per
    sequence chunk with AttnSpec.seq fixed (transformer/forward.rs:314-336),
    issued from Python.  A one-sequence call holds only kv_heads groups, so
    that pattern runs on a pool of 256-key partitions (128 workgroups per
    call; the default 4096 gives 8); the batched call on the default.  Events
    around `steps` passes; us per layer."""
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    pl = 32

    def make(part_len):
        pool = KvPool(ArenaSpec([ctx] * B, B * (-(-ctx // pl))), nkv, hd, layers=layers, page_len=pl,
                      kv_dtype="bf16", part_len=part_len)
        scattered_alloc(pool, [ctx] * B, random.Random(1012), pl)
        pool.sync()
        gg = torch.Generator(device=dev)
        gg.manual_seed(1012)
        for layer in range(layers):
            for t in pool.layer_tensors(layer):
                t.view(torch.bfloat16).normal_(generator=gg)
        return pool

    g = torch.Generator(device=dev)
    g.manual_seed(1013)
    rows = RowMeta(B)
    rows.write([ctx - 1] * B, list(range(B)), B)
    q = torch.randn(B, nq, hd, device=dev, generator=g)
    k = torch.randn(B, nkv, hd, device=dev, generator=g)
    v = torch.randn(B, nkv, hd, device=dev, generator=g)
    y = torch.empty_like(q)
    scale = 1.0 / math.sqrt(hd)
    batched = ops.AttnSpec(q_heads=nq, window=0, scale=scale, m=B, causal=True, seq=None, args=rows)
    per_seq = [ops.AttnSpec(q_heads=nq, window=0, scale=scale, m=1, causal=True, seq=s, args=rows, row_off=s)
               for s in range(B)]

    def one_call(pool):
        for layer in range(layers):
            ops.kv_store_attn(k, v, q, pool, layer, y, batched)

    def reference_pattern(pool):
        for layer in range(layers):
            ops.kv_store(k, v, pool, layer, B, rows)
            for s in range(B):
                ops.attn(q[s:s + 1], pool, layer, y[s:s + 1], per_seq[s])

    out = {}
    for name, fn, part_len in (("batched", one_call, 0), ("per_sequence", reference_pattern, 256)):
        pool = make(part_len)
        out[name] = _time_steps(torch, lambda: fn(pool), steps, 2) / layers
        pool.close()
        torch.cuda.empty_cache()
    return out


def time_hbm_ceiling(torch, dev, mib=1024, reps=5):
    """The device's achievable linear HBM rate, measured next to the 8 TB/s
    specification: thb_hbm_stream over `mib` MiB with 16-byte non-temporal
    accesses (the attention and page-move kernels' access kind), read-only
    and copy, the best of a sweep of workgroup counts (median of `reps`
    launches each, HIP events on the launch stream); and torch's own
    device copy of the same buffers for comparison.  Copy rates count the
    bytes read plus the bytes written."""
    import ctypes

    from flint_amd import _lib
    from flint_amd.pool import _stream_ptr

    nbytes = mib << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    src.random_(0, 255)
    dst = torch.empty_like(src)
    L = _lib.lib()
    stream = _stream_ptr(None)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e-3)
        ts.sort()
        return ts[len(ts) // 2]

    best = {}
    for mode, name in ((0, "read"), (1, "copy")):
        for wg in (256, 512, 1024, 2048, 4096):
            def run(mode=mode, wg=wg):
                _lib.check(L.thb_hbm_stream(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                            nbytes, mode, wg, stream))
            t = timed(run)
            moved = nbytes * (2 if mode else 1)
            gbps = moved / t / 1e9
            if gbps > best.get(name, (0.0, 0))[0]:
                best[name] = (gbps, wg)
    t_torch = timed(lambda: dst.copy_(src))
    del src, dst
    torch.cuda.empty_cache()
    return {"read_GBps": round(best["read"][0], 1), "read_workgroups": best["read"][1],
            "copy_GBps": round(best["copy"][0], 1), "copy_workgroups": best["copy"][1],
            "torch_copy_GBps": round(2 * nbytes / t_torch / 1e9, 1), "bytes": nbytes,
            "read_frac_of_spec": round(best["read"][0] / PEAK_HBM_GBPS, 4),
            "copy_frac_of_spec": round(best["copy"][0] / PEAK_HBM_GBPS, 4),
            "note": f"thb_hbm_stream over {mib} MiB, linear 16-byte non-temporal accesses, 512-lane workgroups "
                    f"(best of 256-4096), median of {reps} launches; copy = read + write bytes"}


def time_gather_copy(torch, ops, pool, layer, B, ctx, nkv, hd, pl, dev, reps=3):
    """Gather of every sequence of one layer into contiguous buffers, the
    scatter of those buffers back (the pool is left bit-identical), and a
    block copy of 512 whole pages (every layer) in a second pool of the same
    geometry whose sequences leave 512 pages free (the decode pool holds
    exactly its sequences' pages).  HIP events around `reps` replays of a
    captured graph of the B gather (scatter) calls, and around `reps`
    block-copy calls; algorithmic bytes = 2 x bytes moved."""
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    kb = torch.empty(B, nkv, ctx, hd, dtype=torch.int16, device=dev)
    vb = torch.empty_like(kb)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    def sweep(fn):
        for s in range(B):
            fn(pool, layer, s, 0, ctx, kb[s], vb[s])

    def graph_of_fn(work):
        # one graph of many calls: Python issues a call in ~10 us, longer than the kernel
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            work()  # warm
            side.synchronize()
            with torch.cuda.graph(graph, stream=side):
                work()
        torch.cuda.current_stream().wait_stream(side)
        return graph

    gg, gs = graph_of_fn(lambda: sweep(ops.kv_gather)), graph_of_fn(lambda: sweep(ops.kv_scatter))
    ranges = [(s, layer, 0, ctx) for s in range(B)]
    bg = graph_of_fn(lambda: ops.kv_gather_batch(pool, ranges, kb, vb))
    bs = graph_of_fn(lambda: ops.kv_scatter_batch(pool, ranges, kb, vb))
    for gr in (gg, gs, bg, bs):
        gr.replay()
    torch.cuda.synchronize()
    ev += [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(reps):
        gg.replay()
    ev[1].record()
    for _ in range(reps):
        gs.replay()
    ev[2].record()
    for _ in range(reps):
        bg.replay()
    ev[3].record()
    for _ in range(reps):
        bs.replay()
    ev[4].record()
    torch.cuda.synchronize()
    del gg, gs, bg, bs
    moved = B * nkv * ctx * hd * 2 * 2
    g_us = ev[0].elapsed_time(ev[1]) / reps * 1e3
    s_us = ev[1].elapsed_time(ev[2]) / reps * 1e3
    bg_us = ev[2].elapsed_time(ev[3]) / reps * 1e3
    bs_us = ev[3].elapsed_time(ev[4]) / reps * 1e3
    del kb, vb
    spare, held = 512, 3584  # pages: copy destinations / held by the second pool's sequences
    cpool = KvPool(ArenaSpec([ctx] * (-(-held * pl // ctx)), held + spare), nkv, hd, layers=pool.layers,
                   page_len=pl, kv_dtype="f16")
    scattered_alloc(cpool, [ctx] * (held * pl // ctx), random.Random(7), pl)
    used = [p for s in range(held * pl // ctx) for p in cpool.arena.table_of(s)]
    free = sorted(set(range(cpool.arena.pages())) - set(used))[:spare]
    triples = [[used[i * 7 % len(used)], free[i], pl] for i in range(len(free))]
    ops.block_copy(cpool, triples)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # a spin kernel ahead of the first event keeps the GPU busy while Python
    # prepares the calls (the triple list costs more host time than the copy)
    torch.cuda._sleep(20_000_000)
    c0.record()
    for _ in range(reps):
        ops.block_copy(cpool, triples)
    c1.record()
    torch.cuda.synchronize()
    c_us = c0.elapsed_time(c1) / reps * 1e3
    c_moved = len(triples) * pool.layers * 2 * nkv * pl * hd * 2
    # bulk append: a prefill-sized call (8 sequences x 512 consecutive positions) into the
    # second pool, f16 sources, one layer per call, all layers in turn
    rows_b = RowMeta(4096)
    rows_b.write([p for _ in range(8) for p in range(512)], [s for s in range(8) for _ in range(512)], 4096)
    kb = torch.randn(4096, nkv, hd, device=dev).half()
    vb2 = torch.randn(4096, nkv, hd, device=dev).half()
    def append_all():
        for layer in range(pool.layers):
            ops.kv_store(kb, vb2, cpool, layer, 4096, rows_b)

    ga = graph_of_fn(append_all)  # the runs are uploaded by the warm call, outside the graph
    ga.replay()
    torch.cuda.synchronize()
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record()
    for _ in range(reps):
        ga.replay()
    b1.record()
    torch.cuda.synchronize()
    del ga
    a_us = b0.elapsed_time(b1) / (reps * pool.layers) * 1e3
    a_bytes = 4096 * nkv * hd * 2 * (2 + 2)  # K and V: f16 source read + f16 page write
    cpool.close()

    def rec(us, nbytes, note):
        gbps = 2 * nbytes / (us * 1e-6) / 1e9
        return {"us_per_call": round(us, 1), "GBps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
                "bytes_moved": nbytes, "note": note}

    return {"gather": rec(g_us, moved, f"kv_gather of all {B} sequences x {ctx} tokens of one layer "
                                       f"({B} calls, one graph) into [kv_heads, ctx, head_dim]"),
            "scatter": rec(s_us, moved, f"kv_scatter of the same {B} buffers back ({B} calls, one graph)"),
            "gather_batch": rec(bg_us, moved, f"kv_gather_batch: the same {B} sequences in one call (one launch)"),
            "scatter_batch": rec(bs_us, moved, f"kv_scatter_batch: the same {B} buffers back in one call"),
            "block_copy": rec(c_us, c_moved, f"one block_copy call of {len(triples)} whole pages x "
                                             f"{pool.layers} layers x K,V x {nkv} heads"),
            "append_bulk": {"us_per_call": round(a_us, 2), "GBps": round(a_bytes / (a_us * 1e-6) / 1e9, 1),
                            "frac": round(a_bytes / (a_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4), "bytes": a_bytes,
                            "note": "kv_store of a 4096-row prefill call (8 seqs x 512 positions), f16 source, "
                                    "one graph of a call per layer; bytes = rows x kv_heads x head_dim x "
                                    "(2 B read + 2 B write) x K,V"}}


def time_o_proj(torch, ops, dev, B, nq, hd, layers=32, reps=5):
    """The attention consumer at the C2 shape: o_proj (Llama-3-8B: 4096 x
    4096 bf16 weights, one matrix per layer) on the bf16 attention output of
    B rows, accumulated into the f32 residual (ops::gemm_acc with acc, as
    transformer/forward.rs:338-351 calls it).  A graph of one call per layer,
    replayed `reps` times between events; distinct weights per layer, so
    every launch streams its 32 MiB from HBM."""
    hidden = nq * hd
    w = [(torch.randn(hidden, hidden, device=dev) * 0.02).to(torch.bfloat16) for _ in range(layers)]
    x = torch.randn(B, hidden, device=dev).to(torch.bfloat16)
    y = torch.zeros(B, hidden, device=dev)

    def run():
        for layer in range(layers):
            ops.gemm_acc(x, w[layer], y, B, True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        run()
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / (reps * layers) * 1e3
    nbytes = hidden * hidden * 2 + B * hidden * 2 + 2 * B * hidden * 4  # W, x, y read + write
    del graph, w
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"us_per_call": round(us, 2), "GBps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "bytes_per_call": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                         "frac": round(gbps / PEAK_HBM_GBPS, 4)},
            "note": f"thb_gemm_acc (gemm_split at 17-64 rows): y[{B}, {hidden}] += x[{B}, {hidden}] bf16 . W[{hidden}, {hidden}]^T "
                    f"bf16, acc into f32, distinct W per layer, graph of {layers} calls; bytes = W + x + y read/write"}


def time_identity_leg(torch, ops, cfg, q, k_new, v_new, steps=5):
    """The reference's attention probe (thuban_bench/src/probes/attn.rs
    :97-133) times one attention with an identity block table and with a
    shuffled one.  Here: the same fused append + decode step over a second
    pool whose sequences own consecutive pages (sequence s holds pages
    s * ctx / P ...), events around layers 1..L-1 of `steps` steps; returns
    us per layer."""
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    L, B, ctx = cfg["layers"], cfg["batch"], cfg["ctx"]
    nq, nkv, hd, pl = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"], cfg["page_len"]
    pool = KvPool(ArenaSpec([ctx] * B, B * (-(-ctx // pl))), nkv, hd, layers=L, page_len=pl, kv_dtype="f16")
    for s in range(B):
        pool.alloc(s, 0, ctx)
    g = torch.Generator(device=q.device)
    g.manual_seed(1002)
    for layer in range(L):
        for t in pool.layer_tensors(layer):
            t.view(torch.float16).normal_(generator=g)
    rows = RowMeta(B)
    rows.write([ctx - 1] * B, list(range(B)), B)
    y = torch.empty_like(q[0])
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1.0 / math.sqrt(hd), m=B, causal=True, seq=None, args=rows)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for i in range(-2, steps):
        for layer in range(L):
            if i >= 0 and layer == 1:
                ev[i][0].record()
            ops.kv_store_attn(k_new[layer], v_new[layer], q[layer], pool, layer, y, spec)
        if i >= 0:
            ev[i][1].record()
    torch.cuda.synchronize()
    us = sum(e[0].elapsed_time(e[1]) for e in ev) / steps / (L - 1) * 1e3
    pool.close()
    return us


def time_rope_step(torch, ops, pool, rows, positions, seqs, q, k_new, v_new, L, B, nq, hd, scale, steps=5):
    """The per-layer step with rotary embedding (Llama-3: theta 500000,
    rot = head_dim) three ways: the reference's four launches (rope q, rope
    k, kv_store, attn; transformer/forward.rs:265-336), thb_attn_append_rope
    (one launch), and the step captured in a HIP graph over a device plan
    (one thb_dplan_build per step, thb_attn_step_dplan with the rope and the
    append per layer).  Copies of q and k are rotated, so the main
    workload's buffers stay as they were.  Events around `steps` passes over
    the layers; returns us per layer for each."""
    from flint_amd.rope import Rope, kv_store_attn_rope, rope_rows

    ctx = max(positions) + 1
    rope = Rope.from_theta(ctx, hd, 500000.0)
    qr, kr = q.clone(), k_new.clone()
    y = torch.empty_like(q[0])
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=scale, m=B, causal=True, seq=None, args=rows)
    nkv = k_new.shape[2]

    def unfused():
        for layer in range(L):
            rope_rows(qr[layer], nq, rope, rows, B)
            rope_rows(kr[layer], nkv, rope, rows, B)
            ops.kv_store(kr[layer], v_new[layer], pool, layer, B, rows)
            ops.attn(qr[layer], pool, layer, y, spec)

    def fused():
        for layer in range(L):
            kv_store_attn_rope(k_new[layer], v_new[layer], q[layer], pool, layer, y, spec, rope)

    plan = ops.DevicePlan(pool, max_m=B, q_heads=nq, append=True)
    plan.set_pos_limit(rope.max_pos)

    def planned():
        plan.build(spec, q[0], y)
        for layer in range(L):
            plan.step(layer, q[layer], y, k_src=k_new[layer], v_src=v_new[layer], rope=rope)

    planned()  # outside the capture first: nothing left to set up
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            planned()
    torch.cuda.current_stream().wait_stream(side)

    out = {}
    for name, fn in (("unfused", unfused), ("fused", fused), ("graph", graph.replay)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) / (steps * L) * 1e3
    pool.status()  # every replay's plan checks passed
    del graph
    plan.close()
    return out


def cpu_model():
    """The host CPU's model name and logical core count (nproc)."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return name, os.cpu_count()


def cpu_median(fn, seconds, min_runs=20, warmup=3):
    """Median wall time of fn() over at least min_runs runs (and at least
    `seconds` of work) after `warmup` untimed runs; returns (median s, runs,
    last result)."""
    for _ in range(warmup):
        out = fn()
    times, t_start = [], time.perf_counter()
    while len(times) < min_runs or time.perf_counter() - t_start < seconds:
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times), out


def cpu_baseline_record(value_gbps, median_s, runs, sample):
    import oracle

    name, nproc = cpu_model()
    return {"value": round(value_gbps, 3), "unit": "GB/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": sample, "median_us": round(median_s * 1e6, 1), "runs": runs, "warmup": 3, "nproc": nproc,
            "cpu_model": name,
            "label": "restatement of reference algorithm (oracle/oracle.c, f32 online softmax of attn.wgsl), "
                     "not reference binary"}


def cpu_baseline(torch, pool, q0, y0, cfg, scale, seconds):
    """Times the oracle on layer 0 of the workload: median of >= 20 runs
    after 3 warm-ups."""
    import numpy as np

    import oracle

    kw, vw = pool.read_layer(0)
    info = pool.arena.info()
    ref = oracle.Layer(cfg["kv_heads"], cfg["head_dim"], info.pages, cfg["page_len"],
                       np.array(pool.arena.table(), np.uint32), info.max_pages, oracle.KV_F16, k=kw, v=vw)
    B, ctx = cfg["batch"], cfg["ctx"]
    args = oracle.row_meta([ctx - 1] * B, list(range(B)))
    qn = q0.float().cpu().numpy()
    med, runs, y = cpu_median(lambda: ref.attn(qn, args, B, cfg["q_heads"], scale, precision=1), seconds)
    err = float(np.max(np.abs(y - y0.float().cpu().numpy())))
    log(f"cpu baseline: median {med * 1e3:.1f} ms over {runs} runs; max |cpu - gpu| = {err:.2e}")
    return med, runs, err


def c1_cpu_baseline(torch, pool, rows, k, v, q, y, ctx, nq, hd, byts, seconds):
    """C1, the shape BASELINE.json defines on the reference's CPU path: the
    oracle's append (kv_store.wgsl) + f32 blockwise attention (attn.wgsl) of
    the 4-row step on a host copy of the layer, median of >= 20 runs after 3
    warm-ups."""
    import numpy as np

    import oracle

    torch.cuda.synchronize()
    kw, vw = pool.read_layer(0)
    info = pool.arena.info()
    ref = oracle.Layer(pool.kv_heads, hd, info.pages, pool.page_len, np.array(pool.arena.table(), np.uint32),
                       info.max_pages, oracle.KV_F16, k=kw, v=vw)
    B = len(ctx)
    args = oracle.row_meta(ctx, list(range(B)))
    kn, vn, qn = k.float().cpu().numpy(), v.float().cpu().numpy(), q.float().cpu().numpy()

    def step():
        ref.kv_store(kn, vn, args, B)
        return ref.attn(qn, args, B, nq, 1.0 / math.sqrt(hd), precision=1)

    med, runs, yc = cpu_median(step, seconds)
    err = float(np.max(np.abs(yc - y.float().cpu().numpy())))
    log(f"C1 cpu baseline: median {med * 1e6:.1f} us over {runs} runs; max |cpu - gpu| = {err:.2e}")
    return cpu_baseline_record(byts / med / 1e9, med, runs,
                               f"the C1 step (append 1 token + decode of {B} seqs, ctx {ctx}), median of {runs} "
                               f"runs after 3 warm-ups, {med * 1e6:.1f} us/run, max |cpu-gpu| {err:.1e}")


def _time_steps(torch, step, steps, warmup):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        step()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps * 1e3  # us per step


def measure_secondary(name, args):
    """One of the other BASELINE configurations (see the module docstring):
    its record as a dict.  Synthetic N(0,1) data, block tables scattered."""
    import numpy as np
    import torch

    from flint_amd import ops
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    out = {"metric": "paged attention us/step + achieved HBM GB/s (% peak) [secondary config]", "unit": "GB/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16", "data": "synthetic N(0,1), block tables randomly scattered",
           "cpu_baseline": None}

    def make(seq_lens, pages, nkv, hd, layers, pl=16):
        return KvPool(ArenaSpec(list(seq_lens), pages), nkv, hd, layers=layers, page_len=pl, kv_dtype="f16",
                      part_len=args.part_len)

    def randomize(pool, layers, seed):
        g.manual_seed(seed)
        for layer in layers:
            for t in pool.layer_tensors(layer):
                t.view(torch.float16).normal_(generator=g)

    def spec(rows, nq, hd, m, window=0, softcap=0.0):
        return ops.AttnSpec(q_heads=nq, window=window, scale=1.0 / math.sqrt(hd), m=m, causal=True, seq=None,
                            args=rows, softcap=softcap)

    if name == "qwen2-0.5b":  # C1: one layer, B=4, ctx U[128, 512], 256-page pool
        rng = random.Random(1001)
        nq, nkv, hd, L, B = 14, 2, 64, 1, 4
        ctx = [rng.randint(128, 512) for _ in range(B)]
        budget = [c + 1 for c in ctx]
        pool = make(budget, 256, nkv, hd, L)
        scattered_alloc(pool, budget, rng, 16)
        randomize(pool, range(L), 1001)
        rows = RowMeta(B)
        rows.write(ctx, list(range(B)), B)
        k = torch.randn(B, nkv, hd, device=dev, generator=g)
        v = torch.randn(B, nkv, hd, device=dev, generator=g)
        q = torch.randn(B, nq, hd, device=dev, generator=g)
        y = torch.empty_like(q)
        sp = spec(rows, nq, hd, B)
        # ~8 us steps issued from Python: at least 100 of them, so that a stall of the host
        # thread does not dominate the average
        us = _time_steps(torch, lambda: ops.kv_store_attn(k, v, q, pool, 0, y, sp), max(args.steps, 100),
                         max(args.warmup, 10))
        byts = sum(c + 1 for c in ctx) * nkv * hd * 2 * 2
        # the same step as a serving loop replays it, captured once in a HIP graph (thb_attn plans
        # on the host and cannot be captured), 20 steps per graph: thb_dplan_build +
        # thb_attn_append_dplan (the append inside the attention launch), and for comparison
        # kv_store + thb_dplan_build + thb_attn_dplan
        def graph_us(fused):
            plan = ops.DevicePlan(pool, max_m=B, q_heads=nq, append=fused)
            yg = torch.empty_like(q)

            def body():
                if not fused:
                    ops.kv_store(k, v, pool, 0, B, rows)
                plan.build(sp, q, yg)
                if fused:
                    plan.attn_append(0, k, v, q, yg)
                else:
                    plan.attn(0, q, yg)

            body()  # outside the capture first: nothing left to set up
            torch.cuda.synchronize()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(graph, stream=side):
                    for _ in range(20):
                        body()
            torch.cuda.current_stream().wait_stream(side)
            yg.fill_(float("nan"))
            t = _time_steps(torch, graph.replay, max(1, args.steps // 5), 2) / 20
            ops.kv_store_attn(k, v, q, pool, 0, y, sp)
            torch.cuda.synchronize()
            same = bool(torch.equal(y, yg))
            pool.status()
            del graph
            plan.close()
            return t, same

        gus, same = graph_us(True)
        gus3, same3 = graph_us(False)
        out["graph_step"] = {"us_per_step": round(gus, 2), "GBps": round(byts / (gus * 1e-6) / 1e9, 1),
                             "bit_identical_to_eager": same and same3,
                             "three_launch_us_per_step": round(gus3, 2),
                             "note": "thb_dplan_build + thb_attn_append_dplan (append and decode in one launch) "
                                     "captured in a HIP graph (20 steps per graph), replayed; "
                                     "three_launch_us_per_step: kv_store + thb_dplan_build + thb_attn_dplan "
                                     "the same way; the eager line above is one fused launch per step issued "
                                     "from Python with the plan made on the host"}
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = c1_cpu_baseline(torch, pool, rows, k, v, q, y, ctx, nq, hd, byts,
                                                  min(args.cpu_seconds, 3.0))
        out["config"] = {"workload": f"qwen2-0.5b C1: 1 layer, B=4, ctx {ctx}, 14q/2kv/hd64, page 16, f16 KV, "
                                     "step = append 1 token + decode (fused), f32 sources"}
    elif name == "qwen3-8b":  # C3: 64 ragged decode rows + 8 x 512 prefill rows in one call per layer
        rng = random.Random(1003)
        nprng = np.random.default_rng(1003)
        nq, nkv, hd, L, pre = 32, 8, 128, 4, 512
        ctx = np.clip(np.round(nprng.lognormal(math.log(2048), 1.0, 64)), 256, 32768).astype(int).tolist()
        budget = [c + 1 for c in ctx] + [pre] * 8
        need = sum(-(-b // 16) for b in budget)
        n_fill = 256
        pages = int(need / 0.4) + 64
        fill_cap = -(-pages // n_fill) * 4 * 16
        pool = make([fill_cap] * n_fill + budget, pages, nkv, hd, L)
        owners = [rng.randrange(n_fill) for _ in range(pages)]  # 60% pre-occupied, fragmented free list
        have = [0] * n_fill
        for s in owners:
            pool.alloc(s, have[s] * 16, 16)
            have[s] += 1
        order = list(range(n_fill))
        rng.shuffle(order)
        freed = 0
        for s in order:
            if freed >= 0.4 * pages:
                break
            freed += have[s]
            pool.free_seq(s)
        for i, b in enumerate(budget):
            pool.alloc(n_fill + i, 0, b)
        randomize(pool, range(L), 1003)
        positions = list(ctx) + [p for _ in range(8) for p in range(pre)]
        seqs = [n_fill + i for i in range(64)] + [n_fill + 64 + i for i in range(8) for _ in range(pre)]
        m = len(seqs)
        rows = RowMeta(m)
        rows.write(positions, seqs, m)
        k = torch.randn(m, nkv, hd, device=dev, generator=g).half()
        v = torch.randn(m, nkv, hd, device=dev, generator=g).half()
        q = torch.randn(m, nq, hd, device=dev, generator=g).half()
        y = torch.empty_like(q)
        sp = spec(rows, nq, hd, m)

        def step():
            for layer in range(L):
                ops.kv_store_attn(k, v, q, pool, layer, y, sp)
        us = _time_steps(torch, step, args.steps, args.warmup) / L
        byts = sum(c + 1 for c in ctx) * nkv * hd * 2 * 2 + 8 * pre * nkv * hd * 2 * 2
        flops = 8 * (pre * (pre + 1) // 2) * nq * hd * 4
        # the same mixed step planned on the device (work-list plan) and captured in a HIP graph as a
        # serving loop runs it: one thb_dplan_build per model step, then for each of Qwen3-8B's 36
        # layers (the L layer pools cycled) kv_store + thb_attn_dplan; 2 steps per graph
        n_model = 36
        plan = ops.DevicePlan(pool, max_m=m, q_heads=nq, prefill=True)
        yg = torch.empty_like(q)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for _ in range(2):
                    plan.build(sp, q, yg)
                    for i in range(n_model):
                        ops.kv_store(k, v, pool, i % L, m, rows)
                        plan.attn(i % L, q, yg)
        torch.cuda.current_stream().wait_stream(side)
        gus = _time_steps(torch, graph.replay, max(1, args.steps // 10), 1) / (2 * n_model)
        bus = _time_steps(torch, lambda: [plan.build(sp, q, yg) for _ in range(20)], 3, 1) / 20
        ops.kv_store_attn(k, v, q, pool, (n_model - 1) % L, y, sp)
        torch.cuda.synchronize()
        same = bool(torch.equal(y, yg))
        del graph
        plan.close()
        out["list_plan_graph"] = {"us_per_layer": round(gus, 1), "eager_us_per_layer": round(us, 1),
                                  "ratio_to_eager": round(gus / us, 3), "build_us": round(bus, 1),
                                  "bit_identical_to_eager": same,
                                  "note": "thb_dplan_create_ex(THB_DPLAN_PREFILL): decode rows and the 8 prefill "
                                          "chunks planned on the device (thb_dplan_build once per 36-layer model "
                                          "step, build_us alone), kv_store + thb_attn_dplan per layer, captured "
                                          "(2 steps per graph) and replayed; eager = kv_store + thb_attn per layer "
                                          "with the host plan cached across layers and steps"}
        # the prefill rows alone (their K/V already appended), for the matrix-core roofline
        rp = RowMeta(8 * pre)
        rp.write(positions[64:], seqs[64:], 8 * pre)
        qp, yp = q[64:].contiguous(), torch.empty_like(q[64:])
        spp = spec(rp, nq, hd, 8 * pre)
        pus = _time_steps(torch, lambda: [ops.attn(qp, pool, layer, yp, spp) for layer in range(L)],
                          args.steps, args.warmup) / L
        out["prefill"] = {"us_per_layer": round(pus, 1), "TFLOPs": round(flops / (pus * 1e-6) / 1e12, 1),
                          "mfma_frac_of_2.5PF": round(flops / (pus * 1e-6) / 2.5e15, 4),
                          "flops": flops, "note": "8 x 512 causal rows; unmasked (q,k) pairs x 4 x nq x hd"}
        # Qwen3's layer step proper: q_norm/k_norm + rotation (norm_rope), append, attention,
        # as the reference's four dispatches vs one thb_attn_step
        from flint_amd.rope import Rope, kv_store_rope, rope_rows
        wq = torch.rand(hd, device=dev, generator=g) + 0.5
        wk = torch.rand(hd, device=dev, generator=g) + 0.5
        rope = Rope.from_theta(max(positions) + 1, hd, 1e6, q_norm=wq, k_norm=wk)
        qr, kr = q.clone(), k.clone()

        def unfused():
            for layer in range(L):
                rope_rows(qr, nq, rope, rows, m, norm_w=wq)
                rope_rows(kr, nkv, rope, rows, m, norm_w=wk)
                ops.kv_store(kr, v, pool, layer, m, rows)
                ops.attn(qr, pool, layer, y, sp)

        def fused():
            for layer in range(L):
                ops.attn_step(pool, layer, sp, q, y, k_src=k, v_src=v, rope=rope)

        r_un = _time_steps(torch, unfused, args.steps, args.warmup) / L
        r_fu = _time_steps(torch, fused, args.steps, args.warmup) / L
        out["norm_rope_step"] = {"fused_us_per_layer": round(r_fu, 1), "unfused_us_per_layer": round(r_un, 1),
                                 "note": "the same mixed call with q/k RMSNorm + rotation: rope_rows(q), "
                                         "rope_rows(k), kv_store, attn vs one thb_attn_step"}
        out["config"] = {"workload": "qwen3-8b C3: 64 decode rows (log-normal ctx in [256, 32768], median 2048) "
                                     "+ 8 x 512-token causal prefill chunks in one call per layer, 32q/8kv/hd128, "
                                     f"page 16, f16 KV, pool {pages} pages 60% pre-occupied, {L} layers cycled"}
    elif name == "gemma2-9b":  # C4: verify 4 drafts per sequence, window / global layers alternating
        rng = random.Random(1004)
        nq, nkv, hd, L, B, ctx = 16, 8, 256, 4, 16, 8192
        pool = make([ctx + 4] * B, None, nkv, hd, L)
        scattered_alloc(pool, [ctx + 4] * B, rng, 16)
        randomize(pool, range(L), 1004)
        m = 4 * B
        rows = RowMeta(m)
        rows.write([ctx + i for _ in range(B) for i in range(4)], [s for s in range(B) for _ in range(4)], m)
        k = torch.randn(m, nkv, hd, device=dev, generator=g).half()
        v = torch.randn(m, nkv, hd, device=dev, generator=g).half()
        q = torch.randn(m, nq, hd, device=dev, generator=g).half()
        y = torch.empty_like(q)
        specs = [spec(rows, nq, hd, m, window=4096 if layer % 2 == 0 else 0, softcap=50.0) for layer in range(L)]

        def step():
            for layer in range(L):
                ops.kv_store_attn(k, v, q, pool, layer, y, specs[layer])
        us = _time_steps(torch, step, args.steps, args.warmup) / L
        for kind, first in (("window", 0), ("global", 1)):
            def half_step(first=first):
                for layer in range(first, L, 2):
                    ops.kv_store_attn(k, v, q, pool, layer, y, specs[layer])
            lus = _time_steps(torch, half_step, args.steps, args.warmup) / (L // 2)
            keys = 4096 + 4 if kind == "window" else ctx + 4
            lb = B * keys * nkv * hd * 2 * 2 + m * nkv * hd * 2 * 2
            out[f"{kind}_layer"] = {"us": round(lus, 1), "pct_of_peak": round(100 * lb / (lus * 1e3) / PEAK_HBM_GBPS, 1)}
        byts = B * (4096 + ctx + 8) // 2 * nkv * hd * 2 * 2 + m * nkv * hd * 2 * 2
        # Gemma-2-shaped chunked prefill: 8 fresh 512-token causal chunks, window 4096, soft-cap 50
        # (the head_dim-256 path of attn_prefill_wide), two layers of their own pool
        npre, pre = 8, 512
        pp = make([pre] * npre, npre * pre // 16, nkv, hd, 2)
        for s_ in range(npre):
            pp.alloc(s_, 0, pre)
        randomize(pp, range(2), 1014)
        rp = RowMeta(npre * pre)
        rp.write([p for _ in range(npre) for p in range(pre)], [s_ for s_ in range(npre) for _ in range(pre)],
                 npre * pre)
        qp = torch.randn(npre * pre, nq, hd, device=dev, generator=g).half()
        yp = torch.empty_like(qp)
        spp = spec(rp, nq, hd, npre * pre, window=4096, softcap=50.0)
        pus = _time_steps(torch, lambda: [ops.attn(qp, pp, layer, yp, spp) for layer in range(2)],
                          args.steps, args.warmup) / 2
        pflops = npre * (pre * (pre + 1) // 2) * nq * hd * 4
        out["gemma_prefill"] = {"us_per_layer": round(pus, 1), "TFLOPs": round(pflops / (pus * 1e-6) / 1e12, 1),
                                "mfma_frac_of_2.5PF": round(pflops / (pus * 1e-6) / 2.5e15, 4), "flops": pflops,
                                "note": "8 x 512 causal rows, 16q/8kv/hd256, window 4096, soft-cap 50, f16 queries "
                                        "and outputs; unmasked (q,k) pairs x 4 x nq x hd"}
        pp.close()
        out["config"] = {"workload": "gemma2-9b C4: B=16 at ctx 8192, 16q/8kv/hd256, soft-cap 50, layers alternate "
                                     "window 4096 / global; step = append 4 drafts + 4-row causal verify (fused), "
                                     f"{L} layers"}
    else:  # qwen2.5-32b, C5: 64 layers, 4 x 131072 forked to 8, 25% evicted and reallocated, decode
        rng = random.Random(1005)
        nq, nkv, hd, L = 40, 8, 128, 64
        ctx, new_ctx = 131072 - 5, 20000
        pages = 4 * (131072 // 16) + 4 + 2 * (-(-(new_ctx + 1) // 16)) + 64
        pool = make([131072 + 8] * 8 + [new_ctx + 8] * 2, pages, nkv, hd, L)
        scattered_alloc(pool, [ctx] * 4, rng, 16)
        for s in range(4):
            pool.fork(s, 4 + s, ctx)
        evict = rng.sample(range(8), 2)
        for s in evict:
            pool.free_seq(s)
        live = [s for s in range(8) if s not in evict] + [8, 9]
        for s in (8, 9):
            pool.alloc(s, 0, new_ctx)
        pos = [ctx if s < 8 else new_ctx for s in live]
        for s, p in zip(live, pos):
            pool.alloc(s, p, 1)
        randomize(pool, (0, L - 1), 1005)
        m = len(live)
        rows = RowMeta(m)
        rows.write(pos, live, m)
        k = torch.randn(m, nkv, hd, device=dev, generator=g).half()
        v = torch.randn(m, nkv, hd, device=dev, generator=g).half()
        q = torch.randn(m, nq, hd, device=dev, generator=g).half()
        y = torch.empty_like(q)
        sp = spec(rows, nq, hd, m)

        def step():
            for layer in range(L):
                ops.kv_store_attn(k, v, q, pool, layer, y, sp)
        us = _time_steps(torch, step, max(1, args.steps // 5), max(1, args.warmup // 2)) / L
        byts = sum(p + 1 for p in pos) * nkv * hd * 2 * 2
        out["arena_bytes"] = pool.memory()[1]
        out["config"] = {"workload": f"qwen2.5-32b C5: 64 layers, 4 x 131072 forked to 8, evicted {evict} and "
                                     "reallocated to 2 new sequences of 20000, decode step (fused append), "
                                     "40q/8kv/hd128, page 16, f16 KV"}
    gbps = byts / (us * 1e-6) / 1e9
    out.update({"value": round(gbps, 1), "us_per_layer_step": round(us, 1),
                "pct_of_peak": round(100 * gbps / PEAK_HBM_GBPS, 1), "ms_per_step": round(us * 1e-3, 4),
                "bytes_per_layer_step": byts})
    out["config"]["config_name"] = name
    pool.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="llama3-8b", choices=sorted(CONFIGS) + list(SECONDARY))
    ap.add_argument("--part-len", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the C1, C3, C4 and C5 fields of the default line")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the timed steps, run 3 device copies of this many MiB (scale factor for the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for {max(args.gpus, world)}); "
              "the paged KV path has no multi-GPU code.", file=sys.stderr)
        sys.exit(2)

    if args.config in SECONDARY:
        print(json.dumps(measure_secondary(args.config, args)), flush=True)
        return

    import torch

    from flint_amd import ops
    from flint_amd.pool import ArenaSpec, KvPool, RowMeta

    cfg = CONFIGS[args.config]
    L, B, ctx = cfg["layers"], cfg["batch"], cfg["ctx"]
    nq, nkv, hd, pl = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"], cfg["page_len"]
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    pages = B * (-(-ctx // pl))
    log(f"pool: {L} layers x {pages} pages of {pl} tokens, {nkv} kv heads, hd {hd}")
    pool = KvPool(ArenaSpec([ctx] * B, pages), nkv, hd, layers=L, page_len=pl, kv_dtype="f16",
                  part_len=args.part_len)
    scattered_alloc(pool, [ctx] * B, random.Random(1002), pl)
    pool.sync()
    g = torch.Generator(device=dev)
    g.manual_seed(1002)
    for layer in range(L):
        k, v = pool.layer_tensors(layer)
        k.view(torch.float16).normal_(generator=g)
        v.view(torch.float16).normal_(generator=g)
    q = torch.randn(L, B, nq, hd, device=dev, generator=g).half()
    y = torch.empty_like(q)
    k_new = torch.randn(L, B, nkv, hd, device=dev, generator=g).half()
    v_new = torch.randn(L, B, nkv, hd, device=dev, generator=g).half()
    rows = RowMeta(B)
    scale = 1.0 / math.sqrt(hd)
    positions, seqs = [ctx - 1] * B, list(range(B))
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=scale, m=B, causal=True, seq=None, args=rows)
    torch.cuda.synchronize()

    # ev[i] = (before layer 1, after layer L-1) of timed step i
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]

    def step(i=None):
        rows.write(positions, seqs, B)
        for layer in range(L):
            if i is not None and layer == min(1, L - 1):
                ev[i][0].record()
            # kv_store + attn of the layer (transformer/forward.rs:300-336), one launch
            ops.kv_store_attn(k_new[layer], v_new[layer], q[layer], pool, layer, y[layer], spec)
        if i is not None:
            ev[i][1].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    t_start.record()
    for i in range(args.steps):
        step(i)
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = t_start.elapsed_time(t_end) / args.steps
    timed = ev
    per_run = max(L - 1, 1)
    attn_us = sum(e[0].elapsed_time(e[1]) for e in timed) / len(timed) / per_run * 1e3
    append_us = time_append_graph(torch, ops, pool, rows, k_new[1 % L], v_new[1 % L], 1 % L, B)
    log(f"step {ms_step:.3f} ms (host wall {wall / args.steps * 1e3:.3f} ms); fused append+attention "
        f"{attn_us:.1f} us/launch; standalone append {append_us} us/launch")
    rope_us = time_rope_step(torch, ops, pool, rows, positions, seqs, q, k_new, v_new, L, B, nq, hd, scale)
    step()  # re-append the unrotated keys: the pool and y agree again for the CPU baseline
    torch.cuda.synchronize()
    log(f"rope step: reference-shaped 4 launches {rope_us['unfused']:.1f} us/layer, "
        f"fused {rope_us['fused']:.1f} us/layer, captured over a device plan {rope_us['graph']:.1f} us/layer")
    graph_us, graph_same = time_decode_graph(torch, ops, pool, spec, q, k_new, v_new, y, L, B, nq,
                                             max(2, min(args.steps, 10)))
    log(f"captured step: {graph_us:.2f} us/layer (eager {attn_us:.2f}), bit-identical {graph_same}")

    kv_bytes = B * nkv * ctx * hd * 2 * 2
    qo_bytes = 2 * B * nq * hd * 2
    bt_bytes = B * (-(-ctx // pl)) * 4 + B * 32
    attn_bytes = kv_bytes + qo_bytes + bt_bytes
    append_bytes = B * nkv * hd * 2 * (2 + 2)
    fused_bytes = attn_bytes + append_bytes  # one fused launch per layer
    step_bytes = L * fused_bytes
    value = step_bytes / (ms_step * 1e-3) / 1e9
    achieved = fused_bytes / (attn_us * 1e-6) / 1e9
    traffic = load_traffic(f"attn_mfma_{args.config}-decode_traffic.json")

    out = {
        "metric": "paged decode us/step + achieved HBM GB/s (% peak); KV append GB/s @Llama-3-8B",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: N(0,1) f16 K/V and queries, block tables randomly scattered over the pool",
        "config": {"workload": f"{args.config}-decode: {L} layers, batch {B}, ctx {ctx}, {nq}q/{nkv}kv, "
                               f"hd {hd}, page {pl}, f16 KV; step = append 1 token/seq/layer + paged decode",
                   "layers": L, "batch": B, "ctx": ctx, "q_heads": nq, "kv_heads": nkv, "head_dim": hd,
                   "page_len": pl, "kv_dtype": "f16", "part_len": args.part_len or 4096},
        "us_per_step": round(ms_step * 1e3, 1),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 1),
        "decode": {"us_per_layer": round(attn_us, 2), "GBps": round(achieved, 1),
                   "bytes_per_launch": fused_bytes, "note": "one launch per layer: append fused into attention"},
        "append": {"us_per_launch": round(append_us, 2) if append_us else None,
                   "GBps": round(append_bytes / (append_us * 1e-6) / 1e9, 1) if append_us else None,
                   "bytes_per_launch": append_bytes,
                   "note": "standalone kv_store kernel (32 rows), graph of back-to-back launches after the steps"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic,
                     "kernel": "attn_mfma<128,f16,8 waves,ring 2> with fused append",
                     "traffic_source": "profiles/attn_mfma_llama3-8b-decode_traffic.json: rocprofv3 FETCH_SIZE and "
                                       "WRITE_SIZE passes of this kernel (committed), scaled by a 256 MiB copy; "
                                       "not counted in this run",
                     "algorithmic_bytes": fused_bytes, "launches_timed": len(timed) * per_run},
        "cpu_baseline": None,
    }
    out["graph_step"] = {"us_per_step": round(graph_us * L, 1), "eager_us_per_step": round(ms_step * 1e3, 1),
                         "us_per_layer": round(graph_us, 2), "eager_us_per_layer": round(attn_us, 2),
                         "ratio_to_eager": round(graph_us / attn_us, 4),
                         "GBps": round(fused_bytes / (graph_us * 1e-6) / 1e9, 1),
                         "bit_identical_to_eager": graph_same,
                         "note": "the step captured once in a HIP graph and replayed: one thb_dplan_build per "
                                 "step, then per layer thb_attn_append_dplan (append + decode planned on the "
                                 "device, one launch); us_per_layer includes the plan build's share"}
    out["rope"] = {"fused_us_per_layer": round(rope_us["fused"], 2),
                   "unfused_us_per_layer": round(rope_us["unfused"], 2),
                   "graph_us_per_layer": round(rope_us["graph"], 2),
                   "fused_GBps": round(fused_bytes / (rope_us["fused"] * 1e-6) / 1e9, 1),
                   "note": "step with rotary embedding (theta 5e5, rot = head_dim): rope(q), rope(k), kv_store, "
                           "attn as four launches vs thb_attn_append_rope as one; graph: the step captured over a "
                           "device plan (thb_dplan_build + thb_attn_step_dplan with the rope and the append per "
                           "layer) and replayed"}
    ident_us = time_identity_leg(torch, ops, cfg, q, k_new, v_new)
    log(f"identity block tables: {ident_us:.2f} us/layer vs scattered {attn_us:.2f}")
    out["identity_vs_scattered"] = {
        "identity_us_per_layer": round(ident_us, 2), "scattered_us_per_layer": round(attn_us, 2),
        "scattered_over_identity": round(attn_us / ident_us, 4),
        "note": "the same fused append + decode with every sequence on consecutive pages vs pages scattered "
                "at random (thuban_bench probes/attn.rs:97-133 compares identity and shuffled tables)"}
    ref_us = time_reference_mode(torch, ops, dev, B, ctx, nq, nkv, hd)
    ref_bytes = B * nkv * ctx * hd * 2 * 2 + 2 * B * nq * hd * 4 + B * nkv * hd * 4 * 2 + B * nkv * hd * 2 * 2
    log(f"reference mode (bf16 KV, page 32, f32 q/y): batched {ref_us['batched']:.1f} us/layer, "
        f"one call per sequence {ref_us['per_sequence']:.1f} us/layer")
    out["reference_mode"] = {
        "batched_us_per_layer": round(ref_us["batched"], 2),
        "batched_GBps": round(ref_bytes / (ref_us["batched"] * 1e-6) / 1e9, 1),
        "per_sequence_us_per_layer": round(ref_us["per_sequence"], 2),
        "note": "the headline shape in the reference's storage and layout (bf16 KV by truncation, page 32, f32 q, "
                "y and appended rows), 4 layers: one batched thb_attn_append per layer, and the reference's "
                "dispatch pattern (kv_store, then one attn per sequence with AttnSpec.seq fixed, 32 calls "
                "issued from Python, on a pool of 256-key partitions so that each call fills 128 CUs)"}
    out["o_proj"] = time_o_proj(torch, ops, dev, B, nq, hd, layers=L)
    ceiling = time_hbm_ceiling(torch, dev)
    out["hbm_ceiling"] = ceiling
    log(f"hbm ceiling: read {ceiling['read_GBps']} GB/s, copy {ceiling['copy_GBps']} GB/s")
    rd, cp = ceiling["read_GBps"], ceiling["copy_GBps"]
    out["roofline"]["frac_of_ceiling"] = round(achieved / rd, 4)
    out["decode"]["frac_of_read_ceiling"] = round(achieved / rd, 4)
    out["o_proj"]["frac_of_read_ceiling"] = round(out["o_proj"]["GBps"] / rd, 4)
    log(f"o_proj: {out['o_proj']['us_per_call']} us/call, {out['o_proj']['GBps']} GB/s")
    moves = time_gather_copy(torch, ops, pool, 1 % L, B, ctx, nkv, hd, pl, dev)
    log("gather/scatter/copy: " + ", ".join(f"{k} {v['us_per_call']} us {v['GBps']} GB/s" for k, v in moves.items()))
    for rec in moves.values():
        rec["frac_of_copy_ceiling"] = round(rec["GBps"] / cp, 4)
    out.update(moves)
    if args.calibrate_copy_mib:
        src = torch.empty(args.calibrate_copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration: 3 copies of {args.calibrate_copy_mib} MiB")
    if not args.no_cpu_baseline:
        med, runs, err = cpu_baseline(torch, pool, q[0], y[0], cfg, scale, args.cpu_seconds)
        out["cpu_baseline"] = cpu_baseline_record(
            attn_bytes / med / 1e9, med, runs,
            f"layer 0 of the step (decode of {B} seqs x {nq} heads x {ctx} keys), median of {runs} runs after 3 "
            f"warm-ups, {med * 1e3:.1f} ms/run, max |cpu-gpu| {err:.1e}")
    if not args.no_secondary:
        # C1, C3, C4 and C5 on the same box, in the driver's line (their own lines: --config)
        pool.close()
        del q, y, k_new, v_new
        torch.cuda.empty_cache()
        sec = argparse.Namespace(**vars(args))
        sec.steps, sec.warmup, sec.no_cpu_baseline = min(args.steps, 10), min(args.warmup, 3), True
        for name, key in (("qwen2-0.5b", "c1_qwen2_0_5b"), ("qwen3-8b", "c3_qwen3_8b"),
                          ("gemma2-9b", "c4_gemma2_9b"), ("qwen2.5-32b", "c5_qwen2_5_32b")):
            sec.no_cpu_baseline = name != "qwen2-0.5b" or args.no_cpu_baseline
            rec = measure_secondary(name, sec)
            out[key] = {k: rec[k] for k in ("value", "unit", "us_per_layer_step", "pct_of_peak", "bytes_per_layer_step",
                                            "prefill", "norm_rope_step", "window_layer", "global_layer",
                                            "gemma_prefill", "graph_step", "list_plan_graph", "arena_bytes",
                                            "cpu_baseline")
                        if k in rec and rec[k] is not None}
            out[key]["pct_of_read_ceiling"] = round(100 * rec["value"] / rd, 1)
            out[key]["workload"] = rec["config"]["workload"]
            log(f"{name}: {rec['us_per_layer_step']} us/layer, {rec['value']} GB/s ({rec['pct_of_peak']}%)")
            torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
