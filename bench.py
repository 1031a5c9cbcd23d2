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


def cpu_baseline(torch, pool, q0, y0, cfg, scale, seconds):
    """Times the oracle on layer 0 of the workload (bounded sample)."""
    import numpy as np

    import oracle

    kw, vw = pool.read_layer(0)
    info = pool.arena.info()
    ref = oracle.Layer(cfg["kv_heads"], cfg["head_dim"], info.pages, cfg["page_len"],
                       np.array(pool.arena.table(), np.uint32), info.max_pages, oracle.KV_F16, k=kw, v=vw)
    B, ctx = cfg["batch"], cfg["ctx"]
    args = oracle.row_meta([ctx - 1] * B, list(range(B)))
    qn = q0.float().cpu().numpy()
    runs, t0 = 0, time.perf_counter()
    y = None
    while True:
        y = ref.attn(qn, args, B, cfg["q_heads"], scale, precision=1)
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    err = float(np.max(np.abs(y - y0.float().cpu().numpy())))
    log(f"cpu baseline: {runs} runs in {el:.2f}s; max |cpu - gpu| = {err:.2e}")
    return el / runs, runs, err


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="llama3-8b", choices=sorted(CONFIGS))
    ap.add_argument("--part-len", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the timed steps, run 3 device copies of this many MiB (scale factor for the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for {max(args.gpus, world)}); "
              "the paged KV path has no multi-GPU code.", file=sys.stderr)
        sys.exit(2)

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
                     "algorithmic_bytes": fused_bytes, "launches_timed": len(timed) * per_run},
        "cpu_baseline": None,
    }
    if args.calibrate_copy_mib:
        src = torch.empty(args.calibrate_copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration: 3 copies of {args.calibrate_copy_mib} MiB")
    if not args.no_cpu_baseline:
        per_run, runs, err = cpu_baseline(torch, pool, q[0], y[0], cfg, scale, args.cpu_seconds)
        threads = __import__("oracle").num_threads()
        out["cpu_baseline"] = {
            "value": round(attn_bytes / per_run / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"layer 0 of the step (decode of {B} seqs x {nq} heads x {ctx} keys), oracle f32 "
                      f"online-softmax restatement of attn.wgsl, {runs} runs, {per_run * 1e3:.1f} ms/run, "
                      f"max |cpu-gpu| {err:.1e}",
            "us_per_layer": round(per_run * 1e6, 1)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
