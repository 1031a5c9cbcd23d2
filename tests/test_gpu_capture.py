"""Graph capture of a decode step (no reference counterpart: the reference
records wgpu command buffers per step).  A step of the engine's per-plan page
allocation (thuban_generate/src/engine.rs:197-200 -> KvArena::alloc,
crates/thuban_model/src/pool.rs:47-65), kv_store and attention
(transformer/forward.rs:300-336) is captured once with thb_pool_alloc_rows,
thb_kv_store, thb_dplan_build and thb_attn_dplan, then replayed while the
rows move, sequences fork and speculative rollbacks truncate into shared
pages (so replays must copy on write).  Every replay equals the eager path
bit for bit, and the device allocator's state equals oracle/arena.py; the
same holds for a continuous batch (decode rows and a walking prefill chunk)
captured with the work-list plan.  Calls
that cannot replay correctly refuse a capturing stream, and once the page
allocation is captured the host reloads its mirror from the device before
every host-side call."""

import math
import random

import numpy as np
import pytest

from gpu_util import fill, make_pool, say, scattered_alloc
from oracle.arena import KvArena

pytestmark = pytest.mark.gpu


def _capture(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    return graph


def _state(pool):
    free, refs, table = pool.read_state()
    return free, refs, table


def test_captured_step_with_fork_and_rollback_matches_eager(torch_cuda):
    """Two pools set up identically.  E runs each step eagerly (alloc_rows,
    kv_store and thb_attn per layer); G replays one captured graph of
    (alloc_rows, kv_store and the device-planned attention per layer).
    Between replays the host only writes the row meta, and at three steps
    runs a page-API call (after an explicit pull, or relying on graph mode's
    reload at step 12): a rollback of a fork into the
    page it shares with its source (step 7; the next replay's alloc_rows
    copies it), a fork of a partial page whose target takes over a row (step
    12), and a rollback of the fork's source into a page still shared (step
    16).  20 steps: outputs, pool bytes and allocator state are identical,
    and the state equals the oracle's."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd, P, L, T = 8, 2, 128, 16, 2, 20
    prompts = [103, 257, 31, 64]
    budgets = [512] * 6
    pools = []
    for _ in range(2):
        pool = make_pool(budgets, kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16", layers=L)
        scattered_alloc(pool, prompts, random.Random(17), P)
        fr = RowMeta(256)
        for layer in range(L):
            fill(torch, pool, fr, prompts, layer=layer, seed=40 + layer)
        pool.fork(1, 4, 256)  # 16 full pages shared
        pool.sync()
        pools.append(pool)
    E, G = pools
    orc = KvArena(budgets, pages=E.arena.pages(), page_len=P)
    rng = random.Random(17)
    need = [-(-n // P) for n in prompts]
    have = [0] * len(prompts)
    order = [s for s in range(len(prompts)) for _ in range(need[s])]
    rng.shuffle(order)
    for s in order:  # scattered_alloc's calls, in its order
        orc.alloc(s, have[s] * P, P if (have[s] + 1) * P <= prompts[s] else prompts[s] - have[s] * P)
        have[s] += 1
    orc.fork(1, 4, 256)
    orc.copies.clear()
    assert _state(E) == _state(G) == (orc.free, orc.refs, orc.table())

    B = 5
    active = [0, 1, 2, 3, 4]
    pos = {0: 103, 1: 257, 2: 31, 3: 64, 4: 256}
    rows = {"E": RowMeta(B), "G": RowMeta(B)}
    k_in = [torch.empty(B, nkv, hd, device="cuda", dtype=torch.float16) for _ in range(L)]
    v_in = [torch.empty_like(k_in[0]) for _ in range(L)]
    q_in = [torch.empty(B, nq, hd, device="cuda", dtype=torch.float16) for _ in range(L)]
    y = {"E": [torch.empty(B, nq, hd, device="cuda") for _ in range(L)],
         "G": [torch.empty(B, nq, hd, device="cuda") for _ in range(L)]}
    specs = {w: ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=B, causal=True, seq=None,
                             args=rows[w]) for w in rows}

    def eager_step():
        E.alloc_rows(rows["E"], B)
        for layer in range(L):
            ops.kv_store(k_in[layer], v_in[layer], E, layer, B, rows["E"])
            ops.attn(q_in[layer], E, layer, y["E"][layer], specs["E"])

    plan = ops.DevicePlan(G, max_m=B, q_heads=nq)  # the plan's buffers: nothing to allocate inside the capture

    def graph_step():
        G.alloc_rows(rows["G"], B)
        for layer in range(L):
            ops.kv_store(k_in[layer], v_in[layer], G, layer, B, rows["G"])
        plan.build(specs["G"], q_in[0], y["G"][0])
        for layer in range(L):
            plan.attn(layer, q_in[layer], y["G"][layer])

    graph = _capture(torch, graph_step)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    copies_seen = 0
    for step in range(T):
        if step in (7, 12, 16):
            if step != 12:  # at step 12 the fork reloads the mirror itself (graph mode)
                G.pull()
                assert G.arena.table() == E.arena.table(), step
            if step == 7:  # reject 7 drafts of seq 4: back into page 15, shared with seq 1
                for pool in pools:
                    pool.truncate(4, 250)
                orc.truncate(4, 250)
                pos[4] = 250
            elif step == 12:  # fork seq 0 mid-page into seq 5, which replaces seq 3's row
                for pool in pools:
                    pool.fork(0, 5, pos[0])
                orc.fork(0, 5, pos[0])
                active[3] = 5
                pos[5] = pos[0]
            else:  # roll seq 1 back into page 14, still shared with seq 4
                for pool in pools:
                    pool.truncate(1, 230)
                orc.truncate(1, 230)
                pos[1] = 230
            for pool in pools:
                pool.sync()
            orc.copies.clear()
        positions = [pos[s] for s in active]
        for w in rows:
            rows[w].write(positions, active, B)
        for layer in range(L):
            k_in[layer].copy_(torch.randn(B, nkv, hd, device="cuda", generator=gen))
            v_in[layer].copy_(torch.randn(B, nkv, hd, device="cuda", generator=gen))
            q_in[layer].copy_(torch.randn(B, nq, hd, device="cuda", generator=gen))
        for w in ("E", "G"):
            for layer in range(L):
                y[w][layer].fill_(float("nan"))
        torch.cuda.synchronize()
        eager_step()
        graph.replay()
        orc.alloc_rows(positions, active)
        copies_seen += len(orc.copies)
        orc.copies.clear()
        torch.cuda.synchronize()
        say("captured step", step, "rows", list(zip(active, positions)))
        for layer in range(L):
            assert torch.isfinite(y["E"][layer]).all(), (step, layer)
            assert torch.equal(y["G"][layer], y["E"][layer]), (step, layer,
                                                               float((y["G"][layer] - y["E"][layer]).abs().max()))
        for s in active:
            pos[s] += 1
    assert copies_seen == 2  # the two rollbacks into shared pages copied on write
    G.status()
    G.pull()
    want = (orc.free, orc.refs, orc.table())
    assert _state(G) == want
    assert _state(E) == want
    assert G.arena.table() == orc.table() and G.arena.refs() == orc.refs and G.arena.free_list() == orc.free
    for layer in range(L):
        ka, va = E.read_layer(layer)
        kb, vb = G.read_layer(layer)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), layer
    del graph
    plan.close()


def test_capture_refusals_and_graph_mode(torch_cuda):
    """A host-planned attention call, queued host page ops and a state read
    refuse a capturing stream (THB_ERR_INVALID).  Once alloc_rows has been
    captured the pool is in graph mode: a host call reloads the mirror from
    the device first, so it sees what replays allocated without a pull."""
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    lens = [200, 90]
    pool = make_pool([400, 400], kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16")
    for s, n in enumerate(lens):
        pool.alloc(s, 0, n)
    fill(torch, pool, RowMeta(64), lens, seed=2)
    rows = RowMeta(2)
    rows.write([200, 90], [0, 1], 2)
    pool.alloc_rows(rows, 2)
    q = torch.randn(2, 4, 64, device="cuda")
    y = torch.empty_like(q)
    spec = ops.AttnSpec(q_heads=4, window=0, scale=0.125, m=2, causal=True, seq=None, args=rows)
    ops.attn(q, pool, 0, y, spec)
    torch.cuda.synchronize()

    def refused(fn, text):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            graph.capture_begin()
            try:
                y.zero_()
                with pytest.raises(ThubanError) as e:
                    fn()
            finally:
                graph.capture_end()
        torch.cuda.synchronize()
        assert e.value.kind == "Invalid" and text in str(e.value), str(e.value)
        say("refused under capture:", str(e.value)[:100])

    refused(lambda: ops.attn(q, pool, 0, y, spec), "not capturable: thb_attn plans")
    refused(lambda: pool.status(), "not capturable")
    pool.alloc(1, 96, 1)  # a new page: queued for the device
    refused(lambda: pool.alloc_rows(rows, 2), "must run before the capture")
    pool.sync()
    graph = _capture(torch, lambda: pool.alloc_rows(rows, 2))
    n0, n1 = len(pool.arena.table_of(0)), len(pool.arena.table_of(1))
    rows.write([300, 150], [0, 1], 2)
    graph.replay()
    torch.cuda.synchronize()
    assert len(pool.arena.table_of(0)) == n0  # the host has not looked yet
    ops.attn(q, pool, 0, y, spec)  # graph mode: the mirror is reloaded first
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert len(pool.arena.table_of(0)) == 19 and len(pool.arena.table_of(1)) == 10 > n1
    free, refs, table = pool.read_state()
    assert pool.arena.table() == table and pool.arena.refs() == refs and pool.arena.free_list() == free
    pool.alloc(1, 160, 1)  # host page API in graph mode: on the reloaded mirror
    pool.sync()
    assert pool.read_state()[2] == pool.arena.table()
    del graph


def test_replayed_alloc_rows_rejects_bad_and_repeated_sequences(torch_cuda):
    """The host rejects a call whose rows name a sequence out of range or a
    sequence heading two runs before anything is allocated.  A replay reads
    its rows on the device, which now makes the same checks: the replay
    allocates nothing, and thb_pool_status reports the first offending row
    with the host's message."""
    torch = torch_cuda
    from flint_amd import ThubanError
    from flint_amd.pool import RowMeta

    pool = make_pool([300, 300, 300], kv_heads=2, head_dim=64, page_len=16, kv_dtype="f16")
    rows = RowMeta(4)
    rows.write([0, 0, 1, 0], [0, 1, 1, 2], 4)
    graph = _capture(torch, lambda: pool.alloc_rows(rows, 4))
    graph.replay()
    torch.cuda.synchronize()
    pool.status()
    pool.pull()
    before = _state(pool)
    assert pool.arena.table_of(0) == [0] and pool.arena.table_of(2) == [2]
    for positions, seqs, msg in [
        ([16, 2, 16, 17], [0, 1, 0, 0], "sequence 0 heads two runs of rows in one call (one run per sequence)"),
        ([16, 2, 3, 16], [0, 1, 7, 2], "sequence 7 out of range (3 sequences)"),
        ([16, 2, 16, 3], [0, 2, 0, 7], "sequence 0 heads two runs of rows in one call (one run per sequence)"),
    ]:
        rows.write(positions, seqs, 4)
        graph.replay()
        torch.cuda.synchronize()
        with pytest.raises(ThubanError) as e:
            pool.status()
        assert str(e.value) == msg and e.value.kind == "Invalid", str(e.value)
        assert _state(pool) == before
    rows.write([16, 2, 3, 16], [0, 1, 1, 2], 4)
    graph.replay()
    torch.cuda.synchronize()
    pool.status()
    pool.pull()
    assert len(pool.arena.table_of(0)) == 2 and len(pool.arena.table_of(2)) == 2
    del graph


def test_captured_continuous_batch_with_list_plan_matches_eager(torch_cuda):
    """Continuous batching in a captured step (the engine's mixed plans,
    thuban_generate/src/engine.rs:237-300, one forward over decode rows and
    prefill chunks, transformer/forward.rs:314-336): four sequences decode
    one token per step while a 256-row prefill chunk walks through three
    arriving 512-token prompts, two chunks each.  E runs each step eagerly
    (alloc_rows, kv_store and thb_attn per layer); G replays one captured
    graph of (alloc_rows, kv_store per layer, one build of a work-list device
    plan, thb_attn_dplan per layer).  Every step's outputs are identical bit
    for bit, and at the end both pools' bytes and allocator states are equal
    and equal the oracle's."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd, P, L, C, plen = 32, 8, 128, 16, 2, 256, 512
    prompts = [300, 1200, 77, 640]
    arriving = [4, 5, 6]
    budgets = [n + 16 for n in prompts] + [plen] * len(arriving)
    pools = []
    for _ in range(2):
        pool = make_pool(budgets, kv_heads=nkv, head_dim=hd, page_len=P, kv_dtype="f16", layers=L)
        scattered_alloc(pool, prompts, random.Random(23), P)
        fr = RowMeta(256)
        for layer in range(L):
            fill(torch, pool, fr, prompts, layer=layer, seed=60 + layer)
        pool.sync()
        pools.append(pool)
    E, G = pools
    orc = KvArena(budgets, pages=E.arena.pages(), page_len=P)
    rng = random.Random(23)
    need = [-(-n // P) for n in prompts]
    have = [0] * len(prompts)
    order = [s for s in range(len(prompts)) for _ in range(need[s])]
    rng.shuffle(order)
    for s in order:  # scattered_alloc's calls, in its order
        orc.alloc(s, have[s] * P, P if (have[s] + 1) * P <= prompts[s] else prompts[s] - have[s] * P)
        have[s] += 1
    orc.copies.clear()
    assert _state(E) == _state(G) == (orc.free, orc.refs, orc.table())

    m = len(prompts) + C
    rows = {"E": RowMeta(m), "G": RowMeta(m)}
    k_in = [torch.empty(m, nkv, hd, device="cuda", dtype=torch.float16) for _ in range(L)]
    v_in = [torch.empty_like(k_in[0]) for _ in range(L)]
    q_in = [torch.empty(m, nq, hd, device="cuda", dtype=torch.float16) for _ in range(L)]
    y = {"E": [torch.empty(m, nq, hd, device="cuda") for _ in range(L)],
         "G": [torch.empty(m, nq, hd, device="cuda") for _ in range(L)]}
    specs = {w: ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=m, causal=True, seq=None,
                             args=rows[w]) for w in rows}

    def eager_step():
        E.alloc_rows(rows["E"], m)
        for layer in range(L):
            ops.kv_store(k_in[layer], v_in[layer], E, layer, m, rows["E"])
            ops.attn(q_in[layer], E, layer, y["E"][layer], specs["E"])

    plan = ops.DevicePlan(G, max_m=m, q_heads=nq, prefill=True)

    def graph_step():
        G.alloc_rows(rows["G"], m)
        for layer in range(L):
            ops.kv_store(k_in[layer], v_in[layer], G, layer, m, rows["G"])
        plan.build(specs["G"], q_in[0], y["G"][0])
        for layer in range(L):
            plan.attn(layer, q_in[layer], y["G"][layer])

    graph = _capture(torch, graph_step)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(61)
    dpos = list(prompts)
    for step in range(2 * len(arriving)):
        seq, c0 = arriving[step // 2], (step % 2) * C
        positions = dpos + list(range(c0, c0 + C))
        seqs = list(range(len(prompts))) + [seq] * C
        for w in rows:
            rows[w].write(positions, seqs, m)
        for layer in range(L):
            k_in[layer].copy_(torch.randn(m, nkv, hd, device="cuda", generator=gen))
            v_in[layer].copy_(torch.randn(m, nkv, hd, device="cuda", generator=gen))
            q_in[layer].copy_(torch.randn(m, nq, hd, device="cuda", generator=gen))
        for w in ("E", "G"):
            for layer in range(L):
                y[w][layer].fill_(float("nan"))
        torch.cuda.synchronize()
        eager_step()
        graph.replay()
        orc.alloc_rows(positions, seqs)
        orc.copies.clear()
        torch.cuda.synchronize()
        say("captured continuous batch step", step, "prefill seq", seq, "rows", c0, "..", c0 + C - 1)
        for layer in range(L):
            assert torch.isfinite(y["E"][layer]).all(), (step, layer)
            assert torch.equal(y["G"][layer], y["E"][layer]), (step, layer,
                                                               float((y["G"][layer] - y["E"][layer]).abs().max()))
        dpos = [p + 1 for p in dpos]
    G.status()
    G.pull()
    want = (orc.free, orc.refs, orc.table())
    assert _state(G) == want
    assert _state(E) == want
    for layer in range(L):
        ka, va = E.read_layer(layer)
        kb, vb = G.read_layer(layer)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), layer
    del graph
    plan.close()
