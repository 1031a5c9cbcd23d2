"""thb_attn_noalloc (the attention call that allocates nothing: its plan and
split-K partial results live in a fixed device array) against thb_attn, the
entry point it varies, through the C ABI: bit-identical outputs on two calls
in a row, the second smaller, both with contexts split over many partitions
so that the partial results and the merge run; and a call too large for the
array is refused."""

import ctypes
import math
import random

import pytest

from gpu_util import fill, make_pool, say, scattered_alloc

pytestmark = pytest.mark.gpu


def _noalloc(pool, layer, q, y, spec):
    from flint_amd import _lib, ops
    from flint_amd.pool import _stream_ptr

    c = ops._spec_c(spec, q, y)
    return _lib.lib().thb_attn_noalloc(pool.handle, layer, q.data_ptr(), y.data_ptr(), ctypes.byref(c),
                                       spec.args.handle, _stream_ptr(None))


def test_noalloc_matches_attn_twice(torch_cuda):
    torch = torch_cuda
    from flint_amd import _lib, ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd = 32, 8, 128
    lens = [3000, 1700, 2500, 900, 4100, 60]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", part_len=256)
    scattered_alloc(pool, lens, random.Random(31), 16)
    fill_rows = RowMeta(256)
    fill(torch, pool, fill_rows, lens, seed=31)
    g = torch.Generator(device="cuda")
    g.manual_seed(32)
    calls = [(list(range(6)), [n - 1 for n in lens]),  # six rows, up to 16 partitions each
             ([4, 1], [2000, 1500])]                       # then a smaller call
    for i, (seqs, positions) in enumerate(calls):
        m = len(seqs)
        say("no-alloc call", i, "rows", m)
        rows = RowMeta(m)
        rows.write(positions, seqs, m)
        q = torch.randn(m, nq, hd, device="cuda", generator=g)
        spec = ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows)
        y_ref = torch.empty_like(q)
        ops.attn(q, pool, 0, y_ref, spec)
        y = torch.full_like(q, float("nan"))
        rc = _noalloc(pool, 0, q, y, spec)
        assert rc == 0, _lib.lib().thb_last_error().decode()
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        assert torch.equal(y, y_ref), (i, float((y - y_ref).abs().max()))


def test_noalloc_refuses_calls_beyond_the_scratch(torch_cuda):
    """Two 8192-token rows cut into 512 partitions of 16 tokens need 68 MB
    of partial results, beyond the 32 MiB array: THB_ERR_INVALID."""
    torch = torch_cuda
    from flint_amd import _lib, ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd = 8, 8, 128
    lens = [8192, 8192]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", part_len=16)
    for s, n in enumerate(lens):
        pool.alloc(s, 0, n)
    rows = RowMeta(2)
    rows.write([8191, 8191], [0, 1], 2)
    q = torch.zeros(2, nq, hd, device="cuda")
    y = torch.empty_like(q)
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=0.1, m=2, causal=True, seq=None, args=rows)
    rc = _noalloc(pool, 0, q, y, spec)
    assert rc == _lib.THB_ERR_INVALID
    assert "exceed the no-allocation scratch" in _lib.lib().thb_last_error().decode()
    torch.cuda.synchronize()


def test_noalloc_captured_calls_replay_their_own_plans(torch_cuda):
    """Two no-allocation calls with different plans (both split into
    partitions) captured in one graph, then an eager call with a third plan
    that overwrites the array, then replays: each replay writes its own
    plans into the array (they travel in the graph's kernel arguments), so
    both outputs equal thb_attn's bit for bit, also after another eager
    call between replays."""
    torch = torch_cuda
    from flint_amd import _lib, ops
    from flint_amd.pool import RowMeta

    nq, nkv, hd = 16, 4, 128
    lens = [2100, 700, 1500, 3000]
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype="f16", part_len=256)
    scattered_alloc(pool, lens, random.Random(41), 16)
    fill(torch, pool, RowMeta(256), lens, seed=41)
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    calls = {"a": ([0, 2, 3], [2099, 1499, 2999]), "b": ([1, 3], [699, 1200]), "c": ([3, 0, 1, 2], [10, 700, 600, 1400])}
    rows, qs, ys, want, specs = {}, {}, {}, {}, {}
    for name, (seqs, positions) in calls.items():
        m = len(seqs)
        rows[name] = RowMeta(m)
        rows[name].write(positions, seqs, m)
        qs[name] = torch.randn(m, nq, hd, device="cuda", generator=g)
        ys[name] = torch.empty_like(qs[name])
        want[name] = torch.empty_like(qs[name])
        specs[name] = ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=m, causal=True, seq=None,
                                   args=rows[name])
        ops.attn(qs[name], pool, 0, want[name], specs[name])

    def call(name):
        rc = _noalloc(pool, 0, qs[name], ys[name], specs[name])
        assert rc == 0, _lib.lib().thb_last_error().decode()

    call("a")  # resolves the device's scratch address outside the capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call("a")
            call("b")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        call("c")  # another plan in the array
        torch.cuda.synchronize()
        assert torch.equal(ys["c"], want["c"]), rep
        ys["a"].fill_(float("nan"))
        ys["b"].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        say("no-alloc graph replay", rep)
        for name in ("a", "b"):
            assert torch.equal(ys[name], want[name]), (rep, name, float((ys[name] - want[name]).abs().max()))
    del graph
