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
