"""Host-side argument checks of flint_amd.ops: a tensor that is strided,
of the wrong type, too small or not on the GPU is rejected with
ThubanError (kind "Invalid") before any pointer reaches the C ABI, where a
kernel would read or write out of bounds.  CPU only: every case fails in
Python, before a library call."""

import pytest
import torch

from flint_amd import ThubanError, ops


class _Pool:
    """Only what the checks read from a KvPool (no device memory)."""

    kv_heads, head_dim, handle, _hd_arr = 2, 64, 0, None


class _Rows:
    handle = 0


def _spec(m=3, q_heads=4):
    return ops.AttnSpec(q_heads=q_heads, window=0, scale=0.125, m=m, causal=True, seq=None, args=_Rows())


def _raises(fn, text):
    with pytest.raises(ThubanError) as e:
        fn()
    assert text in str(e.value), str(e.value)
    assert e.value.kind == "Invalid"


def test_attn_rejects_bad_queries_and_outputs():
    pool, spec = _Pool(), _spec()
    q = torch.zeros(3, 4, 64)
    y = torch.zeros(3, 4, 64)
    _raises(lambda: ops.attn(q.transpose(0, 1), pool, 0, y, spec), "q must be contiguous")
    _raises(lambda: ops.attn(q.int(), pool, 0, y, spec), "q: dtype int32")
    _raises(lambda: ops.attn(q[:2], pool, 0, y, spec), "q holds 512 elements, the call needs 768")
    _raises(lambda: ops.attn(q, pool, 0, y[:, :3], spec), "y must be contiguous")
    _raises(lambda: ops.attn(q, pool, 0, y, _spec(m=4)), "holds 768 elements, the call needs 1024")
    _raises(lambda: ops.attn(q, pool, 0, y, spec), "q must be a GPU tensor")


def test_append_rejects_bad_sources():
    pool, spec = _Pool(), _spec()
    k = torch.zeros(3, 2, 64, dtype=torch.float16)
    q = torch.zeros(3, 4, 64)
    _raises(lambda: ops.kv_store(k[:1], k, pool, 0, 3, _Rows()), "k_src holds 128 elements, the call needs 384")
    _raises(lambda: ops.kv_store(k, k.float(), pool, 0, 3, _Rows()), "dtypes differ")
    _raises(lambda: ops.kv_store(k, k.to(torch.float64), pool, 0, 3, _Rows()), "v_src: dtype float64")
    _raises(lambda: ops.kv_store_attn(k, k[:, :1], q, pool, 0, q, spec), "v_src must be contiguous")
    _raises(lambda: ops.kv_store(k, k, pool, 0, 3, _Rows()), "k_src must be a GPU tensor")


def test_strided_query_checks_the_storage():
    """attn_step reads heads q_stride elements apart: a view into a fused
    q|gate projection is fine as long as its storage covers the last head."""
    pool, spec = _Pool(), _spec()
    qg = torch.zeros(3, 4, 128)
    y = torch.zeros(3, 4, 64)
    _raises(lambda: ops.attn_step(pool, 0, spec, qg[..., :64], y, q_stride=128, gate=qg[..., 64:],
                                  gate_stride=128), "q must be a GPU tensor")
    short = torch.zeros(3 * 4 * 128 - 100)
    _raises(lambda: ops.attn_step(pool, 0, spec, short, y, q_stride=128), "storage holds 1436 elements")
    _raises(lambda: ops.attn_step(pool, 0, spec, qg, y, q_stride=128, gate=qg[1:, :, 64:], gate_stride=128),
            "gate: storage holds")
    _raises(lambda: ops.attn_step(pool, 0, spec, qg[..., :64], y), "q must be contiguous")


def test_gather_rejects_non_16_bit_buffers():
    pool = _Pool()
    k = torch.zeros(2, 10, 64, dtype=torch.int16)
    _raises(lambda: ops.kv_gather(pool, 0, 0, 0, 10, k.float(), k), "k_dst: dtype float32")
    _raises(lambda: ops.kv_gather(pool, 0, 0, 0, 11, k, k), "k_dst holds 1280 elements, the call needs 1408")
    _raises(lambda: ops.kv_scatter(pool, 0, 0, 0, 10, k, k[:, ::2]), "v_src must be contiguous")
    _raises(lambda: ops.kv_gather(pool, 0, 0, 0, 10, k, k), "k_dst must be a GPU tensor")
