"""Operators of the paged KV path, mirroring ``thuban_model::ops::attn``
(crates/thuban_model/src/ops/attn.rs:8-90).

``kv_store`` and ``attn`` keep the reference's names and argument meaning;
``kv_gather``, ``kv_scatter`` and ``block_copy`` have no reference
counterpart (fork, copy-on-write, rollback and eviction support).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Sequence

from . import _lib
from ._lib import ThubanError, check, lib
from .pool import KvPool, RowMeta, _ptr, _stream_ptr

_DTYPES = {"f32": _lib.DT_F32, "f16": _lib.DT_F16, "bf16": _lib.DT_BF16}


_DTYPE_OF = {}  # dtype object -> code, filled on first use


def _dtype_code(x, default="f32") -> int:
    if x is None:
        return _DTYPES[default]
    code = _DTYPE_OF.get(x)
    if code is not None:
        return code
    if isinstance(x, str):
        return _DTYPES[x]
    name = str(x).replace("torch.", "")
    code = {"float32": _lib.DT_F32, "float16": _lib.DT_F16, "bfloat16": _lib.DT_BF16}[name]
    _DTYPE_OF[x] = code
    return code


@dataclass
class AttnSpec:
    """ops/attn.rs:8-16 plus this backend's extensions (softcap, dtypes)."""

    q_heads: int
    window: int
    scale: float
    m: int
    causal: bool
    seq: Optional[int]  # None = per-row sequence from the row meta (batched)
    args: RowMeta
    row_off: int = 0
    softcap: float = 0.0


def check_head_dim(head_dim: int) -> None:
    """ops/attn.rs:83-90 (raises ThubanError kind "Config")."""
    check(lib().thb_check_head_dim(head_dim))


def kv_store(k_src, v_src, kv: KvPool, layer: int, m: int, meta: RowMeta, row_off: int = 0, stream=None) -> None:
    """ops/attn.rs:53-81: append rows [row_off, row_off+m) of K/V (shape
    [m, kv_heads, head_dim], f32/f16/bf16) into the paged cache."""
    check(lib().thb_kv_store(kv.handle, layer, _ptr(k_src), _ptr(v_src), _dtype_code(getattr(k_src, "dtype", None)),
                             meta.handle, row_off, m, _stream_ptr(stream)))


def _spec_c(spec: AttnSpec, q, y) -> _lib.AttnSpecC:
    c = _lib.AttnSpecC()
    c.q_heads, c.window, c.scale, c.m = spec.q_heads, spec.window, spec.scale, spec.m
    c.causal = 1 if spec.causal else 0
    c.seq = _lib.SEQ_PER_ROW if spec.seq is None else spec.seq
    c.row_off, c.softcap = spec.row_off, spec.softcap
    c.q_dtype = _dtype_code(getattr(q, "dtype", None))
    c.y_dtype = _dtype_code(getattr(y, "dtype", None))
    return c


def attn(q, kv: KvPool, layer: int, y, spec: AttnSpec, stream=None) -> None:
    """ops/attn.rs:18-51: paged attention of spec.m rows; q and y are
    [m, q_heads, head_dim] (f32 as the reference, or f16)."""
    c = _spec_c(spec, q, y)
    check(lib().thb_attn(kv.handle, layer, _ptr(q), _ptr(y), ctypes.byref(c), spec.args.handle, _stream_ptr(stream)))


def kv_store_attn(k_src, v_src, q, kv: KvPool, layer: int, y, spec: AttnSpec, stream=None) -> None:
    """kv_store of the spec's rows followed by attn (the per-layer step of
    transformer/forward.rs:300-336), in one launch where the rows allow it;
    bit-identical to calling the two."""
    c = _spec_c(spec, q, y)
    check(lib().thb_attn_append(kv.handle, layer, _ptr(k_src), _ptr(v_src),
                                _dtype_code(getattr(k_src, "dtype", None)), _ptr(q), _ptr(y), ctypes.byref(c),
                                spec.args.handle, _stream_ptr(stream)))


def attn_step(kv: KvPool, layer: int, spec: AttnSpec, q, y, q_stride: int = 0, gate=None, gate_stride: int = 0,
              k_src=None, v_src=None, rope=None, stream=None) -> None:
    """thb_attn_step: attention with every extension of the C ABI's
    thb_attn_io.  q heads are q_stride elements apart (0 = head_dim; pass
    2 * head_dim and a view of a fused q|gate projection); gate, when given,
    multiplies the output by sigmoid(gate) (qwen35/layers.rs:231-238); k_src
    and v_src are appended first; rope (flint_amd.rope.Rope) rotates q and k.
    q, gate and y are device tensors or raw device addresses."""
    c = _spec_c(spec, q, y)
    io = _lib.AttnIoC()
    io.q_dev, io.y_dev, io.q_stride = _ptr(q), _ptr(y), q_stride
    io.gate_dev = _ptr(gate) if gate is not None else None
    io.gate_stride = gate_stride
    if k_src is not None:
        io.k_src_dev, io.v_src_dev = _ptr(k_src), _ptr(v_src)
        io.src_dtype = _dtype_code(getattr(k_src, "dtype", None))
    io.rope = ctypes.pointer(rope._c) if rope is not None else None
    check(lib().thb_attn_step(kv.handle, layer, ctypes.byref(io), ctypes.byref(c), spec.args.handle,
                              _stream_ptr(stream)))


def default_scale(head_dim: int) -> float:
    """forward.rs:328: attn_scale or 1/sqrt(head_dim)."""
    return 1.0 / math.sqrt(head_dim)


def kv_gather(kv: KvPool, layer: int, seq: int, t0: int, n: int, k_dst, v_dst, stream=None) -> None:
    check(lib().thb_kv_gather(kv.handle, layer, seq, t0, n, _ptr(k_dst), _ptr(v_dst), _stream_ptr(stream)))


def kv_scatter(kv: KvPool, layer: int, seq: int, t0: int, n: int, k_src, v_src, stream=None) -> None:
    check(lib().thb_kv_scatter(kv.handle, layer, seq, t0, n, _ptr(k_src), _ptr(v_src), _stream_ptr(stream)))


def block_copy(kv: KvPool, triples: Sequence[Sequence[int]], stream=None) -> None:
    flat = [int(x) for t in triples for x in t]
    check(lib().thb_block_copy(kv.handle, _lib.u32_array(flat) if flat else None, len(flat) // 3,
                               _stream_ptr(stream)))


__all__ = ["AttnSpec", "ThubanError", "attn", "attn_step", "block_copy", "check_head_dim", "default_scale", "kv_gather",
           "kv_scatter", "kv_store", "kv_store_attn"]
