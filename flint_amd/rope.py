"""Rotary position embedding of the paged KV path, mirroring
``thuban_model::ops::rope`` (crates/thuban_model/src/ops/rope.rs:1-87) and
``ops::norm_rope`` (crates/thuban_model/src/ops/norm.rs:73-111).

``rope_tables`` is the reference's host-side table builder; ``Rope`` carries
the device tables (and optional RMSNorm weights) that the rotary entry
points of the C ABI take.  ``rope_rows`` is the standalone op;
``kv_store_rope``, ``attn_rope`` and ``kv_store_attn_rope`` fuse the rotation
into the append and the attention launches.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

from . import _lib
from ._lib import check, lib
from .ops import AttnSpec, _dtype_code, _spec_c
from .pool import KvPool, RowMeta, _ptr, _stream_ptr


@dataclass
class RopeScaling:
    """ops/rope.rs:46-50: per-frequency divisors for positions below
    ``original_max`` (short) and from it on (long)."""

    short: Sequence[float]
    long: Sequence[float]
    original_max: int


def rope_tables(max_seq: int, rotary_dim: int, freq_dim: int, theta: float, partial: Optional[int] = None,
                scaling: Optional[RopeScaling] = None):
    """ops/rope.rs:52-87: cos and sin tables, float32 numpy arrays of shape
    [max_seq, rotary_dim / 2].  Angles are computed in double precision:
    inv_i = theta^(-2i / freq_dim) (0 for i >= partial), divided by the
    scaling factor of frequency i when one applies, times the position."""
    import numpy as np

    half = rotary_dim // 2
    i = np.arange(half, dtype=np.float64)
    inv = 1.0 / np.power(float(theta), 2.0 * i / float(freq_dim))
    if partial is not None:
        inv[np.arange(half) >= partial] = 0.0
    pos = np.arange(max_seq, dtype=np.float64)
    inv_rows = np.broadcast_to(inv, (max_seq, half)).copy()
    if scaling is not None:
        for p in range(max_seq):
            for k in range(half):
                f = None
                if p < scaling.original_max and k < len(scaling.short):
                    f = scaling.short[k]
                elif k < len(scaling.long):
                    f = scaling.long[k]
                if f is not None:
                    inv_rows[p, k] = inv[k] / float(np.float32(f))
    angle = pos[:, None] * inv_rows
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)


class Rope:
    """Device tables of one rotary configuration (the reference's
    RopeInputs, ops/rope.rs:13-17), plus the RMSNorm weights of norm_rope
    for queries and keys (Qwen3's q_norm / k_norm), float32 on cuda:0."""

    def __init__(self, cos, sin, rot: int, q_norm=None, k_norm=None, eps: float = 1e-6):
        import numpy as np
        import torch

        dev = torch.device("cuda", torch.cuda.current_device())

        def dev_f32(a):
            if a is None:
                return None
            t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a, np.float32))
            return t.to(device=dev, dtype=torch.float32).contiguous()

        self.cos, self.sin = dev_f32(cos), dev_f32(sin)
        self.q_norm, self.k_norm = dev_f32(q_norm), dev_f32(k_norm)
        self.rot, self.eps = int(rot), float(eps)
        self.max_pos = int(self.cos.shape[0])
        c = _lib.RopeC()
        c.cos_dev, c.sin_dev = self.cos.data_ptr(), self.sin.data_ptr()
        c.rot, c.max_pos, c.eps = self.rot, self.max_pos, self.eps
        c.q_norm_dev = self.q_norm.data_ptr() if self.q_norm is not None else None
        c.k_norm_dev = self.k_norm.data_ptr() if self.k_norm is not None else None
        self._c = c

    @classmethod
    def from_theta(cls, max_seq: int, rotary_dim: int, theta: float, freq_dim: Optional[int] = None, **kw):
        cos, sin = rope_tables(max_seq, rotary_dim, freq_dim or rotary_dim, theta)
        return cls(cos, sin, rotary_dim, **kw)

    @property
    def c(self):
        return ctypes.byref(self._c)


def rope_rows(x, heads: int, rope: Rope, meta: RowMeta, m: int, norm_w=None, row_off: int = 0, stream=None) -> None:
    """ops::rope (ops/rope.rs:19-43) on rows [row_off, row_off + m) of x
    [m, heads, head_dim] (f32 or f16), in place; with norm_w, ops::norm_rope
    (RMSNorm with that weight, then the rotation)."""
    hd = int(x.shape[-1])
    w = _ptr(norm_w) if norm_w is not None else None
    check(lib().thb_rope_rows(_ptr(x), _dtype_code(getattr(x, "dtype", None)), m, heads, hd, w, rope.c,
                              meta.handle, row_off, _stream_ptr(stream)))


def kv_store_rope(k_src, v_src, kv: KvPool, layer: int, m: int, meta: RowMeta, rope: Rope, row_off: int = 0,
                  stream=None) -> None:
    """rope(k) (norm_rope with rope.k_norm) + kv_store in one pass: the
    rotated K is encoded straight into the pages."""
    check(lib().thb_kv_store_rope(kv.handle, layer, _ptr(k_src), _ptr(v_src),
                                  _dtype_code(getattr(k_src, "dtype", None)), rope.c, meta.handle, row_off, m,
                                  _stream_ptr(stream)))


def attn_rope(q, kv: KvPool, layer: int, y, spec: AttnSpec, rope: Rope, stream=None) -> None:
    """rope(q) (norm_rope with rope.q_norm) + attn in one launch."""
    c = _spec_c(spec, q, y)
    check(lib().thb_attn_rope(kv.handle, layer, _ptr(q), _ptr(y), ctypes.byref(c), rope.c, spec.args.handle,
                              _stream_ptr(stream)))


def kv_store_attn_rope(k_src, v_src, q, kv: KvPool, layer: int, y, spec: AttnSpec, rope: Rope, stream=None) -> None:
    """The per-layer step of transformer/forward.rs:186-336 (rope of q and
    k, kv_store, attn), in one launch where the rows allow it."""
    c = _spec_c(spec, q, y)
    check(lib().thb_attn_append_rope(kv.handle, layer, _ptr(k_src), _ptr(v_src),
                                     _dtype_code(getattr(k_src, "dtype", None)), _ptr(q), _ptr(y), ctypes.byref(c),
                                     rope.c, spec.args.handle, _stream_ptr(stream)))


__all__ = ["Rope", "RopeScaling", "attn_rope", "kv_store_attn_rope", "kv_store_rope", "rope_rows", "rope_tables"]
