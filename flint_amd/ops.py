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
from .pool import KvPool, RowMeta, _stream_ptr

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


_HALF = ("float16", "bfloat16", "int16")  # 16-bit words (KV types) in gather/scatter buffers
_ACT = ("float32", "float16", "bfloat16")   # sources, queries, outputs and gates


_NAME_OF = {}  # dtype object -> name, filled on first use


def _dtype_name(t) -> str:
    dt = t.dtype
    name = _NAME_OF.get(dt)
    if name is None:
        name = _NAME_OF[dt] = str(dt).replace("torch.", "")
    return name


def _buf(name: str, x, elems: int, dtypes, extent: Optional[int] = None):
    """Checks argument ``x`` and returns it.  A torch tensor must have one of
    ``dtypes``, be contiguous and hold ``elems`` elements; with ``extent``
    (a strided view such as a query read q_stride elements apart) it may be
    non-contiguous, but its storage must hold ``extent`` elements from its
    first one.  A raw int address passes unchecked, as at the C ABI.
    Raises ThubanError (kind "Invalid") instead of letting a kernel read or
    write out of bounds.  _addr then checks the device."""
    if isinstance(x, int):
        return x
    if x is None:
        raise ThubanError(_lib.THB_ERR_INVALID, f"{name} is None")
    dt = _dtype_name(x)
    if dt not in dtypes:
        raise ThubanError(_lib.THB_ERR_INVALID, f"{name}: dtype {dt} is not one of {', '.join(dtypes)}")
    if extent is None:
        if not x.is_contiguous():
            raise ThubanError(_lib.THB_ERR_INVALID, f"{name} must be contiguous")
        if x.numel() < elems:
            raise ThubanError(_lib.THB_ERR_INVALID, f"{name} holds {x.numel()} elements, the call needs {elems}")
    else:
        have = x.untyped_storage().nbytes() // x.element_size() - x.storage_offset()
        if have < extent:
            raise ThubanError(_lib.THB_ERR_INVALID,
                              f"{name}: storage holds {have} elements from the view's start, the call reads {extent}")
    return x


def _addr(name: str, x) -> int:
    """Device address of a checked argument; a tensor must live on the GPU."""
    if isinstance(x, int):
        return x
    if not x.is_cuda:
        raise ThubanError(_lib.THB_ERR_INVALID, f"{name} must be a GPU tensor (device {x.device})")
    return x.data_ptr()


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


def _head_dim(kv: KvPool, layer: int) -> int:
    hds = getattr(kv, "_hd_arr", None)
    if hds is not None and 0 <= layer < len(hds):
        return hds[layer]
    return kv.head_dim


def _src_bufs(kv: KvPool, layer: int, m: int, k_src, v_src):
    n = m * kv.kv_heads * _head_dim(kv, layer)
    _buf("k_src", k_src, n, _ACT)
    _buf("v_src", v_src, n, _ACT)
    if not isinstance(k_src, int) and not isinstance(v_src, int) and k_src.dtype != v_src.dtype:
        raise ThubanError(_lib.THB_ERR_INVALID, f"k_src and v_src dtypes differ ({k_src.dtype}, {v_src.dtype})")


def kv_store(k_src, v_src, kv: KvPool, layer: int, m: int, meta: RowMeta, row_off: int = 0, stream=None) -> None:
    """ops/attn.rs:53-81: append rows [row_off, row_off+m) of K/V (shape
    [m, kv_heads, head_dim], f32/f16/bf16) into the paged cache."""
    _src_bufs(kv, layer, m, k_src, v_src)
    k, v = _addr("k_src", k_src), _addr("v_src", v_src)
    check(lib().thb_kv_store(kv.handle, layer, k, v, _dtype_code(getattr(k_src, "dtype", None)),
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


def _qy_bufs(kv: KvPool, layer: int, spec: AttnSpec, q, y):
    n = spec.m * spec.q_heads * _head_dim(kv, layer)
    _buf("q", q, n, _ACT)
    _buf("y", y, n, _ACT)


def attn(q, kv: KvPool, layer: int, y, spec: AttnSpec, stream=None) -> None:
    """ops/attn.rs:18-51: paged attention of spec.m rows; q and y are
    [m, q_heads, head_dim] (f32 as the reference, or f16)."""
    _qy_bufs(kv, layer, spec, q, y)
    qp, yp = _addr("q", q), _addr("y", y)
    c = _spec_c(spec, q, y)
    check(lib().thb_attn(kv.handle, layer, qp, yp, ctypes.byref(c), spec.args.handle, _stream_ptr(stream)))


class DevicePlan:
    """thb_dplan_*: an attention call planned on the device from the row meta
    in device memory (no reference counterpart), so that a step can be
    captured in a graph once and replayed while positions move.  ``build``
    plans the spec's rows (q and y give the spec's dtypes); ``attn`` runs
    attention of one layer over the plan.  Each (group, partition) computes
    what ``attn`` computes, bit for bit; in a work-list plan (prefill=True) a
    prefill block whose keys span several partitions runs as decode groups,
    whose sums are ordered differently from ``attn``'s.  ``attn_append``
    (append=True) is ``kv_store_attn`` over the plan, in one launch; ``step``
    is ``attn_step`` over the plan (a rope needs ``set_pos_limit`` first)."""

    def __init__(self, kv: KvPool, max_m: int, q_heads: int, prefill: bool = False, append: bool = False):
        """prefill=True: a work-list plan (thb_dplan_create_ex with
        THB_DPLAN_PREFILL) that also runs prefill chunks on the prefill
        kernel.  append=True (THB_DPLAN_APPEND, fixed-grid plans): each build
        also checks on the device that the call's append can run inside the
        attention launch, for ``attn_append``."""
        h = ctypes.c_void_p()
        flags = (1 if prefill else 0) | (2 if append else 0)
        check(lib().thb_dplan_create_ex(kv.handle, max_m, q_heads, flags, ctypes.byref(h)))
        self._h = h.value
        self.kv, self.max_m, self.q_heads = kv, max_m, q_heads
        self.spec = None
        self._dt = None

    def build(self, spec: AttnSpec, q, y, stream=None) -> None:
        c = _spec_c(spec, q, y)
        check(lib().thb_dplan_build(self._h, ctypes.byref(c), spec.args.handle, _stream_ptr(stream)))
        self.spec = spec
        self._dt = (_dtype_name(q), _dtype_name(y))

    def attn(self, layer: int, q, y, stream=None) -> None:
        if self.spec is None:
            raise ThubanError(_lib.THB_ERR_INVALID, "the plan has not been built")
        n = self.spec.m * self.spec.q_heads * _head_dim(self.kv, layer)
        _buf("q", q, n, (self._dt[0],))
        _buf("y", y, n, (self._dt[1],))
        check(lib().thb_attn_dplan(self.kv.handle, layer, _addr("q", q), _addr("y", y), self._h,
                                   _stream_ptr(stream)))

    def attn_append(self, layer: int, k_src, v_src, q, y, stream=None) -> None:
        """thb_attn_append_dplan: the plan's rows of k_src / v_src appended
        and attention run in one launch, bit-identical to ``kv_store_attn``."""
        if self.spec is None:
            raise ThubanError(_lib.THB_ERR_INVALID, "the plan has not been built")
        _src_bufs(self.kv, layer, self.spec.m, k_src, v_src)
        n = self.spec.m * self.spec.q_heads * _head_dim(self.kv, layer)
        _buf("q", q, n, (self._dt[0],))
        _buf("y", y, n, (self._dt[1],))
        check(lib().thb_attn_append_dplan(self.kv.handle, layer, _addr("k_src", k_src), _addr("v_src", v_src),
                                          _dtype_code(getattr(k_src, "dtype", None)), _addr("q", q), _addr("y", y),
                                          self._h, _stream_ptr(stream)))

    def set_pos_limit(self, max_pos: int) -> None:
        """thb_dplan_set_pos_limit: later builds report rows at or past
        max_pos (the rope tables' rows) and give them no keys; needed by
        ``step`` with a rope.  Build again before the next launch."""
        check(lib().thb_dplan_set_pos_limit(self._h, max_pos))
        self.spec = None

    def step(self, layer: int, q, y, q_stride: int = 0, gate=None, gate_stride: int = 0, k_src=None, v_src=None,
             rope=None, stream=None) -> None:
        """thb_attn_step_dplan: ``attn_step``'s extensions over the plan
        (k_src / v_src appended inside the launch need append=True)."""
        if self.spec is None:
            raise ThubanError(_lib.THB_ERR_INVALID, "the plan has not been built")
        for name, x, dt in (("q", q, self._dt[0]), ("y", y, self._dt[1])):
            if not isinstance(x, int) and _dtype_name(x) != dt:
                raise ThubanError(_lib.THB_ERR_INVALID, f"{name}: dtype {_dtype_name(x)} is not the plan's {dt}")
        io = _attn_io(self.kv, layer, self.spec.m, self.spec.q_heads, q, y, q_stride, gate, gate_stride, k_src, v_src,
                      rope)
        check(lib().thb_attn_step_dplan(self.kv.handle, layer, ctypes.byref(io), self._h, _stream_ptr(stream)))

    def close(self) -> None:
        if self._h:
            lib().thb_dplan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def kv_store_attn(k_src, v_src, q, kv: KvPool, layer: int, y, spec: AttnSpec, stream=None) -> None:
    """kv_store of the spec's rows followed by attn (the per-layer step of
    transformer/forward.rs:300-336), in one launch where the rows allow it;
    bit-identical to calling the two."""
    _src_bufs(kv, layer, spec.m, k_src, v_src)
    _qy_bufs(kv, layer, spec, q, y)
    k, v, qp, yp = _addr("k_src", k_src), _addr("v_src", v_src), _addr("q", q), _addr("y", y)
    c = _spec_c(spec, q, y)
    check(lib().thb_attn_append(kv.handle, layer, k, v, _dtype_code(getattr(k_src, "dtype", None)), qp, yp,
                                ctypes.byref(c), spec.args.handle, _stream_ptr(stream)))


def _attn_io(kv: KvPool, layer: int, m: int, q_heads: int, q, y, q_stride, gate, gate_stride, k_src, v_src,
             rope) -> _lib.AttnIoC:
    """The thb_attn_io of a call of m rows, its buffers checked."""
    hd = _head_dim(kv, layer)
    heads = m * q_heads
    io = _lib.AttnIoC()
    q_ext = (heads - 1) * q_stride + hd if q_stride and heads else None
    _buf("q", q, heads * hd, _ACT, extent=q_ext)
    _buf("y", y, heads * hd, _ACT)
    if gate is not None:
        g_ext = (heads - 1) * (gate_stride or hd) + hd if heads else 0
        _buf("gate", gate, heads * hd, _ACT, extent=g_ext if gate_stride else None)
    if k_src is not None:
        _src_bufs(kv, layer, m, k_src, v_src)
    io.q_dev, io.y_dev, io.q_stride = _addr("q", q), _addr("y", y), q_stride
    io.gate_dev = _addr("gate", gate) if gate is not None else None
    io.gate_stride = gate_stride
    if k_src is not None:
        io.k_src_dev, io.v_src_dev = _addr("k_src", k_src), _addr("v_src", v_src)
        io.src_dtype = _dtype_code(getattr(k_src, "dtype", None))
    io.rope = ctypes.pointer(rope._c) if rope is not None else None
    return io


def attn_step(kv: KvPool, layer: int, spec: AttnSpec, q, y, q_stride: int = 0, gate=None, gate_stride: int = 0,
              k_src=None, v_src=None, rope=None, stream=None) -> None:
    """thb_attn_step: attention with every extension of the C ABI's
    thb_attn_io.  q heads are q_stride elements apart (0 = head_dim; pass
    2 * head_dim and a view of a fused q|gate projection); gate, when given,
    multiplies the output by sigmoid(gate) (qwen35/layers.rs:231-238); k_src
    and v_src are appended first; rope (flint_amd.rope.Rope) rotates q and k.
    q, gate and y are device tensors or raw device addresses."""
    io = _attn_io(kv, layer, spec.m, spec.q_heads, q, y, q_stride, gate, gate_stride, k_src, v_src, rope)
    c = _spec_c(spec, q, y)
    check(lib().thb_attn_step(kv.handle, layer, ctypes.byref(io), ctypes.byref(c), spec.args.handle,
                              _stream_ptr(stream)))


def default_scale(head_dim: int) -> float:
    """forward.rs:328: attn_scale or 1/sqrt(head_dim)."""
    return 1.0 / math.sqrt(head_dim)


def kv_gather(kv: KvPool, layer: int, seq: int, t0: int, n: int, k_dst, v_dst, stream=None) -> None:
    """Tokens [t0, t0+n) of seq into contiguous [kv_heads, n, head_dim]
    16-bit buffers (no reference counterpart)."""
    e = n * kv.kv_heads * _head_dim(kv, layer)
    _buf("k_dst", k_dst, e, _HALF)
    _buf("v_dst", v_dst, e, _HALF)
    check(lib().thb_kv_gather(kv.handle, layer, seq, t0, n, _addr("k_dst", k_dst), _addr("v_dst", v_dst),
                              _stream_ptr(stream)))


def kv_scatter(kv: KvPool, layer: int, seq: int, t0: int, n: int, k_src, v_src, stream=None) -> None:
    """Inverse of kv_gather (no reference counterpart)."""
    e = n * kv.kv_heads * _head_dim(kv, layer)
    _buf("k_src", k_src, e, _HALF)
    _buf("v_src", v_src, e, _HALF)
    check(lib().thb_kv_scatter(kv.handle, layer, seq, t0, n, _addr("k_src", k_src), _addr("v_src", v_src),
                               _stream_ptr(stream)))


def _ranges_c(kv: KvPool, ranges):
    arr = (_lib.KvRangeC * max(len(ranges), 1))()
    hd, total = None, 0
    for i, (seq, layer, t0, n) in enumerate(ranges):
        arr[i].seq, arr[i].layer, arr[i].t0, arr[i].n = seq, layer, t0, n
        if n:
            hd = _head_dim(kv, layer) if hd is None else hd
            total += n * kv.kv_heads * hd
    return arr, total


def kv_gather_batch(kv: KvPool, ranges: Sequence[Sequence[int]], k_dst, v_dst, stream=None) -> None:
    """kv_gather of many (seq, layer, t0, n) ranges in one launch; range i
    lands after ranges 0..i-1, each [kv_heads, n_i, head_dim] (no reference
    counterpart)."""
    arr, total = _ranges_c(kv, ranges)
    _buf("k_dst", k_dst, total, _HALF)
    _buf("v_dst", v_dst, total, _HALF)
    check(lib().thb_kv_gather_batch(kv.handle, arr, len(ranges), _addr("k_dst", k_dst), _addr("v_dst", v_dst),
                                    _stream_ptr(stream)))


def kv_scatter_batch(kv: KvPool, ranges: Sequence[Sequence[int]], k_src, v_src, stream=None) -> None:
    """Inverse of kv_gather_batch (no reference counterpart)."""
    arr, total = _ranges_c(kv, ranges)
    _buf("k_src", k_src, total, _HALF)
    _buf("v_src", v_src, total, _HALF)
    check(lib().thb_kv_scatter_batch(kv.handle, arr, len(ranges), _addr("k_src", k_src), _addr("v_src", v_src),
                                     _stream_ptr(stream)))


def check_gemm_dims(pairs: Sequence[Sequence[int]]) -> None:
    """ops::check_gemm_dims (crates/thuban_model/src/ops/gemm.rs:133-146):
    every (N, K) pair needs N % 16 == 0 and K % 64 == 0 (ThubanError kind
    "Config" otherwise)."""
    for n, k in pairs:
        check(lib().thb_check_gemm_dims(n, k))


def gemm_acc(x, w, y, rows: int, acc: bool, stream=None) -> None:
    """ops::gemm_acc (crates/thuban_model/src/ops/gemm.rs:113-131): y[rows, n]
    = x[rows, k] . w[n, k]^T (+ y when acc); rows == 1 is the gemv.  x is
    f32, f16 or bf16 (the attention output), w bf16 or f16 [n, k], y f32."""
    n, k = w.shape
    _buf("x", x, rows * k, _ACT)
    _buf("w", w, n * k, ("bfloat16", "float16"))
    _buf("y", y, rows * n, ("float32",))
    check(lib().thb_gemm_acc(_addr("x", x), _dtype_code(x.dtype), _addr("w", w), _dtype_code(w.dtype),
                             _addr("y", y), rows, n, k, 1 if acc else 0, _stream_ptr(stream)))


def block_copy(kv: KvPool, triples: Sequence[Sequence[int]], stream=None) -> None:
    flat = [int(x) for t in triples for x in t]
    check(lib().thb_block_copy(kv.handle, _lib.u32_array(flat) if flat else None, len(flat) // 3,
                               _stream_ptr(stream)))


__all__ = ["AttnSpec", "ThubanError", "attn", "attn_step", "block_copy", "check_gemm_dims", "check_head_dim",
           "default_scale", "gemm_acc", "kv_gather", "kv_gather_batch", "kv_scatter", "kv_scatter_batch", "kv_store",
           "kv_store_attn"]
