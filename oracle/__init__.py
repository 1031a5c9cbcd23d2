"""CPU oracle for the paged KV-cache path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
package ``flint_amd`` never imports it.

``oracle.c`` restates the reference's kernels (``kv_store.wgsl``,
``attn.wgsl``) and codecs (``thuban_num``); ``arena.py`` restates the host
page allocator (``thuban_model/src/pool.rs``).  Each function cites the
reference lines it follows; how each is pinned is listed at the top of
``oracle.c`` and ``arena.py``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

KV_BF16 = 0  # bf16 by truncation (reference parity)
KV_F16 = 1  # f16, round to nearest even
SRC_F32, SRC_F16, SRC_BF16 = 0, 1, 2


def build() -> str:
    """Compile oracle.c with the committed Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class OrcLayer(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("pool_len", ctypes.c_uint32),
        ("max_pages", ctypes.c_uint32),
        ("page_len", ctypes.c_uint32),
        ("kv_dtype", ctypes.c_int32),
    ]


class OrcAttnSpec(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_uint32),
        ("q_heads", ctypes.c_uint32),
        ("nq_per_kv", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("window", ctypes.c_uint32),
        ("causal", ctypes.c_int32),
        ("seq", ctypes.c_int64),
        ("softcap", ctypes.c_float),
        ("precision", ctypes.c_int32),
    ]


def _declare(L: ctypes.CDLL) -> None:
    vp, u32, sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f32_to_f16.argtypes = [ctypes.c_float]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_bf16_to_f32.restype = ctypes.c_float
    L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    for name in ("orc_f32_to_f16_n", "orc_f16_to_f32_n", "orc_f32_to_bf16_n"):
        getattr(L, name).argtypes = [vp, vp, sz]
        getattr(L, name).restype = None
    L.orc_kv_store.argtypes = [ctypes.POINTER(OrcLayer), vp, vp, ctypes.c_int, vp, u32]
    L.orc_kv_store.restype = ctypes.c_int
    L.orc_attn_ranges.argtypes = [vp, u32, ctypes.c_int64, ctypes.c_int, u32, vp, vp, vp]
    L.orc_attn_ranges.restype = None
    L.orc_attn.argtypes = [ctypes.POINTER(OrcLayer), vp, vp, vp, ctypes.POINTER(OrcAttnSpec)]
    L.orc_attn.restype = ctypes.c_int
    L.orc_kv_gather.argtypes = [ctypes.POINTER(OrcLayer), u32, u32, u32, vp, vp]
    L.orc_kv_gather.restype = ctypes.c_int
    L.orc_block_copy.argtypes = [ctypes.POINTER(OrcLayer), vp, u32]
    L.orc_block_copy.restype = None
    L.orc_rope_rows.argtypes = [vp, u32, u32, u32, u32, vp, vp, u32, vp, vp, ctypes.c_float]
    L.orc_rope_rows.restype = ctypes.c_int
    L.orc_gemm.argtypes = [vp, vp, vp, u32, u32, u32, ctypes.c_int, ctypes.c_int]
    L.orc_gemm.restype = None
    L.orc_num_threads.argtypes = []
    L.orc_num_threads.restype = ctypes.c_int


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ------------------------------------------------------------------ codecs
def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def decode_kv(bits: np.ndarray, kv_dtype: int) -> np.ndarray:
    return f16_to_f32(bits) if kv_dtype == KV_F16 else bf16_to_f32(bits)


def encode_kv(x: np.ndarray, kv_dtype: int) -> np.ndarray:
    return f32_to_f16(x) if kv_dtype == KV_F16 else f32_to_bf16(x)


# -------------------------------------------------------------- the layer
class Layer:
    """One layer of a paged pool on the host: K, V [kv_heads, pool_len,
    head_dim] as uint16 words plus a flattened block table (pool.rs:120-163)."""

    def __init__(self, kv_heads, head_dim, pages, page_len, block_table, max_pages, kv_dtype,
                 k=None, v=None):
        self.kv_heads, self.head_dim, self.page_len = kv_heads, head_dim, page_len
        self.pool_len = pages * page_len
        self.max_pages, self.kv_dtype = max_pages, kv_dtype
        shape = (kv_heads, self.pool_len, head_dim)
        self.k = np.zeros(shape, np.uint16) if k is None else np.ascontiguousarray(k, np.uint16).reshape(shape)
        self.v = np.zeros(shape, np.uint16) if v is None else np.ascontiguousarray(v, np.uint16).reshape(shape)
        self.block_table = np.ascontiguousarray(block_table, dtype=np.uint32)

    def _struct(self) -> OrcLayer:
        return OrcLayer(_ptr(self.k), _ptr(self.v), _ptr(self.block_table), self.kv_heads, self.head_dim,
                        self.pool_len, self.max_pages, self.page_len, self.kv_dtype)

    def kv_store(self, k_src, v_src, args, m, src_dtype=SRC_F32) -> None:
        dt = np.float32 if src_dtype == SRC_F32 else np.uint16
        k_src = np.ascontiguousarray(k_src, dtype=dt)
        v_src = np.ascontiguousarray(v_src, dtype=dt)
        args = np.ascontiguousarray(args, dtype=np.uint32)
        s = self._struct()
        rc = lib().orc_kv_store(ctypes.byref(s), _ptr(k_src), _ptr(v_src), src_dtype, _ptr(args), m)
        if rc != 0:
            raise ValueError(f"oracle kv_store: row {-rc - 1} has no page")

    def attn(self, q, args, m, q_heads, scale, window=0, causal=True, seq=None, softcap=0.0,
             precision=0) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float32)
        args = np.ascontiguousarray(args, dtype=np.uint32)
        nq_per_kv = q_heads // self.kv_heads
        spec = OrcAttnSpec(m, q_heads, nq_per_kv, scale, window, int(bool(causal)),
                           -1 if seq is None else int(seq), softcap, precision)
        y = np.empty((m, q_heads, self.head_dim), dtype=np.float64 if precision == 0 else np.float32)
        s = self._struct()
        rc = lib().orc_attn(ctypes.byref(s), _ptr(q), _ptr(y), _ptr(args), ctypes.byref(spec))
        if rc != 0:
            raise ValueError("oracle attn: a key's page is missing")
        return y

    def gather(self, seq, t0, n):
        k = np.empty((self.kv_heads, n, self.head_dim), np.uint16)
        v = np.empty_like(k)
        s = self._struct()
        if lib().orc_kv_gather(ctypes.byref(s), seq, t0, n, _ptr(k), _ptr(v)) != 0:
            raise ValueError("oracle gather: page missing")
        return k, v

    def block_copy(self, triples) -> None:
        t = np.ascontiguousarray(triples, dtype=np.uint32).reshape(-1)
        s = self._struct()
        lib().orc_block_copy(ctypes.byref(s), _ptr(t), len(t) // 3)


def rope_rows(x, pos, rot, cos, sin, w=None, eps=1e-6) -> np.ndarray:
    """rope.wgsl:16-40 / norm.wgsl MODE 4 on x [m, heads, hd] (float32;
    float16 input is widened and the result rounded back to float16 with
    f32_to_f16).  pos: the m row positions; cos/sin [max_pos, rot/2]."""
    x = np.asarray(x)
    half_out = x.dtype == np.float16
    v = np.ascontiguousarray(x.astype(np.float32))
    m, heads, hd = v.shape
    p = np.ascontiguousarray(np.asarray(pos, np.uint32))
    c = np.ascontiguousarray(cos, np.float32)
    s = np.ascontiguousarray(sin, np.float32)
    wv = None if w is None else np.ascontiguousarray(w, np.float32)
    rc = lib().orc_rope_rows(_ptr(v), m, heads, hd, rot, _ptr(c), _ptr(s), c.shape[0], _ptr(p),
                             _ptr(wv) if wv is not None else None, eps)
    if rc != 0:
        raise ValueError(f"oracle rope: bad input (code {rc})")
    if half_out:
        return f32_to_f16(v).view(np.float16)
    return v


def attn_ranges(args, m, seq=None, causal=True, window=0):
    """Per-row [lo, hi) key range and seq, following attn.wgsl:78-88,169."""
    args = np.ascontiguousarray(args, dtype=np.uint32)
    lo = np.empty(m, np.uint32)
    hi = np.empty(m, np.uint32)
    sq = np.empty(m, np.uint32)
    lib().orc_attn_ranges(_ptr(args), m, -1 if seq is None else int(seq), int(bool(causal)), window,
                          _ptr(lo), _ptr(hi), _ptr(sq))
    return lo, hi, sq


def row_meta(positions, seqs) -> np.ndarray:
    """8 u32 per row: [pos, seq, 0 x 6] (rows.rs:19-30)."""
    m = len(positions)
    a = np.zeros(8 * m, np.uint32)
    a[0::8] = np.asarray(positions, np.uint32)
    a[1::8] = np.asarray(seqs, np.uint32)
    return a


def gemm(x, w, m, n, k, y0=None, exact=False) -> np.ndarray:
    """cpu_ref::gemm / gemv (cpu_ref.rs:11-35): x [m, k] . w[n, k]^T as f32
    sums in k order, + y0 when given (acc).  exact=True sums in double and
    rounds once."""
    x = np.ascontiguousarray(x, np.float32).reshape(m, k)
    w = np.ascontiguousarray(w, np.float32).reshape(n, k)
    y = np.zeros((m, n), np.float32) if y0 is None else np.array(y0, np.float32).reshape(m, n)
    lib().orc_gemm(_ptr(x), _ptr(w), _ptr(y), m, n, k, int(y0 is not None), int(bool(exact)))
    return y


def lcg_fill(seed: int, n: int) -> np.ndarray:
    """The reference tests' Rng (crates/thuban_backend/tests/kernels.rs
    :112-124): a 64-bit LCG, each draw (state >> 33) / 2^31 * 2 - 1 in f32."""
    out = np.empty(n, np.float32)
    state = seed & 0xFFFFFFFFFFFFFFFF
    mul, inc, mask = 6364136223846793005, 1442695040888963407, 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        state = (state * mul + inc) & mask
        out[i] = np.float32(np.float32(state >> 33) / np.float32(1 << 31)) * np.float32(2.0) - np.float32(1.0)
    return out


def num_threads() -> int:
    return lib().orc_num_threads()
