"""KV pool API mirroring the reference's ``thuban_model::pool`` and ``rows``.

* ``ArenaSpec`` / ``KvArena``: crates/thuban_model/src/pool.rs:6-118, a host
  page allocator (here backed by the C++ allocator in libthuban_hip.so).
* ``KvPool``: pool.rs:120-163, the device KV of every layer in one HIP
  allocation plus a device block table; also exposes the page API of
  ``LanguageModel::{alloc,free,truncate}_pages`` (traits.rs:39-41).
* ``RowMeta``: rows.rs:7-30 (``row_meta`` + ``write_row_meta``).

Device buffers are plain device pointers; torch tensors are accepted for
convenience and only their ``data_ptr()`` is used.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

from . import _lib
from ._lib import check, lib


_current_stream = None  # callable: address of torch's current HIP stream, or None without a GPU


def _current_stream_fn():
    """Resolved once.  torch's raw-stream accessor returns the address
    without building a Stream object (~0.3 us against ~3 us per call)."""
    global _current_stream
    if _current_stream is None:
        try:
            import torch

            if not torch.cuda.is_available():
                _current_stream = lambda: None
            else:
                get_dev = getattr(torch._C, "_cuda_getDevice", None)
                get_raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
                if get_dev is not None and get_raw is not None:
                    _current_stream = lambda: get_raw(get_dev())
                else:
                    _current_stream = lambda: torch.cuda.current_stream().cuda_stream
        except ImportError:
            _current_stream = lambda: None
    return _current_stream


def _stream_ptr(stream) -> Optional[int]:
    if stream is None:
        return _current_stream_fn()()
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _ptr(buf) -> int:
    if isinstance(buf, int):
        return buf
    return buf.data_ptr()


@dataclass
class ArenaSpec:
    """pool.rs:6-9."""

    seq_lens: List[int]
    pages: Optional[int] = None


class KvArena:
    """Host page allocator, KvArena (pool.rs:11-118) with a runtime page
    length and the fork / copy-on-write extension."""

    def __init__(self, spec: ArenaSpec, page_len: int = 32, _handle=None, _owner=None):
        self._owner = _owner
        if _handle is not None:
            self._h = _handle
            self._own = False
            return
        n = len(spec.seq_lens)
        arr = _lib.u32_array(spec.seq_lens) if n else None
        h = ctypes.c_void_p()
        check(lib().thb_arena_create(arr, n, -1 if spec.pages is None else spec.pages, page_len, ctypes.byref(h)))
        self._h = h.value
        self._own = True

    def __del__(self):
        # at interpreter shutdown the loader may already be gone: nothing to release then
        try:
            if getattr(self, "_own", False) and self._h:
                lib().thb_arena_destroy(self._h)
                self._h = None
        except (AttributeError, ImportError, TypeError):
            pass

    def alloc(self, seq: int, pos: int, tokens: int) -> None:
        check(lib().thb_arena_alloc(self._h, seq, pos, tokens))

    def free_seq(self, seq: int) -> None:
        check(lib().thb_arena_free_seq(self._h, seq))

    def truncate(self, seq: int, keep_tokens: int) -> None:
        check(lib().thb_arena_truncate(self._h, seq, keep_tokens))

    def covers(self, seq: int, tokens: int) -> bool:
        return check(lib().thb_arena_covers(self._h, seq, tokens)) == 1

    def fork(self, src: int, dst: int, tokens: int) -> None:
        check(lib().thb_arena_fork(self._h, src, dst, tokens))

    def info(self) -> _lib.ArenaInfo:
        info = _lib.ArenaInfo()
        check(lib().thb_arena_info_get(self._h, ctypes.byref(info)))
        return info

    def pages(self) -> int:
        return self.info().pages

    def used(self) -> int:
        return self.info().used

    def max_pages(self) -> int:
        return self.info().max_pages

    def seqs(self) -> int:
        return self.info().seqs

    def seq_len(self, seq: int) -> int:
        v = ctypes.c_uint32()
        check(lib().thb_arena_seq_len(self._h, seq, ctypes.byref(v)))
        return v.value

    def table(self) -> List[int]:
        info = self.info()
        n = info.seqs * info.max_pages
        out = (ctypes.c_uint32 * max(n, 1))()
        check(lib().thb_arena_table(self._h, out, n))
        return list(out[:n])

    def table_of(self, seq: int) -> List[int]:
        n = ctypes.c_uint32()
        check(lib().thb_arena_table_of(self._h, seq, None, 0, ctypes.byref(n)))
        out = (ctypes.c_uint32 * max(n.value, 1))()
        check(lib().thb_arena_table_of(self._h, seq, out, n.value, ctypes.byref(n)))
        return list(out[: n.value])

    def free_list(self) -> List[int]:
        """The free stack, bottom first: the last entry is the next page
        handed out (KvArena::free, pool.rs:16)."""
        n = ctypes.c_uint32()
        check(lib().thb_arena_free_list(self._h, None, 0, ctypes.byref(n)))
        out = (ctypes.c_uint32 * max(n.value, 1))()
        check(lib().thb_arena_free_list(self._h, out, n.value, ctypes.byref(n)))
        return list(out[: n.value])

    def refs(self) -> List[int]:
        pages = self.pages()
        out = (ctypes.c_uint32 * max(pages, 1))()
        check(lib().thb_arena_refs(self._h, out, pages))
        return list(out[:pages])

    def take_copies(self) -> List[tuple]:
        pending = self.info().pending_copies
        out = (ctypes.c_uint32 * max(3 * pending, 1))()
        n = ctypes.c_uint32()
        check(lib().thb_arena_take_copies(self._h, out, pending, ctypes.byref(n)))
        return [tuple(out[3 * i: 3 * i + 3]) for i in range(n.value)]


class KvPool:
    """Device KV of ``layers`` layers sharing one page allocator
    (KvArena + one KvPool per layer in the reference, model.rs:103-124)."""

    def __init__(self, spec: ArenaSpec, kv_heads: int, head_dim: int, layers: int = 1, page_len: int = 32,
                 kv_dtype: str = "bf16", head_dims: Optional[Sequence[int]] = None, part_len: int = 0,
                 arena=None):
        kv = {"bf16": _lib.KV_BF16_TRUNC, "f16": _lib.KV_F16_RNE}[kv_dtype]
        d = _lib.PoolDesc()
        d.layers, d.kv_heads, d.head_dim = layers, kv_heads, head_dim
        self._hd_arr = _lib.u32_array(list(head_dims)) if head_dims is not None else None
        d.head_dims = self._hd_arr
        d.page_len, d.kv_dtype = page_len, kv
        self._sl = _lib.u32_array(spec.seq_lens) if spec.seq_lens else None
        d.seqs, d.seq_lens = len(spec.seq_lens), self._sl
        d.pages = -1 if spec.pages is None else spec.pages
        d.part_len = part_len
        self._arena_buf = arena
        if arena is not None:
            d.arena_dev = _ptr(arena)
            d.arena_bytes = arena.numel() * arena.element_size()
        h = ctypes.c_void_p()
        check(lib().thb_pool_create(ctypes.byref(d), ctypes.byref(h)))
        self._h = h.value
        self.layers, self.kv_heads, self.page_len = layers, kv_heads, page_len
        self.head_dim = head_dim
        self.kv_dtype = kv_dtype
        self.arena = KvArena(spec, _handle=lib().thb_pool_arena(self._h), _owner=self)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().thb_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except (AttributeError, ImportError, TypeError):  # interpreter shutdown
            pass

    @property
    def handle(self) -> int:
        return self._h

    # LanguageModel page API (traits.rs:39-41) -----------------------------
    def alloc(self, seq: int, pos: int, tokens: int) -> None:
        check(lib().thb_pool_alloc(self._h, seq, pos, tokens))

    def free_seq(self, seq: int) -> None:
        check(lib().thb_pool_free_seq(self._h, seq))

    def truncate(self, seq: int, keep_tokens: int) -> None:
        check(lib().thb_pool_truncate(self._h, seq, keep_tokens))

    def fork(self, src: int, dst: int, tokens: int) -> None:
        check(lib().thb_pool_fork(self._h, src, dst, tokens))

    def sync(self, stream=None) -> None:
        check(lib().thb_pool_sync(self._h, _stream_ptr(stream)))

    # device page allocator ------------------------------------------------
    def alloc_rows(self, rows: "RowMeta", m: int, row_off: int = 0, stream=None) -> None:
        """The engine's per-plan alloc_pages loop (engine.rs:197-200) for
        rows [row_off, row_off + m) of the row meta, on the device."""
        check(lib().thb_pool_alloc_rows(self._h, rows.handle, row_off, m, _stream_ptr(stream)))

    def status(self, stream=None) -> None:
        """Raises the first failure the device allocator met since the last
        call (ThubanError with the reference's message), and clears it."""
        check(lib().thb_pool_status(self._h, _stream_ptr(stream)))

    def read_state(self, stream=None):
        """(free stack bottom first, reference counts, flattened block
        table) of the device allocator after the stream's work."""
        info = self.arena.info()
        n_tab = info.seqs * info.max_pages
        free = (ctypes.c_uint32 * max(info.pages, 1))()
        refs = (ctypes.c_uint32 * max(info.pages, 1))()
        table = (ctypes.c_uint32 * max(n_tab, 1))()
        n_free = ctypes.c_uint32()
        check(lib().thb_pool_read_state(self._h, _stream_ptr(stream), free, info.pages, ctypes.byref(n_free), refs,
                                        info.pages, table, n_tab))
        return list(free[: n_free.value]), list(refs[: info.pages]), list(table[:n_tab])

    def pull(self, stream=None) -> None:
        """Reloads the host mirror from the device allocator."""
        check(lib().thb_pool_pull(self._h, _stream_ptr(stream)))

    # device views ---------------------------------------------------------
    def layer_info(self, layer: int) -> _lib.LayerInfo:
        info = _lib.LayerInfo()
        check(lib().thb_pool_layer(self._h, layer, None, None, ctypes.byref(info)))
        return info

    def layer_ptrs(self, layer: int):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib().thb_pool_layer(self._h, layer, ctypes.byref(k), ctypes.byref(v), None))
        return k.value, v.value

    def block_table_ptr(self) -> int:
        p = ctypes.c_void_p()
        check(lib().thb_pool_block_table(self._h, ctypes.byref(p)))
        return p.value

    def memory(self):
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        check(lib().thb_pool_memory(self._h, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def layer_tensors(self, layer: int):
        """torch views (16-bit words, no copy) of the layer's device planes as
        stored, one flat page per row: [kv_heads, pages, page_len * head_dim]
        (the element order inside a page is page_offsets())."""
        import torch

        info = self.layer_info(layer)
        k, v = self.layer_ptrs(layer)
        pages = info.pool_len // info.page_len
        n = info.page_len * info.head_dim
        return (_device_view(k, (info.kv_heads, pages, n), torch.int16),
                _device_view(v, (info.kv_heads, pages, n), torch.int16))

    @staticmethod
    def page_offsets(page_len: int, head_dim: int):
        """Offsets of element (slot j, dim d) inside a K and a V page, as
        numpy arrays [page_len, head_dim] (THB_PAGE_LAYOUT_MFMA of
        include/thuban_hip.h): K in 32-dimension groups, group g of width
        w = min(32, head_dim - 32 g) at 32 P g + w j + d % 32; V in 4-slot
        groups at (j / 4) 4 head_dim + 4 d + j % 4."""
        import numpy as np

        j = np.arange(page_len)[:, None]
        d = np.arange(head_dim)[None, :]
        g0 = d & ~31
        w = np.minimum(32, head_dim - g0)
        k = g0 * page_len + w * j + (d & 31)
        v = (j >> 2) * (4 * head_dim) + 4 * d + (j & 3)
        return k.astype(np.int64), v.astype(np.int64)

    def read_layer(self, layer: int):
        """Host copies (numpy uint16) of the layer's K and V in the
        reference's KvPool layout [kv_heads, pool_len, head_dim]
        (pool.rs:131-153)."""
        import torch

        k, v = self.layer_tensors(layer)
        torch.cuda.synchronize()
        info = self.layer_info(layer)
        P, hd = info.page_len, info.head_dim
        ko, vo = self.page_offsets(P, hd)
        shape = (info.kv_heads, info.pool_len, hd)
        kn = k.cpu().numpy().view("uint16")[..., ko.reshape(-1)].reshape(shape)
        vn = v.cpu().numpy().view("uint16")[..., vo.reshape(-1)].reshape(shape)
        return kn, vn

    def write_layer(self, layer: int, k_words, v_words) -> None:
        """Uploads K and V words given in the reference layout [kv_heads,
        pool_len, head_dim] (numpy uint16) into the device page layout."""
        import numpy as np
        import torch

        info = self.layer_info(layer)
        k, v = self.layer_tensors(layer)
        pages = info.pool_len // info.page_len
        P, hd = info.page_len, info.head_dim
        ko, vo = self.page_offsets(P, hd)
        for dev, words, off in ((k, k_words, ko), (v, v_words, vo)):
            flat = np.empty((info.kv_heads, pages, P * hd), np.uint16)
            flat[..., off.reshape(-1)] = np.asarray(words, np.uint16).reshape(info.kv_heads, pages, P * hd)
            dev.copy_(torch.from_numpy(flat.view(np.int16)))
        torch.cuda.synchronize()

    def block_table_tensor(self):
        import torch

        info = self.arena.info()
        return _device_view(self.block_table_ptr(), (info.seqs * info.max_pages,), torch.int32)


class _CudaArray:
    """Minimal __cuda_array_interface__ wrapper over a raw device pointer."""

    _TYPESTR = {"int16": "<i2", "int32": "<i4", "float32": "<f4", "float16": "<f2", "uint8": "|u1"}

    def __init__(self, ptr, shape, typestr):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr, "data": (ptr, False),
                                         "version": 2, "strides": None}


def _device_view(ptr, shape, dtype):
    import torch

    name = str(dtype).replace("torch.", "")
    return torch.as_tensor(_CudaArray(ptr, shape, _CudaArray._TYPESTR[name]), device="cuda")


class RowMeta:
    """rows::row_meta + write_row_meta (rows.rs:11-30): 8 u32 per row."""

    def __init__(self, max_m: int = 128):
        h = ctypes.c_void_p()
        check(lib().thb_rows_create(max_m, ctypes.byref(h)))
        self._h = h.value
        self.max_m = max_m

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().thb_rows_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except (AttributeError, ImportError, TypeError):  # interpreter shutdown
            pass

    @property
    def handle(self) -> int:
        return self._h

    def write(self, positions: Sequence[int], seqs: Sequence[int], m: Optional[int] = None, stream=None) -> None:
        m = len(positions) if m is None else m
        check(lib().thb_rows_write(self._h, _lib.u32_array(list(positions)[:m]) if m else None,
                                   _lib.u32_array(list(seqs)[:m]) if m else None, m, _stream_ptr(stream)))

    def device_ptr(self) -> int:
        return lib().thb_rows_device(self._h)


def row_meta(max_m: int = 128) -> RowMeta:
    return RowMeta(max_m)


def write_row_meta(meta: RowMeta, positions, seqs, m: int, stream=None) -> None:
    """rows.rs:19-30."""
    if len(positions) < m or len(seqs) < m:
        raise ValueError("row meta arrays must cover the chunk size")
    meta.write(positions, seqs, m, stream)
