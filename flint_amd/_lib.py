"""ctypes binding of ``libthuban_hip.so`` (declarations in include/thuban_hip.h).

The library is built in-tree by ``flint_amd.build.build()``.  Loading fails
loudly when it is missing: there is no CPU fallback for any entry point.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libthuban_hip.so")

ABI_VERSION = 8  # THB_ABI_VERSION of include/thuban_hip.h

THB_OK = 0
THB_ERR_MODEL = -1
THB_ERR_CONFIG = -2
THB_ERR_GPU = -3
THB_ERR_INVALID = -4

DT_F32, DT_F16, DT_BF16 = 0, 1, 2
KV_BF16_TRUNC, KV_F16_RNE = 0, 1
NO_PAGE = 0xFFFFFFFF
SEQ_PER_ROW = 0xFFFFFFFF


class ThubanError(RuntimeError):
    """Raised for a non-zero status; ``kind`` mirrors thuban_error::Error."""

    KINDS = {THB_ERR_MODEL: "Model", THB_ERR_CONFIG: "Config", THB_ERR_GPU: "Gpu", THB_ERR_INVALID: "Invalid"}

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = self.KINDS.get(code, "Unknown")
        super().__init__(message)


class ArenaInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("pages", "used", "max_pages", "seqs", "page_len", "pending_copies")]


class PoolDesc(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("head_dims", ctypes.POINTER(ctypes.c_uint32)),
        ("page_len", ctypes.c_uint32),
        ("kv_dtype", ctypes.c_uint32),
        ("seqs", ctypes.c_uint32),
        ("seq_lens", ctypes.POINTER(ctypes.c_uint32)),
        ("pages", ctypes.c_int64),
        ("part_len", ctypes.c_uint32),
        ("arena_dev", ctypes.c_void_p),
        ("arena_bytes", ctypes.c_uint64),
    ]


class LayerInfo(ctypes.Structure):
    _fields_ = [
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("pool_len", ctypes.c_uint32),
        ("max_pages", ctypes.c_uint32),
        ("page_len", ctypes.c_uint32),
        ("kv_dtype", ctypes.c_uint32),
        ("plane_elems", ctypes.c_uint64),
        ("page_layout", ctypes.c_uint32),
    ]


class AttnSpecC(ctypes.Structure):
    _fields_ = [
        ("q_heads", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("m", ctypes.c_uint32),
        ("causal", ctypes.c_uint32),
        ("seq", ctypes.c_uint32),
        ("row_off", ctypes.c_uint32),
        ("softcap", ctypes.c_float),
        ("q_dtype", ctypes.c_uint32),
        ("y_dtype", ctypes.c_uint32),
    ]


class RopeC(ctypes.Structure):
    _fields_ = [
        ("cos_dev", ctypes.c_void_p),
        ("sin_dev", ctypes.c_void_p),
        ("rot", ctypes.c_uint32),
        ("max_pos", ctypes.c_uint32),
        ("q_norm_dev", ctypes.c_void_p),
        ("k_norm_dev", ctypes.c_void_p),
        ("eps", ctypes.c_float),
    ]


class AttnIoC(ctypes.Structure):
    _fields_ = [
        ("q_dev", ctypes.c_void_p),
        ("q_stride", ctypes.c_uint32),
        ("y_dev", ctypes.c_void_p),
        ("gate_dev", ctypes.c_void_p),
        ("gate_stride", ctypes.c_uint32),
        ("k_src_dev", ctypes.c_void_p),
        ("v_src_dev", ctypes.c_void_p),
        ("src_dtype", ctypes.c_uint32),
        ("rope", ctypes.POINTER(RopeC)),
    ]


class KvRangeC(ctypes.Structure):
    _fields_ = [("seq", ctypes.c_uint32), ("layer", ctypes.c_uint32), ("t0", ctypes.c_uint32), ("n", ctypes.c_uint32)]


# (name, restype, argtypes) for every symbol declared in include/thuban_hip.h.
_vp, _u32, _u64, _i64, _sz, _int = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64,
                                    ctypes.c_size_t, ctypes.c_int)
_pu32 = ctypes.POINTER(ctypes.c_uint32)
SIGNATURES = [
    ("thb_last_error", ctypes.c_char_p, []),
    ("thb_abi_version", _u32, []),
    ("thb_check_head_dim", _int, [_u32]),
    ("thb_backend_head_dim", _int, [_u32]),
    ("thb_arena_create", _int, [_pu32, _u32, _i64, _u32, ctypes.POINTER(_vp)]),
    ("thb_arena_destroy", None, [_vp]),
    ("thb_arena_alloc", _int, [_vp, _u32, _u32, _u32]),
    ("thb_arena_free_seq", _int, [_vp, _u32]),
    ("thb_arena_truncate", _int, [_vp, _u32, _u32]),
    ("thb_arena_covers", _int, [_vp, _u32, _u32]),
    ("thb_arena_fork", _int, [_vp, _u32, _u32, _u32]),
    ("thb_arena_table", _int, [_vp, _pu32, _sz]),
    ("thb_arena_table_of", _int, [_vp, _u32, _pu32, _sz, _pu32]),
    ("thb_arena_seq_len", _int, [_vp, _u32, _pu32]),
    ("thb_arena_info_get", _int, [_vp, ctypes.POINTER(ArenaInfo)]),
    ("thb_arena_take_copies", _int, [_vp, _pu32, _sz, _pu32]),
    ("thb_arena_free_list", _int, [_vp, _pu32, _sz, _pu32]),
    ("thb_arena_refs", _int, [_vp, _pu32, _sz]),
    ("thb_pool_create", _int, [ctypes.POINTER(PoolDesc), ctypes.POINTER(_vp)]),
    ("thb_pool_destroy", None, [_vp]),
    ("thb_pool_alloc", _int, [_vp, _u32, _u32, _u32]),
    ("thb_pool_free_seq", _int, [_vp, _u32]),
    ("thb_pool_truncate", _int, [_vp, _u32, _u32]),
    ("thb_pool_fork", _int, [_vp, _u32, _u32, _u32]),
    ("thb_pool_sync", _int, [_vp, _vp]),
    ("thb_pool_alloc_rows", _int, [_vp, _vp, _u32, _u32, _vp]),
    ("thb_pool_status", _int, [_vp, _vp]),
    ("thb_pool_read_state", _int, [_vp, _vp, _pu32, _sz, _pu32, _pu32, _sz, _pu32, _sz]),
    ("thb_pool_pull", _int, [_vp, _vp]),
    ("thb_pool_arena", _vp, [_vp]),
    ("thb_pool_layer", _int, [_vp, _u32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(LayerInfo)]),
    ("thb_pool_block_table", _int, [_vp, ctypes.POINTER(_vp)]),
    ("thb_pool_memory", _int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_u64)]),
    ("thb_rows_create", _int, [_u32, ctypes.POINTER(_vp)]),
    ("thb_rows_destroy", None, [_vp]),
    ("thb_rows_write", _int, [_vp, _pu32, _pu32, _u32, _vp]),
    ("thb_rows_device", _vp, [_vp]),
    ("thb_kv_store", _int, [_vp, _u32, _vp, _vp, _u32, _vp, _u32, _u32, _vp]),
    ("thb_attn", _int, [_vp, _u32, _vp, _vp, ctypes.POINTER(AttnSpecC), _vp, _vp]),
    ("thb_attn_append", _int, [_vp, _u32, _vp, _vp, _u32, _vp, _vp, ctypes.POINTER(AttnSpecC), _vp, _vp]),
    ("thb_rope_rows", _int, [_vp, _u32, _u32, _u32, _u32, _vp, ctypes.POINTER(RopeC), _vp, _u32, _vp]),
    ("thb_kv_store_rope", _int, [_vp, _u32, _vp, _vp, _u32, ctypes.POINTER(RopeC), _vp, _u32, _u32, _vp]),
    ("thb_attn_rope", _int, [_vp, _u32, _vp, _vp, ctypes.POINTER(AttnSpecC), ctypes.POINTER(RopeC), _vp, _vp]),
    ("thb_attn_append_rope", _int, [_vp, _u32, _vp, _vp, _u32, _vp, _vp, ctypes.POINTER(AttnSpecC),
                                    ctypes.POINTER(RopeC), _vp, _vp]),
    ("thb_attn_step", _int, [_vp, _u32, ctypes.POINTER(AttnIoC), ctypes.POINTER(AttnSpecC), _vp, _vp]),
    ("thb_check_gemm_dims", _int, [_u32, _u32]),
    ("thb_gemm_acc", _int, [_vp, _u32, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _vp]),
    ("thb_attn_noalloc", _int, [_vp, _u32, _vp, _vp, ctypes.POINTER(AttnSpecC), _vp, _vp]),
    ("thb_dplan_create", _int, [_vp, _u32, _u32, ctypes.POINTER(_vp)]),
    ("thb_dplan_create_ex", _int, [_vp, _u32, _u32, _u32, ctypes.POINTER(_vp)]),
    ("thb_dplan_destroy", None, [_vp]),
    ("thb_dplan_build", _int, [_vp, ctypes.POINTER(AttnSpecC), _vp, _vp]),
    ("thb_attn_dplan", _int, [_vp, _u32, _vp, _vp, _vp, _vp]),
    ("thb_attn_append_dplan", _int, [_vp, _u32, _vp, _vp, _u32, _vp, _vp, _vp, _vp]),
    ("thb_dplan_set_pos_limit", _int, [_vp, _u32]),
    ("thb_attn_step_dplan", _int, [_vp, _u32, ctypes.POINTER(AttnIoC), _vp, _vp]),
    ("thb_kv_gather", _int, [_vp, _u32, _u32, _u32, _u32, _vp, _vp, _vp]),
    ("thb_kv_scatter", _int, [_vp, _u32, _u32, _u32, _u32, _vp, _vp, _vp]),
    ("thb_kv_gather_batch", _int, [_vp, ctypes.POINTER(KvRangeC), _u32, _vp, _vp, _vp]),
    ("thb_kv_scatter_batch", _int, [_vp, ctypes.POINTER(KvRangeC), _u32, _vp, _vp, _vp]),
    ("thb_block_copy", _int, [_vp, _pu32, _u32, _vp]),
    ("thb_hbm_stream", _int, [_vp, _vp, ctypes.c_uint64, _u32, _u32, _vp]),
]

_lib = None


def lib() -> ctypes.CDLL:
    """Loads the in-tree library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP backend first "
                "(python -c 'import __graft_entry__ as g; g.build()' or make -C flint_amd/csrc)")
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> int:
    """Raises ThubanError for a negative status, returns rc otherwise."""
    if rc < 0:
        raise ThubanError(rc, lib().thb_last_error().decode())
    return rc


def u32_array(values):
    arr = (ctypes.c_uint32 * len(values))(*values)
    return arr
