"""flint_amd -- MI355X-native paged KV-cache path for the Thuban engine.

Hand-written HIP kernels for gfx950 behind the C ABI in include/thuban_hip.h
(libthuban_hip.so, built in-tree).  This package is the host-side mirror of
the reference's pool / ops interface for that path:

* ``flint_amd.pool``: ArenaSpec, KvArena, KvPool, RowMeta
  (reference crates/thuban_model/src/{pool,rows}.rs)
* ``flint_amd.ops``: AttnSpec, attn, kv_store, check_head_dim
  (reference crates/thuban_model/src/ops/attn.rs) plus gather / scatter /
  block_copy.
"""

from ._lib import ThubanError, lib  # noqa: F401
from .ops import (AttnSpec, attn, block_copy, check_head_dim, default_scale, kv_gather, kv_scatter,  # noqa: F401
                  kv_store, kv_store_attn)
from .pool import ArenaSpec, KvArena, KvPool, RowMeta, row_meta, write_row_meta  # noqa: F401
