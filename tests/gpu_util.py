"""Shared helpers of the GPU parity tests: build a pool, fill it through the
product's kv_store, and mirror its contents into an oracle Layer."""

from __future__ import annotations

import sys

import numpy as np

import oracle
from flint_amd import ops
from flint_amd.pool import ArenaSpec, KvPool, RowMeta

KV_CODE = {"bf16": oracle.KV_BF16, "f16": oracle.KV_F16}


def say(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


def scattered_alloc(pool: KvPool, lens, rng, page_len):
    """Allocates pages for every sequence one page at a time in random order,
    so that each sequence's pages are scattered across the pool."""
    need = [-(-n // page_len) for n in lens]
    have = [0] * len(lens)
    order = [s for s in range(len(lens)) for _ in range(need[s])]
    rng.shuffle(order)
    for s in order:
        pool.alloc(s, have[s] * page_len, page_len if (have[s] + 1) * page_len <= lens[s] else lens[s] - have[s] * page_len)
        have[s] += 1


def fill(torch, pool: KvPool, rows: RowMeta, lens, layer=0, src_dtype=None, seed=0, scale=1.0):
    """Appends N(0,1) K/V for tokens [0, lens[s]) of every sequence through
    the product kv_store.  Returns nothing; the oracle reads the pool back."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dt = torch.float32 if src_dtype is None else src_dtype
    pairs = [(p, s) for s, n in enumerate(lens) for p in range(n)]
    nkv, hd = pool.kv_heads, pool.layer_info(layer).head_dim
    for i in range(0, len(pairs), rows.max_m):
        chunk = pairs[i: i + rows.max_m]
        m = len(chunk)
        rows.write([p for p, _ in chunk], [s for _, s in chunk], m)
        k = (torch.randn(m, nkv, hd, device="cuda", generator=g) * scale).to(dt)
        v = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
        ops.kv_store(k, v, pool, layer, m, rows)
    torch.cuda.synchronize()


def oracle_layer(torch, pool: KvPool, layer=0) -> oracle.Layer:
    info = pool.layer_info(layer)
    k, v = pool.read_layer(layer)  # reference layout, V pages un-transposed
    a = pool.arena.info()
    return oracle.Layer(info.kv_heads, info.head_dim, a.pages, info.page_len,
                        np.array(pool.arena.table(), np.uint32), a.max_pages, KV_CODE[pool.kv_dtype], k=k, v=v)


def make_pool(lens, kv_heads, head_dim, page_len=16, kv_dtype="f16", layers=1, extra_pages=0, part_len=0,
              seq_lens=None, head_dims=None):
    seq_lens = list(seq_lens) if seq_lens is not None else [max(n, 1) for n in lens]
    pages = sum(-(-n // page_len) for n in seq_lens) + extra_pages
    return KvPool(ArenaSpec(seq_lens, pages), kv_heads, head_dim, layers=layers, page_len=page_len,
                  kv_dtype=kv_dtype, part_len=part_len, head_dims=head_dims)
