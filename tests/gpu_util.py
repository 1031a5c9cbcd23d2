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


def oracle_seq(torch, pool: KvPool, layer: int, seq: int, n: int) -> oracle.Layer:
    """Oracle layer holding only tokens [0, n) of `seq`, gathered through the
    product's gather kernel into contiguous pages (identity block table,
    the sequence is oracle sequence 0).  Works at any pool size."""
    from flint_amd import ops

    info = pool.layer_info(layer)
    P = info.page_len
    pages = -(-n // P)
    kd = torch.empty(info.kv_heads, n, info.head_dim, dtype=torch.int16, device="cuda")
    vd = torch.empty_like(kd)
    ops.kv_gather(pool, layer, seq, 0, n, kd, vd)  # contiguous [kv_heads, n, head_dim]
    torch.cuda.synchronize()
    k = np.zeros((info.kv_heads, pages * P, info.head_dim), np.uint16)
    v = np.zeros_like(k)
    k[:, :n] = kd.cpu().numpy().view(np.uint16)
    v[:, :n] = vd.cpu().numpy().view(np.uint16)
    return oracle.Layer(info.kv_heads, info.head_dim, pages, P, np.arange(pages, dtype=np.uint32), pages,
                        KV_CODE[pool.kv_dtype], k=k, v=v)


def fill_layer_random(torch, pool: KvPool, layer: int, seed: int, scale: float = 1.0) -> None:
    """N(0, scale^2) f16/bf16 words in every slot of a layer (layout-agnostic)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dt = torch.float16 if pool.kv_dtype == "f16" else torch.bfloat16
    for t in pool.layer_tensors(layer):
        w = t.view(dt)
        w.normal_(generator=g)
        if scale != 1.0:
            w.mul_(scale)
    torch.cuda.synchronize()


def fragment(pool: KvPool, filler_seqs, occupied_frac: float, rng) -> None:
    """Fills the free list with a random scattering: every page goes to a
    random filler sequence one page at a time, then a random subset of the
    filler sequences is freed so that `occupied_frac` of the pages stay
    held.  Filler sequence budgets must cover their share of the pool."""
    pages = pool.arena.pages()
    owners = [filler_seqs[rng.randrange(len(filler_seqs))] for _ in range(pages)]
    have = {s: 0 for s in filler_seqs}
    P = pool.page_len
    for s in owners:
        pool.alloc(s, have[s] * P, P)
        have[s] += 1
    order = list(filler_seqs)
    rng.shuffle(order)
    freed = 0
    for s in order:
        if freed >= (1.0 - occupied_frac) * pages:
            break
        freed += have[s]
        pool.free_seq(s)
