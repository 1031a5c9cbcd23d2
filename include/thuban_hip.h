/*
 * thuban_hip.h -- C ABI of the MI355X-native paged KV-cache path.
 *
 * Drop-in replacement for the paged-KV part of the reference engine
 * (formetaohy/Flint, crate family "Thuban").  Citations are path:line in the
 * reference tree.  Every entry point returns an int status (THB_OK == 0,
 * negative on error) and leaves a reference-style message in
 * thb_last_error() (thread-local), e.g. "KV arena exhausted: 3 pages
 * requested, 1 free" or "context limit 32 reached" (pool.rs:49-59).
 *
 * Pointers named *_dev are device pointers; every other pointer is host
 * memory.  `stream` is a hipStream_t passed as void* (NULL = the null
 * stream).  Device work of one pool is ordered on the stream the caller
 * passes; a pool, like the reference's Backend (thuban_backend/src/lib.rs
 * :57-69), has one owner and is not thread-safe.
 *
 * HIP graph capture (no reference counterpart).  On a capturing stream:
 *  - thb_pool_alloc_rows, thb_kv_store, thb_dplan_build and the attention
 *    calls over a device plan (thb_attn_dplan, thb_attn_append_dplan,
 *    thb_attn_step_dplan) read everything a step changes (row meta, page
 *    counts, block table) from device memory, so a graph of them replays
 *    correctly while the rows move and pages are forked, truncated or freed
 *    between replays.
 *    Once thb_pool_alloc_rows has been captured the pool is in graph mode
 *    for good: every later call that reads the host arena (page API,
 *    thb_attn, gather, ...) first waits for the device and reloads the host
 *    arena from the device allocator, as thb_pool_pull does.
 *  - Other entry points that can be captured replay the captured call: the
 *    host data they upload travels in the graph's own kernel arguments (up
 *    to 256 KiB per upload), and a library buffer a graph uses is not freed
 *    before its pool.  Such a replay is valid while what the call read on
 *    the host at capture time (positions, pages) still holds.
 *  - These refuse with THB_ERR_INVALID: thb_attn and its variants (host
 *    plans; thb_attn_step_dplan is their capturable form), thb_kv_store_rope
 *    and thb_rope_rows (host position checks),
 *    thb_pool_status / _read_state / _pull (they wait for the stream), any
 *    call while page-API calls queued on the host have not run (flush with
 *    thb_pool_sync before capturing), and any call that would have to grow
 *    a library buffer (run it once outside the capture first).
 */
#ifndef THUBAN_HIP_H
#define THUBAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ----------------------------------------------------------- conventions */

/* Status codes.  THB_ERR_MODEL / THB_ERR_CONFIG / THB_ERR_GPU correspond to
 * thuban_error::Error::{Model, Config, Gpu} (thuban_error/src/lib.rs:5-21). */
#define THB_OK 0
#define THB_ERR_MODEL (-1)
#define THB_ERR_CONFIG (-2)
#define THB_ERR_GPU (-3)
#define THB_ERR_INVALID (-4)

/* Element types of source / query / output buffers. */
#define THB_DT_F32 0u
#define THB_DT_F16 1u
#define THB_DT_BF16 2u

/* KV storage types.  BF16_TRUNC is the reference's storage: bf16 by
 * truncating an f32 (kv_store.wgsl:20-22, thuban_num/src/lib.rs:66-68).
 * F16_RNE is IEEE half with round-to-nearest-even (thuban_num lib.rs:25-60). */
#define THB_KV_BF16_TRUNC 0u
#define THB_KV_F16_RNE 1u

/* Block-table sentinel for a missing page (u32::MAX, pool.rs:85-93). */
#define THB_NO_PAGE 0xFFFFFFFFu
/* thb_attn_spec.seq value that takes each row's sequence from row meta. */
#define THB_SEQ_PER_ROW 0xFFFFFFFFu

/* Message of the last failed call on this thread ("" if none). */
const char* thb_last_error(void);
/* ABI revision of this header. */
uint32_t thb_abi_version(void);
#define THB_ABI_VERSION 8u

/* head_dim guard, replaces ops::check_head_dim (ops/attn.rs:83-90) exactly:
 * THB_ERR_CONFIG "head_dim {hd} outside [64, 512]". */
int thb_check_head_dim(uint32_t head_dim);
/* No reference counterpart: what this backend accepts, thb_check_head_dim
 * plus head_dim % 8 == 0 (16-byte vector lanes); THB_ERR_CONFIG otherwise.
 * thb_pool_create and thb_rope_rows apply it. */
int thb_backend_head_dim(uint32_t head_dim);

/* ------------------------------------------------ host page allocator */

/* KvArena (pool.rs:11-118) with the page length as a parameter (the
 * reference fixes PAGE_LEN = 32, thuban_kernel/src/lib.rs:9) and an
 * extension for shared pages: fork() shares full pages between sequences
 * with reference counts, and alloc() copies a shared page before a write
 * lands in it (copy-on-write).  Pure host code: usable without a GPU. */
typedef struct thb_arena thb_arena;

typedef struct thb_arena_info {
    uint32_t pages;     /* KvArena::pages (pool.rs:95-97) */
    uint32_t used;      /* KvArena::used (pool.rs:99-101) */
    uint32_t max_pages; /* KvArena::max_pages (pool.rs:103-105) */
    uint32_t seqs;      /* KvArena::seqs (pool.rs:107-109) */
    uint32_t page_len;
    uint32_t pending_copies; /* copy-on-write copies not yet executed */
} thb_arena_info;

/* KvArena::new (pool.rs:20-45).  pages < 0 means ArenaSpec.pages = None
 * (sum of ceil(seq_len / page_len)).  page_len must be a power of two in
 * [1, 256]. */
int thb_arena_create(const uint32_t* seq_lens, uint32_t seqs, int64_t pages, uint32_t page_len,
                     thb_arena** out);
void thb_arena_destroy(thb_arena* arena);
/* KvArena::alloc (pool.rs:47-65), plus copy-on-write of shared pages that
 * [pos, pos+tokens) touches. */
int thb_arena_alloc(thb_arena* arena, uint32_t seq, uint32_t pos, uint32_t tokens);
/* KvArena::free_seq (pool.rs:67-71). */
int thb_arena_free_seq(thb_arena* arena, uint32_t seq);
/* KvArena::truncate (pool.rs:73-79). */
int thb_arena_truncate(thb_arena* arena, uint32_t seq, uint32_t keep_tokens);
/* KvArena::covers (pool.rs:81-83): 1 or 0, negative on error. */
int thb_arena_covers(const thb_arena* arena, uint32_t seq, uint32_t tokens);
/* No reference counterpart: dst (empty) shares src's pages holding tokens
 * [0, tokens); a partial last page is copied so that both can append. */
int thb_arena_fork(thb_arena* arena, uint32_t src, uint32_t dst, uint32_t tokens);
/* KvArena::table (pool.rs:85-93): n must be seqs * max_pages. */
int thb_arena_table(const thb_arena* arena, uint32_t* out, size_t n);
/* KvArena::table_of (pool.rs:115-117): writes min(cap, len) entries. */
int thb_arena_table_of(const thb_arena* arena, uint32_t seq, uint32_t* out, size_t cap, uint32_t* len);
/* KvArena::seq_len (pool.rs:111-113). */
int thb_arena_seq_len(const thb_arena* arena, uint32_t seq, uint32_t* len);
int thb_arena_info_get(const thb_arena* arena, thb_arena_info* info);
/* Moves the pending copy-on-write copies (src_page, dst_page, tokens) out of
 * the arena; a device pool executes them itself before its next kernel. */
int thb_arena_take_copies(thb_arena* arena, uint32_t* triples, size_t cap, uint32_t* n);
/* The free stack, bottom first (free_list[n - 1] is the next page handed
 * out; KvArena::free, pool.rs:16), and the reference counts [pages]. */
int thb_arena_free_list(const thb_arena* arena, uint32_t* free_list, size_t cap, uint32_t* n);
int thb_arena_refs(const thb_arena* arena, uint32_t* refs, size_t cap);

/* ---------------------------------------------------------- device pool */

/* One hipMalloc'd arena holding K and V of every layer, plus one device
 * block table [seqs * max_pages] shared by all layers (the reference keeps a
 * copy per layer, model.rs:413-418).  Each plane holds the elements of the
 * reference's KvPool tensors [kv_heads, pages * page_len, head_dim]
 * (pool.rs:131-153) with every page reordered for the attention kernel's
 * matrix-core operands (THB_PAGE_LAYOUT_MFMA).  With P = page_len, page
 * base B = (h * pages + s / P) * head_dim * P, j = s % P, g0 = d - d % 32
 * and w = min(32, head_dim - g0), element (head h, slot s, dim d) sits at
 *   K: B + g0 * P + w * j + d % 32               ([head_dim/32][P][32] groups)
 *   V: B + (j / 4) * 4 * head_dim + 4 * d + j % 4  ([P/4][head_dim][4] groups)
 * so a token appended to a page dirties head_dim / 32 K and head_dim / 16 V
 * cache lines.  thb_kv_gather returns both in the reference's token-major
 * layout. */
#define THB_PAGE_LAYOUT_MFMA 2u
typedef struct thb_pool thb_pool;

typedef struct thb_pool_desc {
    uint32_t layers;
    uint32_t kv_heads;
    uint32_t head_dim;          /* used when head_dims == NULL */
    const uint32_t* head_dims;  /* optional per-layer head_dim [layers] */
    uint32_t page_len;          /* power of two, 8..256; 16 and 32 are tuned */
    uint32_t kv_dtype;          /* THB_KV_* */
    uint32_t seqs;
    const uint32_t* seq_lens;   /* ArenaSpec.seq_lens [seqs] */
    int64_t pages;              /* ArenaSpec.pages; < 0 = None */
    uint32_t part_len;          /* split-K partition in tokens (0 = 4096);
                                   multiple of 16 and of page_len, at most
                                   1008 pages */
    void* arena_dev;            /* optional caller-owned device memory */
    uint64_t arena_bytes;       /* its size; 0 = let the pool hipMalloc */
} thb_pool_desc;

typedef struct thb_layer_info {
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t pool_len;          /* KvPool::capacity = pages * page_len */
    uint32_t max_pages;
    uint32_t page_len;
    uint32_t kv_dtype;
    uint64_t plane_elems;       /* elements per head plane = pool_len * head_dim */
    uint32_t page_layout;       /* THB_PAGE_LAYOUT_* of the K and V pages */
} thb_layer_info;

/* KvArena::new + KvPool::new for every layer (pool.rs:20-45,131-153).  The
 * memory is zero-filled, as Backend::zero_tensor does (lib.rs:192-206).
 *
 * The page allocator lives on the device: the free stack, per-page reference
 * counts and per-sequence page counts sit in HBM next to the block table,
 * and kernels change them with KvArena's semantics (pops yield pages 0, 1,
 * 2, ...; freed pages return in table order).  The pool's host arena
 * (thb_pool_arena) is a mirror that runs every page-API call first, so that
 * errors return synchronously with the reference's messages and attention
 * can plan its launch without reading the GPU. */
int thb_pool_create(const thb_pool_desc* desc, thb_pool** out);
void thb_pool_destroy(thb_pool* pool);
/* Page API of LanguageModel::{alloc,free,truncate}_pages (traits.rs:39-41,
 * transformer/forward.rs:534-550).  Runs on the host mirror now and on the
 * device allocator (with any copy-on-write copies) before the pool's next
 * kernel, or at thb_pool_sync; no block table is uploaded (the reference
 * re-uploads the whole table to every layer, model.rs:413-418). */
int thb_pool_alloc(thb_pool* pool, uint32_t seq, uint32_t pos, uint32_t tokens);
int thb_pool_free_seq(thb_pool* pool, uint32_t seq);
int thb_pool_truncate(thb_pool* pool, uint32_t seq, uint32_t keep_tokens);
/* No reference counterpart: fork with block sharing + partial-page copy. */
int thb_pool_fork(thb_pool* pool, uint32_t src, uint32_t dst, uint32_t tokens);
/* Runs the queued page-API calls on the device allocator, on stream. */
int thb_pool_sync(thb_pool* pool, void* stream);

typedef struct thb_rows thb_rows;
/* The engine's per-plan allocation (thuban_generate/src/engine.rs:197-200:
 * alloc_pages(seq, tokens) -> KvArena::alloc(seq, pos, tokens), pool.rs
 * :47-65) for the rows [row_off, row_off + m) of the row meta, run by the
 * device allocator on stream: each maximal run of rows of one sequence is
 * KvArena::alloc(seq, position of its first row, rows in the run), in row
 * order, with copy-on-write of shared pages the write touches.  Each
 * sequence may head one run only (THB_ERR_INVALID).  A failing run (context
 * limit, arena exhausted) ends the call with the reference's message; the
 * runs before it keep their pages, as the engine's loop does.  Captured in a
 * graph, each replay validates its own rows on the device (a bad or
 * repeated sequence allocates nothing and is reported by thb_pool_status
 * with the message above) and copies shared pages it writes into (copy on
 * write) over a launch sized by the device's own copy count; the pool enters
 * graph mode (see the top of this file). */
int thb_pool_alloc_rows(thb_pool* pool, const thb_rows* rows, uint32_t row_off, uint32_t m, void* stream);
/* First failure the device allocator met since the last call (THB_OK if
 * none), with the reference's message; clears it.  Synchronises stream. */
int thb_pool_status(thb_pool* pool, void* stream);
/* Copies the device allocator's state to host memory after stream's work:
 * the free stack (bottom first, so free_list[n_free - 1] is the next page
 * handed out), the reference counts [pages] and the flattened block table
 * [seqs * max_pages] (KvArena::table layout, pool.rs:85-93).  Any pointer
 * may be NULL. */
int thb_pool_read_state(thb_pool* pool, void* stream, uint32_t* free_list, size_t free_cap, uint32_t* n_free,
                        uint32_t* refs, size_t refs_cap, uint32_t* table, size_t table_n);
/* Reloads the host mirror from the device allocator (after changes the host
 * did not see, such as replays of a captured thb_pool_alloc_rows; in graph
 * mode every call that reads the host arena does this first). */
int thb_pool_pull(thb_pool* pool, void* stream);
/* The pool's allocator (queries; mutate through thb_pool_* instead). */
const thb_arena* thb_pool_arena(const thb_pool* pool);
/* Device pointers of layer `layer`'s K and V planes (KvPool::k / ::v, in the
 * page layout above). */
int thb_pool_layer(const thb_pool* pool, uint32_t layer, void** k_dev, void** v_dev, thb_layer_info* info);
/* Device block table [seqs * max_pages] (KvPool::block_table). */
int thb_pool_block_table(const thb_pool* pool, const uint32_t** table_dev);
/* Whole arena: base pointer and size in bytes. */
int thb_pool_memory(const thb_pool* pool, void** base_dev, uint64_t* bytes);

/* -------------------------------------------------------------- row meta */

/* Row metadata, rows::row_meta / write_row_meta (rows.rs:11-30): 8 u32 per
 * row, [pos, seq, 0 x 6].  The object keeps a host mirror of what it last
 * wrote so that attention can plan its launch without reading the GPU. */
int thb_rows_create(uint32_t max_m, thb_rows** out);
void thb_rows_destroy(thb_rows* rows);
/* rows::write_row_meta: uploads rows [0, m) on stream. */
int thb_rows_write(thb_rows* rows, const uint32_t* positions, const uint32_t* seqs, uint32_t m, void* stream);
/* Device pointer of the 8 x max_m u32 buffer. */
const uint32_t* thb_rows_device(const thb_rows* rows);

/* --------------------------------------------------------------- kernels */

/* ops::kv_store (ops/attn.rs:53-81) / kv_store.wgsl:24-46: for each row r of
 * [row_off, row_off + m): slot = block_table[seq][pos / page_len] * page_len
 * + pos % page_len, and K/V[h][slot][:] = encode(src[r - row_off][h][:]) for
 * every KV head.  src_dtype is THB_DT_*; src is [m, kv_heads, head_dim],
 * 16-byte aligned.  Bit-exact: bf16 truncation or f16 RNE as thuban_num. */
int thb_kv_store(thb_pool* pool, uint32_t layer, const void* k_src_dev, const void* v_src_dev, uint32_t src_dtype,
                 const thb_rows* rows, uint32_t row_off, uint32_t m, void* stream);

/* ops::AttnSpec (ops/attn.rs:8-16) plus the extensions of this backend. */
typedef struct thb_attn_spec {
    uint32_t q_heads;  /* AttnSpec.q_heads; multiple of kv_heads */
    uint32_t window;   /* AttnSpec.window; 0 = none (causal only) */
    float scale;       /* AttnSpec.scale */
    uint32_t m;        /* AttnSpec.m: rows in this call */
    uint32_t causal;   /* AttnSpec.causal */
    uint32_t seq;      /* AttnSpec.seq, or THB_SEQ_PER_ROW (batched rows) */
    uint32_t row_off;  /* first row in the row meta (the reference binds a
                          slice at row_off * 32 bytes, forward.rs:332) */
    float softcap;     /* extension: 0 = off, else s = cap * tanh(s / cap) */
    uint32_t q_dtype;  /* THB_DT_F32 (reference), THB_DT_F16 or THB_DT_BF16 */
    uint32_t y_dtype;  /* THB_DT_F32 (reference), THB_DT_F16 or THB_DT_BF16 (round to
                          nearest even; the o_proj GEMM's operand type) */
} thb_attn_spec;

/* ops::attn (ops/attn.rs:18-51) / attn.wgsl:53-365.  q, y: [m, q_heads,
 * head_dim], 16-byte aligned.  Key ranges per row follow attn.wgsl:78-88,169
 * exactly.  One launch covers every row (batched over sequences), as a
 * split-K pass with a deterministic log-sum-exp merge when a row's keys span
 * several part_len partitions (in the same launch, by the workgroup that
 * finishes the group's last partition; a second kernel for prefill blocks):
 * output is independent of physical page placement and of the other rows in
 * the batch.  Products on the matrix cores with q and p split into high and
 * low halves, f32 accumulation; within 2e-3 of an exact softmax.  The pool
 * holds the split-K partial results and the merge counters: calls on one
 * pool run in stream order, and calls on one pool from several streams at
 * once race. */
int thb_attn(thb_pool* pool, uint32_t layer, const void* q_dev, void* y_dev, const thb_attn_spec* spec,
             const thb_rows* rows, void* stream);

/* thb_kv_store of rows [spec->row_off, spec->row_off + spec->m) followed by
 * thb_attn(spec): the step the model runs per layer (transformer/forward.rs
 * :300-336).  Results are bit-identical to the two calls.  When the call is
 * causal, each sequence's rows fit in one query group (decode, and verify
 * chunks of up to 16 / (q_heads / kv_heads) rows) and every row's new token
 * is its last key, the append runs inside the attention launch (one kernel
 * instead of two); otherwise the two kernels run in order. */
int thb_attn_append(thb_pool* pool, uint32_t layer, const void* k_src_dev, const void* v_src_dev, uint32_t src_dtype,
                    const void* q_dev, void* y_dev, const thb_attn_spec* spec, const thb_rows* rows, void* stream);

/* ----------------------------------------------------------------- RoPE */

/* Rotary position embedding as rope.wgsl:16-40 / ops::rope (ops/rope.rs:22-48)
 * and, with a weight, the RMSNorm + rotation of norm.wgsl MODE 4 /
 * ops::norm_rope (ops/norm.rs:73-109), keyed off each row's row-meta pos.
 * With half = rot / 2 and c = cos[pos][d % half], s = sin[pos][d % half]:
 *   y[d] = x[d] c - x[d + half] s   (d < half)
 *   y[d] = x[d] c + x[d - half] s   (half <= d < rot)
 *   y[d] = x[d]                     (d >= rot)
 * where x is the head vector, first scaled by w[d] / sqrt(mean(x^2) + eps)
 * when a norm weight is given.  The tables are the reference's rope_tables
 * (ops/rope.rs:50-80): f32 [max_pos][rot / 2], on the device.  Arithmetic is
 * f32 without fused multiply-adds; the sum of squares runs over 8-element
 * chunks in order, then over the chunks in order. */
typedef struct thb_rope {
    const float* cos_dev;    /* [max_pos][rot / 2] */
    const float* sin_dev;
    uint32_t rot;            /* rotated leading dims: a multiple of 16, <= head_dim */
    uint32_t max_pos;        /* table rows; every row's pos must be below it */
    const float* q_norm_dev; /* [head_dim] RMSNorm weight of query heads, or NULL (rope only) */
    const float* k_norm_dev; /* [head_dim] RMSNorm weight of key heads, or NULL */
    float eps;               /* RMSNorm epsilon */
} thb_rope;

/* ops::rope / ops::norm_rope on rows [row_off, row_off + m) of x [m, heads,
 * head_dim] (dtype THB_DT_F32 or THB_DT_F16, 16-byte aligned), in place.
 * norm_w_dev: [head_dim] weight (norm_rope) or NULL (rope only). */
int thb_rope_rows(void* x_dev, uint32_t dtype, uint32_t m, uint32_t heads, uint32_t head_dim,
                  const float* norm_w_dev, const thb_rope* rope, const thb_rows* rows, uint32_t row_off,
                  void* stream);

/* No reference counterpart: the model's ops::rope(k) (or norm_rope with
 * rope->k_norm_dev) followed by ops::kv_store (transformer/forward.rs
 * :186-313) in one pass: the rotated K is encoded straight into the pages,
 * never written back.  V is stored as by thb_kv_store.  The pool contents
 * are bit-identical to thb_rope_rows on K followed by thb_kv_store. */
int thb_kv_store_rope(thb_pool* pool, uint32_t layer, const void* k_src_dev, const void* v_src_dev,
                      uint32_t src_dtype, const thb_rope* rope, const thb_rows* rows, uint32_t row_off, uint32_t m,
                      void* stream);

/* thb_attn with the query rotated (and normalised with rope->q_norm_dev) as
 * it is loaded: ops::rope(q) / norm_rope(q) + ops::attn in one launch. */
int thb_attn_rope(thb_pool* pool, uint32_t layer, const void* q_dev, void* y_dev, const thb_attn_spec* spec,
                  const thb_rope* rope, const thb_rows* rows, void* stream);

/* The whole per-layer step (transformer/forward.rs:186-336): rope of q and
 * k, kv_store, attention.  When thb_attn_append would fuse, one launch does
 * all of it; otherwise thb_kv_store_rope then thb_attn_rope.  Results are
 * bit-identical either way. */
int thb_attn_append_rope(thb_pool* pool, uint32_t layer, const void* k_src_dev, const void* v_src_dev,
                         uint32_t src_dtype, const void* q_dev, void* y_dev, const thb_attn_spec* spec,
                         const thb_rope* rope, const thb_rows* rows, void* stream);

/* ------------------------------------------------------ the whole step */

/* Inputs and outputs of one attention call beyond thb_attn_spec.  Only q_dev
 * and y_dev are required; the other members extend the call. */
typedef struct thb_attn_io {
    const void* q_dev;     /* head h of row r at (r * q_heads + h) * q_stride elements (spec->q_dtype) */
    uint32_t q_stride;     /* 0 = head_dim.  2 * head_dim reads the query straight out of a fused
                              q|gate projection, as split_q_gate.wgsl lays it out (qwen35/layers.rs
                              :138-149) */
    void* y_dev;           /* [m, q_heads, head_dim] of spec->y_dtype */
    const void* gate_dev;  /* output gate, or NULL: y = attention * 1 / (1 + exp(-gate))
                              (sigmoid_mul.wgsl, qwen35/layers.rs:231-238), in spec->q_dtype */
    uint32_t gate_stride;  /* 0 = head_dim; elements from one gate head to the next */
    const void* k_src_dev; /* rows appended first, as thb_attn_append, or NULL */
    const void* v_src_dev;
    uint32_t src_dtype;
    const thb_rope* rope;  /* rotary embedding of q (and of the appended k), or NULL */
} thb_attn_io;

/* thb_attn with every extension of io: the layer's attention from the
 * projected q|gate and k, v to the gated output the o_proj GEMM consumes
 * (transformer/forward.rs:184-351, qwen35/layers.rs:138-238), in one launch
 * at decode.  thb_attn, thb_attn_rope, thb_attn_append and
 * thb_attn_append_rope are this call with some members NULL. */
int thb_attn_step(thb_pool* pool, uint32_t layer, const thb_attn_io* io, const thb_attn_spec* spec,
                  const thb_rows* rows, void* stream);

/* ------------------------------------------------ the attention consumer */

/* ops::check_gemm_dims (crates/thuban_model/src/ops/gemm.rs:133-146) for one
 * pair: THB_ERR_CONFIG "dimension pair (N={n}, K={k}) does not satisfy N%16
 * and K%64". */
int thb_check_gemm_dims(uint32_t n, uint32_t k);
/* ops::gemm_acc (crates/thuban_model/src/ops/gemm.rs:113-131), the o_proj
 * product after attention (transformer/forward.rs:338-351), for plain 16-bit
 * weights: y[rows, n] = x[rows, k] . w[n, k]^T, plus y's old value when acc
 * (the reference adds into the residual stream).  rows == 1 is the
 * reference's gemv.  x: THB_DT_F32 (the reference's activations),
 * THB_DT_F16 or THB_DT_BF16 (thb_attn_spec.y_dtype); w: THB_DT_BF16 or
 * THB_DT_F16; y: f32; all 16-byte aligned; n and k as thb_check_gemm_dims.
 * Products on the matrix cores in f32 accumulation; an x wider than the
 * weight type is split into high and low parts (f32-grade products).
 * Deterministic: the same inputs give the same bits.  At 17-64 rows the
 * split-K partial sums and their merge counters live in one buffer per
 * device: calls on one device from several streams at once race. */
int thb_gemm_acc(const void* x_dev, uint32_t x_dtype, const void* w_dev, uint32_t w_dtype, float* y_dev,
                 uint32_t rows, uint32_t n, uint32_t k, uint32_t acc, void* stream);

/* No reference counterpart.  thb_attn for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc): the launch plan and the split-K partial results go
 * to a fixed device array of THB_NOALLOC_SCRATCH_BYTES that the library
 * holds on each device until the process ends, and the plan is staged
 * through pinned memory the pool allocated at creation, so the call runs no
 * hipMalloc, hipFree or other allocating routine.  The first
 * THB_NOALLOC_PLAN_BYTES hold the plan, the rest the partial results; a call
 * needing more returns THB_ERR_INVALID.  Results are bit-identical to
 * thb_attn.  Every call on a device shares the array: calls that overlap on
 * one device (other streams, other threads) race.  The pool's device must be
 * current.  It can be captured in a graph: the plan then travels in the
 * graph's own kernel arguments and every replay writes it into the array
 * before the attention launch, so a replay recomputes the captured call (at
 * its captured positions) whatever other calls left in the array. */
#define THB_NOALLOC_SCRATCH_BYTES (32u << 20)
#define THB_NOALLOC_PLAN_BYTES (256u << 10)
int thb_attn_noalloc(thb_pool* pool, uint32_t layer, const void* q_dev, void* y_dev, const thb_attn_spec* spec,
                     const thb_rows* rows, void* stream);

/* No reference counterpart: ops::attn (ops/attn.rs:18-51) for decode steps
 * captured once in a graph and replayed while the rows' positions move.
 * thb_dplan_build plans the call on the device from the row meta in device
 * memory (the key ranges, groups and partitions thb_attn's host planner
 * makes, by the same rules) into buffers the plan owns; thb_attn_dplan then
 * launches attention over a fixed grid whose slots past the call's groups or
 * a group's partitions do nothing.  Neither allocates, uploads or reads
 * anything on the host, so both can be captured; a replay computes each
 * (group, partition) as thb_attn does, bit for bit, at the row meta's
 * positions of that replay.  Chunks of four or more groups (prefill) run on
 * the decode kernel (correct, slower: use thb_attn).  A row whose sequence's
 * pages do not cover its keys reads nothing (its output is NaN) and the
 * first such row is reported by thb_pool_status ("pages must cover the
 * chunk: ...").  A plan serves calls of up to max_m rows (at most 4096) and
 * q_heads query heads; its grid holds max_m x (partitions of the pool's
 * longest sequence) x kv_heads workgroups, the unused ones returning at
 * once.  Build it after the row meta it plans (stream order), and rebuild it
 * when the rows, the spec or the pages change.  One plan is one set of
 * buffers: calls that use it must not overlap. */
typedef struct thb_dplan thb_dplan;
int thb_dplan_create(thb_pool* pool, uint32_t max_m, uint32_t q_heads, thb_dplan** out);
/* No reference counterpart: thb_dplan_create with flags.  THB_DPLAN_PREFILL
 * makes the plan a work list (calls of up to 8192 rows, head_dim <= 256):
 * thb_dplan_build also cuts chunks of four or more groups into blocks of
 * consecutive groups (thb_attn's prefill blocks) and runs each block whose
 * keys fit one partition on the prefill kernel, the other groups as decode
 * items, and orders every entry longest first; thb_attn_dplan launches one
 * workgroup per compute unit that claims entries from a counter in the plan
 * (reset by the launch's last workgroup).  Decode rows, and chunks whose
 * blocks each fit one partition, give thb_attn's outputs bit for bit; a
 * block spanning several partitions runs as decode items where thb_attn
 * runs the prefill kernel and a merge, so its rows differ from thb_attn's
 * in the order of the sums only (within 1e-5 on the tested cases). */
#define THB_DPLAN_PREFILL 1u
/* THB_DPLAN_APPEND (fixed-grid plans only; causal calls) makes the plan
 * serve thb_attn_append_dplan as well: each thb_dplan_build also checks, on
 * the device, the conditions under which thb_attn_append appends inside its
 * attention launch (each chunk fits one group, every row's keys end at its
 * new token with positions rising in the chunk, every row in the fixed
 * sequence when spec.seq is fixed, no sequence heading two chunks).  A call
 * that fails them is not planned at all: thb_pool_status reports the first
 * failing row ("the append cannot run inside the attention launch: ..."),
 * the launch appends nothing and every output is NaN. */
#define THB_DPLAN_APPEND 2u
int thb_dplan_create_ex(thb_pool* pool, uint32_t max_m, uint32_t q_heads, uint32_t flags, thb_dplan** out);
void thb_dplan_destroy(thb_dplan* plan);
int thb_dplan_build(thb_dplan* plan, const thb_attn_spec* spec, const thb_rows* rows, void* stream);
int thb_attn_dplan(thb_pool* pool, uint32_t layer, const void* q_dev, void* y_dev, const thb_dplan* plan,
                   void* stream);
/* No reference counterpart: kv_store then attention of a decode step
 * (transformer/forward.rs:300-336, as thb_attn_append) over a plan made with
 * THB_DPLAN_APPEND, in one launch: the workgroup whose keys hold a row's new
 * token stores the row's K and V (rows [0, m) of k_src_dev / v_src_dev,
 * [m, kv_heads, head_dim] in src_dtype, as thb_kv_store) before reading
 * them.  Outputs and pool bytes equal thb_attn_append's bit for bit; it can
 * be captured with thb_dplan_build, so a replayed step is two launches. */
int thb_attn_append_dplan(thb_pool* pool, uint32_t layer, const void* k_src_dev, const void* v_src_dev,
                          uint32_t src_dtype, const void* q_dev, void* y_dev, const thb_dplan* plan, void* stream);
/* No reference counterpart: the rotary tables' bound for device-planned
 * calls (thb_rope.max_pos; 0 removes it).  Each later thb_dplan_build
 * reports a row whose position is not below it ("row position P outside
 * the rope tables (N positions)", thb_pool_status) and gives that row no
 * keys (a NaN output; with THB_DPLAN_APPEND the whole call is planned
 * empty).  The plan must be built again before its next launch. */
int thb_dplan_set_pos_limit(thb_dplan* plan, uint32_t max_pos);
/* No reference counterpart: thb_attn_step over a device plan, either form
 * (ops::attn with the thb_attn_io extensions: query stride, sigmoid gate,
 * rotary embedding with optional q/k norm, and with k_src/v_src the append
 * inside the launch, which needs THB_DPLAN_APPEND).  io->rope needs a plan
 * built with a position limit of at most io->rope->max_pos.  Outputs (and,
 * with the append, pool bytes) equal thb_attn_step's bit for bit, the
 * work-list form as thb_attn_dplan describes; it can be captured. */
int thb_attn_step_dplan(thb_pool* pool, uint32_t layer, const thb_attn_io* io, const thb_dplan* plan,
                        void* stream);

/* No reference counterpart.  Copies tokens [t0, t0 + n) of seq, layer
 * `layer`, into contiguous k_dst/v_dst [kv_heads, n, head_dim] in the KV type
 * (bit copy). */
int thb_kv_gather(thb_pool* pool, uint32_t layer, uint32_t seq, uint32_t t0, uint32_t n, void* k_dst_dev,
                  void* v_dst_dev, void* stream);

/* No reference counterpart.  Inverse of thb_kv_gather: writes contiguous
 * [kv_heads, n, head_dim] words (KV type) into tokens [t0, t0 + n) of seq.
 * Writes in place, so a page the sequence shares with another (after
 * thb_pool_fork) is refused with THB_ERR_MODEL. */
int thb_kv_scatter(thb_pool* pool, uint32_t layer, uint32_t seq, uint32_t t0, uint32_t n, const void* k_src_dev,
                   const void* v_src_dev, void* stream);

/* One range of a batched gather or scatter: tokens [t0, t0 + n) of seq in
 * layer `layer`. */
typedef struct thb_kv_range {
    uint32_t seq;
    uint32_t layer;
    uint32_t t0;
    uint32_t n;
} thb_kv_range;

/* No reference counterpart.  thb_kv_gather of `count` ranges in one launch:
 * range i lands in k_dst / v_dst at element offset sum_{j < i} kv_heads *
 * n_j * head_dim, laid out [kv_heads, n_i, head_dim].  The ranges' layers
 * share one head_dim. */
int thb_kv_gather_batch(thb_pool* pool, const thb_kv_range* ranges, uint32_t count, void* k_dst_dev,
                        void* v_dst_dev, void* stream);
/* No reference counterpart.  The inverse of thb_kv_gather_batch.  Like
 * thb_kv_scatter, pages shared with another sequence are refused
 * (THB_ERR_MODEL), and so are ranges of one sequence and layer that overlap
 * (THB_ERR_INVALID). */
int thb_kv_scatter_batch(thb_pool* pool, const thb_kv_range* ranges, uint32_t count, const void* k_src_dev,
                         const void* v_src_dev, void* stream);

/* No reference counterpart.  For each host triple (src_page, dst_page,
 * tokens) copies slots [0, tokens) of src_page to dst_page, K and V, every
 * head of every layer.  Triples must not chain (no page both a source and a
 * destination). */
int thb_block_copy(thb_pool* pool, const uint32_t* triples, uint32_t n, void* stream);

/* ----------------------------------------------------------- measurement */

/* No reference counterpart: a measurement aid.  Streams `bytes` of src_dev
 * with 16-byte non-temporal loads (mode 0, read: folds them into registers
 * and writes workgroups x 2 KiB of dst_dev) or copies them to dst_dev (mode
 * 1), each of `workgroups` workgroups of 512 lanes taking one contiguous
 * slab.  The benchmark times it to state the device's achievable linear
 * HBM rate next to the specification's. */
int thb_hbm_stream(const void* src_dev, void* dst_dev, uint64_t bytes, uint32_t mode, uint32_t workgroups,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* THUBAN_HIP_H */
