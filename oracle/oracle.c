/*
 * CPU oracle for the paged KV-cache path.  TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic of the reference engine
 * ("Thuban", formetaohy/Flint) for the paged KV path so that the HIP product
 * can be checked against it.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker.  The
 * product (flint_amd/) never links or calls it.
 *
 * Reference files restated here (paths relative to the reference root):
 *   crates/thuban_num/src/lib.rs:1-68            f16/bf16 codecs
 *   crates/thuban_kernel/wgsl/kv_store.wgsl:20-46 append/scatter
 *   crates/thuban_kernel/wgsl/attn.wgsl:42-365    paged attention masks/kv_len
 *   crates/thuban_backend/tests/support/cpu_ref.rs:172-228 exact softmax
 *   crates/thuban_kernel/wgsl/rope.wgsl:16-40     rotary embedding
 *   crates/thuban_kernel/wgsl/norm.wgsl:122-160   RMSNorm + rotation (MODE 4)
 *   crates/thuban_backend/tests/support/cpu_ref.rs:11-35 gemm / gemv
 *
 * How each function is pinned (checked by tests/test_oracle.py):
 *   codecs        thuban_num known-answer tests (lib.rs:78-139) + exhaustive
 *                 f16->f32->f16 round trip + brute force vs numpy's IEEE cast
 *   kv_store      reference anchors kernels.rs:1396-1407 and the LCG vector
 *                 test kernels.rs:1266-1308 (closed form cpu_ref.rs:154-170)
 *   attn          reference anchors kernels.rs:1439-1481 ([2,3] / [3,4]),
 *                 one-valid-key and uniform-weight closed forms, paged ==
 *                 contiguous (batch.rs:302-347), window >= context == no window
 *   attn_f32      agrees with attn (double) within 1e-5 on random inputs
 *   gather/copy   memcpy closed form (no reference counterpart; pinned by
 *                 round trips against kv_store)
 *   softcap       closed form cap*tanh(s/cap); parity vs the reference is
 *                 unpinned because the reference has no attention soft-cap.
 *   gemm          cpu_ref::gemm/gemv (cpu_ref.rs:11-35): f32 sums in k order;
 *                 pinned by numpy's float64 matmul within the f32 rounding
 *                 bound, the identity-weight closed form y = x (+ y0), and
 *                 rows == 1 equal to gemv
 *   rope_rows     reference anchor kernels.rs:1410-1436, the rope_case vectors
 *                 of kernels.rs:1200-1263 (LCG inputs) against a double-
 *                 precision rotation, position 0 = identity, dims >= rot
 *                 untouched, pair norms kept; the RMSNorm against a double-
 *                 precision RMS.  Sums of squares run over 8-element chunks in
 *                 order, then over the chunks in order (the WGSL kernel sums
 *                 4-element vectors per thread and reduces by a tree; float
 *                 association differs, within the reference tests' 1e-5).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_KV_BF16 0 /* bf16 by truncation (reference parity) */
#define ORC_KV_F16 1  /* f16 round-to-nearest-even            */

#define ORC_SRC_F32 0
#define ORC_SRC_F16 1
#define ORC_SRC_BF16 2

/* ---------------------------------------------------------------- codecs */

/* thuban_num/src/lib.rs:1-23 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            int32_t e = 127 - 15 + 1;
            uint32_t m = mant;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            bits = (sign << 31) | ((uint32_t)e << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) {
        bits = (sign << 31) | 0x7f800000u | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* thuban_num/src/lib.rs:25-60: round to nearest even, subnormals kept,
 * overflow saturates to infinity, every NaN becomes sign|0x7E00. */
uint16_t orc_f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xff) return mant == 0 ? (uint16_t)(sign | 0x7c00u) : (uint16_t)(sign | 0x7e00u);
    int32_t half_exp = exp - 127 + 15;
    if (half_exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (half_exp <= 0) {
        if (half_exp < -10) return sign;
        uint32_t m = mant | 0x800000u;
        uint32_t shift = (uint32_t)(14 - half_exp);
        uint32_t shifted = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        int round = rem > half || (rem == half && (shifted & 1u) == 1u);
        return (uint16_t)(sign | (uint16_t)(shifted + (uint32_t)round));
    }
    uint16_t frac = (uint16_t)(mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    uint16_t result = (uint16_t)(sign | (uint16_t)(half_exp << 10) | frac);
    if (rem > 0x1000u || (rem == 0x1000u && (frac & 1u) == 1u)) result = (uint16_t)(result + 1u);
    return result;
}

/* thuban_num/src/lib.rs:62-64 */
float orc_bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* thuban_num/src/lib.rs:66-68 and pack2 at kv_store.wgsl:20-22: truncation. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    return (uint16_t)(bits >> 16);
}

void orc_f32_to_f16_n(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_n(const uint16_t* x, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(x[i]);
}
void orc_f32_to_bf16_n(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(x[i]);
}

static float src_value(const void* src, int src_dtype, size_t i) {
    switch (src_dtype) {
        case ORC_SRC_F16: return orc_f16_to_f32(((const uint16_t*)src)[i]);
        case ORC_SRC_BF16: return orc_bf16_to_f32(((const uint16_t*)src)[i]);
        default: return ((const float*)src)[i];
    }
}

static uint16_t encode_kv(float v, int kv_dtype) {
    return kv_dtype == ORC_KV_F16 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
}

static double decode_kv(uint16_t b, int kv_dtype) {
    return kv_dtype == ORC_KV_F16 ? (double)orc_f16_to_f32(b) : (double)orc_bf16_to_f32(b);
}

/* ----------------------------------------------------------- paged view */

/* One layer of the pool: K and V each [kv_heads, pool_len, head_dim] in
 * 16-bit words, as KvPool allocates them (pool.rs:131-153), and the flattened
 * block table [seqs * max_pages] with u32::MAX sentinels (pool.rs:85-93). */
typedef struct {
    uint16_t* k;
    uint16_t* v;
    const uint32_t* block_table;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t pool_len; /* pages * page_len */
    uint32_t max_pages;
    uint32_t page_len;
    int32_t kv_dtype;
} orc_layer;

/* Physical slot of logical token `pos` of `seq` (kv_store.wgsl:40-41,
 * attn.wgsl:42-51,111).  Returns -1 if the page is missing. */
static int64_t slot_of(const orc_layer* L, uint32_t seq, uint32_t pos) {
    uint32_t lp = pos / L->page_len;
    if (lp >= L->max_pages) return -1;
    uint32_t page = L->block_table[(size_t)seq * L->max_pages + lp];
    if (page == 0xffffffffu) return -1;
    int64_t slot = (int64_t)page * L->page_len + pos % L->page_len;
    if (slot >= (int64_t)L->pool_len) return -1;
    return slot;
}

/* kv_store.wgsl:24-46.  For each of the m rows: pos = args[8r], seq =
 * args[8r+1]; every (head, dim) element of the row is encoded to the KV type
 * and stored at the row's slot in both caches.  src is [m, kv_heads, head_dim].
 * Returns 0, or -(r+1) for the first row whose page is missing. */
int orc_kv_store(orc_layer* L, const void* k_src, const void* v_src, int src_dtype,
                 const uint32_t* args, uint32_t m) {
    const uint32_t nkv = L->kv_heads, hd = L->head_dim;
    for (uint32_t r = 0; r < m; r++) {
        uint32_t pos = args[8 * r], seq = args[8 * r + 1];
        int64_t slot = slot_of(L, seq, pos);
        if (slot < 0) return -(int)(r + 1);
        for (uint32_t h = 0; h < nkv; h++) {
            size_t s_base = ((size_t)r * nkv + h) * hd;
            size_t c_base = ((size_t)h * L->pool_len + (size_t)slot) * hd;
            for (uint32_t d = 0; d < hd; d++) {
                L->k[c_base + d] = encode_kv(src_value(k_src, src_dtype, s_base + d), L->kv_dtype);
                L->v[c_base + d] = encode_kv(src_value(v_src, src_dtype, s_base + d), L->kv_dtype);
            }
        }
    }
    return 0;
}

/* --------------------------------------------------------- attention */

/* Per-row key range, following attn.wgsl.  Rows are taken in "chunks": the
 * reference dispatches attn once per sequence chunk with SEQ fixed
 * (forward.rs:316-336).  In per-row mode (seq_fixed < 0) a chunk is a maximal
 * run of consecutive rows with equal seq, the batched generalisation.
 *   kv_len (attn.wgsl:84-88): causal -> pos of the last row of the row's
 *          8-row block within the chunk, +1; else pos of the chunk's last
 *          row, +1.
 *   window start (attn.wgsl:79-82): causal && W>0 && pos+1>W ? pos+1-W : 0.
 *   key j valid (attn.wgsl:169): (!causal || j<=pos) && j>=ws && j<kv_len.
 * Writes lo[r], hi[r] (valid keys are lo <= j < hi) and seq[r]. */
void orc_attn_ranges(const uint32_t* args, uint32_t m, int64_t seq_fixed, int causal, uint32_t window,
                     uint32_t* lo, uint32_t* hi, uint32_t* seq_out) {
    uint32_t start = 0;
    while (start < m) {
        uint32_t seq = seq_fixed >= 0 ? (uint32_t)seq_fixed : args[8 * start + 1];
        uint32_t end = start + 1;
        if (seq_fixed < 0)
            while (end < m && args[8 * end + 1] == seq) end++;
        else
            end = m;
        uint32_t n = end - start;
        for (uint32_t i = 0; i < n; i++) {
            uint32_t r = start + i;
            uint32_t pos = args[8 * r];
            uint32_t blk_last = (i / 8) * 8 + 8;
            if (blk_last > n) blk_last = n;
            uint32_t kv_len = causal ? args[8 * (start + blk_last - 1)] + 1 : args[8 * (end - 1)] + 1;
            uint32_t ws = 0;
            if (causal && window != 0 && pos + 1 > window) ws = pos + 1 - window;
            uint32_t h = kv_len;
            if (causal && pos + 1 < h) h = pos + 1;
            lo[r] = ws;
            hi[r] = h;
            seq_out[r] = seq;
        }
        start = end;
    }
}

typedef struct {
    uint32_t m;
    uint32_t q_heads;
    uint32_t nq_per_kv;
    float scale;
    uint32_t window;
    int32_t causal;
    int64_t seq; /* >= 0: fixed sequence (reference AttnSpec.seq); < 0: per row */
    float softcap; /* 0 = off; else s = cap * tanh(s / cap) (extension) */
    int32_t precision; /* 0: double, exact softmax (checker); 1: f32 blockwise
                          online softmax in the order of attn.wgsl (baseline) */
} orc_attn_spec;

static int attn_row_head_double(const orc_layer* L, const float* q, double* out, uint32_t seq, uint32_t lo,
                                uint32_t hi, uint32_t kvh, double scale, double cap, double* scores) {
    const uint32_t hd = L->head_dim;
    double mx = -INFINITY;
    for (uint32_t j = lo; j < hi; j++) {
        int64_t slot = slot_of(L, seq, j);
        if (slot < 0) return -1;
        const uint16_t* kr = L->k + ((size_t)kvh * L->pool_len + (size_t)slot) * hd;
        double dot = 0.0;
        for (uint32_t d = 0; d < hd; d++) dot += (double)q[d] * decode_kv(kr[d], L->kv_dtype);
        double s = dot * scale;
        if (cap > 0.0) s = cap * tanh(s / cap);
        scores[j - lo] = s;
        if (s > mx) mx = s;
    }
    double sum = 0.0;
    for (uint32_t j = lo; j < hi; j++) {
        double e = exp(scores[j - lo] - mx);
        scores[j - lo] = e;
        sum += e;
    }
    for (uint32_t d = 0; d < hd; d++) out[d] = 0.0;
    for (uint32_t j = lo; j < hi; j++) {
        int64_t slot = slot_of(L, seq, j);
        const uint16_t* vr = L->v + ((size_t)kvh * L->pool_len + (size_t)slot) * hd;
        double w = scores[j - lo] / sum;
        for (uint32_t d = 0; d < hd; d++) out[d] += w * decode_kv(vr[d], L->kv_dtype);
    }
    return 0;
}

/* The reference kernel's own order (attn.wgsl:119-339), in f32: keys in
 * blocks of 128, running max m_old / sum s_old, rescale on a new max, exp in
 * base e, final division by s_old.  Used as the timed CPU baseline. */
static int attn_row_head_f32(const orc_layer* L, const float* q, float* out, uint32_t seq, uint32_t lo, uint32_t hi,
                             uint32_t kvh, float scale, float cap, float* e_blk) {
    const uint32_t hd = L->head_dim;
    const uint32_t BC = 128;
    float m_old = -3.4e38f, s_old = 0.0f;
    for (uint32_t d = 0; d < hd; d++) out[d] = 0.0f;
    uint32_t c0 = (lo / BC) * BC;
    for (; c0 < hi; c0 += BC) {
        uint32_t lim = hi - c0 < BC ? hi - c0 : BC;
        float m_cur = -3.4e38f;
        for (uint32_t c = 0; c < lim; c++) {
            uint32_t j = c0 + c;
            float s = -3.4e38f;
            if (j >= lo) {
                int64_t slot = slot_of(L, seq, j);
                if (slot < 0) return -1;
                const uint16_t* kr = L->k + ((size_t)kvh * L->pool_len + (size_t)slot) * hd;
                float dot = 0.0f;
                if (L->kv_dtype == ORC_KV_F16)
                    for (uint32_t d = 0; d < hd; d++) dot += q[d] * orc_f16_to_f32(kr[d]);
                else
                    for (uint32_t d = 0; d < hd; d++) dot += q[d] * orc_bf16_to_f32(kr[d]);
                s = dot * scale;
                if (cap > 0.0f) s = cap * tanhf(s / cap);
            }
            e_blk[c] = s;
            if (s > m_cur) m_cur = s;
        }
        float s_cur = 0.0f;
        if (m_cur > m_old) {
            float r = expf(m_old - m_cur);
            s_old *= r;
            for (uint32_t d = 0; d < hd; d++) out[d] *= r;
            m_old = m_cur;
        }
        for (uint32_t c = 0; c < lim; c++) {
            float e = e_blk[c] == -3.4e38f ? 0.0f : expf(e_blk[c] - m_old);
            e_blk[c] = e;
            s_cur += e;
        }
        s_old += s_cur;
        for (uint32_t c = 0; c < lim; c++) {
            if (e_blk[c] == 0.0f) continue;
            int64_t slot = slot_of(L, seq, c0 + c);
            const uint16_t* vr = L->v + ((size_t)kvh * L->pool_len + (size_t)slot) * hd;
            float e = e_blk[c];
            if (L->kv_dtype == ORC_KV_F16)
                for (uint32_t d = 0; d < hd; d++) out[d] += e * orc_f16_to_f32(vr[d]);
            else
                for (uint32_t d = 0; d < hd; d++) out[d] += e * orc_bf16_to_f32(vr[d]);
        }
    }
    for (uint32_t d = 0; d < hd; d++) out[d] /= s_old;
    return 0;
}

/* Paged attention (attn.wgsl:53-365 semantics; exact softmax as cpu_ref.rs
 * :172-228 when precision==0).  q [m, q_heads, head_dim] f32, args 8 u32 per
 * row (rows.rs:11-30), y [m, q_heads, head_dim] f64 (precision 0) or f32
 * (precision 1).  Parallel over (row, head) with OpenMP when built with it.
 * Returns 0, or -1 if a key's page is missing. */
int orc_attn(const orc_layer* L, const float* q, void* y, const uint32_t* args, const orc_attn_spec* spec) {
    const uint32_t m = spec->m, nq = spec->q_heads, hd = L->head_dim;
    uint32_t* lo = (uint32_t*)malloc(sizeof(uint32_t) * m * 3 + 4);
    uint32_t* hi = lo + m;
    uint32_t* sq = hi + m;
    orc_attn_ranges(args, m, spec->seq, spec->causal, spec->window, lo, hi, sq);
    uint32_t maxlen = 1;
    for (uint32_t r = 0; r < m; r++)
        if (hi[r] > lo[r] && hi[r] - lo[r] > maxlen) maxlen = hi[r] - lo[r];
    int status = 0;
    const int64_t total = (int64_t)m * nq;
#pragma omp parallel
    {
        double* scores = (double*)malloc(sizeof(double) * (maxlen + 128));
        float* eblk = (float*)malloc(sizeof(float) * 128);
#pragma omp for schedule(dynamic, 1)
        for (int64_t idx = 0; idx < total; idx++) {
            uint32_t r = (uint32_t)(idx / nq), h = (uint32_t)(idx % nq);
            uint32_t kvh = h / spec->nq_per_kv;
            const float* qr = q + ((size_t)r * nq + h) * hd;
            int rc;
            if (spec->precision == 0) {
                double* out = (double*)y + ((size_t)r * nq + h) * hd;
                if (hi[r] <= lo[r]) {
                    for (uint32_t d = 0; d < hd; d++) out[d] = NAN;
                    rc = 0;
                } else {
                    rc = attn_row_head_double(L, qr, out, sq[r], lo[r], hi[r], kvh, (double)spec->scale,
                                              (double)spec->softcap, scores);
                }
            } else {
                float* out = (float*)y + ((size_t)r * nq + h) * hd;
                rc = attn_row_head_f32(L, qr, out, sq[r], lo[r], hi[r], kvh, spec->scale, spec->softcap, eblk);
            }
            if (rc != 0) {
#pragma omp atomic write
                status = -1;
            }
        }
        free(scores);
        free(eblk);
    }
    free(lo);
    return status;
}

/* ------------------------------------------------------------------ rope */

/* rope.wgsl:16-40 (cpu_ref.rs:132-152) and, with a weight w, norm.wgsl
 * MODE 4 (:122-160): x [m][heads][hd] in place; row r is at position
 * pos[r] (its row meta).  Products and sums are separate roundings (this
 * file is compiled with -ffp-contract=off).  Returns -1 when a position is
 * outside the tables, -2 for a shape it does not take. */
int orc_rope_rows(float* x, uint32_t m, uint32_t heads, uint32_t hd, uint32_t rot, const float* cos_t,
                  const float* sin_t, uint32_t max_pos, const uint32_t* pos, const float* w, float eps) {
    const uint32_t half = rot / 2;
    float t[512];
    if (hd > 512 || rot > hd || rot % 2) return -2;
    for (uint32_t r = 0; r < m; r++) {
        if (pos[r] >= max_pos) return -1;
        for (uint32_t h = 0; h < heads; h++) {
            float* v = x + ((size_t)r * heads + h) * hd;
            float inv = 1.0f;
            if (w) {
                float ss = 0.0f;
                for (uint32_t c = 0; c < hd / 8; c++) {
                    float sc = 0.0f;
                    for (uint32_t e = 0; e < 8; e++) sc = sc + v[8 * c + e] * v[8 * c + e];
                    ss = ss + sc;
                }
                inv = 1.0f / sqrtf(ss / (float)hd + eps);
            }
            for (uint32_t d = 0; d < hd; d++) t[d] = w ? (v[d] * inv) * w[d] : v[d];
            for (uint32_t d = 0; d < hd; d++) {
                if (d >= rot) {
                    v[d] = t[d];
                    continue;
                }
                const size_t ti = (size_t)pos[r] * half + d % half;
                const float c = cos_t[ti], s = sin_t[ti];
                v[d] = d < half ? t[d] * c - t[d + half] * s : t[d] * c + t[d - half] * s;
            }
        }
    }
    return 0;
}

/* ------------------------------------------------- gather / block copy */

/* Gather tokens [t0, t0+n) of `seq` into contiguous dst [kv_heads, n,
 * head_dim] (bit copy).  No reference counterpart: the closed form is the
 * inverse of the block-table lookup above.  Returns -1 on a missing page. */
int orc_kv_gather(const orc_layer* L, uint32_t seq, uint32_t t0, uint32_t n, uint16_t* k_dst, uint16_t* v_dst) {
    const uint32_t hd = L->head_dim;
    for (uint32_t t = 0; t < n; t++) {
        int64_t slot = slot_of(L, seq, t0 + t);
        if (slot < 0) return -1;
        for (uint32_t h = 0; h < L->kv_heads; h++) {
            size_t src = ((size_t)h * L->pool_len + (size_t)slot) * hd;
            size_t dst = ((size_t)h * n + t) * hd;
            memcpy(k_dst + dst, L->k + src, hd * 2);
            memcpy(v_dst + dst, L->v + src, hd * 2);
        }
    }
    return 0;
}

/* Block copy: for each triple (src_page, dst_page, ntok) copy slots
 * [0, ntok) of src_page to dst_page in K and V of every head (one layer). */
void orc_block_copy(orc_layer* L, const uint32_t* triples, uint32_t n) {
    const uint32_t hd = L->head_dim;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t sp = triples[3 * i], dp = triples[3 * i + 1], nt = triples[3 * i + 2];
        for (uint32_t h = 0; h < L->kv_heads; h++) {
            size_t s = ((size_t)h * L->pool_len + (size_t)sp * L->page_len) * hd;
            size_t d = ((size_t)h * L->pool_len + (size_t)dp * L->page_len) * hd;
            memmove(L->k + d, L->k + s, (size_t)nt * hd * 2);
            memmove(L->v + d, L->v + s, (size_t)nt * hd * 2);
        }
    }
}

/* ----------------------------------------------------------------- gemm */

/* cpu_ref::gemm (cpu_ref.rs:11-25): y[mi][ni] = sum over k in order of
 * x[mi][k] * w[ni][k], an f32 sum, plus y's old value when acc (the
 * reference's acc tests add y0 afterwards, kernels.rs:566-571).  rows == 1
 * is cpu_ref::gemv (cpu_ref.rs:27-35), the same loop.  With exact != 0 the
 * sums are taken in double and rounded once (the tight check). */
void orc_gemm(const float* x, const float* w, float* y, uint32_t m, uint32_t n, uint32_t k, int acc, int exact) {
#pragma omp parallel for schedule(static)
    for (int64_t mi = 0; mi < (int64_t)m; mi++) {
        for (uint32_t ni = 0; ni < n; ni++) {
            const float* xr = x + (size_t)mi * k;
            const float* wr = w + (size_t)ni * k;
            float out;
            if (exact) {
                double s = 0.0;
                for (uint32_t ki = 0; ki < k; ki++) s += (double)xr[ki] * (double)wr[ki];
                if (acc) s += (double)y[(size_t)mi * n + ni];
                out = (float)s;
            } else {
                float s = 0.0f;
                for (uint32_t ki = 0; ki < k; ki++) s += xr[ki] * wr[ki];
                out = acc ? s + y[(size_t)mi * n + ni] : s;
            }
            y[(size_t)mi * n + ni] = out;
        }
    }
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
