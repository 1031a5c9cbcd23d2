// Paged attention on gfx950: one launch over every row of the batch.
//
// Semantics follow the reference kernel attn.wgsl:53-365: for row i, key j
// is valid iff (!causal || j <= pos_i) && j >= window_start_i && j < kv_len,
// with kv_len and window_start exactly as attn.wgsl:78-88 (computed on the
// host into per-row [lo, hi) ranges).  Softmax in f32, base 2 internally.
//
// Work decomposition:
//  * A "group" holds up to 16 query vectors that read the same keys: R rows
//    of one sequence x H query heads of one KV head.  Every K/V byte of a
//    group is loaded once for all of its query vectors (GQA packing).
//  * A group's key span (from its first key rounded down to the page and tile
//    size) is cut into n equal partitions, n = ceil(span / part_len) rounded
//    up to a power of two (so that groups of similar spans tile the 256 CUs
//    evenly: 3 partitions per group on 128 groups leave half the CUs idle
//    for the last third of the launch, 4 do not; a span a few keys over
//    k * part_len, k >= 2, takes k slightly longer partitions).  One
//    workgroup of W waves handles one (group, partition, KV head); the waves
//    split the partition into W contiguous runs of 16-token tiles.  All
//    boundaries depend only on the group's own key range, so a row's
//    arithmetic is the same whatever else is in the batch and wherever its
//    pages sit: batch == solo and paged == contiguous hold bit-exactly.
//    Work items are launched longest first.
//  * Scores come from MFMA: S^T[16 tokens x 16 columns] = K Q^T with
//    v_mfma_f32_16x16x32_{f16,bf16}.  The A operand is 16 bytes of one key
//    per lane; the pool keeps K pages in 32-dimension groups ([head_dim/32]
//    [page_len][32], layout.hpp) so that one load instruction covers 1 KiB of
//    contiguous memory.  The B
//    operand is Q^T held in registers.  Q is split into a high and a low
//    half-precision part and both are multiplied, which keeps the products
//    at f32 accuracy; the softmax scale is applied to the f32 scores.
//  * S^T leaves lane (a, c) holding tokens 4a..4a+3 of column c.  That is
//    exactly the B-operand layout of v_mfma_f32_16x16x16 for P^T, so the
//    probabilities feed the PV product without any lane exchange.  The A
//    operand is V^T: the pool stores V in 4-slot groups inside each page
//    ([page_len/4][head_dim][4]), so 4 consecutive tokens of one dimension
//    are 8 contiguous bytes.  P is split into high and low halves as well.
//  * Online softmax per column with a lazy rescale (the running max moves
//    only when a score beats it by more than 2^8).  The waves' states are
//    merged through LDS in a fixed tree.  A group split over several
//    partitions writes (m, l, o) per partition and a second kernel merges
//    them in partition order; there are no device-wide fences or atomics.
#include <algorithm>
#include <array>
#include <cmath>
#include <map>
#include <memory>
#include <mutex>
#include <queue>
#include <string>

#include "codec.hpp"
#include "layout.hpp"
#include "partition.hpp"
#include "pool.hpp"
#include "rope.hpp"

namespace thb {
namespace {

constexpr float kTau = 8.0f;          // lazy-rescale threshold (log2 units)
constexpr float kFloor = -1.0e30f;    // initial running max (finite on purpose)
constexpr uint32_t kGroupWords = 11;  // r0, R, h0, H, seq, lo, hi, n_parts, base, plen, item0
constexpr uint32_t kMaxPartPages = 1024;
// Longest part_len in pages: its partitions, up to part_len + part_len / 64
// rounded up to the alignment, fit kMaxPartPages pages.
constexpr uint32_t kMaxPartLenPages = kMaxPartPages - kMaxPartPages / 64;

// Raw buffer resources (decode tile loads): word 3 of a gfx9 descriptor
// with a 32-bit data format (untyped loads need a nonzero one), the
// non-temporal cache-policy bit of a buffer load, and an offset that is out
// of range of every resource the kernels build (loads there return zeros).
constexpr int kBufferFlags = 0x00020000;
constexpr int kBufferNt = 2;
constexpr uint32_t kBufferOob = 0xFFFFFFF0u;
constexpr uint32_t kMaxParts = 512;   // partitions of one group the merge kernel takes
constexpr uint32_t kCols = 16;        // query vectors per group (MFMA N)
constexpr uint32_t kMergeWords = 8;   // merge record: r0, R, h0, H, n_parts, item0, 0, 0
constexpr uint32_t kBlockWords = 9;   // g0, ng, seq, lo, hi, n_parts, base, plen, bitem0
// Work-item records carry their group's (or block's) words and the
// partition index, so a workgroup finds its work in one dependent load.
constexpr uint32_t kItemWords = kGroupWords + 1;
constexpr uint32_t kNoItem = 0xFFFFFFFFu;  // the empty second half of a prefill pair
constexpr uint32_t kBItemWords = kBlockWords + 1;

// Waves per workgroup and tiles in flight per wave of each head_dim
// template: up to head_dim 256, 8 waves (2 per SIMD, 256 registers each),
// with two tiles in flight up to 128 and one at 256 (the query, output and
// load registers grow with head_dim; at 256 the second wave per SIMD hides
// more than a second tile, 1.5% on Gemma-2 layers, and a second tile with
// the query halves in LDS measured 2% slower); at 512, 4 waves with one
// tile and the query halves in LDS.
#ifndef THB_ATTN_WAVES
#define THB_ATTN_WAVES 8
#endif
#ifndef THB_ATTN_RING
#define THB_ATTN_RING 2
#endif
#ifndef THB_ATTN_WAVES_256
#define THB_ATTN_WAVES_256 8
#endif
#ifndef THB_ATTN_RING_256
#define THB_ATTN_RING_256 1
#endif
constexpr int waves_for(int hd) { return hd >= 512 ? 4 : THB_ATTN_WAVES; }
constexpr int ring_for(int hd) { return hd >= 512 ? 1 : hd >= 256 ? THB_ATTN_RING_256 : THB_ATTN_RING; }
// Decode workgroups: head_dim 256 has its own wave count (fewer waves hold
// more tiles in flight each).
constexpr int decode_waves(int hd) { return hd == 256 ? THB_ATTN_WAVES_256 : waves_for(hd); }
// Decode keeps the query's high and low halves in LDS (one copy for the
// workgroup's waves, which share the query group) instead of registers.
constexpr bool q_in_lds(int hd) { return hd >= 512; }

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct AttnArgs {
    const void* q;
    void* y;
    const uint32_t* groups;
    const uint32_t* items;   // decode work items: group words + partition (kItemWords each)
    const uint32_t* ranges;  // [m][2]: lo, hi
    const uint32_t* bitems;  // prefill work items: block words + partition (kBItemWords each)
    // attn_prefill_wide: pairs of prefill work items one workgroup runs in
    // turn (first, second or kNoItem), 2 words each
    const uint32_t* bpairs;
    const uint32_t* order;   // attn_mixed: launch order of decode items and prefill pairs (bit 31)
    // attn_list: the device plan's header (entries, claim counter, done counter)
    uint32_t* list;
    const uint32_t* merge_groups;  // attn_merge: the groups that span several partitions
    const uint32_t* table;
    uint16_t* k;
    uint16_t* v;
    const void* k_src;  // fused append: new K/V rows [m, n_kvh, hd] (null: none)
    const void* v_src;
    uint32_t src_dtype;
    float* part_o;   // [n_items][n_kvh][16][hd_t]
    float* part_ml;  // [n_items][n_kvh][16][2]
    // Arrival counters of the decode groups of several partitions, one per
    // (first item, KV head), zero between launches; null: attn_merge combines
    // every group's partitions after the launch.
    uint32_t* merge_cnt;
    uint64_t plane;  // 16-bit elements per head plane
    uint32_t max_pages, page_shift, q_heads, nq_per_kv, head_dim, part_len, n_kvh;
    uint32_t pages;  // pages of the pool
    float qscale;  // scale * log2(e), or scale / softcap
    float cap2;    // softcap * log2(e), 0 = no soft-cap
    // attn_prefill_wide: the query carries qpre = the sign of qscale (an exact
    // multiply), and qpost = |qscale| scales its products inside the
    // exponent's fma.  (Splitting q * qscale into f16 halves instead measured
    // ~100x larger errors against an exact softmax, 2.6e-5 vs 3e-7.)
    float qpre, qpost;
    uint32_t q_dt, y_dt;       // THB_DT_* of the query (and gate) and of the output
    uint32_t q_stride;         // elements from one query head to the next
    const void* gate;          // sigmoid gate of the output (q_dt), or null
    uint32_t gate_stride;      // elements from one gate head to the next
    // full = 1 selects the kernels with the extensions of thb_attn_io (query
    // stride, gate, bf16 query/output, rope) and the logit soft-cap; the
    // others take f32/f16 q and y only and are the lean path of the common
    // call.
    uint32_t full;
    // Rotary position embedding (FULL kernels): the query is normalised and
    // rotated as it is loaded, the fused append rotates the key.
    uint32_t rope_on;
    const uint32_t* meta;  // row meta of the call's rows (positions)
    RopeDev qrope, krope;
};

// Loads 8 query elements of dims [d0, d0 + 8) as f32: f32 or f16, and
// bf16 in the FULL kernels.
template <bool FULL>
__device__ inline void load_q8(const AttnArgs& a, uint64_t qbase, uint32_t d0, float (&x)[8]) {
    if (a.q_dt == THB_DT_F16) {
        const f16x8 w = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(a.q) + qbase + d0);
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = static_cast<float>(w[e]);
    } else if (FULL && a.q_dt == THB_DT_BF16) {
        const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qbase + d0);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[2 * e] = __uint_as_float(ws[e] << 16);
            x[2 * e + 1] = __uint_as_float(ws[e] & 0xffff0000u);
        }
    } else {
        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.q) + qbase + d0);
        const f32x4 u0 = p[0], u1 = p[1];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = u0[e];
            x[4 + e] = u1[e];
        }
    }
}

// The lane's KS chunks of 8 query elements as f32 (load_q8 for every k-step):
// every load is issued before the first conversion, from the query's first
// element where a chunk is out of range (then zeroed), so the KS round trips
// overlap instead of each waiting behind a branch.
template <int KS, bool FULL>
__device__ inline void load_q_all(const AttnArgs& a, bool con, uint64_t qbase, uint32_t a4, float (&x)[KS][8]) {
    const uint32_t hd = a.head_dim;
    bool ok[KS];
    uint64_t off[KS];
#pragma unroll
    for (int j = 0; j < KS; j++) {
        const uint32_t d0 = 32u * j + 8u * a4;
        ok[j] = con && d0 < hd;
        off[j] = ok[j] ? qbase + d0 : 0u;
    }
    if (a.q_dt == THB_DT_F16) {
        f16x8 w[KS];
#pragma unroll
        for (int j = 0; j < KS; j++) w[j] = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(a.q) + off[j]);
#pragma unroll
        for (int j = 0; j < KS; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) x[j][e] = ok[j] ? static_cast<float>(w[j][e]) : 0.0f;
    } else if (FULL && a.q_dt == THB_DT_BF16) {
        uint4 w[KS];
#pragma unroll
        for (int j = 0; j < KS; j++) w[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + off[j]);
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const uint32_t ws[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[j][2 * e] = ok[j] ? __uint_as_float(ws[e] << 16) : 0.0f;
                x[j][2 * e + 1] = ok[j] ? __uint_as_float(ws[e] & 0xffff0000u) : 0.0f;
            }
        }
    } else {
        f32x4 u[KS][2];
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.q) + off[j]);
            u[j][0] = p[0];
            u[j][1] = p[1];
        }
#pragma unroll
        for (int j = 0; j < KS; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[j][e] = ok[j] ? u[j][0][e] : 0.0f;
                x[j][4 + e] = ok[j] ? u[j][1][e] : 0.0f;
            }
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float tanh_approx(float x) {
    // tanh(x) = 1 - 2 / (exp(2x) + 1); saturates cleanly at +-1.
    const float e = fast_exp2(x * 2.8853900817779268f);  // 2 * log2(e)
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}
// tanh(x * c2 / (2 log2 e)) for a scale c2 folded into the exponent.
__device__ __forceinline__ float tanh_scaled(float x, float c2) {
    const float e = fast_exp2(x * c2);
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

// Max / sum over the four lanes c, c+16, c+32, c+48 (one MFMA column).
__device__ __forceinline__ float col_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float col_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

// Operand types of one KV encoding.
template <bool F16>
struct Ops;

template <>
struct Ops<true> {
    typedef f16x8 in8;
    typedef f16x4 in4;
    // hi + lo split of an f32 (hi = RNE(x), lo = RNE(x - hi)).
    __device__ static void split(float x, _Float16& h, _Float16& l) {
        h = static_cast<_Float16>(x);
        l = static_cast<_Float16>(x - static_cast<float>(h));
    }
    __device__ static f32x4 qk(const u32x4& k, const in8& q, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(in8, k), q, acc, 0, 0, 0);
    }
    __device__ static f32x4 pv(const u32x2& v, const in4& p, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(in4, v), p, acc, 0, 0, 0);
    }
    // PV over 32 tokens: 8 tokens of one dimension (A) against 8 probabilities
    // of one column (B).
    __device__ static f32x4 pv32(const u32x4& v, const in8& p, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(in8, v), p, acc, 0, 0, 0);
    }
    __device__ static void split4(const float* p, in4& h, in4& l) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            _Float16 a, b;
            split(p[e], a, b);
            h[e] = a;
            l[e] = b;
        }
    }
    __device__ static void split8(const float* x, in8& h, in8& l) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            _Float16 a, b;
            split(x[e], a, b);
            h[e] = a;
            l[e] = b;
        }
    }
    // The same split (both halves rounded to nearest even), two elements per
    // conversion: three vector instructions per element.
    __device__ static void split8_fast(const float* x, in8& h, in8& l) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const f16x2 hh = __builtin_convertvector((f32x2{x[e], x[e + 1]}), f16x2);
            const f16x2 ll = __builtin_convertvector(
                (f32x2{x[e] - static_cast<float>(hh[0]), x[e + 1] - static_cast<float>(hh[1])}), f16x2);
            h[e] = hh[0];
            h[e + 1] = hh[1];
            l[e] = ll[0];
            l[e + 1] = ll[1];
        }
    }
};

template <>
struct Ops<false> {
    typedef bf16x8 in8;
    typedef i16x4 in4;
    __device__ static void split(float x, __bf16& h, __bf16& l) {
        h = static_cast<__bf16>(x);
        l = static_cast<__bf16>(x - static_cast<float>(h));
    }
    __device__ static f32x4 qk(const u32x4& k, const in8& q, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(in8, k), q, acc, 0, 0, 0);
    }
    __device__ static f32x4 pv(const u32x2& v, const in4& p, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(in4, v), p, acc, 0, 0, 0);
    }
    __device__ static f32x4 pv32(const u32x4& v, const in8& p, f32x4 acc) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(in8, v), p, acc, 0, 0, 0);
    }
    __device__ static void split4(const float* p, in4& h, in4& l) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            __bf16 a, b;
            split(p[e], a, b);
            h[e] = __builtin_bit_cast(short, a);
            l[e] = __builtin_bit_cast(short, b);
        }
    }
    __device__ static void split8(const float* x, in8& h, in8& l) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            __bf16 a, b;
            split(x[e], a, b);
            h[e] = a;
            l[e] = b;
        }
    }
    __device__ static void split8_fast(const float* x, in8& h, in8& l) { split8(x, h, l); }
};

// One scalar of the sigmoid gate (same type as the query).
__device__ inline float gate_at(const AttnArgs& a, uint64_t i) {
    if (a.q_dt == THB_DT_F16) return static_cast<float>(static_cast<const _Float16*>(a.gate)[i]);
    if (a.q_dt == THB_DT_BF16) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(a.gate)[i]) << 16);
    return static_cast<const float*>(a.gate)[i];
}

// f32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ inline uint16_t f32_to_bf16_rne(float x) {
    const uint32_t b = __float_as_uint(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((b >> 16) | 0x40u);
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// Writes n (1 or 4) output values of (row, head) at dims [d, d + n): y =
// o / l, times the sigmoid gate 1 / (1 + exp(-g)) when there is one
// (sigmoid_mul.wgsl), in the output type.  The gate and bf16 outputs exist
// in the FULL kernels only.
template <int N, bool FULL>
__device__ inline void store_y(const AttnArgs& a, uint32_t row, uint32_t head, uint32_t d, const float (&v)[N]) {
    float yv[N];
#pragma unroll
    for (int e = 0; e < N; e++) yv[e] = v[e];
    if (FULL && a.gate) {
        const uint64_t gi = (static_cast<uint64_t>(row) * a.q_heads + head) * a.gate_stride + d;
#pragma unroll
        for (int e = 0; e < N; e++) yv[e] = yv[e] / (1.0f + __expf(-gate_at(a, gi + e)));
    }
    const uint64_t yi = (static_cast<uint64_t>(row) * a.q_heads + head) * a.head_dim + d;
    if constexpr (N == 4) {
        if (a.y_dt == THB_DT_F32) {
            *reinterpret_cast<f32x4*>(static_cast<float*>(a.y) + yi) = f32x4{yv[0], yv[1], yv[2], yv[3]};
        } else if (!FULL || a.y_dt == THB_DT_F16) {
            f16x4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = static_cast<_Float16>(yv[e]);
            *reinterpret_cast<f16x4*>(static_cast<_Float16*>(a.y) + yi) = h;
        } else {
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + yi) =
                u32x2{f32_to_bf16_rne(yv[0]) | (static_cast<uint32_t>(f32_to_bf16_rne(yv[1])) << 16),
                      f32_to_bf16_rne(yv[2]) | (static_cast<uint32_t>(f32_to_bf16_rne(yv[3])) << 16)};
        }
    } else {
        if (a.y_dt == THB_DT_F32)
            static_cast<float*>(a.y)[yi] = yv[0];
        else if (!FULL || a.y_dt == THB_DT_F16)
            static_cast<_Float16*>(a.y)[yi] = static_cast<_Float16>(yv[0]);
        else
            static_cast<uint16_t*>(a.y)[yi] = f32_to_bf16_rne(yv[0]);
    }
}

// Q^T operand of a lane: column (row, head), dims 32j + 8 a4 .. + 8 of k-step
// j, split into high and low halves.  The raw query is split (the prefill
// kernel passes pre = the sign of the score scale, an exact multiply) and the
// f32 scores are scaled afterwards, so the low half stays out of the f16
// subnormal range.  In the FULL kernels: query heads q_stride apart and,
// with rope on, the query head is first normalised (q_norm; the four lanes
// of the column add their sums of squares) and rotated at the row's
// position.  Every lane must call it (column sums).
template <int KS, class O, bool FULL>
__device__ inline void load_q(const AttnArgs& a, bool con, uint32_t row, uint32_t head, uint32_t a4,
                              typename O::in8 (&qh)[KS], typename O::in8 (&ql)[KS], float pre = 1.0f) {
    const uint32_t hd = a.head_dim;
    const uint64_t qbase = (static_cast<uint64_t>(row) * a.q_heads + head) * (FULL ? a.q_stride : hd);
    const bool rope = FULL && a.rope_on;
    if (!rope) {
        float x[KS][8];
        load_q_all<KS, FULL>(a, con, qbase, a4, x);
#pragma unroll
        for (int j = 0; j < KS; j++) {
#pragma unroll
            for (int e = 0; e < 8; e++) x[j][e] *= pre;
            O::split8(x[j], qh[j], ql[j]);
        }
        return;
    }
    // Rotary path: the lane's chunks in registers, normalised in place.
    const RopeDev& r = a.qrope;
    const uint32_t pos = con ? a.meta[8 * row] : 0u;
    float x[KS][8];
    load_q_all<KS, FULL>(a, con, qbase, a4, x);
    float inv = 1.0f;
    if (r.w) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < KS; j++) ss += sumsq8(x[j]);
        inv = rms_inv(col_sum(ss), hd, r.eps);
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const uint32_t d0 = 32u * j + 8u * a4;
            if (con && d0 < hd) norm8(x[j], inv, r.w + d0);
        }
    }
    if (r.rot == hd && hd == 32u * KS) {
        // Full rotation at the template width: the partner of chunk j is
        // chunk j + KS / 2 of the same lane.
#pragma unroll
        for (int j = 0; j < KS / 2; j++) {
            float lo[8], hi[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                lo[e] = x[j][e];
                hi[e] = x[j + KS / 2][e];
            }
            const uint32_t d0 = 32u * j + 8u * a4;
            rotate8(x[j], hi, d0, pos, r);
            rotate8(x[j + KS / 2], lo, d0 + r.half, pos, r);
        }
    } else {
        // Partial rotation or a narrower head: partners from memory.
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const uint32_t d0 = 32u * j + 8u * a4;
            if (con && d0 < r.rot) {
                const uint32_t dp = d0 < r.half ? d0 + r.half : d0 - r.half;
                float y[8];
                load_q8<FULL>(a, qbase, dp, y);
                if (r.w) norm8(y, inv, r.w + dp);
                rotate8(x[j], y, d0, pos, r);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < KS; j++) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[j][e] *= pre;
        O::split8(x[j], qh[j], ql[j]);
    }
}

// The query operand in LDS (head_dim 512 only: QLDS), else nothing.
template <typename T, int KS, bool QLDS>
struct DecodeQLds {
    T q[KS][2][64];
};
template <typename T, int KS>
struct DecodeQLds<T, KS, false> {};

// ------------------------------------------------ split-K partition merge
// A group whose keys span several partitions has one partial result (m, l,
// o) per partition.  The partials are written with relaxed agent-scope
// atomic stores and read with relaxed agent-scope atomic loads (coherent
// across the XCDs' L2 caches: the stores reach the device's coherence point,
// the loads do not hit a stale copy), so a workgroup of the same launch can
// read another's partial once that partial's stores have completed.
__device__ inline void publish_o(float* p, const f32x4& v) {
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __hip_atomic_store(q, (uint64_t(__float_as_uint(v[1])) << 32) | __float_as_uint(v[0]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (uint64_t(__float_as_uint(v[3])) << 32) | __float_as_uint(v[2]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void publish_ml(float* p, float m, float l) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t(__float_as_uint(l)) << 32) | __float_as_uint(m),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool COH>
__device__ inline uint64_t load_u64(const float* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    if constexpr (COH)
        return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        return *q;
}
template <bool COH>
__device__ inline f32x4 load_o(const float* p) {
    const uint64_t lo = load_u64<COH>(p), hi = load_u64<COH>(p + 2);
    return f32x4{__uint_as_float(static_cast<uint32_t>(lo)), __uint_as_float(static_cast<uint32_t>(lo >> 32)),
                 __uint_as_float(static_cast<uint32_t>(hi)), __uint_as_float(static_cast<uint32_t>(hi >> 32))};
}

// Combines the partitions of one (group, KV head) in partition order.  Each
// of NT threads owns 4-dimension units of the group's outputs (unit u:
// column u / q4, dims 4 (u % q4) .. + 4) and reads its column's (m, l)
// itself; up to U partitions are requested at once, (m, l) and o together.
// The arithmetic does not depend on NT or on where it runs (the merge
// kernel, or the workgroup of the group's last partition), so neither does
// the output.
template <int HD, bool FULL, int NT, bool COH>
__device__ __forceinline__ void merge_group(const AttnArgs& a, uint32_t r0, uint32_t R, uint32_t h0, uint32_t H,
                                            uint32_t n_parts, uint32_t item0, uint32_t kvh, uint32_t tid) {
    const uint32_t ncols = R * H, hd = a.head_dim, q4 = hd >> 2;
    const uint64_t base = static_cast<uint64_t>(item0) * a.n_kvh + kvh;  // partition pi: base + pi * n_kvh
    const uint64_t mstep = 2 * static_cast<uint64_t>(a.n_kvh) * kCols;   // (m, l) of the next partition
    const uint64_t ostep = static_cast<uint64_t>(a.n_kvh) * kCols * HD;  // o of the next partition
    constexpr uint32_t U = 8, NU = (kCols * HD / 4 + NT - 1) / NT;
    for (uint32_t u0 = 0; u0 < NU; u0++) {
        const uint32_t u = tid + NT * u0;
        if (u >= ncols * q4) break;
        const uint32_t c = u / q4, d = 4u * (u - c * q4);
        const float* ml = a.part_ml + 2 * (base * kCols + c);
        const float* op = a.part_o + (base * kCols + c) * HD + d;
        float M = kFloor;
        if (n_parts > U) {  // long merges: the maximum first
            for (uint32_t p0 = 0; p0 < n_parts; p0 += U) {
                float mv[U];
#pragma unroll
                for (uint32_t k = 0; k < U; k++)
                    mv[k] = p0 + k < n_parts ? __uint_as_float(static_cast<uint32_t>(load_u64<COH>(ml + (p0 + k) * mstep)))
                                             : kFloor;
#pragma unroll
                for (uint32_t k = 0; k < U; k++) M = fmaxf(M, mv[k]);
            }
        }
        float L = 0.0f;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t p0 = 0; p0 < n_parts; p0 += U) {
            float mv[U], lv[U];
            f32x4 ov[U];
#pragma unroll
            for (uint32_t k = 0; k < U; k++) {
                const bool in = p0 + k < n_parts;
                const uint64_t w = in ? load_u64<COH>(ml + (p0 + k) * mstep) : 0ull;
                mv[k] = in ? __uint_as_float(static_cast<uint32_t>(w)) : kFloor;
                lv[k] = in ? __uint_as_float(static_cast<uint32_t>(w >> 32)) : 0.0f;
                ov[k] = in ? load_o<COH>(op + (p0 + k) * ostep) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            if (n_parts <= U) {
#pragma unroll
                for (uint32_t k = 0; k < U; k++) M = fmaxf(M, mv[k]);
            }
#pragma unroll
            for (uint32_t k = 0; k < U; k++) {
                if (p0 + k >= n_parts) break;
                const float w = fast_exp2(mv[k] - M);
                L += w * lv[k];
                acc += w * ov[k];
            }
        }
        const float inv = 1.0f / L;
        const float yv[4] = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        const uint32_t rr = c / H, hh = c - rr * H;
        store_y<4, FULL>(a, r0 + rr, kvh * a.nq_per_kv + h0 + hh, d, yv);
    }
}

// Run by every thread of a decode workgroup of a group with several
// partitions once its partial is published: the workgroup that finishes
// the group's last partition combines them all (merge_group) and clears the
// group's counter for the next launch.  Each thread waits until its partial
// stores have completed before the barrier, the counter add (relaxed, agent
// scope) is issued after it, and the combining loads only after the add has
// returned, so the last workgroup's loads find every partition's stores
// done.  No workgroup waits for another.  Every partial store and merge load
// is an agent-scope atomic (sc1 on gfx950: not held in an XCD's L2), so this
// is the memory model's agent-scope release/acquire sequence without the L2
// write-back and invalidate, which only plain accesses need.
template <int HD, bool FULL, int NT>
__device__ __forceinline__ void merge_if_last(const AttnArgs& a, uint32_t& s_arrived, uint32_t r0, uint32_t R,
                                              uint32_t h0, uint32_t H, uint32_t n_parts, uint32_t item0,
                                              uint32_t kvh, uint32_t tid) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint32_t* cnt = a.merge_cnt + static_cast<uint64_t>(item0) * a.n_kvh + kvh;
    if (tid == 0) s_arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived + 1u != n_parts) return;
    merge_group<HD, FULL, NT, true>(a, r0, R, h0, H, n_parts, item0, kvh, tid);
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS of one decode workgroup.  The W waves' states are merged in one step
// (every state in LDS, each wave merging and storing its own 16-dimension
// tiles) up to head_dim 256 (128 KiB at 8 waves); head_dim 512 uses a fixed
// tree over W / 2 states.
template <int HD, bool F16, int W>
struct DecodeLds : DecodeQLds<typename Ops<F16>::in8, HD / 32, q_in_lds(HD)> {
    static constexpr bool FLAT = HD <= 256;
    static constexpr int NSTATE = FLAT ? W : (W / 2 > 0 ? W / 2 : 1);
    uint32_t page[kMaxPartPages];
    f32x4 o[NSTATE][HD / 16][64];
    float m[NSTATE][64];
    float l[NSTATE][64];
    uint32_t arrived;  // partitions of the group finished before this one
};

// One (group, partition, KV head) per workgroup of W waves.  NB tiles of
// loads are kept in flight per wave: tile i + NB is requested as soon as
// tile i has been consumed.
template <int HD, bool F16, int W, int NB, bool FULL>
__device__ __forceinline__ void decode_wg(const AttnArgs& a, uint32_t bid, DecodeLds<HD, F16, W>& L,
                                          uint32_t tid_arg) {
    using O = Ops<F16>;
    typedef typename O::in8 in8;
    typedef typename O::in4 in4;
    constexpr int KS = HD / 32;  // QK k-steps of 32 dimensions
    constexpr int MT = HD / 16;  // PV tiles of 16 dimensions
    constexpr bool FLAT = DecodeLds<HD, F16, W>::FLAT;
    auto& s_page = L.page;
    auto& s_o = L.o;
    auto& s_m = L.m;
    auto& s_l = L.l;
    auto& s_arrived = L.arrived;

    const uint32_t tid = tid_arg;  // threadIdx.x (opaque in attn_list)
    const uint32_t lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t a4 = lane >> 4, c = lane & 15u;
    // 1-D grid, KV head fastest: consecutive workgroups share a work item,
    // and items are ordered longest first (the host sorts them).
    const uint32_t item = bid / a.n_kvh, kvh = bid - item * a.n_kvh;

    const uint32_t* G = a.items + static_cast<uint64_t>(item) * kItemWords;
    const uint32_t r0 = G[0], R = G[1], h0 = G[2], H = G[3], seq = G[4];
    const uint32_t glo = G[5], ghi = G[6], n_parts = G[7], gbase = G[8], P = G[9], item0 = G[10];
    // A device-planned call's fixed grid holds slots past a group's last
    // partition (and groups past the call's last): they do nothing.
    if (G[kGroupWords] >= n_parts) return;
    const uint32_t pbeg = gbase + G[kGroupWords] * P;
    const uint32_t tb = max(glo, pbeg), te = min(ghi, pbeg + P);
    const uint32_t hd = a.head_dim;
    const uint32_t pshift = a.page_shift;
    const uint32_t pmask = (1u << pshift) - 1u;

    // Physical pages of this partition that hold keys of the group.
    {
        const uint32_t npg = P >> pshift;
        const uint32_t lp0 = pbeg >> pshift;
        const uint32_t* trow = a.table + static_cast<uint64_t>(seq) * a.max_pages;
        for (uint32_t i = tid; i < npg; i += 64 * W) {
            const uint32_t lp = lp0 + i;
            const bool used = tb < te && (lp << pshift) < te && ((lp + 1) << pshift) > tb;
            const uint32_t pg = used ? trow[lp] : 0u;
            s_page[i] = pg < a.pages ? pg : 0u;  // block_pages: a page outside the pool reads page 0
        }
    }

    // Column c of this lane: row r0 + c / H, head h0 + c % H of the KV head.
    const uint32_t ncols = R * H;
    const bool con = c < ncols;
    const uint32_t rr = con ? c / H : 0u;
    const uint32_t row = r0 + rr;
    const uint32_t head = kvh * a.nq_per_kv + h0 + (con ? c - rr * H : 0u);
    uint32_t clo = 0, chi = 0;
    if (con) {
        clo = max(a.ranges[2 * row], tb);
        chi = min(a.ranges[2 * row + 1], te);
    }
    const uint32_t cspan = chi > clo ? chi - clo : 0u;  // key t is read iff t - clo < cspan

    // Q^T operand: lane (a4, c) holds q[c][32j + 8a4 .. +8], split hi/lo; at
    // head_dim 512 in LDS (wave 0 writes it before the barrier below).
    constexpr bool QLDS = q_in_lds(HD);
    [[maybe_unused]] in8 qh[QLDS ? 1 : KS], ql[QLDS ? 1 : KS];
    if constexpr (QLDS) {
        if (wave == 0) {
            in8 th[KS], tl[KS];
            load_q<KS, O, FULL>(a, con, row, head, a4, th, tl);
#pragma unroll
            for (int j = 0; j < KS; j++) {
                L.q[j][0][lane] = th[j];
                L.q[j][1][lane] = tl[j];
            }
        }
    } else {
        load_q<KS, O, FULL>(a, con, row, head, a4, qh, ql);
    }


    // This wave's run of 16-token tiles inside [tb, te).  For groups of
    // several rows, and with the rotary embedding, runs are handed out last
    // key first: wave 0 takes the run that ends at te, which holds the rows'
    // new tokens, so a fused append's stores (~3.5 us for a 4-row verify
    // chunk at head_dim 256) delay the older wave of its SIMD pair, which
    // the SIMD's issue arbiter favours (over equal runs the younger waves
    // 4-7 take 9-14% longer).  The order depends on the group and the call's
    // kind only, not on whether the append is fused, so fused and separate
    // calls stay bit-identical.
    const uint32_t tb16 = tb & ~15u;
    const uint32_t span = te > tb16 ? te - tb16 : 0u;
    const uint32_t run = ((span + W - 1) / W + 15u) & ~15u;
    const bool last_first = R > 1 || (FULL && a.rope_on);
    const uint32_t ws = tb16 + (last_first ? W - 1u - wave : wave) * run;
    const uint32_t we = min(ws + run, te);

    // Fused append (thb_attn_append).  A row's new token sits at position
    // hi - 1 of the row, and the only wave that ever loads it is the wave
    // whose run holds that position.  That wave encodes and stores the row's
    // K and V of this KV head (exactly as kv_store) before its first tile
    // load; one wave's accesses to an address are ordered, so its tile loads
    // read the stored token.  Work item t of the group: row t / (2 cpr), K or
    // V, 8-element chunk.
    const uint32_t cpr = hd >> 3;
    const uint32_t app_items = a.k_src != nullptr ? R * 2 * cpr : 0u;
    constexpr uint32_t KVE = F16 ? THB_KV_F16_RNE : THB_KV_BF16_TRUNC;
    auto app_decode = [&](uint32_t t, uint32_t& pos, bool& is_v, uint32_t& d, uint64_t& e) -> bool {
        const uint32_t ar = t / (2 * cpr), rem = t - ar * 2 * cpr;
        is_v = rem >= cpr;
        d = (is_v ? rem - cpr : rem) << 3;
        pos = a.ranges[2 * (r0 + ar) + 1] - 1;
        e = (static_cast<uint64_t>(r0 + ar) * a.n_kvh + kvh) * hd + d;
        return pos >= ws && pos < we;
    };
    auto app_store_at = [&](uint32_t page, uint32_t pos, bool is_v, uint32_t d, const uint4& w) {
        const uint64_t base = ((static_cast<uint64_t>(page) * hd) << pshift) + static_cast<uint64_t>(kvh) * a.plane;
        if (!is_v) {
            *reinterpret_cast<uint4*>(a.k + base + k_off(pos & pmask, d, hd, pshift)) = w;
        } else {
            uint16_t* dst = a.v + base + v_off(pos & pmask, d, hd);  // dim d + e at + 4 e
            const uint32_t ws4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int q2 = 0; q2 < 4; q2++) {
                dst[8 * q2] = static_cast<uint16_t>(ws4[q2] & 0xffffu);
                dst[8 * q2 + 4] = static_cast<uint16_t>(ws4[q2] >> 16);
            }
        }
    };
    auto app_store = [&](uint32_t pos, bool is_v, uint32_t d, const uint4& w) {
        app_store_at(s_page[(pos - pbeg) >> pshift], pos, is_v, d, w);
    };
    // The first kAppLane items of each lane (items lane + 64 k): their
    // positions, and the sources of the items this wave owns, are loaded
    // beside the query loads, before the barrier (the source loads overlap
    // the page-table round trips the barrier waits for); the owning lanes
    // encode and store them after the barrier, before the first tile load.
    // A 4-row verify chunk at head_dim 256 (256 items, all in one wave's
    // run) thus costs one round trip instead of four in a row.  The tile
    // loop then holds no store.
    constexpr int kAppLane = 4;
    uint32_t app_pos[kAppLane], app_d[kAppLane];
    uint64_t app_e[kAppLane];
    bool app_v[kAppLane], app_own[kAppLane];
    Raw8 app_raw[kAppLane];
    const bool rope = FULL && a.rope_on;
#pragma unroll
    for (int k = 0; k < kAppLane; k++) {
        const uint32_t t = lane + 64u * k;
        app_own[k] = false;
        if (t < app_items && !rope) {
            app_own[k] = app_decode(t, app_pos[k], app_v[k], app_d[k], app_e[k]);
            if (app_own[k]) app_raw[k] = load_raw8_rt(a.src_dtype, app_v[k] ? a.v_src : a.k_src, app_e[k]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kAppLane; k++)
        if (app_own[k]) app_store(app_pos[k], app_v[k], app_d[k], encode8_rt<KVE>(a.src_dtype, app_raw[k]));
    if (rope) {
        if (app_items != 0) {
            // Rotary append: the key head of each row this wave owns, one chunk
            // of 8 dims per lane (the norm and the rotation need the whole head),
            // exactly as kv_store_rope_kernel.
            for (uint32_t ar = 0; ar < R; ar++) {
                const uint32_t pos = a.ranges[2 * (r0 + ar) + 1] - 1;
                if (pos < ws || pos >= we) continue;  // wave-uniform
                const uint64_t e = (static_cast<uint64_t>(r0 + ar) * a.n_kvh + kvh) * hd + 8u * lane;
                float x[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                if (lane < cpr) load8_f32(a.src_dtype, a.k_src, e, x);
                rope_head_seg(x, lane, cpr, 0, pos, a.krope);
                if (lane < cpr) {
                    uint32_t w[4];
#pragma unroll
                    for (int q2 = 0; q2 < 4; q2++) {
                        if (a.src_dtype == THB_DT_F16)
                            w[q2] = conv16<THB_DT_F16, KVE>(f32_to_f16_rne(x[2 * q2])) |
                                    (conv16<THB_DT_F16, KVE>(f32_to_f16_rne(x[2 * q2 + 1])) << 16);
                        else
                            w[q2] = conv32<KVE>(__float_as_uint(x[2 * q2])) |
                                    (conv32<KVE>(__float_as_uint(x[2 * q2 + 1])) << 16);
                    }
                    app_store(pos, false, 8u * lane, make_uint4(w[0], w[1], w[2], w[3]));
                    app_store(pos, true, 8u * lane, load_encode8_rt<KVE>(a.src_dtype, a.v_src, e));
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        }
    } else if (app_items > 64u * kAppLane) {
        for (uint32_t t = lane + 64u * kAppLane; t < app_items; t += 64) {
            uint32_t pos2, d2;
            uint64_t e2;
            bool v2;
            if (app_decode(t, pos2, v2, d2, e2))
                app_store(pos2, v2, d2, load_encode8_rt<KVE>(a.src_dtype, v2 ? a.v_src : a.k_src, e2));
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }

    float m = kFloor, l = 0.0f;
    f32x4 o[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* kplane = a.k + static_cast<uint64_t>(kvh) * a.plane;
    const uint16_t* vplane = a.v + static_cast<uint64_t>(kvh) * a.plane;
    const uint32_t last = te > 0 ? te - 1 : 0;
    const uint32_t page_elems = hd << pshift;

    // Loads one 16-token tile with buffer loads.  Tokens outside [tb, te)
    // are clamped into it (their scores are masked).  The tile's tokens lie
    // in the pages of its first and last clamped token (one page unless
    // page_len is 8); the buffer resource starts at the lower of the two, so
    // every lane's byte offset is non-negative (below 4 GiB: the pool checks
    // the plane size for page_len 8).  A tile past the wave's run gets a
    // resource of size 0 and a lane past head_dim an offset beyond the size:
    // such loads return zeros without touching memory (K dims past head_dim
    // must be zeros: the query is zero there).  Every load is thus
    // issued unconditionally, and the compiler's wait counts stay exact
    // through the tile loop (a skipped load would force a full drain).
    // K pages hold 32-dimension groups ([hd/32][page_len][32]): for a fixed
    // k-step j the 64 lanes read 16 tokens x 64 bytes, 1 KiB contiguous.  V
    // pages hold 4-slot groups ([page_len/4][hd][4]): a lane's 4 slots of one
    // dim are 8 bytes, and 16 lanes read 128 contiguous bytes.  The loads are
    // non-temporal (every byte is read once).
    struct TileRes {
        __amdgpu_buffer_rsrc_t k, v;
        uint32_t pa, pb, pmin, first_lp;
    };
    auto tile_res = [&](uint32_t t0) {
        TileRes r;
        const bool on = t0 < we;  // then tb <= tf <= tl <= last: pages of the partition
        const uint32_t tf = min(max(t0, tb), last), tl = min(max(t0 + 15u, tb), last);
        r.first_lp = tf >> pshift;
        r.pa = __builtin_amdgcn_readfirstlane(s_page[on ? r.first_lp - (pbeg >> pshift) : 0u]);
        r.pb = __builtin_amdgcn_readfirstlane(s_page[on ? (tl >> pshift) - (pbeg >> pshift) : 0u]);
        r.pmin = min(r.pa, r.pb);
        const uint32_t nrec = on ? (max(r.pa, r.pb) - r.pmin + 1u) * 2u * page_elems : 0u;
        const uint64_t off = static_cast<uint64_t>(r.pmin) * page_elems;
        r.k = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kplane + off), 0, nrec, kBufferFlags);
        r.v = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vplane + off), 0, nrec, kBufferFlags);
        return r;
    };
    // Byte offset of token t's page from the resource base.
    auto page_bytes_off = [&](const TileRes& r, uint32_t t) {
        return ((t >> pshift) == r.first_lp ? r.pa - r.pmin : r.pb - r.pmin) * 2u * page_elems;
    };
    auto load_k = [&](uint32_t t0, u32x4 (&kr)[KS]) {
        const TileRes r = tile_res(t0);
        const uint32_t tk = min(max(t0 + c, tb), last);
        const uint32_t base = page_bytes_off(r, tk);
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const uint32_t d0 = 32u * j + 8u * a4;
            const uint32_t off = d0 < hd ? base + 2u * k_off(tk & pmask, d0, hd, pshift) : kBufferOob;
            kr[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r.k, off, 0, kBufferNt));
        }
    };
    auto load_v = [&](uint32_t t0, u32x2 (&vr)[MT]) {
        const TileRes r = tile_res(t0);
        const uint32_t tv = min(max(t0 + 4u * a4, tb & ~3u), last & ~3u);
        const uint32_t base = page_bytes_off(r, tv) + 2u * v_off(tv & pmask, 0, hd);
        // Dims past head_dim read whatever lies there (or zeros): each PV
        // output row is one dim, so they only reach outputs never stored.
#pragma unroll
        for (int i = 0; i < MT; i++)
            vr[i] = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(r.v, base + 8u * (16u * i + c), 0, kBufferNt));
    };
    auto load = [&](uint32_t t0, u32x4 (&kr)[KS], u32x2 (&vr)[MT]) {
        load_k(t0, kr);
        load_v(t0, vr);
    };

    // after_qk runs once the tile's K operands are consumed (one tile in
    // flight: the next tile's K is requested there, before the softmax and
    // the PV products of this one).
    auto compute = [&](uint32_t t0, const u32x4 (&kr)[KS], const u32x2 (&vr)[MT], auto&& after_qk) {
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < KS; j++) {
            if constexpr (QLDS) {
                s = O::qk(kr[j], L.q[j][0][lane], s);
                s = O::qk(kr[j], L.q[j][1][lane], s);
            } else {
                s = O::qk(kr[j], qh[j], s);
                s = O::qk(kr[j], ql[j], s);
            }
        }
        after_qk();
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float x = s[e] * a.qscale;
            if (FULL && a.cap2 != 0.0f) x = a.cap2 * tanh_approx(x);  // soft-cap: FULL kernels only
            const uint32_t t = t0 + 4u * a4 + e;
            x = t - clo < cspan ? x : -INFINITY;
            sv[e] = x;
            mx = fmaxf(mx, x);
        }
        // The column max (two cross-lane steps) is taken only when some score
        // beats its column's running max by more than kTau; without one, no
        // column rescales, exactly as if the max had been taken.
        if (__builtin_amdgcn_ballot_w64(mx > m + kTau) != 0) {
            mx = col_max(mx);
            if (mx > m + kTau) {
                const float alpha = fast_exp2(m - mx);
                l *= alpha;
#pragma unroll
                for (int i = 0; i < MT; i++) o[i] *= alpha;
                m = mx;
            }
        }
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            p[e] = fast_exp2(sv[e] - m);
            l += p[e];
        }
        in4 ph, pl;
        O::split4(p, ph, pl);
#pragma unroll
        for (int i = 0; i < MT; i++) {
            o[i] = O::pv(vr[i], ph, o[i]);
            o[i] = O::pv(vr[i], pl, o[i]);
        }
    };

    {
        // NB tiles in flight per wave.  Loads of tiles past the run are
        // issued too (they read nothing), so every iteration issues the same
        // loads and only the products are skipped.
        u32x4 kr[NB][KS];
        u32x2 vr[NB][MT];
#pragma unroll
        for (int b = 0; b < NB; b++) load(ws + 16u * b, kr[b], vr[b]);
        for (uint32_t t0 = ws; t0 < we; t0 += 16u * NB) {
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const uint32_t t = t0 + 16u * b, tn = t + 16u * NB;
                if constexpr (NB == 1 && HD < 512) {
                    // One tile in flight: the next tile's K goes out as soon
                    // as this tile's K is consumed, its V after the PV.  (At
                    // head_dim 512 the next K beside this tile's V and the
                    // 128 output registers spilled ~90 registers: 246 us for
                    // a 16 x 4096-token decode, against 106 us with the whole
                    // next tile requested after the PV, below.)
                    compute(t, kr[b], vr[b], [&]() { load_k(tn, kr[b]); });
                    load_v(tn, vr[b]);
                } else {
                    if (t < we) compute(t, kr[b], vr[b], []() {});
                    load(tn, kr[b], vr[b]);
                }
            }
        }
    }
    l = col_sum(l);

    if constexpr (FLAT) {
        // ---- merge the W waves' states in one step ----------------------
#pragma unroll
        for (int i = 0; i < MT; i++) s_o[wave][i][lane] = o[i];
        s_m[wave][lane] = m;
        s_l[wave][lane] = l;
        __syncthreads();
        float M = s_m[0][lane];
#pragma unroll
        for (int w = 1; w < W; w++) M = fmaxf(M, s_m[w][lane]);
        float f[W];
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            f[w] = fast_exp2(s_m[w][lane] - M);
            L += s_l[w][lane] * f[w];
        }
        const uint64_t pb = (static_cast<uint64_t>(item) * a.n_kvh + kvh) * kCols + c;
        for (uint32_t i = wave; i < static_cast<uint32_t>(MT); i += W) {  // this wave's tiles
            f32x4 acc = s_o[0][i][lane] * f[0];
#pragma unroll
            for (int w = 1; w < W; w++) acc += s_o[w][i][lane] * f[w];
            const uint32_t d = 16u * i + 4u * a4;
            if (!con || d >= hd) continue;
            if (n_parts == 1) {
                const f32x4 yv = acc * (1.0f / L);
                const float v4[4] = {yv[0], yv[1], yv[2], yv[3]};
                store_y<4, FULL>(a, row, head, d, v4);
            } else {
                // several partitions: publish this one's (m, l, o) for the
                // workgroup of the last partition (or the merge kernel)
                publish_o(a.part_o + pb * HD + d, acc);
            }
        }
        if (n_parts > 1 && wave == 0 && con && a4 == 0) publish_ml(a.part_ml + 2 * pb, M, L);
        if (n_parts > 1 && a.merge_cnt)
            merge_if_last<HD, FULL, 64 * W>(a, s_arrived, r0, R, h0, H, n_parts, item0, kvh, tid);
        return;
    }

    // ---- merge the W waves' states through LDS (fixed tree) -------------
    for (uint32_t half = W / 2; half >= 1; half >>= 1) {
        if (wave >= half && wave < 2 * half) {
            const uint32_t sl = wave - half;
#pragma unroll
            for (int i = 0; i < MT; i++) s_o[sl][i][lane] = o[i];
            s_m[sl][lane] = m;
            s_l[sl][lane] = l;
        }
        __syncthreads();
        if (wave < half) {
            const float m2 = s_m[wave][lane], l2 = s_l[wave][lane];
            const float M = fmaxf(m, m2);
            const float f1 = fast_exp2(m - M), f2 = fast_exp2(m2 - M);
#pragma unroll
            for (int i = 0; i < MT; i++) o[i] = o[i] * f1 + s_o[wave][i][lane] * f2;
            l = l * f1 + l2 * f2;
            m = M;
        }
        __syncthreads();
    }
    if (wave == 0 && con) {
        if (n_parts == 1) {
            const float inv = 1.0f / l;
#pragma unroll
            for (int i = 0; i < MT; i++) {
                const uint32_t d = 16u * i + 4u * a4;
                if (d >= hd) continue;
                const f32x4 yv = o[i] * inv;
                const float v4[4] = {yv[0], yv[1], yv[2], yv[3]};
                store_y<4, FULL>(a, row, head, d, v4);
            }
        } else {
            // Several partitions: publish this one's (m, l, o) for the
            // workgroup of the last partition (or the merge kernel).
            const uint64_t pb = (static_cast<uint64_t>(item) * a.n_kvh + kvh) * kCols + c;
#pragma unroll
            for (int i = 0; i < MT; i++) publish_o(a.part_o + pb * HD + 16u * i + 4u * a4, o[i]);
            if (a4 == 0) publish_ml(a.part_ml + 2 * pb, m, l);
        }
    }
    if (n_parts > 1 && a.merge_cnt)
        merge_if_last<HD, FULL, 64 * W>(a, s_arrived, r0, R, h0, H, n_parts, item0, kvh, tid);
}

template <int HD, bool F16, int W, int NB, bool FULL>
__global__ __launch_bounds__(64 * W) void attn_mfma(AttnArgs a) {
    __shared__ DecodeLds<HD, F16, W> lds;
    decode_wg<HD, F16, W, NB, FULL>(a, blockIdx.x, lds, threadIdx.x);
}

// Merges the partitions of every group that has more than one, in
// partition order.  One workgroup per (such group, KV head): the plan lists
// them, so a call of many single-partition groups launches no idle
// workgroups.
template <int HD, bool FULL>
__global__ __launch_bounds__(256) void attn_merge(AttnArgs a) {
    // Merge record (kMergeWords): the group's r0, R, h0, H, n_parts, item0,
    // so the partials are requested one round trip after the launch.
    const uint32_t* E = a.merge_groups + static_cast<uint64_t>(blockIdx.x) * kMergeWords;
    const uint32_t n_parts = E[4];
    if (n_parts <= 1) return;  // a device-planned call's slot of a one-partition group (or none)
    merge_group<HD, FULL, 256, false>(a, E[0], E[1], E[2], E[3], n_parts, E[5], blockIdx.y, threadIdx.x);
}

// Chunked prefill (and any sequence chunk that needs more than one group).
// One workgroup of W waves handles a block of up to W consecutive groups of
// one chunk (wave w: group g0 + w) for one KV head and one partition of the
// block's key span.  K and V tiles of TT tokens are loaded once per
// workgroup into LDS (double-buffered: the next tile's global loads are in
// flight while the waves compute on the current one) and shared by all
// waves; each wave skips the 16-token slices outside its group's keys (the
// causal triangle).  The per-slice arithmetic is the decode kernel's: split
// Q and P, MFMA, online softmax with the lazy rescale.
//   K tile in LDS: [TT/16 slices][HD/8 chunks][16 tokens] x 16 bytes, so 8
//     lanes of an operand read are 128 contiguous bytes.
//   V tile in LDS: [TT/16 slices][HD dims][4 groups of 4 tokens] x 8 bytes,
//     the group index XOR-ed with (dim / 8) % 4 so that the 16 lanes of a
//     PV operand read hit distinct banks.
template <int HD, bool F16, int W, bool FULL>
__global__ __launch_bounds__(64 * W, HD <= 128 ? 4 : 1) void attn_prefill(AttnArgs a) {
    using O = Ops<F16>;
    typedef typename O::in8 in8;
    typedef typename O::in4 in4;
    constexpr int KS = HD / 32;
    constexpr int MT = HD / 16;
    constexpr int TT = HD <= 128 ? 64 : (HD == 256 ? 32 : 16);
    constexpr int ST = TT / 16;
    constexpr int KU = TT * HD / 8;  // 16-byte K units per tile
    constexpr int VU = TT * HD / 8;  // 16-byte V units per tile (8 tokens of one dim)
    constexpr int NT = 64 * W;
    constexpr int KPT = (KU + NT - 1) / NT;
    constexpr int VPT = (VU + NT - 1) / NT;

    __shared__ u32x4 s_k[2][KU];
    __shared__ u32x2 s_v[2][ST * HD * 4];
    __shared__ uint32_t s_page[kMaxPartPages];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t a4 = lane >> 4, c = lane & 15u;
    const uint32_t bitem = blockIdx.x / a.n_kvh, kvh = blockIdx.x - bitem * a.n_kvh;

    const uint32_t* Bk = a.bitems + static_cast<uint64_t>(bitem) * kBItemWords;
    const uint32_t g0 = Bk[0], ng = Bk[1], seq = Bk[2], blo = Bk[3], bhi = Bk[4];
    const uint32_t n_parts = Bk[5], bbase = Bk[6], P = Bk[7];
    const uint32_t part = Bk[kBlockWords];
    const uint32_t pbeg = bbase + part * P;
    const uint32_t tb = max(blo, pbeg), te = min(bhi, pbeg + P);
    const uint32_t hd = a.head_dim;
    const uint32_t pshift = a.page_shift;
    const uint32_t pmask = (1u << pshift) - 1u;
    const uint32_t last = te > 0 ? te - 1 : 0;

    {
        const uint32_t npg = P >> pshift;
        const uint32_t lp0 = pbeg >> pshift;
        const uint32_t* trow = a.table + static_cast<uint64_t>(seq) * a.max_pages;
        for (uint32_t i = tid; i < npg; i += NT) {
            const uint32_t lp = lp0 + i;
            const bool used = tb < te && (lp << pshift) < te && ((lp + 1) << pshift) > tb;
            const uint32_t pg = used ? trow[lp] : 0u;
            s_page[i] = pg < a.pages ? pg : 0u;  // block_pages: a page outside the pool reads page 0
        }
    }

    // This wave's group and its columns.
    const bool gon = wave < ng;
    const uint32_t* G = a.groups + (g0 + (gon ? wave : 0u)) * kGroupWords;
    const uint32_t r0 = G[0], R = G[1], h0 = G[2], H = G[3], item0 = G[10];
    const uint32_t wlo = max(G[5], tb), whi = min(G[6], te);
    const uint32_t ncols = gon ? R * H : 0u;
    const bool con = c < ncols;
    const uint32_t rr = con ? c / H : 0u;
    const uint32_t row = r0 + rr;
    const uint32_t head = kvh * a.nq_per_kv + h0 + (con ? c - rr * H : 0u);
    uint32_t clo = 0, chi = 0;
    if (con) {
        clo = max(a.ranges[2 * row], tb);
        chi = min(a.ranges[2 * row + 1], te);
    }
    in8 qh[KS], ql[KS];

    const uint16_t* kplane = a.k + static_cast<uint64_t>(kvh) * a.plane;
    const uint16_t* vplane = a.v + static_cast<uint64_t>(kvh) * a.plane;
    const uint32_t cph = HD / 8;

    // Global -> registers for one tile; tokens outside [tb, te) are clamped
    // into it (their scores are masked).
    auto load = [&](uint32_t t0, u32x4 (&kr)[KPT], u32x4 (&vr)[VPT]) {
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const uint32_t u = tid + k * NT;
            const uint32_t st = u / (16 * cph), rem = u - st * (16 * cph);
            const uint32_t ch = rem >> 4, tok = rem & 15u;
            const uint32_t t = min(max(t0 + 16u * st + tok, tb), last);
            const uint32_t page = s_page[(t - pbeg) >> pshift];
            const bool ok = u < static_cast<uint32_t>(KU) && 8u * ch < hd;
            kr[k] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                             kplane + ((static_cast<uint64_t>(page) * hd) << pshift) + k_off(t & pmask, 8u * ch, hd, pshift)))
                       : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < VPT; k++) {  // unit: dims (d, d + 1) x 4-slot group g4 of a 16-token slice
            const uint32_t u = tid + k * NT;
            const uint32_t st = u / (2 * HD), rem = u - st * (2 * HD);
            const uint32_t g4 = rem / (HD / 2), d = 2u * (rem - g4 * (HD / 2));
            const uint32_t t = min(max(t0 + 16u * st + 4u * g4, tb & ~3u), last & ~3u);
            const uint32_t page = s_page[(t - pbeg) >> pshift];
            const bool ok = u < static_cast<uint32_t>(VU) && d < hd;
            vr[k] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                             vplane + ((static_cast<uint64_t>(page) * hd) << pshift) + v_off(t & pmask, d, hd)))
                       : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store = [&](int buf, const u32x4 (&kr)[KPT], const u32x4 (&vr)[VPT]) {
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const uint32_t u = tid + k * NT;
            if (u < static_cast<uint32_t>(KU)) s_k[buf][u] = kr[k];
        }
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const uint32_t u = tid + k * NT;
            if (u >= static_cast<uint32_t>(VU)) continue;
            const uint32_t st = u / (2 * HD), rem = u - st * (2 * HD);
            const uint32_t g4 = rem / (HD / 2), d = 2u * (rem - g4 * (HD / 2));
            const uint32_t sw = (d >> 3) & 3u;  // the same for d and d + 1
            s_v[buf][(st * HD + d) * 4 + (g4 ^ sw)] = u32x2{vr[k].x, vr[k].y};
            s_v[buf][(st * HD + d + 1u) * 4 + (g4 ^ sw)] = u32x2{vr[k].z, vr[k].w};
        }
    };

    float m = kFloor, l = 0.0f;
    f32x4 o[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int buf, uint32_t t0) {
#pragma unroll
        for (int st = 0; st < ST; st++) {
            const uint32_t ts = t0 + 16u * st;
            if (ts >= whi || ts + 16u <= wlo) continue;  // outside this wave's keys
            f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < KS; j++) {
                const u32x4 kv = s_k[buf][(st * cph + 4u * j + a4) * 16u + c];
                s = O::qk(kv, qh[j], s);
                s = O::qk(kv, ql[j], s);
            }
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float x = s[e] * a.qscale;
                if (a.cap2 != 0.0f) x = a.cap2 * tanh_approx(x);
                const uint32_t t = ts + 4u * a4 + e;
                x = (t >= clo && t < chi) ? x : -INFINITY;
                sv[e] = x;
                mx = fmaxf(mx, x);
            }
            mx = col_max(mx);
            if (mx > m + kTau) {
                const float alpha = fast_exp2(m - mx);
                l *= alpha;
#pragma unroll
                for (int i = 0; i < MT; i++) o[i] *= alpha;
                m = mx;
            }
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                p[e] = fast_exp2(sv[e] - m);
                l += p[e];
            }
            in4 ph, pl;
            O::split4(p, ph, pl);
#pragma unroll
            for (int i = 0; i < MT; i++) {
                const uint32_t d = 16u * i + c;
                const u32x2 vv = s_v[buf][(st * HD + d) * 4 + (a4 ^ ((d >> 3) & 3u))];
                o[i] = O::pv(vv, ph, o[i]);
                o[i] = O::pv(vv, pl, o[i]);
            }
        }
    };

    const uint32_t t_first = tb & ~15u;
    const uint32_t n_tiles = te > t_first ? (te - t_first + TT - 1) / TT : 0u;
    __syncthreads();  // s_page complete
    {
        u32x4 kr[KPT], vr[VPT];
        // The first tile's loads are in flight while the query is loaded
        // (and normalised / rotated, which takes dependent round trips).
        if (n_tiles) load(t_first, kr, vr);
        load_q<KS, O, FULL>(a, con, row, head, a4, qh, ql);
        if (n_tiles) store(0, kr, vr);
        __syncthreads();
        for (uint32_t i = 0; i < n_tiles; i++) {
            const uint32_t t0 = t_first + i * TT;
            const bool more = i + 1 < n_tiles;
            if (more) load(t0 + TT, kr, vr);
            if (gon) compute(static_cast<int>(i & 1u), t0);
            if (more) store(static_cast<int>((i + 1) & 1u), kr, vr);
            __syncthreads();
        }
    }
    l = col_sum(l);
    if (!con) return;

    if (n_parts == 1) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int i = 0; i < MT; i++) {
            const uint32_t d = 16u * i + 4u * a4;
            if (d >= hd) continue;
            const f32x4 yv = o[i] * inv;
            const float v4[4] = {yv[0], yv[1], yv[2], yv[3]};
            store_y<4, FULL>(a, row, head, d, v4);
        }
        return;
    }
    const uint64_t pb = (static_cast<uint64_t>(item0 + part) * a.n_kvh + kvh) * kCols + c;
#pragma unroll
    for (int i = 0; i < MT; i++)
        *reinterpret_cast<f32x4*>(a.part_o + pb * HD + 16u * i + 4u * a4) = o[i];
    if (a4 == 0) {
        a.part_ml[2 * pb] = m;
        a.part_ml[2 * pb + 1] = l;
    }
}

// Chunked prefill at head_dim <= 128 (attn_prefill serves wider heads and
// scales above one), as the workgroup body of attn_prefill_wide and
// attn_mixed.  One workgroup of W waves handles a block of up to NCG * W
// consecutive groups of one chunk, for one KV head and one partition of the
// block's key span.  Wave w owns groups g0 + NCG w .. + NCG - 1 (16 NCG query
// columns), so every K and V operand read from LDS feeds a product for each
// of its groups (two for the query's high and low halves in QK^T).  Keys
// advance 32 at a time:
//  * QK^T: two 16-token products per column group (S^T[16 tok x 16 col],
//    v_mfma_f32_16x16x32), which leave lane (a, c) with tokens 4a..4a+3 of
//    each half;
//  * PV: one v_mfma_f32_16x16x32 per 16 dims over all 32 tokens.  Its B
//    operand (8 probabilities of one column) is the lane's two score
//    quadruples, so its k index runs over tokens {4a..4a+3, 16+4a..16+4a+3};
//    the A operand (V^T) is read from LDS in that same token order.
// K and V tiles of 64 tokens are double-buffered in LDS and shared by all
// waves; the next tile's global loads are in flight during the compute.
// They are ordinary cached loads: the blocks of a chunk read the same keys
// (one KV head's blocks run on one XCD, whose L2 keeps them), where the
// streaming hint of the decode kernels sent every tile to HBM.
//   K tile: [4 slices of 16][HD/8 chunks][16 tokens] x 16 bytes (as attn_prefill).
//   V tile: [2 steps of 32][HD dims][4 lane groups] x 16 bytes.  Entry
//     (s, d, a) holds dim d of tokens 32s + 4a..+3 and 32s + 16 + 4a..+3; the
//     lane-group index is XOR-ed with (d / 4) % 4, so the 16 lanes of an
//     operand read hit distinct banks.
#ifndef THB_PREFILL_TILE
#define THB_PREFILL_TILE 64
#endif
#ifndef THB_PREFILL_NCG
#define THB_PREFILL_NCG 2
#endif
// Wave priority by phase in attn_prefill_wide (0: none; 1: the products'
// phases high, the probabilities' low; 2: the reverse).
#ifndef THB_PREFILL_PRIO
#define THB_PREFILL_PRIO 0
#endif
// Query groups per wave of attn_prefill_wide: two up to head_dim 128 (every
// K or V operand read from LDS feeds both), one at 256 (its accumulators
// alone take 64 registers).
constexpr int prefill_ncg(int hd) { return hd > 128 ? 1 : THB_PREFILL_NCG; }

template <bool MATRIX>
__device__ __forceinline__ void phase_prio() {
    if constexpr (THB_PREFILL_PRIO == 1) __builtin_amdgcn_s_setprio(MATRIX ? 1 : 0);
    if constexpr (THB_PREFILL_PRIO == 2) __builtin_amdgcn_s_setprio(MATRIX ? 0 : 1);
}
// LDS of one prefill workgroup: the double-buffered K and V tiles and the
// partition's page list.
template <int HD>
struct PrefillLds {
    u32x4 k[2][THB_PREFILL_TILE * HD / 8];
    u32x4 v[2][THB_PREFILL_TILE / 32 * HD * 4];
    uint32_t page[kMaxPartPages];
};

template <int HD, bool F16, int W, bool FULL, bool CAP, bool QLO = true>
__device__ __forceinline__ void prefill_wide_wg(const AttnArgs& a, uint32_t bid, PrefillLds<HD>& L,
                                                uint32_t tid_arg) {
    using O = Ops<F16>;
    typedef typename O::in8 in8;
    constexpr int KS = HD / 32;
    constexpr int MT = HD / 16;
    constexpr int NCG = prefill_ncg(HD);   // column groups per wave
    constexpr int TT = THB_PREFILL_TILE;   // tokens per tile
    constexpr int NS = TT / 32;            // 32-token steps per tile
    constexpr int CPH = HD / 8;            // 8-dim chunks of a key
    constexpr int KU = TT * HD / 8;        // 16-byte K units per tile
    constexpr int VE = NS * HD * 4;        // 16-byte V entries per tile
    constexpr int VP = NS * 4 * (HD / 2);  // V load units (step, lane group, dim pair): two loads each
    constexpr int NT = 64 * W;
    constexpr int KPT = (KU + NT - 1) / NT;
    constexpr int VPT = (VP + NT - 1) / NT;

    static_assert(sizeof(L.k[0]) == KU * 16 && sizeof(L.v[0]) == VE * 16, "prefill LDS tiles");
    auto& s_k = L.k;
    auto& s_v = L.v;
    auto& s_page = L.page;

    const uint32_t tid = tid_arg;  // threadIdx.x (opaque in attn_list)
    const uint32_t lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t a4 = lane >> 4, c = lane & 15u;
    const uint32_t pr = bid / a.n_kvh, kvh = bid - pr * a.n_kvh;

    // A pair of prefill work items of one sequence and partition (the host
    // pairs a chunk's longest block with its shortest): the workgroup runs
    // the first, then the second, over one stream of tiles (the second's
    // first tile is loaded while the first's last is computed) and one page
    // list (the union of their keys), so the launch's fixed costs are paid
    // once per pair.  Each item's arithmetic is exactly that of a workgroup
    // of its own.
    const uint32_t it0 = a.bpairs[2 * pr], it1 = a.bpairs[2 * pr + 1];
    const bool two = it1 != kNoItem;
    const uint32_t* B0 = a.bitems + static_cast<uint64_t>(it0) * kBItemWords;
    const uint32_t* B1 = a.bitems + static_cast<uint64_t>(two ? it1 : it0) * kBItemWords;
    // Both items start their partition at the same key (the host pairs
    // only such items); the page list spans the longer of the two.
    const uint32_t seq = B0[2];
    const uint32_t pbeg = B0[6] + B0[kBlockWords] * B0[7];
    const uint32_t P = max(B0[7], B1[7]);
    const uint32_t hd = a.head_dim;
    const uint32_t pshift = a.page_shift;
    const uint32_t pmask = (1u << pshift) - 1u;
    // Per item: its keys [tb, te) in this partition, its first tile and tile
    // count (scalars, selected by the item index: no indexed arrays).
    const uint32_t tb0 = max(B0[3], pbeg), te0 = min(B0[4], pbeg + B0[7]);
    const uint32_t tb1 = max(B1[3], pbeg), te1 = two ? min(B1[4], pbeg + B1[7]) : tb1;
    const uint32_t tf0 = tb0 & ~31u, tf1 = tb1 & ~31u;
    const uint32_t nt0 = te0 > tf0 ? (te0 - tf0 + TT - 1) / TT : 0u;
    const uint32_t nt1 = te1 > tf1 ? (te1 - tf1 + TT - 1) / TT : 0u;

    {
        const uint32_t npg = P >> pshift;
        const uint32_t lp0 = pbeg >> pshift;
        const uint32_t* trow = a.table + static_cast<uint64_t>(seq) * a.max_pages;
        for (uint32_t i = tid; i < npg; i += NT) {
            const uint32_t lp = lp0 + i;
            const bool used = (tb0 < te0 && (lp << pshift) < te0 && ((lp + 1) << pshift) > tb0) ||
                              (tb1 < te1 && (lp << pshift) < te1 && ((lp + 1) << pshift) > tb1);
            const uint32_t pg = used ? trow[lp] : 0u;
            s_page[i] = pg < a.pages ? pg : 0u;  // block_pages: a page outside the pool reads page 0
        }
    }

    // This wave's two column groups of the current item; [wlo, whi) spans
    // both groups' keys.  Each column's key range is requested here and used
    // after the first tile's loads and the queries' loads are out, so the
    // round trips overlap.
    bool con[NCG];
    uint32_t row[NCG], head[NCG], clo[NCG], chi[NCG], cspan[NCG], item0[NCG];
    uint32_t wlo = 0xFFFFFFFFu, whi = 0;
    auto setup = [&](const uint32_t* Bk, uint32_t tb, uint32_t te) {
        const uint32_t g0 = Bk[0], ng = Bk[1];
        wlo = 0xFFFFFFFFu;
        whi = 0;
#pragma unroll
        for (int g = 0; g < NCG; g++) {
            const uint32_t gi = NCG * wave + g;
            const bool gon = gi < ng;
            const uint32_t* G = a.groups + (g0 + (gon ? gi : 0u)) * kGroupWords;
            const uint32_t r0 = G[0], R = G[1], h0 = G[2], H = G[3];
            item0[g] = G[10];
            const uint32_t ncols = gon ? R * H : 0u;
            con[g] = c < ncols;
            const uint32_t rr = con[g] ? c / H : 0u;
            row[g] = r0 + rr;
            head[g] = kvh * a.nq_per_kv + h0 + (con[g] ? c - rr * H : 0u);
            clo[g] = a.ranges[2 * row[g]];  // row r0 of an unused column: a valid index
            chi[g] = a.ranges[2 * row[g] + 1];
            if (gon) {
                const uint32_t glo = max(G[5], tb), ghi = min(G[6], te);
                if (glo < ghi) {
                    wlo = min(wlo, glo);
                    whi = max(whi, ghi);
                }
            }
        }
    };
    // Per group, the keys every column reads: a 32-key step inside
    // [lomax, himin) needs no mask.
    uint32_t lomax[NCG], himin[NCG];
    auto column_ranges = [&](uint32_t tb, uint32_t te) {
#pragma unroll
        for (int g = 0; g < NCG; g++) {
            clo[g] = con[g] ? max(clo[g], tb) : 0u;
            chi[g] = con[g] ? min(chi[g], te) : 0u;
            cspan[g] = chi[g] > clo[g] ? chi[g] - clo[g] : 0u;  // key t is read iff t - clo < cspan
            uint32_t lo = con[g] ? clo[g] : 0u, hi = con[g] ? chi[g] : 0xFFFFFFFFu;
#pragma unroll
            for (int sh = 1; sh < 64; sh <<= 1) {
                lo = max(lo, static_cast<uint32_t>(__shfl_xor(static_cast<int>(lo), sh)));
                hi = min(hi, static_cast<uint32_t>(__shfl_xor(static_cast<int>(hi), sh)));
            }
            lomax[g] = __builtin_amdgcn_readfirstlane(lo);
            himin[g] = __builtin_amdgcn_readfirstlane(hi);
        }
    };
    in8 qh[NCG][KS], ql[NCG][KS];

    const uint16_t* kplane = a.k + static_cast<uint64_t>(kvh) * a.plane;
    const uint16_t* vplane = a.v + static_cast<uint64_t>(kvh) * a.plane;

    // Global -> registers for one tile of an item whose keys are [tb, last];
    // tokens outside are clamped into it (their scores are masked).  At the
    // template's own head_dim every unit is in range: the page numbers of all
    // units are read from LDS first (one round trip), then every load is
    // issued, with no guards.
    auto load = [&](uint32_t t0, uint32_t tb, uint32_t last, u32x4 (&kr)[KPT], u32x4 (&vr)[VPT][2]) {
        if constexpr (KU % NT == 0 && VP % NT == 0) {
            if (hd == static_cast<uint32_t>(HD)) {
                uint32_t kpg[KPT], kin[KPT], vpg[VPT][2], vin[VPT][2];
#pragma unroll
                for (int k = 0; k < KPT; k++) {
                    const uint32_t u = tid + k * NT;
                    const uint32_t st = u / (16 * CPH), rem = u - st * (16 * CPH);
                    const uint32_t ch = rem >> 4, tok = rem & 15u;
                    const uint32_t t = min(max(t0 + 16u * st + tok, tb), last);
                    kpg[k] = s_page[(t - pbeg) >> pshift];
                    kin[k] = ((8u * ch & ~31u) << pshift) + 32u * (t & pmask) + (8u * ch & 31u);
                }
#pragma unroll
                for (int k = 0; k < VPT; k++) {
                    const uint32_t u = tid + k * NT;
                    const uint32_t st = u / (4 * (HD / 2)), rem = u - st * (4 * (HD / 2));
                    const uint32_t ag = rem / (HD / 2), d = 2u * (rem - ag * (HD / 2));
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const uint32_t t = min(max(t0 + 32u * st + 16u * h + 4u * ag, tb & ~3u), last & ~3u);
                        vpg[k][h] = s_page[(t - pbeg) >> pshift];
                        vin[k][h] = ((t & pmask) >> 2) * (4u * HD) + 4u * d;
                    }
                }
#pragma unroll
                for (int k = 0; k < KPT; k++)
                    kr[k] = *reinterpret_cast<const u32x4*>(kplane + ((static_cast<uint64_t>(kpg[k]) * HD) << pshift) + kin[k]);
#pragma unroll
                for (int k = 0; k < VPT; k++)
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        vr[k][h] = *reinterpret_cast<const u32x4*>(vplane + ((static_cast<uint64_t>(vpg[k][h]) * HD) << pshift) +
                                                                 vin[k][h]);
                return;
            }
        }
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const uint32_t u = tid + k * NT;
            const uint32_t st = u / (16 * CPH), rem = u - st * (16 * CPH);
            const uint32_t ch = rem >> 4, tok = rem & 15u;
            const uint32_t t = min(max(t0 + 16u * st + tok, tb), last);
            const uint32_t page = s_page[(t - pbeg) >> pshift];
            const bool ok = u < static_cast<uint32_t>(KU) && 8u * ch < hd;
            kr[k] = ok ? *(reinterpret_cast<const u32x4*>(
                             kplane + ((static_cast<uint64_t>(page) * hd) << pshift) + k_off(t & pmask, 8u * ch, hd, pshift)))
                       : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const uint32_t u = tid + k * NT;
            const uint32_t st = u / (4 * (HD / 2)), rem = u - st * (4 * (HD / 2));
            const uint32_t ag = rem / (HD / 2), d = 2u * (rem - ag * (HD / 2));
            const bool ok = u < static_cast<uint32_t>(VP) && d < hd;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t t = min(max(t0 + 32u * st + 16u * h + 4u * ag, tb & ~3u), last & ~3u);
                const uint32_t page = s_page[(t - pbeg) >> pshift];
                vr[k][h] = ok ? *(reinterpret_cast<const u32x4*>(
                                    vplane + ((static_cast<uint64_t>(page) * hd) << pshift) + v_off(t & pmask, d, hd)))
                              : u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store = [&](int buf, const u32x4 (&kr)[KPT], const u32x4 (&vr)[VPT][2]) {
#pragma unroll
        for (int k = 0; k < KPT; k++) {
            const uint32_t u = tid + k * NT;
            if (u < static_cast<uint32_t>(KU)) s_k[buf][u] = kr[k];
        }
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const uint32_t u = tid + k * NT;
            if (u >= static_cast<uint32_t>(VP)) continue;
            const uint32_t st = u / (4 * (HD / 2)), rem = u - st * (4 * (HD / 2));
            const uint32_t ag = rem / (HD / 2), d = 2u * (rem - ag * (HD / 2));
            const uint32_t sw = ag ^ ((d >> 2) & 3u);  // the same for d and d + 1
            s_v[buf][(st * HD + d) * 4 + sw] = u32x4{vr[k][0].x, vr[k][0].y, vr[k][1].x, vr[k][1].y};
            s_v[buf][(st * HD + d + 1u) * 4 + sw] = u32x4{vr[k][0].z, vr[k][0].w, vr[k][1].z, vr[k][1].w};
        }
    };

    // The softmax denominators come from the matrix cores: lsum[g] is a PV
    // product against a row of ones, so every element holds the column's sum
    // of probabilities (all 32 keys of a step, all four lane groups).
    float m[NCG];
    f32x4 o[NCG][MT], lsum[NCG];
    const float tanh_c = 2.8853900817779268f * a.qpost;  // 2 log2(e) |qscale|
    u32x4 ones;  // eight 1.0 in the KV type
    {
        const uint32_t one2 = F16 ? 0x3C003C00u : 0x3F803F80u;
        ones = u32x4{one2, one2, one2, one2};
        asm volatile("" : "+v"(ones));  // held in registers, not rebuilt before every use
    }
    // Lazy-rescale thresholds, in the units of the scores x (m + kTau, over
    // qpost without a cap).
    const float inv_qpost = 1.0f / a.qpost;
    float thr[NCG];
    auto init_state = [&]() {
#pragma unroll
        for (int g = 0; g < NCG; g++) {
            m[g] = kFloor;
            lsum[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < MT; i++) o[g][i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            thr[g] = CAP ? m[g] + kTau : (m[g] + kTau) * inv_qpost;
        }
    };

    // 32-key steps, software-pipelined: the QK^T products of step s + 1 are
    // issued before the softmax of step s, so the matrix cores work on them
    // while the vector ALU computes the probabilities.  Products are ordered
    // so that an accumulator is reused only every fourth MFMA (two column
    // groups x two halves), which covers the matrix pipeline's latency; the
    // mask is one unsigned range compare per score, and steps inside every
    // column's keys skip it.
    auto qk_step = [&](int buf, int st, f32x4 (&sc)[NCG][2]) {
        phase_prio<true>();
#pragma unroll
        for (int g = 0; g < NCG; g++) sc[g][0] = sc[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < KS; j++) {
            u32x4 kv[2];
#pragma unroll
            for (int h = 0; h < 2; h++) kv[h] = s_k[buf][((2 * st + h) * CPH + 4 * j + a4) * 16u + c];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int g = 0; g < NCG; g++) sc[g][h] = O::qk(kv[h], qh[g][j], sc[g][h]);
            // The query's low half is exactly zero (QLO false: an f16 query
            // against f16 keys): its products would add zeros.
            if constexpr (QLO) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int g = 0; g < NCG; g++) sc[g][h] = O::qk(kv[h], ql[g][j], sc[g][h]);
            }
        }
    };
    auto softmax_pv = [&](int buf, int st, uint32_t ts, const f32x4 (&sc)[NCG][2]) {
        phase_prio<false>();
        in8 ph[NCG], pl[NCG];
        // Without the query's low half (the lean f16 kernel, whose registers
        // allow it) the step's V operands are requested before the softmax,
        // whose vector work covers their LDS latency; the other kernels read
        // them pair by pair beside the products.
        constexpr bool VPRE = !FULL && !QLO && HD <= 128;  // 64 more registers at 256
        auto vread = [&](int i) {
            const uint32_t d = 16u * i + c;
            return s_v[buf][(st * HD + d) * 4 + (a4 ^ ((d >> 2) & 3u))];
        };
        u32x4 vop[VPRE ? MT : 1];
        if constexpr (VPRE) {
#pragma unroll
            for (int i = 0; i < MT; i++) vop[i] = vread(i);
        }
#pragma unroll
        for (int g = 0; g < NCG; g++) {
            float x[8];
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // the query carries the scale's sign: without a cap, x
                    // times qpost is the logit; with one, x is the logit
                    float v = sc[g][h][e];
                    if constexpr (CAP) v = a.cap2 * tanh_scaled(v, tanh_c);
                    x[4 * h + e] = v;
                }
            }
            if (!(ts >= lomax[g] && ts + 32u <= himin[g])) {  // wave-uniform
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t t = ts + 16u * (e >> 2) + 4u * a4 + (e & 3);
                    x[e] = t - clo[g] < cspan[g] ? x[e] : -INFINITY;
                }
            }
            // The column max (two cross-lane steps) is needed only when some
            // score beats its column's running max by more than kTau; without
            // one, no column rescales, exactly as if the max had been taken.
            // The test compares each score with the column's threshold
            // (m + kTau in score units, kept with m): eight compares whose
            // lane masks the scalar unit ORs, instead of a max tree.
            uint64_t hit = 0;  // lanes with a score above the threshold (2: ordered >)
#pragma unroll
            for (int e = 0; e < 8; e++) hit |= __builtin_amdgcn_fcmpf(x[e], thr[g], 2);
            if (hit != 0) {  // wave-uniform
                float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
                if constexpr (!CAP) mx *= a.qpost;  // log2 units (qpost > 0)
                mx = col_max(mx);
                if (mx > m[g] + kTau) {
                    const float alpha = fast_exp2(m[g] - mx);
                    lsum[g] *= alpha;
#pragma unroll
                    for (int i = 0; i < MT; i++) o[g][i] *= alpha;
                    m[g] = mx;
                    thr[g] = CAP ? mx + kTau : (mx + kTau) * inv_qpost;
                }
            }
            float p[8];
#pragma unroll
            for (int e = 0; e < 8; e++) p[e] = fast_exp2(CAP ? x[e] - m[g] : __builtin_fmaf(x[e], a.qpost, -m[g]));
            // High and low halves, as in the decode kernels: one f16 operand
            // alone (relative error 2^-12) measured 1e-4 .. 5e-4 against the
            // exact softmax on N(0,1) .. N(0,4) data, both halves 3e-7.
            O::split8_fast(p, ph[g], pl[g]);
        }
        phase_prio<true>();
#pragma unroll
        for (int i = 0; i < MT; i += 2) {
            u32x4 vv[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                if constexpr (VPRE)
                    vv[u] = vop[i + u];
                else
                    vv[u] = vread(i + u);
            }
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int g = 0; g < NCG; g++) o[g][i + u] = O::pv32(vv[u], ph[g], o[g][i + u]);
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int g = 0; g < NCG; g++) o[g][i + u] = O::pv32(vv[u], pl[g], o[g][i + u]);
        }
#pragma unroll
        for (int g = 0; g < NCG; g++) lsum[g] = O::pv32(ones, ph[g], lsum[g]);
#pragma unroll
        for (int g = 0; g < NCG; g++) lsum[g] = O::pv32(ones, pl[g], lsum[g]);
    };
    auto compute = [&](int buf, uint32_t t0) {
        bool act[NS];
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const uint32_t ts = t0 + 32u * st;
            act[st] = !(ts >= whi || ts + 32u <= wlo);  // inside this wave's keys
        }
        f32x4 scA[NCG][2], scB[NCG][2];
        if (act[0]) qk_step(buf, 0, scA);
#pragma unroll
        for (int st = 0; st < NS; st++) {
            if (st + 1 < NS && act[st + 1]) qk_step(buf, st + 1, (st & 1) ? scA : scB);
            if (act[st]) softmax_pv(buf, st, t0 + 32u * st, (st & 1) ? scB : scA);
        }
    };

    // Outputs of the current item: the normalised rows, or this partition's
    // (m, l, o) when the item's block spans several partitions.
    auto finish = [&](const uint32_t* Bk) {
        const uint32_t n_parts = Bk[5], part = Bk[kBlockWords];
#pragma unroll
        for (int g = 0; g < NCG; g++) {
            const float lg = lsum[g][0];
            if (!con[g]) continue;
            if (n_parts == 1) {
                const float inv = 1.0f / lg;
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const uint32_t d = 16u * i + 4u * a4;
                    if (d >= hd) continue;
                    const f32x4 yv = o[g][i] * inv;
                    const float v4[4] = {yv[0], yv[1], yv[2], yv[3]};
                    store_y<4, FULL>(a, row[g], head[g], d, v4);
                }
                continue;
            }
            const uint64_t pb = (static_cast<uint64_t>(item0[g] + part) * a.n_kvh + kvh) * kCols + c;
#pragma unroll
            for (int i = 0; i < MT; i++)
                *reinterpret_cast<f32x4*>(a.part_o + pb * HD + 16u * i + 4u * a4) = o[g][i];
            if (a4 == 0) {
                a.part_ml[2 * pb] = m[g];
                a.part_ml[2 * pb + 1] = lg;
            }
        }
    };

    __syncthreads();  // s_page complete
    u32x4 kr[KPT], vr[VPT][2];
    uint32_t k_tile = 0;  // tiles of the pair computed so far (LDS buffer parity)
    const uint32_t last1 = te1 > 0 ? te1 - 1 : 0;
    // One item of the pair: straight-line code per item (a loop over the two
    // items kept both items' state live and spilled).
    auto run_item = [&](auto second_c) {
        constexpr bool second = decltype(second_c)::value;
        const uint32_t* Bk = second ? B1 : B0;
        const uint32_t tb = second ? tb1 : tb0, te = second ? te1 : te0;
        const uint32_t tf = second ? tf1 : tf0, nt = second ? nt1 : nt0;
        const uint32_t last = te > 0 ? te - 1 : 0;
        setup(Bk, tb, te);
        if constexpr (!second) {
            // The pair's first tile: the first item's, or the second's if
            // the first has none.
            if (nt0)
                load(tf0, tb0, last, kr, vr);
            else if (nt1)
                load(tf1, tb1, last1, kr, vr);
        }
        // The queries are loaded and split while the first tile's loads are
        // in flight (their round trips overlap).
#pragma unroll
        for (int g = 0; g < NCG; g++) load_q<KS, O, FULL>(a, con[g], row[g], head[g], a4, qh[g], ql[g], a.qpre);
        column_ranges(tb, te);
        init_state();
        if constexpr (!second)
            if (nt0 || nt1) store(0, kr, vr);
        __syncthreads();
        // The second item's first tile follows the first item's last.
        const uint32_t nt_next = second ? 0u : nt1;
        for (uint32_t i = 0; i < nt; i++, k_tile++) {
            const uint32_t t0 = tf + i * TT;
            const bool own = i + 1 < nt;
            const bool more = own || nt_next > 0;
            if (more) load(own ? t0 + TT : tf1, own ? tb : tb1, own ? last : last1, kr, vr);
            compute(static_cast<int>(k_tile & 1u), t0);
            if (more) store(static_cast<int>((k_tile + 1) & 1u), kr, vr);
            __syncthreads();
        }
        finish(Bk);
    };
    run_item(std::integral_constant<bool, false>{});
    if (two) run_item(std::integral_constant<bool, true>{});
}

template <int HD, bool F16, int W, bool FULL, bool CAP, bool QLO = true>
__global__ __launch_bounds__(64 * W, W >= 8 ? W / 4 : 1) void attn_prefill_wide(AttnArgs a) {
    __shared__ PrefillLds<HD> lds;
    prefill_wide_wg<HD, F16, W, FULL, CAP, QLO>(a, blockIdx.x, lds, threadIdx.x);
}

// A call with decode items and prefill blocks (a continuous batch) as one
// launch: record r of the launch order is a decode item or a prefill block
// (bit 31), and its KV heads are the workgroups r * n_kvh .. + n_kvh - 1.
// The host interleaves the two kinds, so that workgroups streaming KV from
// HBM and workgroups busy on the matrix cores run side by side on different
// CUs instead of one kernel after the other.  Each workgroup runs exactly
// the code (and arithmetic) of its own kernel.  The two bodies' LDS
// overlay each other.
template <int HD, bool F16, int W>
union MixedLds {
    DecodeLds<HD, F16, W> d;
    PrefillLds<HD> p;
};

template <int HD, bool F16, int W, bool FULL, bool CAP, bool QLO = true>
__global__ __launch_bounds__(64 * W, 2) void attn_mixed(AttnArgs a) {
    __shared__ MixedLds<HD, F16, W> lds;
    const uint32_t rec = blockIdx.x / a.n_kvh, kvh = blockIdx.x - rec * a.n_kvh;
    const uint32_t w = a.order[rec];
    const uint32_t bid = (w & 0x7FFFFFFFu) * a.n_kvh + kvh;
    if (w >> 31)
        prefill_wide_wg<HD, F16, W, FULL, CAP, QLO>(a, bid, lds.p, threadIdx.x);
    else
        decode_wg<HD, F16, W, ring_for(HD), FULL>(a, bid, lds.d, threadIdx.x);
}

// A device-planned call in list mode (thb_dplan_create_ex with
// THB_DPLAN_PREFILL): workgroups claim entries of the plan's launch order
// from a counter in its header (entry e covers its record's KV heads as
// workgroups e * n_kvh .. + n_kvh - 1) and run each with its own kernel's
// code, as attn_mixed does; the last workgroup to find no entry left resets
// the counters for the next launch.  Head_dim <= 256 (both bodies 8 waves).
template <int HD, bool F16, int W, bool FULL, bool CAP, bool QLO = true>
__global__ __launch_bounds__(64 * W, 2) void attn_list(AttnArgs a) {
    __shared__ MixedLds<HD, F16, W> lds;
    __shared__ uint32_t s_w;
    // Each entry reads the arguments through a pointer the compiler must
    // take as new on every pass (an empty asm), so their scalar loads stay
    // inside the loop: hoisted, both bodies' loop-invariant values stayed
    // live across the loop and spilled.
    typedef const __attribute__((address_space(4))) AttnArgs* KArgs;
    const KArgs kargs = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t* hdr = a.list;
    const uint32_t n_kvh = a.n_kvh;
    const uint32_t n = hdr[0] * n_kvh;
    for (;;) {
        if (threadIdx.x == 0) s_w = __hip_atomic_fetch_add(&hdr[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const uint32_t w = s_w;
        if (w >= n) break;
        KArgs kp = kargs;
        asm volatile("" : "+s"(kp));
        const AttnArgs& ar = *(const AttnArgs*)kp;
        uint32_t tid = threadIdx.x;  // opaque too: values derived from it stay inside the loop
        asm volatile("" : "+v"(tid));
        const uint32_t rec = w / n_kvh, kvh = w - rec * n_kvh;
        const uint32_t e = ar.order[rec];
        if (e >> 31)
            prefill_wide_wg<HD, F16, W, FULL, CAP, QLO>(ar, (e & 0x7FFFFFFFu) * n_kvh + kvh, lds.p, tid);
        else
            decode_wg<HD, F16, W, ring_for(HD), FULL>(ar, e * n_kvh + kvh, lds.d, tid);
        __syncthreads();
    }
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(&hdr[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u == gridDim.x) {
        __hip_atomic_store(&hdr[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&hdr[2], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------- device-side planning
// Plans a decode call on the device from the row meta in device memory, so
// that a step can be captured in a graph once and replayed while the rows'
// positions move (thb_dplan_*).  The rules are build_plan's: each row's key
// range (plan_rows: kv_len per 8-row block of its chunk, window, causal), the
// chunk's groups of up to 16 query vectors, each group's partitions (the same
// function of its key range), so every (group, partition, KV head) computes
// what thb_attn computes for it.  The layout differs: group g of the call
// owns slot g of a fixed grid of gmax groups and its partition p slot
// g * pmax + p; slots past a group's partitions or past the call's groups do
// nothing.  Chunks of four or more groups (prefill) run as decode groups too.
constexpr uint32_t kDPlanMaxRows = 4096;
constexpr uint32_t kDPlanThreads = 1024;

struct DPlanArgs {
    const uint32_t* meta;  // row meta of the call's first row
    uint32_t* blob;        // [groups gmax | items gmax * pmax | ranges 2 m | merge gmax]
    uint32_t* state;       // device allocator state: page counts, status
    uint32_t npages_off;
    uint32_t m, seq_fixed, causal, window, G, PL, align, pmax, gmax, page_shift, seqs;
    uint32_t items_off, ranges_off, merge_off;
    uint32_t append;     // the plan serves thb_attn_append_dplan: check that the append can run in the launch
    uint32_t pos_limit;  // rows at or past it read nothing (0: none)
};

// build_plan's partition of a key range [lo, hi) (lo = hi = 0 when empty).
__device__ inline void dplan_partition(uint32_t& lo, uint32_t& hi, uint32_t PL, uint32_t align, uint32_t& base,
                                       uint32_t& n_parts, uint32_t& plen) {
    base = 0;
    n_parts = 1;
    plen = align;
    if (hi <= lo || lo == 0xFFFFFFFFu) {
        lo = hi = 0;
        return;
    }
    base = lo & ~(align - 1);
    part_split(uint64_t(hi) - base, PL, align, n_parts, plen);
}

// Inclusive sum over the workgroup; *total gets the sum.  Every thread calls it.
__device__ uint32_t dplan_scan(uint32_t v, uint32_t* red, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(v, d);
        if (lane >= d) v += t;
    }
    if (lane == 63) red[w] = v;
    __syncthreads();
    if (w == 0) {
        uint32_t x = lane < nw ? red[lane] : 0u;
#pragma unroll
        for (uint32_t d = 1; d < 64; d <<= 1) {
            const uint32_t t = __shfl_up(x, d);
            if (lane >= d) x += t;
        }
        if (lane < nw) red[lane] = x;
    }
    __syncthreads();
    if (w > 0) v += red[w - 1];
    *total = red[nw - 1];
    __syncthreads();
    return v;
}

// First failure of the call, in the device allocator's status word
// (thb_pool_status reports it).
__device__ void dplan_fail(uint32_t* hdr, uint32_t code, uint32_t x, uint32_t y, uint32_t z) {
    if (atomicCAS(&hdr[kPageHdrStatus], 0u, code) == 0u) {
        hdr[kPageHdrStatus + 1] = x;
        hdr[kPageHdrStatus + 2] = y;
        hdr[kPageHdrStatus + 3] = z;
    }
}

// The row phases of both planners: chunks (maximal runs of rows of one
// sequence; one chunk with a fixed seq) into s_ck (chunk of each row) and
// s_cs (first row of each chunk, then m; *n_chunks), then each row's key
// range (plan_rows) into s_lo / s_hi and ranges_out; a row its pages do
// not cover, or whose position is not below pos_limit (the rope tables'
// rows, when set), reads nothing and is reported in the allocator's status
// word.
struct DPlanRows {
    const uint32_t* meta;
    uint32_t* ranges_out;
    uint32_t* state;
    uint32_t npages_off, m, seq_fixed, causal, window, page_shift, seqs;
    uint32_t pos_limit;  // 0: none
};

__device__ void dplan_rows(const DPlanRows& a, uint32_t* s_ck, uint32_t* s_cs, uint32_t* s_lo, uint32_t* s_hi,
                           uint32_t* s_red, uint32_t& s_carry) {
    const uint32_t tid = threadIdx.x, m = a.m;
    const bool per_row = a.seq_fixed == THB_SEQ_PER_ROW;
    auto seq_of = [&](uint32_t r) { return per_row ? a.meta[8u * r + 1] : a.seq_fixed; };
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (uint32_t t0 = 0; t0 < m; t0 += kDPlanThreads) {
        const uint32_t r = t0 + tid;
        const bool start = r < m && (r == 0 || (per_row && seq_of(r) != seq_of(r - 1)));
        uint32_t total = 0;
        const uint32_t incl = dplan_scan(start ? 1u : 0u, s_red, &total);
        const uint32_t carry = s_carry;
        if (r < m) {
            s_ck[r] = carry + incl - 1;
            if (start) s_cs[carry + incl - 1] = r;
        }
        __syncthreads();
        if (tid == 0) s_carry = carry + total;
        __syncthreads();
    }
    if (tid == 0) s_cs[s_carry] = m;
    __syncthreads();
    const uint32_t* npages = a.state + a.npages_off;
    for (uint32_t r = tid; r < m; r += kDPlanThreads) {
        const uint32_t ck = s_ck[r], c0 = s_cs[ck], c1 = s_cs[ck + 1];
        const uint32_t n = c1 - c0, i = r - c0, pos = a.meta[8u * r];
        const uint32_t blk_last = min((i / 8u) * 8u + 8u, n);
        const uint64_t kv_len =
            a.causal ? uint64_t(a.meta[8u * (c0 + blk_last - 1)]) + 1 : uint64_t(a.meta[8u * (c1 - 1)]) + 1;
        uint64_t ws = 0;
        if (a.causal && a.window != 0 && uint64_t(pos) + 1 > a.window) ws = uint64_t(pos) + 1 - a.window;
        uint64_t h = kv_len;
        if (a.causal && uint64_t(pos) + 1 < h) h = uint64_t(pos) + 1;
        uint32_t lo = static_cast<uint32_t>(ws), hi = static_cast<uint32_t>(min(h, uint64_t(0xFFFFFFFFu)));
        if (a.pos_limit != 0 && pos >= a.pos_limit) {
            dplan_fail(a.state, kPageStPosLimit, pos, a.pos_limit, 0u);
            lo = hi = 0;
        } else if (hi > lo) {
            const uint32_t seq = seq_of(r);
            if (seq >= a.seqs) {
                dplan_fail(a.state, kPageStBadSeq, seq, a.seqs, 0u);
                lo = hi = 0;
            } else if ((uint64_t(npages[seq]) << a.page_shift) < hi) {
                dplan_fail(a.state, kPageStCover, seq, npages[seq] << a.page_shift, hi);
                lo = hi = 0;
            }
        }
        s_lo[r] = lo;
        s_hi[r] = hi;
        a.ranges_out[2u * r] = lo;
        a.ranges_out[2u * r + 1] = hi;
    }
    __syncthreads();
}

// For a plan that serves thb_attn_append_dplan: build_plan's conditions for
// running the append inside the attention launch, checked on the device at
// every build.  Each chunk fits one group; every row's keys end at its new
// token (hi == pos + 1, lo <= pos) and positions rise within the chunk; with
// a fixed sequence every row's own sequence is that one (the append takes
// the row meta's); no sequence heads two chunks (two groups would append to
// and read one sequence's pages in one launch).  At the first failing row
// (lowest row; code row << 3 | reason) the status is recorded and every
// row's range emptied: the launch then appends nothing and writes NaN.
constexpr uint32_t kFuseSetBits = 13;
constexpr uint32_t kFuseSet = 1u << kFuseSetBits;  // open-addressing set of the chunk heads' sequences
static_assert(kFuseSet >= 2 * kDPlanMaxRows, "the set keeps at least half its slots empty");

__device__ void dplan_check_fused(const DPlanArgs& a, const uint32_t* s_ck, const uint32_t* s_cs, uint32_t* s_lo,
                                  uint32_t* s_hi) {
    constexpr uint32_t kEmpty = 0xFFFFFFFFu;
    __shared__ uint32_t s_key[kFuseSet], s_first[kFuseSet];  // a sequence, its lowest chunk-head row
    __shared__ uint32_t s_bad;
    const uint32_t tid = threadIdx.x, m = a.m;
    const bool per_row = a.seq_fixed == THB_SEQ_PER_ROW;
    const uint32_t rg = a.G <= kCols ? kCols / a.G : 1u;
    for (uint32_t i = tid; i < kFuseSet; i += kDPlanThreads) {
        s_key[i] = kEmpty;
        s_first[i] = kEmpty;
    }
    if (tid == 0) s_bad = kEmpty;
    __syncthreads();
    auto slot = [](uint32_t seq) { return (seq * 0x9E3779B1u) >> (32 - kFuseSetBits); };
    for (uint32_t r = tid; r < m; r += kDPlanThreads) {
        const uint32_t ck = s_ck[r], c0 = s_cs[ck], n = s_cs[ck + 1] - c0;
        const uint32_t pos = a.meta[8u * r], seq = a.meta[8u * r + 1];
        uint32_t why = 0;
        if (n > rg)
            why = kNoFuseChunk;
        else if (uint64_t(s_hi[r]) != uint64_t(pos) + 1 || s_lo[r] > pos || (r > c0 && pos <= a.meta[8u * (r - 1)]))
            why = kNoFuseKeys;  // also a row its pages do not cover (its range is empty)
        else if (!per_row && seq != a.seq_fixed)
            why = kNoFuseSeq;
        if (why) atomicMin(&s_bad, (r << 3) | why);
        if (per_row && r == c0 && seq < a.seqs) {
            uint32_t h = slot(seq);
            for (;;) {
                const uint32_t old = atomicCAS(&s_key[h], kEmpty, seq);
                if (old == kEmpty || old == seq) break;
                h = (h + 1) & (kFuseSet - 1);
            }
            atomicMin(&s_first[h], r);
        }
    }
    __syncthreads();
    for (uint32_t r = tid; r < m; r += kDPlanThreads) {
        const uint32_t seq = a.meta[8u * r + 1];
        if (!per_row || s_cs[s_ck[r]] != r || seq >= a.seqs) continue;
        uint32_t h = slot(seq);
        while (s_key[h] != seq) h = (h + 1) & (kFuseSet - 1);
        if (s_first[h] != r) atomicMin(&s_bad, (r << 3) | kNoFuseTwice);
    }
    __syncthreads();
    const uint32_t bad = s_bad;
    if (bad == kEmpty) return;
    if (tid == 0) {
        const uint32_t r = bad >> 3, why = bad & 7u;
        dplan_fail(a.state, kPageStNoFuse, r, per_row || why == kNoFuseSeq ? a.meta[8u * r + 1] : a.seq_fixed, why);
    }
    uint32_t* ranges = a.blob + a.ranges_off;
    for (uint32_t r = tid; r < m; r += kDPlanThreads) {
        s_lo[r] = s_hi[r] = 0;
        ranges[2u * r] = ranges[2u * r + 1] = 0;
    }
    __syncthreads();
}

__global__ __launch_bounds__(kDPlanThreads) void dplan_kernel(DPlanArgs a) {
    __shared__ uint32_t s_ck[kDPlanMaxRows];      // chunk of each row
    __shared__ uint32_t s_cs[kDPlanMaxRows + 1];  // first row of each chunk, then m
    __shared__ uint32_t s_lo[kDPlanMaxRows], s_hi[kDPlanMaxRows];
    __shared__ uint32_t s_red[kDPlanThreads / 64];
    __shared__ uint32_t s_carry;
    const uint32_t tid = threadIdx.x, m = a.m;
    const bool per_row = a.seq_fixed == THB_SEQ_PER_ROW;
    auto seq_of = [&](uint32_t r) { return per_row ? a.meta[8u * r + 1] : a.seq_fixed; };
    {
        DPlanRows ra;
        ra.meta = a.meta;
        ra.ranges_out = a.blob + a.ranges_off;
        ra.state = a.state;
        ra.npages_off = a.npages_off;
        ra.m = m;
        ra.seq_fixed = a.seq_fixed;
        ra.causal = a.causal;
        ra.window = a.window;
        ra.page_shift = a.page_shift;
        ra.seqs = a.seqs;
        ra.pos_limit = a.pos_limit;
        dplan_rows(ra, s_ck, s_cs, s_lo, s_hi, s_red, s_carry);
    }
    if (a.append) dplan_check_fused(a, s_ck, s_cs, s_lo, s_hi);

    // Groups: rows r0 .. r0 + R - 1 of a chunk (R <= 16 / G), or at G > 16 one
    // row and 16 of its query heads per group; group words as build_plan's.
    const uint32_t rg = a.G <= kCols ? kCols / a.G : 1u;
    const uint32_t hs = a.G <= kCols ? 1u : (a.G + kCols - 1) / kCols;
    auto write_group = [&](uint32_t g, const uint32_t (&w)[kGroupWords]) {
#pragma unroll
        for (uint32_t k = 0; k < kGroupWords; k++) a.blob[g * kGroupWords + k] = w[k];
        for (uint32_t p = 0; p < a.pmax; p++) {
            uint32_t* it = a.blob + a.items_off + (static_cast<size_t>(g) * a.pmax + p) * kItemWords;
#pragma unroll
            for (uint32_t k = 0; k < kGroupWords; k++) it[k] = w[k];
            it[kGroupWords] = p;
        }
        uint32_t* mg = a.blob + a.merge_off + g * kMergeWords;
        mg[0] = w[0];
        mg[1] = w[1];
        mg[2] = w[2];
        mg[3] = w[3];
        mg[4] = w[7];
        mg[5] = w[10];
        mg[6] = mg[7] = 0u;
    };
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (uint32_t t0 = 0; t0 < m; t0 += kDPlanThreads) {
        const uint32_t r = t0 + tid;
        bool head = false;
        uint32_t c1 = 0;
        if (r < m) {
            const uint32_t ck = s_ck[r];
            c1 = s_cs[ck + 1];
            head = (r - s_cs[ck]) % rg == 0;
        }
        uint32_t total = 0;
        const uint32_t incl = dplan_scan(head ? hs : 0u, s_red, &total);
        const uint32_t carry = s_carry;
        if (head) {
            const uint32_t R = min(rg, c1 - r);
            uint32_t lo = 0xFFFFFFFFu, hi = 0;
            for (uint32_t j = r; j < r + R; j++)
                if (s_hi[j] > s_lo[j]) {
                    lo = min(lo, s_lo[j]);
                    hi = max(hi, s_hi[j]);
                }
            uint32_t base, np, plen;
            dplan_partition(lo, hi, a.PL, a.align, base, np, plen);
            np = min(np, a.pmax);  // pmax covers every span the pool's sequences allow
            for (uint32_t k = 0; k < hs; k++) {
                const uint32_t g = carry + incl - hs + k;
                const uint32_t h0 = k * kCols;
                const uint32_t H = a.G <= kCols ? a.G : min(kCols, a.G - h0);
                const uint32_t w[kGroupWords] = {r, a.G <= kCols ? R : 1u, h0, H, seq_of(r), lo, hi, np, base, plen,
                                                 g * a.pmax};
                write_group(g, w);
            }
        }
        __syncthreads();
        if (tid == 0) s_carry = carry + total;
        __syncthreads();
    }
    // Slots past the call's groups: no partitions.
    for (uint32_t g = s_carry + tid; g < a.gmax; g += kDPlanThreads) {
        const uint32_t w[kGroupWords] = {0u, 1u, 0u, 1u, 0u, 0u, 0u, 0u, 0u, a.align, g * a.pmax};
        write_group(g, w);
    }
}

// ---------------------------- device-planned calls with prefill (list mode)
// A plan made by thb_dplan_create_ex(THB_DPLAN_PREFILL) is a compact work
// list instead of the slots of a fixed grid:
//  * decode items: (group, partition), a group's partitions consecutive
//    (their partial-result slots), for every group not in a prefill block;
//  * prefill blocks: a chunk of four or more groups (build_plan's rule) is
//    cut into blocks of WB consecutive groups, and a block whose keys fit
//    one partition runs on attn_prefill_wide (build_plan's block record, so
//    each row's arithmetic is thb_attn's); a block spanning several
//    partitions leaves its groups to the decode items;
//  * the launch order: every entry, longest first by the host planner's
//    cost model (a decode workgroup streams at one CU's rate; a prefill
//    block costs 10 us + 4.5 us per 64-key tile at head_dim 128), by a
//    counting sort over 1-us buckets.
// attn_list then claims entries from a counter in the plan header (the last
// workgroup out resets it), so its grid does not depend on the rows.
constexpr uint32_t kDPlanListMaxRows = 8192;
constexpr uint32_t kListHdrWords = 8;  // entries, claim counter, done counter, decode items, blocks
constexpr uint32_t kListBuckets = 256;

struct DListArgs {
    DPlanRows rows;
    uint32_t* blob;
    uint32_t G, PL, align, WB, hd_t, pmax;
    uint32_t rg_magic, wb_magic;  // div16 multipliers of the rows per group and WB
    uint32_t groups_off, items_off, bitems_off, pairs_off, order_off;
    float dec_us_per_key;  // decode cost model: microseconds per key of a partition
};

// Exclusive sums over the workgroup of C per-thread values (v in, v out),
// totals in tot.  Every thread calls it; red holds (blockDim.x / 64) * C
// words.
template <int C>
__device__ void dplan_scan_c(uint32_t (&v)[C], uint32_t* red, uint32_t (&tot)[C]) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t x[C];
#pragma unroll
    for (int c = 0; c < C; c++) x[c] = v[c];
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
#pragma unroll
        for (int c = 0; c < C; c++) {
            const uint32_t t = __shfl_up(x[c], d);
            if (lane >= d) x[c] += t;
        }
    }
    if (lane == 63) {
#pragma unroll
        for (int c = 0; c < C; c++) red[w * C + c] = x[c];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int c = 0; c < C; c++) {
            uint32_t y = lane < nw ? red[lane * C + c] : 0u;
#pragma unroll
            for (uint32_t d = 1; d < 16; d <<= 1) {
                const uint32_t t = __shfl_up(y, d);
                if (lane >= d) y += t;
            }
            if (lane < nw) red[lane * C + c] = y;
        }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < C; c++) {
        v[c] = x[c] - v[c] + (w > 0 ? red[(w - 1) * C + c] : 0u);
        tot[c] = red[(nw - 1) * C + c];
    }
    __syncthreads();
}

// The list planner.  Each thread owns kListRowsPerThread consecutive rows
// and every phase is one pass over all rows (a sum over the workgroup where
// a phase numbers what it makes), so the plan costs a few memory round
// trips and barriers whatever the row count:
//  1. positions and sequences of the rows (one batch of loads);
//  2. chunks: chunk of each row, first row of each chunk;
//  3. each row's key range (plan_rows), the page-coverage check;
//  4. each group's key range (at its first row) and partition;
//  5. prefill blocks: a block's first group takes the block's range from
//     its groups' ranges and marks them blocked when it fits one partition;
//  6. groups, decode items and blocks numbered in row order, written, and
//     counted into the launch-order histogram;
//  7. the launch order (counting sort, longest first).
constexpr uint32_t kListRowsPerThread = kDPlanListMaxRows / kDPlanThreads;
constexpr uint32_t kListMaxWB = 16;  // groups per prefill block the list planner takes
// s_np word of a row: kRowHead at a group's first row, with the group's
// partition count; for a group of a prefill block kRowBlocked instead of
// the count, and at the block's first group also kRowBlockHead and the
// block's group count.
constexpr uint16_t kRowBlocked = 0x8000u;
constexpr uint16_t kRowBlockHead = 0x4000u;
constexpr uint16_t kRowHead = 0x2000u;
constexpr uint16_t kRowCount = 0x1FFFu;
static_assert(kMaxParts <= kRowCount && kListMaxWB <= kRowCount, "row word fields");

// x / d for x < 2^16 and 1 <= d < 2^16, with mg = floor(2^32 / d) + 1 (0 for
// d = 1): mg = (2^32 + e) / d with 0 < e <= d, so x mg / 2^32 exceeds x / d
// by less than x / 2^32 < 1 / d, which never crosses the next integer.
__device__ inline uint32_t div16(uint32_t x, uint32_t d, uint32_t mg) { return d == 1 ? x : __umulhi(x, mg); }
inline uint32_t div16_magic(uint32_t d) { return d <= 1 ? 0u : static_cast<uint32_t>((1ull << 32) / d + 1); }

// part_split of the list planner: 32-bit arithmetic below 2^31 keys, the
// 64-bit form (one out-of-line copy) from there.
__device__ __noinline__ uint64_t dplan_split_wide(uint32_t span, uint32_t PL, uint32_t align) {
    uint32_t n_parts, plen;
    part_split(span, PL, align, n_parts, plen);
    return (uint64_t(n_parts) << 32) | plen;
}
__device__ inline void dplan_split(uint32_t span, uint32_t PL, uint32_t align, uint32_t& n_parts, uint32_t& plen) {
    if (span < 0x80000000u) {
        part_split32(span, PL, align, n_parts, plen);
    } else {
        const uint64_t np = dplan_split_wide(span, PL, align);
        n_parts = static_cast<uint32_t>(np >> 32);
        plen = static_cast<uint32_t>(np);
    }
}

__global__ __launch_bounds__(kDPlanThreads) void dplan_list_kernel(DListArgs a) {
    constexpr uint32_t K = kListRowsPerThread, T = kDPlanThreads;
    __shared__ uint32_t s_lo[kDPlanListMaxRows], s_hi[kDPlanListMaxRows];
    __shared__ uint32_t s_seq[kDPlanListMaxRows];
    __shared__ uint16_t s_ck[kDPlanListMaxRows];      // chunk of each row
    __shared__ uint16_t s_cs[kDPlanListMaxRows + 1];  // first row of each chunk, then m
    __shared__ uint16_t s_np[kDPlanListMaxRows];      // row word
    __shared__ uint32_t s_red[(kDPlanThreads / 64) * 3];
    __shared__ uint32_t s_hist[kListBuckets];
    const uint32_t tid = threadIdx.x, m = a.rows.m, r0 = tid * K;  // rows r0 .. r0 + K - 1: numbering phases
    const bool per_row = a.rows.seq_fixed == THB_SEQ_PER_ROW;
    const uint32_t rg = a.G <= kCols ? kCols / a.G : 1u;
    const uint32_t hs = a.G <= kCols ? 1u : (a.G + kCols - 1) / kCols;
    const uint32_t amask = ~(a.align - 1);

    // 1. positions and sequences (rows tid + k T: coalesced)
#pragma unroll
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t r = tid + k * T;
        if (r < m) {
            uint32_t pos, sq = a.rows.seq_fixed;
            if (per_row) {
                const uint2 ps = *reinterpret_cast<const uint2*>(a.rows.meta + 8u * r);
                pos = ps.x;
                sq = ps.y;
            } else {
                pos = a.rows.meta[8u * r];
            }
            s_lo[r] = pos;
            s_seq[r] = sq;
            s_np[r] = 0;
        }
    }
    for (uint32_t i = tid; i < kListBuckets; i += T) s_hist[i] = 0;
    __syncthreads();

    // 2. chunks: maximal runs of rows of one sequence
    auto is_start = [&](uint32_t r) { return r < m && (r == 0 || (per_row && s_seq[r] != s_seq[r - 1])); };
    uint32_t nst[1] = {0}, nck[1];
#pragma unroll
    for (uint32_t k = 0; k < K; k++) nst[0] += is_start(r0 + k) ? 1u : 0u;
    dplan_scan_c<1>(nst, s_red, nck);
    {
        uint32_t ck = nst[0];
#pragma unroll
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t r = r0 + k;
            if (r < m) {
                if (is_start(r)) s_cs[ck++] = static_cast<uint16_t>(r);
                s_ck[r] = static_cast<uint16_t>(ck - 1);
            }
        }
    }
    if (tid == 0) s_cs[nck[0]] = static_cast<uint16_t>(m);
    __syncthreads();

    // 3. key range of each row (plan_rows), pages covering it (rows tid + k T)
    {
        uint32_t lo[K], hi[K], np_seq[K];
        const uint32_t* npages = a.rows.state + a.rows.npages_off;
#pragma unroll
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t r = tid + k * T;
            lo[k] = hi[k] = np_seq[k] = 0;
            if (r >= m) continue;
            const uint32_t ck = s_ck[r], c0 = s_cs[ck], c1 = s_cs[ck + 1];
            const uint32_t n = c1 - c0, i = r - c0, pos = s_lo[r];
            const uint32_t blk_last = min((i / 8u) * 8u + 8u, n);
            const uint64_t kv_len = a.rows.causal ? uint64_t(s_lo[c0 + blk_last - 1]) + 1 : uint64_t(s_lo[c1 - 1]) + 1;
            uint64_t ws = 0;
            if (a.rows.causal && a.rows.window != 0 && uint64_t(pos) + 1 > a.rows.window)
                ws = uint64_t(pos) + 1 - a.rows.window;
            uint64_t h = kv_len;
            if (a.rows.causal && uint64_t(pos) + 1 < h) h = uint64_t(pos) + 1;
            lo[k] = static_cast<uint32_t>(ws);
            hi[k] = static_cast<uint32_t>(min(h, uint64_t(0xFFFFFFFFu)));
            if (a.rows.pos_limit != 0 && pos >= a.rows.pos_limit) {
                dplan_fail(a.rows.state, kPageStPosLimit, pos, a.rows.pos_limit, 0u);
                lo[k] = hi[k] = 0;
            }
            const uint32_t sq = s_seq[r];
            if (hi[k] > lo[k] && sq < a.rows.seqs) np_seq[k] = npages[sq];
        }
#pragma unroll
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t r = tid + k * T;
            if (r >= m || hi[k] <= lo[k]) continue;
            const uint32_t sq = s_seq[r];
            if (sq >= a.rows.seqs) {
                dplan_fail(a.rows.state, kPageStBadSeq, sq, a.rows.seqs, 0u);
                lo[k] = hi[k] = 0;
            } else if ((uint64_t(np_seq[k]) << a.rows.page_shift) < hi[k]) {
                dplan_fail(a.rows.state, kPageStCover, sq, np_seq[k] << a.rows.page_shift, hi[k]);
                lo[k] = hi[k] = 0;
            }
        }
        __syncthreads();  // every position read
#pragma unroll
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t r = tid + k * T;
            if (r < m) {
                s_lo[r] = lo[k];
                s_hi[r] = hi[k];
                a.rows.ranges_out[2u * r] = lo[k];  // the ranges may start at an odd word
                a.rows.ranges_out[2u * r + 1] = hi[k];
            }
        }
    }
    __syncthreads();

    // 4. groups (rows r .. r + R - 1 of a chunk, R <= rg): key range at the
    // group's first row (0xFFFFFFFF / 0 when empty) and partition count.
    // Phases 4 to 7 take each thread's consecutive rows, so that the lanes
    // of a wave meet group and block starts together.
#pragma unroll 1
    for (uint32_t r = r0; r < min(m, r0 + K); r++) {
        const uint32_t ck = s_ck[r], c0 = s_cs[ck], c1 = s_cs[ck + 1];
        const uint32_t i = r - c0;
        if (i != div16(i, rg, a.rg_magic) * rg) continue;
        const uint32_t R = min(rg, c1 - r);
        uint32_t glo = 0xFFFFFFFFu, ghi = 0;
#pragma unroll 4
        for (uint32_t j = r; j < r + R; j++) {
            const uint32_t l = s_lo[j], h = s_hi[j];
            if (h > l) {
                glo = min(glo, l);
                ghi = max(ghi, h);
            }
        }
        uint32_t np = 1, plen;
        if (ghi > glo && glo != 0xFFFFFFFFu) dplan_split(ghi - (glo & amask), a.PL, a.align, np, plen);
        s_lo[r] = glo;  // the group's rows r + 1 .. are no other group's
        s_hi[r] = ghi;
        s_np[r] = kRowHead | static_cast<uint16_t>(min(np, a.pmax));  // pmax covers every span of the pool
    }
    __syncthreads();

    // 5. prefill blocks: WB consecutive groups of a chunk of >= 4 groups
    // (build_plan's rule), run on the prefill kernel when their keys fit
    // one partition.  The block's range over its groups' ranges.
    auto block_range = [&](uint32_t r, uint32_t bng, uint32_t& blo, uint32_t& bhi) {
        blo = 0xFFFFFFFFu;
        bhi = 0;
#pragma unroll 4
        for (uint32_t j = 0; j < bng; j++) {
            blo = min(blo, s_lo[r + j * rg]);
            bhi = max(bhi, s_hi[r + j * rg]);
        }
    };
    const bool blocks = a.WB != 0 && hs == 1;
    if (blocks) {
#pragma unroll 1
        for (uint32_t r = r0; r < min(m, r0 + K); r++) {
            if (!(s_np[r] & kRowHead)) continue;
            const uint32_t ck = s_ck[r], c0 = s_cs[ck], c1 = s_cs[ck + 1];
            const uint32_t idx = div16(r - c0, rg, a.rg_magic);
            if (div16(c1 - c0 + rg - 1, rg, a.rg_magic) < 4 || idx != div16(idx, a.WB, a.wb_magic) * a.WB) continue;
            const uint32_t bng = div16(min(c1, r + a.WB * rg) - r + rg - 1, rg, a.rg_magic);
            uint32_t blo, bhi, bnp = 1, bplen;
            block_range(r, bng, blo, bhi);
            if (bhi > blo && blo != 0xFFFFFFFFu) dplan_split(bhi - (blo & amask), a.PL, a.align, bnp, bplen);
            if (bnp == 1) {
                for (uint32_t j = 1; j < bng; j++) s_np[r + j * rg] = kRowHead | kRowBlocked;
                s_np[r] = kRowHead | kRowBlocked | kRowBlockHead | static_cast<uint16_t>(bng);
            }
        }
    }
    __syncthreads();

    // 6. number the groups, items and blocks in row order; write them
    uint32_t cnt[3] = {0, 0, 0}, tot[3];  // groups, decode items, blocks
#pragma unroll
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t w = r0 + k < m ? s_np[r0 + k] : 0u;
        if (!(w & kRowHead)) continue;
        cnt[0] += hs;
        cnt[1] += (w & kRowBlocked) ? 0u : (w & kRowCount) * hs;
        cnt[2] += (w & kRowBlockHead) ? 1u : 0u;
    }
    dplan_scan_c<3>(cnt, s_red, tot);
    const uint32_t n_items = tot[1], n_blocks = tot[2], n_entries = n_items + n_blocks;
    uint32_t* groups = a.blob + a.groups_off;
    uint32_t* items = a.blob + a.items_off;
    uint32_t* bitems = a.blob + a.bitems_off;
    uint32_t* pairs = a.blob + a.pairs_off;
    // launch-order bucket of an entry: kListBuckets - 1 - estimated us
    auto bucket = [&](float us) -> uint32_t {
        return kListBuckets - 1 - static_cast<uint32_t>(min(us, static_cast<float>(kListBuckets - 1)));
    };
    auto item_bucket = [&](uint32_t base, uint32_t plen, uint32_t ghi, uint32_t p) -> uint32_t {
        const uint64_t p0 = uint64_t(base) + uint64_t(p) * plen;
        const uint64_t keys = ghi > p0 ? min(uint64_t(plen), uint64_t(ghi) - p0) : 0;
        return bucket(static_cast<float>(keys) * a.dec_us_per_key);
    };
    auto block_bucket = [&](uint32_t blo, uint32_t bhi) -> uint32_t {
        const uint32_t tb0 = blo & ~31u, tiles = bhi > tb0 ? (bhi - tb0 + 63u) / 64u : 0u;
        return bucket(10.0f + 4.5f * static_cast<float>(tiles) * static_cast<float>(a.hd_t) / 128.0f);
    };
    // a group (or block): lo, hi (0, 0 when empty), base, plen
    auto span_of = [&](uint32_t& lo, uint32_t& hi, uint32_t& base, uint32_t& plen) {
        base = 0;
        plen = a.align;
        if (hi <= lo || lo == 0xFFFFFFFFu) {
            lo = hi = 0;
        } else {
            uint32_t np;
            base = lo & amask;
            dplan_split(hi - base, a.PL, a.align, np, plen);
        }
    };
    {
        uint32_t gi = cnt[0], ii = cnt[1], bi = cnt[2];
#pragma unroll 1
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t r = r0 + k;
            const uint32_t rw = r < m ? s_np[r] : 0u;
            if (!(rw & kRowHead)) continue;
            const uint32_t dn = (rw & kRowBlocked) ? 0u : (rw & kRowCount);
            const uint32_t R = min(rg, static_cast<uint32_t>(s_cs[s_ck[r] + 1]) - r);
            const uint32_t sq = s_seq[r];
            uint32_t glo = s_lo[r], ghi = s_hi[r], base, plen;
            span_of(glo, ghi, base, plen);
            for (uint32_t sub = 0; sub < hs; sub++) {
                const uint32_t g = gi++;
                const uint32_t h0 = sub * kCols;
                const uint32_t H = a.G <= kCols ? a.G : min(kCols, a.G - h0);
                const uint32_t w[kGroupWords] = {r, a.G <= kCols ? R : 1u, h0, H, sq, glo, ghi, dn, base, plen, ii};
#pragma unroll
                for (uint32_t q = 0; q < kGroupWords; q++) groups[g * kGroupWords + q] = w[q];
                for (uint32_t p = 0; p < dn; p++) {
                    uint32_t* it = items + static_cast<size_t>(ii + p) * kItemWords;
#pragma unroll
                    for (uint32_t q = 0; q < kGroupWords; q++) it[q] = w[q];
                    it[kGroupWords] = p;
                    atomicAdd(&s_hist[item_bucket(base, plen, ghi, p)], 1u);
                }
                ii += dn;
            }
            if (rw & kRowBlockHead) {
                const uint32_t bng = rw & kRowCount;
                uint32_t blo, bhi, bbase, bplen;
                block_range(r, bng, blo, bhi);
                span_of(blo, bhi, bbase, bplen);
                const uint32_t b = bi++;
                const uint32_t bw[kBItemWords] = {gi - 1, bng, sq, blo, bhi, 1u, bbase, bplen, b, 0u};
#pragma unroll
                for (uint32_t q = 0; q < kBItemWords; q++) bitems[b * kBItemWords + q] = bw[q];
                pairs[2 * b] = b;
                pairs[2 * b + 1] = kNoItem;
                atomicAdd(&s_hist[block_bucket(blo, bhi)], 1u);
            }
        }
    }
    __syncthreads();

    // 7. launch order: every entry, longest first (counting sort)
    if (tid < 64) {  // exclusive sums of the histogram, four buckets per lane
        uint32_t v[4], sum = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = s_hist[4 * tid + k];
            sum += v[k];
        }
        uint32_t incl = sum;
#pragma unroll
        for (uint32_t d = 1; d < 64; d <<= 1) {
            const uint32_t t = __shfl_up(incl, d);
            if (tid >= d) incl += t;
        }
        uint32_t run = incl - sum;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s_hist[4 * tid + k] = run;
            run += v[k];
        }
    }
    __syncthreads();
    uint32_t* order = a.blob + a.order_off;
    {
        uint32_t ii = cnt[1], bi = cnt[2];
#pragma unroll 1
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t r = r0 + k;
            const uint32_t rw = r < m ? s_np[r] : 0u;
            if (!(rw & kRowHead)) continue;
            if (rw & kRowBlockHead) {
                uint32_t blo, bhi, bbase, bplen;
                block_range(r, rw & kRowCount, blo, bhi);
                span_of(blo, bhi, bbase, bplen);
                order[atomicAdd(&s_hist[block_bucket(blo, bhi)], 1u)] = 0x80000000u | bi++;
            }
            if (rw & kRowBlocked) continue;
            uint32_t glo = s_lo[r], ghi = s_hi[r], base, plen;
            span_of(glo, ghi, base, plen);
            for (uint32_t sub = 0; sub < hs; sub++)
                for (uint32_t p = 0; p < (rw & kRowCount); p++)
                    order[atomicAdd(&s_hist[item_bucket(base, plen, ghi, p)], 1u)] = ii++;
        }
    }
    if (tid == 0) {
        a.blob[0] = n_entries;
        a.blob[1] = 0u;  // claim counter
        a.blob[2] = 0u;  // workgroups done
        a.blob[3] = n_items;
        a.blob[4] = n_blocks;
    }
}

// ------------------------------------------------------------ host side
uint32_t template_hd(uint32_t hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : hd <= 256 ? 256 : 512; }


template <int HD, bool F16>
void launch_hd(dim3 grid, const AttnArgs& a, hipStream_t s) {
    constexpr int W = decode_waves(HD);
    if (a.full)
        hipLaunchKernelGGL((attn_mfma<HD, F16, W, ring_for(HD), true>), grid, dim3(64 * W), 0, s, a);
    else
        hipLaunchKernelGGL((attn_mfma<HD, F16, W, ring_for(HD), false>), grid, dim3(64 * W), 0, s, a);
}

void launch(uint32_t hd_t, bool f16, dim3 grid, const AttnArgs& a, hipStream_t s) {
    switch (hd_t) {
        case 64: f16 ? launch_hd<64, true>(grid, a, s) : launch_hd<64, false>(grid, a, s); break;
        case 128: f16 ? launch_hd<128, true>(grid, a, s) : launch_hd<128, false>(grid, a, s); break;
        case 256: f16 ? launch_hd<256, true>(grid, a, s) : launch_hd<256, false>(grid, a, s); break;
        default: f16 ? launch_hd<512, true>(grid, a, s) : launch_hd<512, false>(grid, a, s); break;
    }
}

// Waves of attn_prefill_wide (head_dim <= 256).
#ifndef THB_PREFILL_WAVES
#define THB_PREFILL_WAVES 8
#endif
// Query groups per prefill block: prefill_ncg per wave of attn_prefill_wide,
// 1 per wave of attn_prefill (head_dim 512).
constexpr uint32_t block_groups(bool wide, uint32_t hd_t) {
    return wide ? static_cast<uint32_t>(prefill_ncg(static_cast<int>(hd_t))) * THB_PREFILL_WAVES
                : static_cast<uint32_t>(waves_for(static_cast<int>(hd_t)));
}

// Score scale applied to the query (log2 units, or 1 / softcap).
float q_scale(const thb_attn_spec& sp) {
    return sp.softcap > 0.0f ? sp.scale / sp.softcap : sp.scale * 1.4426950408889634f;
}

// attn_prefill_wide serves head_dim <= 256; attn_prefill head_dim 512.
bool prefill_wide(uint32_t hd_t) { return hd_t <= 256; }

// An f16 query read as it is (the lean kernels: no rotation, no norm)
// against f16 keys: its low half after the split is exactly zero, and the
// lean prefill kernel skips those products.
bool query_exact(const AttnArgs& a, bool f16_kv) { return f16_kv && !a.full && a.q_dt == THB_DT_F16; }

template <int HD, bool F16>
void launch_prefill_hd(dim3 grid, const AttnArgs& a, hipStream_t s) {
    if constexpr (HD <= 256) {
        constexpr int W = THB_PREFILL_WAVES;
        const bool cap = a.cap2 != 0.0f;
        if (a.full && cap)
            hipLaunchKernelGGL((attn_prefill_wide<HD, F16, W, true, true>), grid, dim3(64 * W), 0, s, a);
        else if (a.full)
            hipLaunchKernelGGL((attn_prefill_wide<HD, F16, W, true, false>), grid, dim3(64 * W), 0, s, a);
        else if (cap)
            hipLaunchKernelGGL((attn_prefill_wide<HD, F16, W, false, true>), grid, dim3(64 * W), 0, s, a);
        else if (query_exact(a, F16))
            hipLaunchKernelGGL((attn_prefill_wide<HD, true, W, false, false, false>), grid, dim3(64 * W), 0, s, a);
        else
            hipLaunchKernelGGL((attn_prefill_wide<HD, F16, W, false, false>), grid, dim3(64 * W), 0, s, a);
    } else {
        constexpr int W = waves_for(HD);  // one group per wave: block_groups(false, HD)
        if (a.full)
            hipLaunchKernelGGL((attn_prefill<HD, F16, W, true>), grid, dim3(64 * W), 0, s, a);
        else
            hipLaunchKernelGGL((attn_prefill<HD, F16, W, false>), grid, dim3(64 * W), 0, s, a);
    }
}

void launch_prefill(uint32_t hd_t, bool f16, dim3 grid, const AttnArgs& a, hipStream_t s) {
    switch (hd_t) {
        case 64: f16 ? launch_prefill_hd<64, true>(grid, a, s) : launch_prefill_hd<64, false>(grid, a, s); break;
        case 128: f16 ? launch_prefill_hd<128, true>(grid, a, s) : launch_prefill_hd<128, false>(grid, a, s); break;
        case 256: f16 ? launch_prefill_hd<256, true>(grid, a, s) : launch_prefill_hd<256, false>(grid, a, s); break;
        default: f16 ? launch_prefill_hd<512, true>(grid, a, s) : launch_prefill_hd<512, false>(grid, a, s); break;
    }
}

template <int HD, bool F16>
void launch_mixed_hd(dim3 grid, const AttnArgs& a, hipStream_t s) {
    constexpr int W = THB_PREFILL_WAVES;
    static_assert(HD > 128 || THB_ATTN_WAVES != THB_PREFILL_WAVES || W == waves_for(HD), "mixed launch waves");
    const bool cap = a.cap2 != 0.0f;
    if (a.full && cap)
        hipLaunchKernelGGL((attn_mixed<HD, F16, W, true, true>), grid, dim3(64 * W), 0, s, a);
    else if (a.full)
        hipLaunchKernelGGL((attn_mixed<HD, F16, W, true, false>), grid, dim3(64 * W), 0, s, a);
    else if (cap)
        hipLaunchKernelGGL((attn_mixed<HD, F16, W, false, true>), grid, dim3(64 * W), 0, s, a);
    else if (query_exact(a, F16))
        hipLaunchKernelGGL((attn_mixed<HD, true, W, false, false, false>), grid, dim3(64 * W), 0, s, a);
    else
        hipLaunchKernelGGL((attn_mixed<HD, F16, W, false, false>), grid, dim3(64 * W), 0, s, a);
}

// Mixed launches exist at head_dim <= 128 (where attn_prefill_wide runs).
void launch_mixed(uint32_t hd_t, bool f16, dim3 grid, const AttnArgs& a, hipStream_t s) {
    if (hd_t == 64)
        f16 ? launch_mixed_hd<64, true>(grid, a, s) : launch_mixed_hd<64, false>(grid, a, s);
    else
        f16 ? launch_mixed_hd<128, true>(grid, a, s) : launch_mixed_hd<128, false>(grid, a, s);
}

template <int HD, bool F16>
void launch_list_hd(dim3 grid, const AttnArgs& a, hipStream_t s) {
    constexpr int W = THB_PREFILL_WAVES;
    static_assert(decode_waves(HD) == W, "list launch waves");
    const bool cap = a.cap2 != 0.0f;
    if (a.full && cap)
        hipLaunchKernelGGL((attn_list<HD, F16, W, true, true>), grid, dim3(64 * W), 0, s, a);
    else if (a.full)
        hipLaunchKernelGGL((attn_list<HD, F16, W, true, false>), grid, dim3(64 * W), 0, s, a);
    else if (cap)
        hipLaunchKernelGGL((attn_list<HD, F16, W, false, true>), grid, dim3(64 * W), 0, s, a);
    else if (query_exact(a, F16))
        hipLaunchKernelGGL((attn_list<HD, true, W, false, false, false>), grid, dim3(64 * W), 0, s, a);
    else
        hipLaunchKernelGGL((attn_list<HD, F16, W, false, false>), grid, dim3(64 * W), 0, s, a);
}

// List-mode device plans exist at head_dim <= 256 (attn_prefill_wide).
void launch_list(uint32_t hd_t, bool f16, dim3 grid, const AttnArgs& a, hipStream_t s) {
    if (hd_t == 64)
        f16 ? launch_list_hd<64, true>(grid, a, s) : launch_list_hd<64, false>(grid, a, s);
    else if (hd_t == 128)
        f16 ? launch_list_hd<128, true>(grid, a, s) : launch_list_hd<128, false>(grid, a, s);
    else
        f16 ? launch_list_hd<256, true>(grid, a, s) : launch_list_hd<256, false>(grid, a, s);
}

template <int HD>
void launch_merge_hd(dim3 grid, const AttnArgs& a, hipStream_t s) {
    if (a.full)
        hipLaunchKernelGGL((attn_merge<HD, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((attn_merge<HD, false>), grid, dim3(256), 0, s, a);
}

void launch_merge(uint32_t hd_t, dim3 grid, const AttnArgs& a, hipStream_t s) {
    switch (hd_t) {
        case 64: launch_merge_hd<64>(grid, a, s); break;
        case 128: launch_merge_hd<128>(grid, a, s); break;
        case 256: launch_merge_hd<256>(grid, a, s); break;
        default: launch_merge_hd<512>(grid, a, s); break;
    }
}

// Per-row key ranges (attn.wgsl:78-88,169).  A chunk is the whole call when
// the sequence is fixed (reference mode, one dispatch per sequence chunk,
// forward.rs:316-336), else each maximal run of rows with equal seq.
struct RowPlan {
    std::vector<uint32_t> lo, hi, seq;
    std::vector<std::pair<uint32_t, uint32_t>> chunks;  // [start, end)
};

RowPlan plan_rows(const uint32_t* args, uint32_t m, uint32_t seq_fixed, bool causal, uint32_t window) {
    RowPlan rp;
    rp.lo.resize(m);
    rp.hi.resize(m);
    rp.seq.resize(m);
    uint32_t start = 0;
    while (start < m) {
        const uint32_t seq = seq_fixed != THB_SEQ_PER_ROW ? seq_fixed : args[8 * start + 1];
        uint32_t end = start + 1;
        if (seq_fixed == THB_SEQ_PER_ROW)
            while (end < m && args[8 * end + 1] == seq) end++;
        else
            end = m;
        const uint32_t n = end - start;
        for (uint32_t i = 0; i < n; i++) {
            const uint32_t r = start + i;
            const uint32_t pos = args[8 * r];
            const uint32_t blk_last = std::min((i / 8) * 8 + 8, n);
            const uint64_t kv_len = causal ? uint64_t(args[8 * (start + blk_last - 1)]) + 1
                                           : uint64_t(args[8 * (end - 1)]) + 1;
            uint64_t ws = 0;
            if (causal && window != 0 && uint64_t(pos) + 1 > window) ws = uint64_t(pos) + 1 - window;
            uint64_t h = kv_len;
            if (causal && uint64_t(pos) + 1 < h) h = uint64_t(pos) + 1;
            rp.lo[r] = static_cast<uint32_t>(ws);
            rp.hi[r] = static_cast<uint32_t>(std::min<uint64_t>(h, 0xFFFFFFFFull));
            rp.seq[r] = seq;
        }
        rp.chunks.push_back({start, end});
        start = end;
    }
    return rp;
}

int build_plan(thb_pool* pool, const thb_rows* rows, const thb_attn_spec& sp, uint32_t hd, AttnPlan& plan) {
    const Arena& arena = pool->arena.a;
    const uint32_t m = sp.m;
    const uint32_t* args = rows->host.data() + 8 * static_cast<size_t>(sp.row_off);
    const uint32_t G = sp.q_heads / pool->kv_heads;
    RowPlan rp = plan_rows(args, m, sp.seq, sp.causal != 0, sp.window);

    // Pages must cover every key a row reads.
    for (uint32_t r = 0; r < m; r++) {
        if (rp.hi[r] <= rp.lo[r]) continue;
        const uint32_t seq = rp.seq[r];
        if (seq >= arena.seqs())
            return fail(THB_ERR_INVALID, "row " + std::to_string(r) + ": sequence " + std::to_string(seq) +
                                             " out of range (" + std::to_string(arena.seqs()) + " sequences)");
        if (!arena.covers(seq, rp.hi[r]))
            return fail(THB_ERR_MODEL, "pages must cover the chunk: sequence " + std::to_string(seq) + " holds " +
                                           std::to_string(arena.table_of(seq).size() * arena.page_len()) +
                                           " slots, row " + std::to_string(r) + " reads " +
                                           std::to_string(rp.hi[r]));
    }

    // Partitions of a group (or of a prefill block) start at its first key
    // (rounded down to the page and tile size) and split its span into
    // n equal parts (part_split: n = ceil(span / part_len) rounded up to a
    // power of two, then lowered if the aligned part length leaves trailing
    // parts empty): a function of its own key range only.
    std::vector<uint32_t> groups, items, blocks, bitems;
    const uint32_t PL = pool->part_len;
    const uint32_t align = std::max<uint32_t>(pool->page_len, 16);
    const uint32_t hd_t = template_hd(hd);
    const bool wide = prefill_wide(hd_t);
    const uint32_t WB = block_groups(wide, hd_t);  // query groups per prefill block
    uint32_t max_parts = 0;
    uint64_t max_span = 0;
    bool any_split = false;
    auto partition = [&](uint32_t& lo, uint32_t& hi, uint32_t& base, uint32_t& n_parts, uint32_t& plen) {
        base = 0;
        n_parts = 1;
        plen = align;
        if (hi <= lo || lo == 0xFFFFFFFFu) {
            lo = hi = 0;  // no keys: one empty partition, output 0/0 = NaN
        } else {
            base = lo & ~(align - 1);
            const uint64_t span = uint64_t(hi) - base;
            max_span = std::max(max_span, span);
            part_split(span, PL, align, n_parts, plen);
        }
        max_parts = std::max(max_parts, n_parts);
        any_split = any_split || n_parts > 1;
    };
    auto add_group = [&](uint32_t r0, uint32_t R, uint32_t h0, uint32_t H, uint32_t seq) {
        uint32_t lo = 0xFFFFFFFFu, hi = 0;
        for (uint32_t r = r0; r < r0 + R; r++) {
            if (rp.hi[r] <= rp.lo[r]) continue;
            lo = std::min(lo, rp.lo[r]);
            hi = std::max(hi, rp.hi[r]);
        }
        uint32_t base, n_parts, plen;
        partition(lo, hi, base, n_parts, plen);
        groups.insert(groups.end(), {r0, R, h0, H, seq, lo, hi, n_parts, base, plen, 0u});
    };
    // A chunk that needs at least 4 groups (a prefill chunk) is cut into
    // blocks of WB consecutive groups for attn_prefill; the others go to the
    // decode kernel.
    std::vector<uint8_t> in_block;
    for (auto& c : rp.chunks) {
        const uint32_t seq = rp.seq[c.first];
        const uint32_t first = static_cast<uint32_t>(groups.size() / kGroupWords);
        if (G <= kCols) {
            const uint32_t rg = kCols / G;
            for (uint32_t r = c.first; r < c.second; r += rg) add_group(r, std::min(rg, c.second - r), 0, G, seq);
        } else {
            for (uint32_t r = c.first; r < c.second; r++)
                for (uint32_t h0 = 0; h0 < G; h0 += kCols) add_group(r, 1, h0, std::min(kCols, G - h0), seq);
        }
        const uint32_t ncg = static_cast<uint32_t>(groups.size() / kGroupWords) - first;
        in_block.resize(first + ncg, 0);
        if (G > kCols || ncg < 4) continue;
        for (uint32_t b = 0; b < ncg; b += WB) {
            const uint32_t g0 = first + b, ng = std::min(WB, ncg - b);
            uint32_t lo = 0xFFFFFFFFu, hi = 0;
            for (uint32_t g = g0; g < g0 + ng; g++) {
                const uint32_t* gr = &groups[static_cast<size_t>(g) * kGroupWords];
                in_block[g] = 1;
                if (gr[6] <= gr[5]) continue;
                lo = std::min(lo, gr[5]);
                hi = std::max(hi, gr[6]);
            }
            uint32_t base, n_parts, plen;
            partition(lo, hi, base, n_parts, plen);
            for (uint32_t g = g0; g < g0 + ng; g++) {  // members share the block's partitions
                uint32_t* gr = &groups[static_cast<size_t>(g) * kGroupWords];
                gr[7] = n_parts;
                gr[8] = base;
                gr[9] = plen;
            }
            blocks.insert(blocks.end(), {g0, ng, seq, lo, hi, n_parts, base, plen, 0u});
        }
    }
    if (max_parts > kMaxParts)
        return fail(THB_ERR_CONFIG, "key span of " + std::to_string(max_span) + " tokens exceeds " + std::to_string(kMaxParts) + " partitions of " +
                                        std::to_string(PL) + " tokens");
    const uint32_t n_groups = static_cast<uint32_t>(groups.size() / kGroupWords);
    const uint32_t n_blocks = static_cast<uint32_t>(blocks.size() / kBlockWords);
    // Work items, longest partitions first, so that the short ones fill in
    // behind them (the order does not change any row's arithmetic).  Decode
    // items come first in the partial-result slots, then block members.
    auto work = [](const uint32_t* r, uint32_t lo_i, uint32_t hi_i, uint32_t base_i, uint32_t plen_i) {
        return std::min(r[plen_i], r[hi_i] - r[base_i]);
    };
    std::vector<uint32_t> order;
    for (uint32_t g = 0; g < n_groups; g++)
        if (!in_block[g]) order.push_back(g);
    std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
        return work(&groups[static_cast<size_t>(x) * kGroupWords], 5, 6, 8, 9) >
               work(&groups[static_cast<size_t>(y) * kGroupWords], 5, 6, 8, 9);
    });
    for (uint32_t g : order) {
        groups[static_cast<size_t>(g) * kGroupWords + 10] = static_cast<uint32_t>(items.size());
        for (uint32_t i = 0; i < groups[static_cast<size_t>(g) * kGroupWords + 7]; i++) items.push_back(g);
    }
    const uint32_t n_items = static_cast<uint32_t>(items.size());
    uint32_t n_slots = n_items;
    for (uint32_t g = 0; g < n_groups; g++)
        if (in_block[g]) {
            groups[static_cast<size_t>(g) * kGroupWords + 10] = n_slots;
            n_slots += groups[static_cast<size_t>(g) * kGroupWords + 7];
        }
    std::vector<uint32_t> border(n_blocks);
    for (uint32_t b = 0; b < n_blocks; b++) border[b] = b;
    std::stable_sort(border.begin(), border.end(), [&](uint32_t x, uint32_t y) {
        return work(&blocks[static_cast<size_t>(x) * kBlockWords], 3, 4, 6, 7) >
               work(&blocks[static_cast<size_t>(y) * kBlockWords], 3, 4, 6, 7);
    });
    for (uint32_t b : border) {
        blocks[static_cast<size_t>(b) * kBlockWords + 8] = static_cast<uint32_t>(bitems.size());
        for (uint32_t i = 0; i < blocks[static_cast<size_t>(b) * kBlockWords + 5]; i++) bitems.push_back(b);
    }
    const uint32_t n_bitems = static_cast<uint32_t>(bitems.size());
    if (n_items > 0x7FFFFFFFu || n_groups > 0x7FFFFFFFu) return fail(THB_ERR_CONFIG, "attention call too large");
    // attn_prefill_wide runs pairs of work items: among the items of one
    // sequence whose partitions start at the same key (one page list serves
    // both), the k-th longest with the k-th shortest, so that each pair holds
    // about the same number of tiles; pairs are launched longest first.  Work
    // per item: its tiles.
    std::vector<uint32_t> bpairs;
    auto bitem_tiles = [&](uint32_t i) {
        const uint32_t* bk = &blocks[static_cast<size_t>(bitems[i]) * kBlockWords];
        const uint64_t p0 = uint64_t(bk[6]) + uint64_t(i - bk[8]) * bk[7];
        const uint64_t tb = std::max<uint64_t>(bk[3], p0), te = std::min<uint64_t>(bk[4], p0 + bk[7]);
        return te > (tb & ~uint64_t(31)) ? (te - (tb & ~uint64_t(31)) + 63) / 64 : uint64_t(0);
    };
    if (wide) {
        // (seq, first key of the item's partition) -> items
        std::map<std::array<uint32_t, 2>, std::vector<uint32_t>> same;
        for (uint32_t i = 0; i < n_bitems; i++) {
            const uint32_t* bk = &blocks[static_cast<size_t>(bitems[i]) * kBlockWords];
            same[{bk[2], bk[6] + (i - bk[8]) * bk[7]}].push_back(i);
        }
        std::vector<std::pair<uint64_t, std::array<uint32_t, 2>>> prs;
        for (auto& kv : same) {
            auto& v = kv.second;
            std::stable_sort(v.begin(), v.end(), [&](uint32_t x, uint32_t y) { return bitem_tiles(x) > bitem_tiles(y); });
            for (size_t k = 0, n = v.size(); k < (n + 1) / 2; k++) {
                const bool solo = 2 * k + 1 == n;
                const uint32_t x = v[k], y = solo ? kNoItem : v[n - 1 - k];
                prs.push_back({bitem_tiles(x) + (solo ? 0 : bitem_tiles(y)), {x, y}});
            }
        }
        std::stable_sort(prs.begin(), prs.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
        for (auto& pp : prs) bpairs.insert(bpairs.end(), {pp.second[0], pp.second[1]});
    }
    const uint32_t n_bpairs = static_cast<uint32_t>(bpairs.size() / 2);

    std::vector<uint32_t> blob;
    blob.reserve(groups.size() + n_items * kItemWords + 2 * m + n_bitems * kBItemWords);
    blob.insert(blob.end(), groups.begin(), groups.end());
    for (uint32_t i = 0; i < n_items; i++) {  // group words + partition index
        const uint32_t* gr = &groups[static_cast<size_t>(items[i]) * kGroupWords];
        blob.insert(blob.end(), gr, gr + kGroupWords);
        blob.push_back(i - gr[10]);
    }
    for (uint32_t r = 0; r < m; r++) {
        blob.push_back(rp.lo[r]);
        blob.push_back(rp.hi[r]);
    }
    for (uint32_t i = 0; i < n_bitems; i++) {  // block words + partition index
        const uint32_t* bk = &blocks[static_cast<size_t>(bitems[i]) * kBlockWords];
        blob.insert(blob.end(), bk, bk + kBlockWords);
        blob.push_back(i - bk[8]);
    }
    blob.insert(blob.end(), bpairs.begin(), bpairs.end());
    // A call with both kinds of work runs them in one launch (attn_mixed).
    // Its order comes from a list schedule over record slots (CUs / KV
    // heads; a record is a decode item or a prefill block over all its KV
    // heads): at most dmax decode records run at once and the prefill blocks
    // fill the other slots (longest first within each kind), so that HBM
    // streams decode while the matrix cores run prefill.  The host simulates
    // up to ~32 values of dmax and keeps the order with the shortest
    // simulated makespan.
    // Model (measured per workgroup): a decode workgroup streams its bytes at
    // min(kCuBytesPerUs, kHbmBytesPerUs / decode workgroups running when it
    // starts); a prefill block costs ~10 us plus ~4.5 us per 64-key tile
    // (head_dim 128, beside streaming decode).  The order changes no row's
    // arithmetic.
    const bool mixed = n_items > 0 && n_bitems > 0 && wide && hd_t <= 128 && THB_ATTN_WAVES == THB_PREFILL_WAVES;
    if (mixed) {
        constexpr double kHbmBytesPerUs = 6.2e6, kCuBytesPerUs = 3.7e4 * THB_PREFILL_WAVES / 8;
        const uint32_t n_kvh = pool->kv_heads;
        std::vector<std::pair<double, uint32_t>> dec, pre;  // (bytes per workgroup | us, record)
        dec.reserve(n_items);
        pre.reserve(n_bpairs);
        for (uint32_t i = 0; i < n_items; i++) {
            const uint32_t* gr = &groups[static_cast<size_t>(items[i]) * kGroupWords];
            const uint64_t p0 = uint64_t(gr[8]) + uint64_t(i - gr[10]) * gr[9];
            const uint64_t keys = gr[6] > p0 ? std::min<uint64_t>(gr[9], gr[6] - p0) : 0;
            dec.push_back({static_cast<double>(keys) * 4.0 * hd, i});
        }
        for (uint32_t i = 0; i < n_bpairs; i++) {  // one fixed cost per pair
            uint64_t tiles = bitem_tiles(bpairs[2 * i]);
            if (bpairs[2 * i + 1] != kNoItem) tiles += bitem_tiles(bpairs[2 * i + 1]);
            pre.push_back({10.0 + static_cast<double>(tiles) * 4.5 * hd_t / 128.0, 0x80000000u | i});
        }
        auto longest_first = [](const std::pair<double, uint32_t>& x, const std::pair<double, uint32_t>& y) {
            return x.first > y.first;
        };
        std::stable_sort(dec.begin(), dec.end(), longest_first);
        std::stable_sort(pre.begin(), pre.end(), longest_first);
        const uint32_t slots = std::max<uint32_t>(2, pool->cus * (8 / THB_PREFILL_WAVES) / n_kvh);
        std::vector<uint32_t> order, best;
        double best_t = INFINITY;
        const uint32_t step = std::max<uint32_t>(1, slots / 32);  // at most ~32 simulations
        for (uint32_t dmax = 1; dmax < slots; dmax += step) {
            std::priority_queue<std::pair<double, bool>, std::vector<std::pair<double, bool>>,
                                std::greater<std::pair<double, bool>>>
                running;  // (end time, decode)
            uint32_t free_slots = slots, n_dec = 0;
            size_t di = 0, pi = 0;
            double t = 0.0, end = 0.0;  // dispatch time of the next record, makespan
            order.clear();
            while (di < dec.size() || pi < pre.size()) {
                while (free_slots == 0) {
                    const auto e = running.top();
                    running.pop();
                    t = e.first;
                    free_slots++;
                    if (e.second) n_dec--;
                }
                double done;
                if (di < dec.size() && (n_dec < dmax || pi == pre.size())) {
                    n_dec++;  // rate from the decode workgroups running once this one starts
                    done = t + dec[di].first / std::min(kCuBytesPerUs,
                                                        kHbmBytesPerUs / (static_cast<double>(n_dec) * n_kvh));
                    running.push({done, true});
                    order.push_back(dec[di++].second);
                } else {
                    done = t + pre[pi].first;
                    running.push({done, false});
                    order.push_back(pre[pi++].second);
                }
                end = std::max(end, done);
                free_slots--;
            }
            if (end < best_t) {
                best_t = end;
                best.swap(order);
            }
        }
        blob.insert(blob.end(), best.begin(), best.end());
    }
    // The groups of more than one partition: decode groups first (their
    // last partition's workgroup combines them where the launch has merge
    // counters), then the prefill blocks' groups (always the merge kernel).
    const size_t merge_off = blob.size();
    uint32_t n_merge_dec = 0;
    for (int blk = 0; blk < 2; blk++)
        for (uint32_t gi = 0; gi < n_groups; gi++) {
            const uint32_t* G = groups.data() + static_cast<size_t>(gi) * kGroupWords;
            if (G[7] > 1 && in_block[gi] == (blk == 1)) {
                blob.insert(blob.end(), {G[0], G[1], G[2], G[3], G[7], G[10], 0u, 0u});
                n_merge_dec += blk == 0;
            }
        }
    const uint32_t n_merge = static_cast<uint32_t>((blob.size() - merge_off) / kMergeWords);
    plan.blob.swap(blob);
    plan.uploaded = false;
    plan.n_groups = n_groups;
    plan.n_items = n_items;
    plan.n_blocks = n_blocks;
    plan.n_bitems = n_bitems;
    plan.n_bpairs = n_bpairs;
    plan.n_slots = n_slots;
    plan.split = any_split;
    plan.n_merge = n_merge;
    plan.n_merge_dec = n_merge_dec;
    plan.merge_off = static_cast<uint32_t>(merge_off);
    plan.hd_t = hd_t;
    plan.wide = wide;
    plan.mixed = mixed;

    // The append can run inside the attention launch when no query reads a
    // token that another workgroup appends: the call is causal, every row's
    // new token is its last key (hi == pos + 1), positions rise within a
    // sequence chunk, each chunk fits in one group, and no sequence appears
    // in two chunks.
    bool fuse = sp.causal != 0;
    std::vector<uint32_t> seen;
    for (auto& c : rp.chunks) {
        if (!fuse) break;
        const uint32_t n = c.second - c.first;
        fuse = G <= kCols ? n <= kCols / G : n == 1;
        for (uint32_t r = c.first; r < c.second && fuse; r++) {
            const uint32_t pos = args[8 * r];
            fuse = rp.hi[r] == static_cast<uint64_t>(pos) + 1 && rp.lo[r] <= pos &&
                   (r == c.first || pos > args[8 * (r - 1)]);
        }
        seen.push_back(rp.seq[c.first]);
    }
    if (fuse) {
        std::sort(seen.begin(), seen.end());
        fuse = std::adjacent_find(seen.begin(), seen.end()) == seen.end();
    }
    plan.fusable = fuse;
    return THB_OK;
}

int check_attn_call(thb_pool* pool, uint32_t layer, const void* q, void* y, const thb_attn_spec& sp,
                    const thb_rows* rows) {
    if (layer >= pool->layers)
        return fail(THB_ERR_INVALID, "layer " + std::to_string(layer) + " out of range (" +
                                         std::to_string(pool->layers) + " layers)");
    if (!q || !y) return fail(THB_ERR_INVALID, "null q or y");
    if (sp.q_heads == 0 || sp.q_heads % pool->kv_heads != 0)
        return fail(THB_ERR_CONFIG, "q_heads " + std::to_string(sp.q_heads) +
                                        " must be a positive multiple of kv_heads " + std::to_string(pool->kv_heads));
    if (sp.q_dtype > THB_DT_BF16 || sp.y_dtype > THB_DT_BF16)
        return fail(THB_ERR_INVALID, "q_dtype and y_dtype must be THB_DT_F32, THB_DT_F16 or THB_DT_BF16");
    if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(y) & 15u))
        return fail(THB_ERR_INVALID, "q and y must be 16-byte aligned");
    if (static_cast<uint64_t>(sp.row_off) + sp.m > rows->m)
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->m) + " rows, call needs " +
                                         std::to_string(static_cast<uint64_t>(sp.row_off) + sp.m));
    if (sp.seq != THB_SEQ_PER_ROW && sp.seq >= pool->arena.a.seqs())
        return fail(THB_ERR_INVALID, "sequence " + std::to_string(sp.seq) + " out of range");
    if (!(sp.softcap >= 0.0f)) return fail(THB_ERR_INVALID, "softcap must be >= 0");
    if (pool->part_len >> pool->page_shift > kMaxPartLenPages)
        return fail(THB_ERR_CONFIG, "part_len / page_len must be at most " + std::to_string(kMaxPartLenPages));
    return THB_OK;
}

// Copies a plan's blob to its own device buffer (once per plan).
void upload_plan(thb_pool* pool, AttnPlan& plan, hipStream_t s) {
    if (plan.uploaded) return;
    void* dev = plan.dev.reserve_rewrite(plan.blob.size() * 4, false, s);
    pool->stager.upload(dev, plan.blob.data(), plan.blob.size() * 4, s);
    plan.uploaded = true;
}

// Finds or builds the launch plan of this call (cached per rows write, call
// shape and allocator state); with `upload`, its blob is on the device in
// plan->dev.  Runs inside guarded().
int get_plan(thb_pool* pool, const thb_rows* rows, const thb_attn_spec& sp, uint32_t hd, hipStream_t s, bool upload,
             AttnPlan** out) {
    const uint64_t av = pool->arena.a.version();
    for (auto& p : pool->plans)
        if (p.rows == rows && p.rows_version == rows->version && p.arena_version == av && p.row_off == sp.row_off &&
            p.m == sp.m && p.seq == sp.seq && p.causal == sp.causal && p.window == sp.window &&
            p.q_heads == sp.q_heads && p.head_dim == hd) {
            p.last_use = ++pool->plan_clock;
            if (upload) upload_plan(pool, p, s);
            *out = &p;
            return THB_OK;
        }
    AttnPlan* plan = &pool->plans[0];
    for (auto& p : pool->plans)
        if (p.last_use < plan->last_use) plan = &p;
    plan->rows = nullptr;
    if (int rc = build_plan(pool, rows, sp, hd, *plan)) return rc;
    if (upload) upload_plan(pool, *plan, s);
    plan->rows = rows;
    plan->rows_version = rows->version;
    plan->arena_version = av;
    plan->row_off = sp.row_off;
    plan->m = sp.m;
    plan->seq = sp.seq;
    plan->causal = sp.causal;
    plan->window = sp.window;
    plan->q_heads = sp.q_heads;
    plan->head_dim = hd;
    plan->last_use = ++pool->plan_clock;
    *out = plan;
    return THB_OK;
}

// Bytes of split-K partial results a plan needs (0 without a split) and,
// in *o_bytes, the size of the partial outputs that come first.
uint64_t partial_bytes(const thb_pool* pool, const AttnPlan& plan, uint64_t* o_bytes) {
    if (!plan.split) {
        *o_bytes = 0;
        return 0;
    }
    const uint64_t n_part = static_cast<uint64_t>(plan.n_slots) * pool->kv_heads * kCols;
    *o_bytes = (n_part * plan.hd_t * 4 + 255) & ~uint64_t(255);
    return *o_bytes + n_part * 8;
}

// The arguments of every attention launch that do not depend on the plan's
// blob: tensors, geometry, score scale, dtypes and the thb_attn_io
// extensions.
void fill_args(thb_pool* pool, uint32_t layer, const thb_attn_io& io, const thb_attn_spec& sp, const uint32_t* meta,
               AttnArgs& a) {
    const thb_rope* rope = io.rope;
    const LayerGeom& g = pool->geom[layer];
    const uint32_t hd = g.head_dim;
    a = AttnArgs{};
    a.q = io.q_dev;
    a.y = io.y_dev;
    a.table = pool->table_dev;
    a.k = reinterpret_cast<uint16_t*>(pool->mem + g.k_off);
    a.v = reinterpret_cast<uint16_t*>(pool->mem + g.v_off);
    a.plane = static_cast<uint64_t>(pool->arena.a.pages()) * pool->page_len * hd;
    a.max_pages = pool->arena.a.max_pages();
    a.pages = pool->arena.a.pages();
    a.page_shift = pool->page_shift;
    a.q_heads = sp.q_heads;
    a.nq_per_kv = sp.q_heads / pool->kv_heads;
    a.head_dim = hd;
    a.part_len = pool->part_len;
    a.n_kvh = pool->kv_heads;
    a.qscale = q_scale(sp);
    a.cap2 = sp.softcap > 0.0f ? sp.softcap * 1.4426950408889634f : 0.0f;
    a.qpre = std::signbit(a.qscale) ? -1.0f : 1.0f;
    a.qpost = std::fabs(a.qscale);
    a.q_dt = sp.q_dtype;
    a.y_dt = sp.y_dtype;
    a.q_stride = io.q_stride ? io.q_stride : hd;
    a.gate = io.gate_dev;
    a.gate_stride = io.gate_stride ? io.gate_stride : hd;
    a.rope_on = rope != nullptr;
    a.full = rope != nullptr || io.gate_dev != nullptr || a.q_stride != hd || sp.q_dtype == THB_DT_BF16 ||
             sp.y_dtype == THB_DT_BF16 || sp.softcap > 0.0f;
    a.meta = meta;
    a.qrope = rope ? rope_dev(*rope, true) : RopeDev{};
    a.krope = rope ? rope_dev(*rope, false) : RopeDev{};
}

// Launches attention (and, when app is set, the fused append) for a plan
// whose blob is at `blob` on the device, with the split-K partial results
// (when the plan splits) at `part`.  With merge_cnt (zeroed counters, one
// per decode item and KV head, left zero again), each split decode group is
// combined by the workgroup of its last partition; without, by the merge
// kernel after the launch.  With rope set, the query is rotated as it is
// loaded (and the fused append rotates the key); meta is the row meta of
// the call's first row.
void launch_plan(thb_pool* pool, uint32_t layer, const thb_attn_io& io, const thb_attn_spec& sp, const AttnPlan& plan,
                 bool fused_append, const uint32_t* meta, const uint32_t* blob, uint8_t* part, uint32_t* merge_cnt,
                 hipStream_t s) {
    const uint32_t hd_t = plan.hd_t;
    float* part_o = nullptr;
    float* part_ml = nullptr;
    if (plan.split) {
        uint64_t o_bytes = 0;
        partial_bytes(pool, plan, &o_bytes);
        part_o = reinterpret_cast<float*>(part);
        part_ml = reinterpret_cast<float*>(part + o_bytes);
    }
    AttnArgs a;
    fill_args(pool, layer, io, sp, meta, a);
    a.groups = blob;
    a.items = blob + static_cast<size_t>(plan.n_groups) * kGroupWords;
    a.ranges = a.items + static_cast<size_t>(plan.n_items) * kItemWords;
    a.bitems = a.ranges + 2 * static_cast<size_t>(sp.m);
    a.bpairs = a.bitems + static_cast<size_t>(plan.n_bitems) * kBItemWords;
    a.order = a.bpairs + 2 * static_cast<size_t>(plan.n_bpairs);
    a.merge_groups = blob + plan.merge_off;
    a.k_src = fused_append ? io.k_src_dev : nullptr;
    a.v_src = fused_append ? io.v_src_dev : nullptr;
    a.src_dtype = fused_append ? io.src_dtype : 0u;
    a.part_o = part_o;
    a.part_ml = part_ml;
    a.merge_cnt = plan.split ? merge_cnt : nullptr;
    const bool f16 = pool->kv_dtype == THB_KV_F16_RNE;
    const uint64_t n_wg = static_cast<uint64_t>(plan.n_items) * pool->kv_heads;
    // attn_prefill_wide runs pairs of prefill items, attn_prefill single items
    const uint64_t n_pwg = static_cast<uint64_t>(plan.wide ? plan.n_bpairs : plan.n_bitems) * pool->kv_heads;
    if (n_wg > 0x7FFFFFFFull || n_pwg > 0x7FFFFFFFull)
        throw HipError{hipErrorInvalidConfiguration, "attention grid too large"};
    // A call with decode items and attn_prefill_wide blocks runs them in one
    // interleaved launch; otherwise the decode items, then the prefill
    // blocks, on the caller's stream.  (Running the prefill kernel on a
    // second stream measured slower: 262 vs 248 us per C3 layer.)
    if (plan.mixed) {
        launch_mixed(hd_t, f16, dim3(static_cast<uint32_t>(n_wg + n_pwg)), a, s);
        THB_HIP(hipGetLastError());
    } else if (n_wg) {
        launch(hd_t, f16, dim3(static_cast<uint32_t>(n_wg)), a, s);
        THB_HIP(hipGetLastError());
    }
    if (n_pwg && !plan.mixed) {
        launch_prefill(hd_t, f16, dim3(static_cast<uint32_t>(n_pwg)), a, s);
        THB_HIP(hipGetLastError());
    }
    const uint32_t m0 = a.merge_cnt ? plan.n_merge_dec : 0u;  // records the launch above combined
    if (plan.split && plan.n_merge > m0) {
        a.merge_groups = blob + plan.merge_off + static_cast<size_t>(m0) * kMergeWords;
        launch_merge(hd_t, dim3(plan.n_merge - m0, pool->kv_heads), a, s);
        THB_HIP(hipGetLastError());
    }
}

}  // namespace
}  // namespace thb

using namespace thb;

namespace {

// Every attention entry point: optional append (fused into the launch where
// the rows allow it), rotary embedding, query stride and output gate.
int step_impl(thb_pool* pool, uint32_t layer, const thb_attn_io* io, const thb_attn_spec* spec, const thb_rows* rows,
              void* stream) {
    if (!pool || !io || !spec || !rows) return fail(THB_ERR_INVALID, "null pool, io, spec or rows");
    // The plan is made on the host from the row meta last written and cached
    // in buffers that later calls reuse: a replay could not follow the rows.
    if (capturing(as_stream(stream)))
        return fail(THB_ERR_INVALID, "not capturable: thb_attn plans each call on the host; capture "
                                     "thb_dplan_build + thb_attn_dplan (planned on the device at every replay) or "
                                     "thb_attn_noalloc (the plan travels in the graph)");
    if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
    if (spec->m == 0)
        return layer < pool->layers ? THB_OK : check_attn_call(pool, layer, io->q_dev, io->y_dev, *spec, rows);
    if (int rc = check_attn_call(pool, layer, io->q_dev, io->y_dev, *spec, rows)) return rc;
    const uint32_t hd = pool->geom[layer].head_dim;
    const uint32_t qes = spec->q_dtype == THB_DT_F32 ? 4u : 2u;
    if (io->q_stride && (io->q_stride < hd || (io->q_stride * qes) % 16 != 0))
        return fail(THB_ERR_INVALID, "q_stride " + std::to_string(io->q_stride) +
                                         " must be 0 or at least head_dim, and a multiple of 16 bytes");
    if (io->gate_dev && io->gate_stride && io->gate_stride < hd)
        return fail(THB_ERR_INVALID, "gate_stride " + std::to_string(io->gate_stride) + " below head_dim");
    const thb_rope* rope = io->rope;
    if (rope)
        if (int rc = check_rope(rope, hd, rows, spec->row_off, spec->m)) return rc;
    const bool append = io->k_src_dev || io->v_src_dev;
    if (append) {
        if (!io->k_src_dev || !io->v_src_dev) return fail(THB_ERR_INVALID, "null source buffer");
        if (io->src_dtype > THB_DT_BF16)
            return fail(THB_ERR_INVALID, "unknown src_dtype " + std::to_string(io->src_dtype));
        if (rope && io->src_dtype == THB_DT_BF16)
            return fail(THB_ERR_INVALID, "rotary append takes f32 or f16 sources (src_dtype 2)");
        if ((reinterpret_cast<uintptr_t>(io->k_src_dev) & 15u) || (reinterpret_cast<uintptr_t>(io->v_src_dev) & 15u))
            return fail(THB_ERR_INVALID, "source buffers must be 16-byte aligned");
        // Pages must cover every appended token (thb_kv_store's check; the
        // append takes each row's sequence from the row meta, kv_store.wgsl:39).
        const Arena& arena = pool->arena.a;
        for (uint32_t r = spec->row_off; r < spec->row_off + spec->m; r++) {
            const uint32_t pos = rows->host[8 * r];
            const uint32_t seq = rows->host[8 * r + 1];
            if (seq >= arena.seqs())
                return fail(THB_ERR_INVALID, "sequence " + std::to_string(seq) + " out of range (" +
                                                 std::to_string(arena.seqs()) + " sequences)");
            if (pos == 0xFFFFFFFFu || !arena.covers(seq, pos + 1))
                return fail(THB_ERR_MODEL, "pages must cover the chunk: sequence " + std::to_string(seq) +
                                               " holds " + std::to_string(arena.table_of(seq).size() * arena.page_len()) +
                                               " slots, needs " + std::to_string(static_cast<uint64_t>(pos) + 1));
        }
    }
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        AttnPlan* plan = nullptr;
        if (int rc = get_plan(pool, rows, *spec, hd, s, true, &plan)) return rc;
        const uint32_t* meta = rows->dev + 8 * static_cast<size_t>(spec->row_off);
        const uint32_t* blob = static_cast<const uint32_t*>(plan->dev.get());
        uint64_t o_bytes = 0;
        const uint64_t pb = partial_bytes(pool, *plan, &o_bytes);
        uint8_t* part = pb ? static_cast<uint8_t*>(pool->partials.reserve(pb, false, s)) : nullptr;
        uint32_t* cnt = plan->n_merge_dec ? static_cast<uint32_t*>(pool->merge_cnt.reserve(
                                                static_cast<size_t>(plan->n_items) * pool->kv_heads * 4, true, s))
                                          : nullptr;
        if (!append) {
            launch_plan(pool, layer, *io, *spec, *plan, false, meta, blob, part, cnt, s);
            return THB_OK;
        }
        // The row meta's sequence must be the one the append uses: a fixed
        // AttnSpec.seq that differs from the rows' own seq is not fused.
        bool fuse = plan->fusable;
        if (fuse && spec->seq != THB_SEQ_PER_ROW)
            for (uint32_t r = spec->row_off; r < spec->row_off + spec->m && fuse; r++)
                fuse = rows->host[8 * r + 1] == spec->seq;
        if (fuse) {
            launch_plan(pool, layer, *io, *spec, *plan, true, meta, blob, part, cnt, s);
            return THB_OK;
        }
        const int rc = rope ? thb_kv_store_rope(pool, layer, io->k_src_dev, io->v_src_dev, io->src_dtype, rope, rows,
                                                spec->row_off, spec->m, stream)
                            : thb_kv_store(pool, layer, io->k_src_dev, io->v_src_dev, io->src_dtype, rows,
                                           spec->row_off, spec->m, stream);
        if (rc) return rc;
        launch_plan(pool, layer, *io, *spec, *plan, false, meta, blob, part, cnt, s);
        return THB_OK;
    });
}

thb_attn_io make_io(const void* q, void* y, const void* k_src, const void* v_src, uint32_t src_dtype,
                    const thb_rope* rope) {
    thb_attn_io io{};
    io.q_dev = q;
    io.y_dev = y;
    io.k_src_dev = k_src;
    io.v_src_dev = v_src;
    io.src_dtype = src_dtype;
    io.rope = rope;
    return io;
}

}  // namespace

extern "C" int thb_attn(thb_pool* pool, uint32_t layer, const void* q, void* y, const thb_attn_spec* spec,
                        const thb_rows* rows, void* stream) {
    const thb_attn_io io = make_io(q, y, nullptr, nullptr, 0, nullptr);
    return step_impl(pool, layer, &io, spec, rows, stream);
}

extern "C" int thb_attn_rope(thb_pool* pool, uint32_t layer, const void* q, void* y, const thb_attn_spec* spec,
                             const thb_rope* rope, const thb_rows* rows, void* stream) {
    if (!rope) return fail(THB_ERR_INVALID, "null rope");
    const thb_attn_io io = make_io(q, y, nullptr, nullptr, 0, rope);
    return step_impl(pool, layer, &io, spec, rows, stream);
}

extern "C" int thb_attn_append(thb_pool* pool, uint32_t layer, const void* k_src, const void* v_src,
                               uint32_t src_dtype, const void* q, void* y, const thb_attn_spec* spec,
                               const thb_rows* rows, void* stream) {
    if (!k_src || !v_src) return fail(THB_ERR_INVALID, "null source buffer");
    const thb_attn_io io = make_io(q, y, k_src, v_src, src_dtype, nullptr);
    return step_impl(pool, layer, &io, spec, rows, stream);
}

extern "C" int thb_attn_append_rope(thb_pool* pool, uint32_t layer, const void* k_src, const void* v_src,
                                    uint32_t src_dtype, const void* q, void* y, const thb_attn_spec* spec,
                                    const thb_rope* rope, const thb_rows* rows, void* stream) {
    if (!rope) return fail(THB_ERR_INVALID, "null rope");
    if (!k_src || !v_src) return fail(THB_ERR_INVALID, "null source buffer");
    const thb_attn_io io = make_io(q, y, k_src, v_src, src_dtype, rope);
    return step_impl(pool, layer, &io, spec, rows, stream);
}

extern "C" int thb_attn_step(thb_pool* pool, uint32_t layer, const thb_attn_io* io, const thb_attn_spec* spec,
                             const thb_rows* rows, void* stream) {
    return step_impl(pool, layer, io, spec, rows, stream);
}

// ------------------------------------------------ no-allocation entry point
// thb_attn_noalloc keeps the launch plan and the split-K partial results of
// one call in this fixed array instead of buffers the pool grows with
// hipMalloc: the plan in its first THB_NOALLOC_PLAN_BYTES, the partial
// results after it.  Each device holds its own copy for the life of the
// process, and every call on a device shares it (the last call's contents
// stay; nothing in it needs to start at zero: each partial slot is written
// before it is read, and the plan is uploaded by each call).  Host code uses
// the address hipGetSymbolAddress returns for the current device, never the
// array's name.
static __device__ __align__(256) uint8_t scratch[THB_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices] = {};

// This device's scratch address, resolved once per device with the device
// current (the first no-allocation call on it).
int scratch_for(int device, uint8_t** out) {
    if (device < 0 || device >= kMaxDevices)
        return fail(THB_ERR_INVALID, "device " + std::to_string(device) + " beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return fail(THB_ERR_GPU, std::string("no-allocation scratch unavailable: ") + hipGetErrorString(e));
        }
        g_scratch[device] = static_cast<uint8_t*>(ptr);
    }
    *out = g_scratch[device];
    return THB_OK;
}

}  // namespace

extern "C" int thb_attn_noalloc(thb_pool* pool, uint32_t layer, const void* q, void* y, const thb_attn_spec* spec,
                                const thb_rows* rows, void* stream) {
    if (!pool || !spec || !rows) return fail(THB_ERR_INVALID, "null pool, spec or rows");
    if (int rc = check_attn_call(pool, layer, q, y, *spec, rows)) return rc;
    if (spec->m == 0) return THB_OK;
    if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
    const uint32_t hd = pool->geom[layer].head_dim;
    return guarded([&]() -> int {
        int device = -1;
        THB_HIP(hipGetDevice(&device));
        if (device != pool->device)
            return fail(THB_ERR_INVALID, "the pool lives on device " + std::to_string(pool->device) + ", device " +
                                             std::to_string(device) + " is current");
        uint8_t* scr = nullptr;
        if (int rc = scratch_for(device, &scr)) return rc;
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);  // page ops in kernel arguments, copies from the device list: no allocation
        AttnPlan* plan = nullptr;
        if (int rc = get_plan(pool, rows, *spec, hd, s, false, &plan)) return rc;
        const uint64_t plan_bytes = plan->blob.size() * 4;
        if (plan_bytes > THB_NOALLOC_PLAN_BYTES)
            return fail(THB_ERR_INVALID, "launch plan of " + std::to_string(plan_bytes) +
                                             " bytes exceeds the no-allocation scratch's " +
                                             std::to_string(THB_NOALLOC_PLAN_BYTES) + " (use thb_attn)");
        uint64_t o_bytes = 0;
        const uint64_t pb = partial_bytes(pool, *plan, &o_bytes);
        constexpr uint64_t kPartCap = static_cast<uint64_t>(THB_NOALLOC_SCRATCH_BYTES) - THB_NOALLOC_PLAN_BYTES;
        if (pb > kPartCap)
            return fail(THB_ERR_INVALID, "split-K partial results of " + std::to_string(pb) +
                                             " bytes exceed the no-allocation scratch's " + std::to_string(kPartCap) +
                                             " (use thb_attn, or a longer part_len)");
        pool->fixed_stager.upload(scr, plan->blob.data(), plan_bytes, s);
        const thb_attn_io io = make_io(q, y, nullptr, nullptr, 0, nullptr);
        const uint32_t* meta = rows->dev + 8 * static_cast<size_t>(spec->row_off);
        launch_plan(pool, layer, io, *spec, *plan, false, meta, reinterpret_cast<const uint32_t*>(scr),
                    scr + THB_NOALLOC_PLAN_BYTES, nullptr, s);
        return THB_OK;
    });
}

// ------------------------------------------- device-planned decode calls
struct thb_dplan {
    thb_pool* pool = nullptr;
    uint32_t max_m = 0, q_heads = 0, gmax = 0, pmax = 0;
    uint32_t items_off = 0, ranges_off = 0, merge_off = 0;
    uint32_t hd_max = 0;  // widest head_dim template of the pool's layers
    // List mode (THB_DPLAN_PREFILL): a work list with prefill blocks, launched
    // as attn_list; the blob is [header | groups | items | ranges | blocks |
    // pairs | order].
    bool list = false;
    bool append = false;  // THB_DPLAN_APPEND: each build checks that the append can run in the launch
    uint32_t pos_limit = 0;  // thb_dplan_set_pos_limit: rows at or past it are reported and read nothing
    uint32_t imax = 0, bmax = 0, wb = 0;
    uint32_t groups_off = 0, bitems_off = 0, pairs_off = 0, order_off = 0;
    bool built = false;
    thb_attn_spec spec{};
    const thb_rows* rows = nullptr;
    thb::DevBuf blob, part;
    thb::DevBuf cnt;  // merge counters (one per item slot and KV head), zero between launches
};

namespace {

// Blob layout of a device plan for calls of up to max_m rows (build_plan's
// order: groups, items, ranges, then the merge records).
void dplan_layout(thb_dplan* p) {
    p->items_off = p->gmax * kGroupWords;
    p->ranges_off = p->items_off + p->gmax * p->pmax * kItemWords;
    p->merge_off = p->ranges_off + 2 * p->max_m;
}

// Blob layout of a list-mode plan.
void dplan_list_layout(thb_dplan* p) {
    p->imax = p->gmax * p->pmax;
    p->bmax = p->gmax / 2 + 1;  // blocks of >= 4 groups, plus each prefill chunk's last partial block
    p->groups_off = kListHdrWords;
    p->items_off = p->groups_off + p->gmax * kGroupWords;
    p->ranges_off = p->items_off + p->imax * kItemWords;
    p->bitems_off = p->ranges_off + 2 * p->max_m;
    p->pairs_off = p->bitems_off + p->bmax * kBItemWords;
    p->order_off = p->pairs_off + 2 * p->bmax;
    p->merge_off = p->order_off + p->imax + p->bmax;
}

// The launch-side plan of a device plan: every slot of the fixed grid (or
// of the list's capacity).
void dplan_shape(const thb_dplan* p, uint32_t hd, AttnPlan& a) {
    a.n_groups = p->gmax;
    a.n_items = p->gmax * p->pmax;
    a.n_slots = a.n_items;
    a.hd_t = template_hd(hd);
    a.split = p->pmax > 1;
    a.n_merge = p->gmax;
    a.n_merge_dec = p->gmax;
    a.merge_off = p->merge_off;
}

// The checks of a launch over a built device plan.
int dplan_call_check(const thb_pool* pool, uint32_t layer, const void* q, const void* y, const thb_dplan* plan) {
    if (!pool || !plan) return fail(THB_ERR_INVALID, "null pool or plan");
    if (plan->pool != pool) return fail(THB_ERR_INVALID, "the plan belongs to another pool");
    if (!plan->built) return fail(THB_ERR_INVALID, "the plan has not been built (thb_dplan_build)");
    if (layer >= pool->layers)
        return fail(THB_ERR_INVALID, "layer " + std::to_string(layer) + " out of range (" +
                                         std::to_string(pool->layers) + " layers)");
    if (!q || !y) return fail(THB_ERR_INVALID, "null q or y");
    if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(y) & 15u))
        return fail(THB_ERR_INVALID, "q and y must be 16-byte aligned");
    return THB_OK;
}

// Attention over a work-list device plan: one workgroup per CU claiming the
// list's entries (decode items with in-launch merges, prefill blocks).
void dplan_launch_list(thb_pool* pool, uint32_t layer, const thb_attn_io& io, const thb_dplan* plan, hipStream_t s) {
    const uint32_t* blob = static_cast<const uint32_t*>(plan->blob.get());
    AttnArgs a;
    fill_args(pool, layer, io, plan->spec, plan->rows->dev + 8 * static_cast<size_t>(plan->spec.row_off), a);
    a.groups = blob + plan->groups_off;
    a.items = blob + plan->items_off;
    a.ranges = blob + plan->ranges_off;
    a.bitems = blob + plan->bitems_off;
    a.bpairs = blob + plan->pairs_off;
    a.order = blob + plan->order_off;
    a.merge_groups = blob + plan->merge_off;
    a.list = const_cast<uint32_t*>(blob);
    AttnPlan shape;
    dplan_shape(plan, plan->hd_max, shape);
    if (shape.split) {
        uint64_t o_bytes = 0;
        partial_bytes(pool, shape, &o_bytes);
        a.part_o = reinterpret_cast<float*>(plan->part.get());
        a.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(plan->part.get()) + o_bytes);
        a.merge_cnt = static_cast<uint32_t*>(plan->cnt.get());
    }
    launch_list(template_hd(pool->geom[layer].head_dim), pool->kv_dtype == THB_KV_F16_RNE, dim3(pool->cus), a, s);
    THB_HIP(hipGetLastError());
}

// Attention over a fixed-grid device plan, with the append inside the
// launch when io carries sources.
void dplan_launch_grid(thb_pool* pool, uint32_t layer, const thb_attn_io& io, const thb_dplan* plan, hipStream_t s) {
    AttnPlan shape;
    dplan_shape(plan, pool->geom[layer].head_dim, shape);
    const uint32_t* meta = plan->rows->dev + 8 * static_cast<size_t>(plan->spec.row_off);
    launch_plan(pool, layer, io, plan->spec, shape, io.k_src_dev != nullptr, meta,
                static_cast<const uint32_t*>(plan->blob.get()), static_cast<uint8_t*>(plan->part.get()),
                static_cast<uint32_t*>(plan->cnt.get()), s);
}

}  // namespace

extern "C" {

int thb_dplan_create(thb_pool* pool, uint32_t max_m, uint32_t q_heads, thb_dplan** out) {
    return thb_dplan_create_ex(pool, max_m, q_heads, 0u, out);
}

int thb_dplan_create_ex(thb_pool* pool, uint32_t max_m, uint32_t q_heads, uint32_t flags, thb_dplan** out) {
    if (!pool || !out) return fail(THB_ERR_INVALID, "null pool or out");
    *out = nullptr;
    if (flags & ~(THB_DPLAN_PREFILL | THB_DPLAN_APPEND))
        return fail(THB_ERR_INVALID, "unknown dplan flags " + std::to_string(flags));
    const bool list = (flags & THB_DPLAN_PREFILL) != 0;
    if (list && (flags & THB_DPLAN_APPEND))
        return fail(THB_ERR_INVALID, "THB_DPLAN_APPEND takes the fixed-grid plan (without THB_DPLAN_PREFILL)");
    const uint32_t max_rows = list ? kDPlanListMaxRows : kDPlanMaxRows;
    if (max_m == 0 || max_m > max_rows)
        return fail(THB_ERR_INVALID, "device-planned calls take 1 to " + std::to_string(max_rows) + " rows, not " +
                                         std::to_string(max_m));
    if (q_heads == 0 || q_heads % pool->kv_heads != 0)
        return fail(THB_ERR_CONFIG, "q_heads " + std::to_string(q_heads) + " must be a positive multiple of kv_heads " +
                                        std::to_string(pool->kv_heads));
    if (pool->part_len >> pool->page_shift > kMaxPartLenPages)
        return fail(THB_ERR_CONFIG, "part_len / page_len must be at most " + std::to_string(kMaxPartLenPages));
    return guarded([&]() -> int {
        auto p = std::make_unique<thb_dplan>();
        p->pool = pool;
        p->max_m = max_m;
        p->q_heads = q_heads;
        p->append = (flags & THB_DPLAN_APPEND) != 0;
        const uint32_t G = q_heads / pool->kv_heads;
        p->gmax = G <= kCols ? max_m : max_m * ((G + kCols - 1) / kCols);
        // Partitions of the longest key range any sequence of the pool allows
        // (partition counts grow with the range).
        const uint64_t span = static_cast<uint64_t>(pool->arena.a.max_pages()) << pool->page_shift;
        uint32_t n = static_cast<uint32_t>(std::max<uint64_t>(1, (span + pool->part_len - 1) / pool->part_len));
        if (n > 1) n = 1u << (32 - __builtin_clz(n - 1));
        if (n > kMaxParts)
            return fail(THB_ERR_CONFIG, "sequences of " + std::to_string(span) + " tokens exceed " +
                                            std::to_string(kMaxParts) + " partitions of " +
                                            std::to_string(pool->part_len) + " tokens");
        p->pmax = n;
        for (const auto& g : pool->geom) p->hd_max = std::max(p->hd_max, template_hd(g.head_dim));
        if (list) {
            if (p->hd_max > 256)
                return fail(THB_ERR_CONFIG, "device plans with prefill blocks take head_dim <= 256");
            p->list = true;
            p->wb = block_groups(true, p->hd_max);
            if (p->wb > kListMaxWB)
                return fail(THB_ERR_CONFIG, "prefill blocks of " + std::to_string(p->wb) + " groups exceed " +
                                                std::to_string(kListMaxWB));
            dplan_list_layout(p.get());
        } else {
            dplan_layout(p.get());
        }
        const size_t words = static_cast<size_t>(p->merge_off) + static_cast<size_t>(p->gmax) * kMergeWords;
        p->blob.reserve(words * 4, true, nullptr);
        AttnPlan shape;
        dplan_shape(p.get(), p->hd_max, shape);
        uint64_t o_bytes = 0;
        const uint64_t pb = partial_bytes(pool, shape, &o_bytes);
        if (pb) {
            p->part.reserve(pb, false, nullptr);
            p->cnt.reserve(static_cast<size_t>(shape.n_items) * pool->kv_heads * 4, true, nullptr);
        }
        *out = p.release();
        return THB_OK;
    });
}

void thb_dplan_destroy(thb_dplan* plan) { delete plan; }

int thb_dplan_build(thb_dplan* plan, const thb_attn_spec* spec, const thb_rows* rows, void* stream) {
    if (!plan || !spec || !rows) return fail(THB_ERR_INVALID, "null plan, spec or rows");
    thb_pool* pool = plan->pool;
    if (spec->m == 0 || spec->m > plan->max_m)
        return fail(THB_ERR_INVALID, "the plan takes 1 to " + std::to_string(plan->max_m) + " rows, the call has " +
                                         std::to_string(spec->m));
    if (spec->q_heads != plan->q_heads)
        return fail(THB_ERR_INVALID, "the plan was made for q_heads " + std::to_string(plan->q_heads) + ", not " +
                                         std::to_string(spec->q_heads));
    if (static_cast<uint64_t>(spec->row_off) + spec->m > rows->max_m)
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->max_m) + " rows, call needs " +
                                         std::to_string(static_cast<uint64_t>(spec->row_off) + spec->m));
    if (spec->seq != THB_SEQ_PER_ROW && spec->seq >= pool->arena.a.seqs())
        return fail(THB_ERR_INVALID, "sequence " + std::to_string(spec->seq) + " out of range");
    if (!(spec->softcap >= 0.0f)) return fail(THB_ERR_INVALID, "softcap must be >= 0");
    if (spec->q_dtype > THB_DT_BF16 || spec->y_dtype > THB_DT_BF16)
        return fail(THB_ERR_INVALID, "q_dtype and y_dtype must be THB_DT_F32, THB_DT_F16 or THB_DT_BF16");
    if (plan->append && !spec->causal)
        return fail(THB_ERR_INVALID, "a plan made with THB_DPLAN_APPEND takes causal calls only (the append runs "
                                     "inside the attention launch)");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);  // queued page-API calls first: the plan reads the page counts
        if (plan->list) {
            DListArgs la;
            la.rows.meta = rows->dev + 8 * static_cast<size_t>(spec->row_off);
            la.rows.ranges_out = static_cast<uint32_t*>(plan->blob.get()) + plan->ranges_off;
            la.rows.state = pool->state_dev;
            la.rows.npages_off = pool->state.npages_off;
            la.rows.m = spec->m;
            la.rows.seq_fixed = spec->seq;
            la.rows.causal = spec->causal;
            la.rows.window = spec->window;
            la.rows.page_shift = pool->page_shift;
            la.rows.seqs = pool->arena.a.seqs();
            la.rows.pos_limit = plan->pos_limit;
            la.blob = static_cast<uint32_t*>(plan->blob.get());
            la.G = spec->q_heads / pool->kv_heads;
            la.PL = pool->part_len;
            la.align = std::max<uint32_t>(pool->page_len, 16);
            la.WB = plan->wb;
            la.rg_magic = div16_magic(la.G <= kCols ? kCols / la.G : 1u);
            la.wb_magic = div16_magic(la.WB);
            la.pmax = plan->pmax;
            la.hd_t = plan->hd_max;
            la.groups_off = plan->groups_off;
            la.items_off = plan->items_off;
            la.bitems_off = plan->bitems_off;
            la.pairs_off = plan->pairs_off;
            la.order_off = plan->order_off;
            // a decode workgroup streams K and V at ~37 GB/s (one CU's share)
            la.dec_us_per_key = static_cast<float>(4.0 * plan->hd_max / 3.7e4);
            hipLaunchKernelGGL(dplan_list_kernel, dim3(1), dim3(kDPlanThreads), 0, s, la);
            THB_HIP(hipGetLastError());
            plan->spec = *spec;
            plan->rows = rows;
            plan->built = true;
            return THB_OK;
        }
        DPlanArgs a;
        a.meta = rows->dev + 8 * static_cast<size_t>(spec->row_off);
        a.blob = static_cast<uint32_t*>(plan->blob.get());
        a.state = pool->state_dev;
        a.npages_off = pool->state.npages_off;
        a.m = spec->m;
        a.seq_fixed = spec->seq;
        a.causal = spec->causal;
        a.window = spec->window;
        a.G = spec->q_heads / pool->kv_heads;
        a.PL = pool->part_len;
        a.align = std::max<uint32_t>(pool->page_len, 16);
        a.pmax = plan->pmax;
        a.gmax = plan->gmax;
        a.page_shift = pool->page_shift;
        a.seqs = pool->arena.a.seqs();
        a.items_off = plan->items_off;
        a.ranges_off = plan->ranges_off;
        a.merge_off = plan->merge_off;
        a.append = plan->append ? 1u : 0u;
        a.pos_limit = plan->pos_limit;
        hipLaunchKernelGGL(dplan_kernel, dim3(1), dim3(kDPlanThreads), 0, s, a);
        THB_HIP(hipGetLastError());
        plan->spec = *spec;
        plan->rows = rows;
        plan->built = true;
        return THB_OK;
    });
}

int thb_attn_dplan(thb_pool* pool, uint32_t layer, const void* q, void* y, const thb_dplan* plan, void* stream) {
    if (int rc = dplan_call_check(pool, layer, q, y, plan)) return rc;
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        const thb_attn_io io = make_io(q, y, nullptr, nullptr, 0, nullptr);
        if (plan->list)
            dplan_launch_list(pool, layer, io, plan, s);
        else
            dplan_launch_grid(pool, layer, io, plan, s);
        return THB_OK;
    });
}

int thb_attn_append_dplan(thb_pool* pool, uint32_t layer, const void* k_src, const void* v_src, uint32_t src_dtype,
                          const void* q, void* y, const thb_dplan* plan, void* stream) {
    if (int rc = dplan_call_check(pool, layer, q, y, plan)) return rc;
    if (!plan->append) return fail(THB_ERR_INVALID, "the plan was not made with THB_DPLAN_APPEND");
    if (!k_src || !v_src) return fail(THB_ERR_INVALID, "null source buffer");
    if (src_dtype > THB_DT_BF16) return fail(THB_ERR_INVALID, "unknown src_dtype " + std::to_string(src_dtype));
    if ((reinterpret_cast<uintptr_t>(k_src) & 15u) || (reinterpret_cast<uintptr_t>(v_src) & 15u))
        return fail(THB_ERR_INVALID, "source buffers must be 16-byte aligned");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        dplan_launch_grid(pool, layer, make_io(q, y, k_src, v_src, src_dtype, nullptr), plan, s);
        return THB_OK;
    });
}

int thb_dplan_set_pos_limit(thb_dplan* plan, uint32_t max_pos) {
    if (!plan) return fail(THB_ERR_INVALID, "null plan");
    plan->pos_limit = max_pos;
    plan->built = false;  // the limit is checked by the next build
    return THB_OK;
}

int thb_attn_step_dplan(thb_pool* pool, uint32_t layer, const thb_attn_io* io, const thb_dplan* plan, void* stream) {
    if (!io) return fail(THB_ERR_INVALID, "null io");
    if (int rc = dplan_call_check(pool, layer, io->q_dev, io->y_dev, plan)) return rc;
    const uint32_t hd = pool->geom[layer].head_dim;
    const uint32_t qes = plan->spec.q_dtype == THB_DT_F32 ? 4u : 2u;
    if (io->q_stride && (io->q_stride < hd || (io->q_stride * qes) % 16 != 0))
        return fail(THB_ERR_INVALID, "q_stride " + std::to_string(io->q_stride) +
                                         " must be 0 or at least head_dim, and a multiple of 16 bytes");
    if (io->gate_dev && io->gate_stride && io->gate_stride < hd)
        return fail(THB_ERR_INVALID, "gate_stride " + std::to_string(io->gate_stride) + " below head_dim");
    if (const thb_rope* rope = io->rope) {
        if (int rc = check_rope_tables(rope, hd)) return rc;
        if (plan->pos_limit == 0 || plan->pos_limit > rope->max_pos)
            return fail(THB_ERR_INVALID, "rotary embedding over a device plan needs the plan's position limit "
                                         "(thb_dplan_set_pos_limit, then thb_dplan_build) at most the tables' " +
                                             std::to_string(rope->max_pos) + " positions; the plan has " +
                                             std::to_string(plan->pos_limit));
    }
    const bool append = io->k_src_dev || io->v_src_dev;
    if (append) {
        if (!plan->append) return fail(THB_ERR_INVALID, "the plan was not made with THB_DPLAN_APPEND");
        if (!io->k_src_dev || !io->v_src_dev) return fail(THB_ERR_INVALID, "null source buffer");
        if (io->src_dtype > THB_DT_BF16)
            return fail(THB_ERR_INVALID, "unknown src_dtype " + std::to_string(io->src_dtype));
        if (io->rope && io->src_dtype == THB_DT_BF16)
            return fail(THB_ERR_INVALID, "rotary append takes f32 or f16 sources (src_dtype 2)");
        if ((reinterpret_cast<uintptr_t>(io->k_src_dev) & 15u) || (reinterpret_cast<uintptr_t>(io->v_src_dev) & 15u))
            return fail(THB_ERR_INVALID, "source buffers must be 16-byte aligned");
    }
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        if (plan->list)
            dplan_launch_list(pool, layer, *io, plan, s);
        else
            dplan_launch_grid(pool, layer, *io, plan, s);
        return THB_OK;
    });
}

}  // extern "C"
