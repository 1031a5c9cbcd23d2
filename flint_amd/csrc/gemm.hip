// The attention consumer's projection on the matrix cores: y[rows, n] =
// x[rows, k] . w[n, k]^T, plus y's old value when acc (ops::gemm_acc,
// crates/thuban_model/src/ops/gemm.rs:113-131; rows == 1 is the reference's
// gemv; the model calls it for o_proj with acc = "add into the residual",
// transformer/forward.rs:338-351).  Weights are bf16 or f16; x is f32 (the
// reference's activations), f16 or bf16 (the attention output the fused
// step writes for this product); y is f32.
//
// Precision: the matrix cores multiply two 16-bit operands.  An x that does
// not fit the weight's type exactly (f32, or f16 against bf16 weights) is
// split into a high and a low part of that type (hi = RNE(x), lo = RNE(x -
// hi)) and both are multiplied, so every product carries ~16 (bf16) or ~22
// (f16) bits of x against the exact weight, accumulated in f32.
//
// Two kernels:
//  * gemm_skinny (rows <= 16, decode): one workgroup per 16 output columns,
//    its 8 waves splitting the k-steps of 32.  Every wave issues the loads of
//    all its weight slices and x operands (a batch of up to NB steps) before
//    its first product, so a CU keeps 128 KiB of weights in flight; each
//    weight byte is read once (non-temporal), x comes from L2.  The 8 waves'
//    partial sums are added through LDS in wave order: one launch, no
//    atomics, deterministic.
//  * gemm_split (rows 17..64): K in slices of 1024, x's slice staged once
//    per workgroup in LDS; the workgroup that finishes a column block's last
//    slice adds the block's partial sums in slice order (the reference's
//    split-K merge_gemm.wgsl order), in the same launch.
//  * gemm_tile (rows > 64, prefill): 128 x 128 output tiles, 4 waves of
//    64 x 64, k-tiles of 64 staged in double-buffered LDS (rows of 144
//    bytes: conflict-free 16-byte operand reads), the next tile's loads in
//    flight during the products.
#include <algorithm>
#include <mutex>
#include <string>

#include "common.hpp"

namespace thb {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct GemmArgs {
    const void* x;      // [m, k] of x_dt
    const uint16_t* w;  // [n, k] bf16 or f16
    float* y;           // [m, n]
    uint32_t m, n, k, acc;
};

// Matrix-core operands of one weight type.
template <bool WF16>
struct WOps;

template <>
struct WOps<false> {
    typedef bf16x8 v8;
    typedef __bf16 e;
    __device__ static f32x4 mfma(const v8& a, const v8& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct WOps<true> {
    typedef f16x8 v8;
    typedef _Float16 e;
    __device__ static f32x4 mfma(const v8& a, const v8& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// x elements fit the weight's operand type exactly (one product), or need
// a low part (two products).
constexpr bool same_type(uint32_t xt, bool wf16) {
    return (xt == THB_DT_BF16 && !wf16) || (xt == THB_DT_F16 && wf16);
}
constexpr bool needs_lo(uint32_t xt, bool wf16) {
    return xt == THB_DT_F32 || (xt == THB_DT_F16 && !wf16);
}
// 32-bit words holding 8 x elements.
constexpr int x_words(uint32_t xt) { return xt == THB_DT_F32 ? 8 : 4; }

template <uint32_t XT>
__device__ inline void load_x8(const void* x, uint64_t e, uint32_t* out) {
    if constexpr (XT == THB_DT_F32) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(static_cast<const float*>(x) + e);
        const u32x4 b = *reinterpret_cast<const u32x4*>(static_cast<const float*>(x) + e + 4);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            out[i] = a[i];
            out[4 + i] = b[i];
        }
    } else {
        const u32x4 a = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + e);
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = a[i];
    }
}

// Element i of 8 x elements held as words, as f32.
template <uint32_t XT>
__device__ inline float x_elem(const uint32_t* w, int i) {
    if constexpr (XT == THB_DT_F32) {
        return __uint_as_float(w[i]);
    } else {
        const uint32_t h = (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
        if constexpr (XT == THB_DT_BF16)
            return __uint_as_float(h << 16);
        else
            return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
    }
}

// The high (and low) operand of 8 x elements in the weight's type.
template <uint32_t XT, bool WF16>
__device__ inline void x_operands(const uint32_t* w, typename WOps<WF16>::v8& hi, typename WOps<WF16>::v8& lo) {
    using E = typename WOps<WF16>::e;
    if constexpr (same_type(XT, WF16)) {
        hi = __builtin_bit_cast(typename WOps<WF16>::v8, u32x4{w[0], w[1], w[2], w[3]});
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float v = x_elem<XT>(w, i);
            const E h = static_cast<E>(v);
            hi[i] = h;
            if constexpr (needs_lo(XT, WF16)) lo[i] = static_cast<E>(v - static_cast<float>(h));
        }
    }
}

__device__ inline u32x4 ld_nt16(const void* p) { return __builtin_nontemporal_load(static_cast<const u32x4*>(p)); }

// Decode-sized rows: see the file comment.  MT = m-tiles of 16 rows (rows
// <= 16 MT), NB = k-steps whose loads are issued before the first product.
template <uint32_t XT, bool WF16, int MT, int NB>
__global__ __launch_bounds__(512) void gemm_skinny(GemmArgs a) {
    using O = WOps<WF16>;
    constexpr bool LO = needs_lo(XT, WF16);
    constexpr int XW = x_words(XT);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t c = lane & 15u, g = lane >> 4;
    const uint32_t n0 = blockIdx.x * 16u;
    const uint32_t steps = a.k >> 5;
    // The wave's chunk of k-steps, rotated by the workgroup index: at any
    // moment the workgroups read different parts of x (every workgroup reads
    // all of x from L2; in the same order they queued on the same lines).
    const uint32_t chunk = (wave + blockIdx.x) & 7u;
    const uint32_t s0 = chunk * steps / 8u, s1 = (chunk + 1) * steps / 8u;
    // A operand: weight row n0 + c, k = 32 s + 8 g .. + 8 (16 bytes).
    const uint16_t* wrow = a.w + static_cast<uint64_t>(n0 + c) * a.k + 8u * g;
    // The accumulated y of the writing waves is requested with the first
    // loads, not after the products (one round trip less).
    f32x4 y_old = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t y_row = 16u * wave + c;
    f32x4* yp = reinterpret_cast<f32x4*>(a.y + static_cast<uint64_t>(y_row) * a.n + n0 + 4u * g);
    if (a.acc && wave < static_cast<uint32_t>(MT) && y_row < a.m) y_old = *yp;
    f32x4 d[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) d[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = s0; sb < s1; sb += NB) {
        u32x4 wv[NB];
        uint32_t xv[NB][MT][XW];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const uint32_t s = sb + i;
            if (s < s1) {
                wv[i] = ld_nt16(wrow + 32u * s);
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const uint32_t row = 16u * t + c;  // B operand: x row, k = 32 s + 8 g .. + 8
                    if (row < a.m) {
                        load_x8<XT>(a.x, static_cast<uint64_t>(row) * a.k + 32u * s + 8u * g, xv[i][t]);
                    } else {
#pragma unroll
                        for (int q = 0; q < XW; q++) xv[i][t][q] = 0u;
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            if (sb + i < s1) {
                const typename O::v8 A = __builtin_bit_cast(typename O::v8, wv[i]);
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    typename O::v8 bh, bl;
                    x_operands<XT, WF16>(xv[i][t], bh, bl);
                    d[t] = O::mfma(A, bh, d[t]);
                    if constexpr (LO) d[t] = O::mfma(A, bl, d[t]);
                }
            }
        }
    }
    // Lane (c, g) holds D[n = 4 g + r][m = c] of each m-tile: add the 8
    // chunks' sums in k order and write y[16 t + c][n0 + 4 g .. + 4].
    __shared__ f32x4 red[8][MT][64];
#pragma unroll
    for (int t = 0; t < MT; t++) red[chunk][t][lane] = d[t];
    __syncthreads();
    if (wave < static_cast<uint32_t>(MT)) {
        f32x4 s = red[0][wave][lane];
#pragma unroll
        for (int q = 1; q < 8; q++) s += red[q][wave][lane];
        if (y_row < a.m) {
            if (a.acc) s += y_old;
            *yp = s;
        }
    }
}

// Rows > 64: 128 x 128 output tiles.  Wave (wn, wm) of the 2 x 2 grid
// computes 64 n x 64 m as 4 x 4 products per k-step of 32.  k-tiles of 64
// columns: the weight tile (128 n rows) and the x tile (128 m rows, its high
// and low parts) sit in LDS as rows of 8 16-byte chunks plus 16 bytes of
// padding (144 bytes), so the 16 lanes of an operand read hit distinct banks.
constexpr uint32_t kTile = 128, kTk = 64, kRowB = 144;

template <uint32_t XT, bool WF16>
__global__ __launch_bounds__(256) void gemm_tile(GemmArgs a) {
    using O = WOps<WF16>;
    constexpr bool LO = needs_lo(XT, WF16);
    constexpr int XW = x_words(XT);
    constexpr uint32_t kMat = kTile * kRowB;  // bytes of one operand tile
    constexpr uint32_t kBuf = (LO ? 3 : 2) * kMat;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kBuf];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t c = lane & 15u, g = lane >> 4, wn = wave & 1u, wm = wave >> 1;
    const uint32_t n0 = blockIdx.x * kTile, m0 = blockIdx.y * kTile;
    const uint32_t tiles = a.k / kTk;
    // Staging: thread t moves chunks q = t + 256 i (i < 4) of each tile:
    // row q / 8, 8-element chunk q % 8.
    u32x4 ws[4];
    uint32_t xs[4][XW];
    auto load_tile = [&](uint32_t kt) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = tid + 256u * i, r = q >> 3, ch = q & 7u;
            const uint32_t kk = kt * kTk + 8u * ch;
            ws[i] = n0 + r < a.n ? *reinterpret_cast<const u32x4*>(a.w + static_cast<uint64_t>(n0 + r) * a.k + kk)
                                 : u32x4{0u, 0u, 0u, 0u};
            if (m0 + r < a.m) {
                load_x8<XT>(a.x, static_cast<uint64_t>(m0 + r) * a.k + kk, xs[i]);
            } else {
#pragma unroll
                for (int w = 0; w < XW; w++) xs[i][w] = 0u;
            }
        }
    };
    auto store_tile = [&](uint32_t buf) {
        uint8_t* base = lds + buf * kBuf;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = tid + 256u * i, r = q >> 3, ch = q & 7u;
            const uint32_t off = r * kRowB + ch * 16u;
            *reinterpret_cast<u32x4*>(base + off) = ws[i];
            typename O::v8 hi, lo;
            x_operands<XT, WF16>(xs[i], hi, lo);
            *reinterpret_cast<typename O::v8*>(base + kMat + off) = hi;
            if constexpr (LO) *reinterpret_cast<typename O::v8*>(base + 2 * kMat + off) = lo;
        }
    };
    f32x4 d[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) d[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < tiles; kt++) {
        const uint32_t buf = kt & 1u;
        if (kt + 1 < tiles) load_tile(kt + 1);
        const uint8_t* base = lds + buf * kBuf;
#pragma unroll
        for (uint32_t ks = 0; ks < kTk / 32; ks++) {
            const uint32_t col = (4u * ks + g) * 16u;  // chunk of this lane's 8 k
            typename O::v8 wa[4], xb[4], xl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                wa[i] = *reinterpret_cast<const typename O::v8*>(base + (64u * wn + 16u * i + c) * kRowB + col);
                xb[i] = *reinterpret_cast<const typename O::v8*>(base + kMat + (64u * wm + 16u * i + c) * kRowB + col);
                if constexpr (LO)
                    xl[i] = *reinterpret_cast<const typename O::v8*>(base + 2 * kMat + (64u * wm + 16u * i + c) * kRowB +
                                                                     col);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    d[i][j] = O::mfma(wa[i], xb[j], d[i][j]);
                    if constexpr (LO) d[i][j] = O::mfma(wa[i], xl[j], d[i][j]);
                }
        }
        if (kt + 1 < tiles) store_tile(buf ^ 1u);
        __syncthreads();
    }
    // d[i][j]: n-tile i, m-tile j; lane (c, g) holds D[n = 4 g + r][m = c].
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t n = n0 + 64u * wn + 16u * i + 4u * g;
        if (n >= a.n) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t row = m0 + 64u * wm + 16u * j + c;
            if (row >= a.m) continue;
            f32x4* yp = reinterpret_cast<f32x4*>(a.y + static_cast<uint64_t>(row) * a.n + n);
            f32x4 s = d[i][j];
            if (a.acc) s += *yp;
            *yp = s;
        }
    }
}

// Rows 17..64: K split into S slices.  Workgroup (n-block of 64 columns, k
// slice q) stages x's slice once in LDS as B operands ([8-element k chunk]
// [row] x 16 bytes, high and low parts), so the 256 workgroups read x's
// slice once instead of all of x once per 16 columns (at 32 rows and k =
// 4096, reading all of x per workgroup measured 8.4 us of L2 traffic that
// did not overlap the 7.5 us weight stream; split: 12.2 us + the merge,
// against 16.3 us in one pass).  Wave w: n-tile
// w % 4, half w / 4 of the slice's k-steps, every weight load issued before
// the first product.  Partial sums go to part[q][m][n] (agent-scope
// atomic stores, coherent across the XCDs' L2 caches); the workgroup that
// finishes the column block's last slice (an arrival counter per block,
// relaxed agent-scope add after every thread's stores have completed) adds
// the block's slices in order, y = (acc ? y : 0) + part[0] + part[1] + ...,
// and clears the counter for the next call.  No workgroup waits for
// another.
struct SplitArgs {
    GemmArgs g;
    float* part;    // [S][m][n]
    uint32_t* cnt;  // [n / 64] arrival counters, zero between launches
    uint32_t S, m16;
};

__device__ inline void publish4(float* p, const f32x4& v) {
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __hip_atomic_store(q, (uint64_t(__float_as_uint(v[1])) << 32) | __float_as_uint(v[0]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (uint64_t(__float_as_uint(v[3])) << 32) | __float_as_uint(v[2]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline f32x4 coherent4(const float* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return f32x4{__uint_as_float(static_cast<uint32_t>(lo)), __uint_as_float(static_cast<uint32_t>(lo >> 32)),
                 __uint_as_float(static_cast<uint32_t>(hi)), __uint_as_float(static_cast<uint32_t>(hi >> 32))};
}

template <uint32_t XT, bool WF16, int MT>
__global__ __launch_bounds__(512) void gemm_split(SplitArgs sa) {
    using O = WOps<WF16>;
    constexpr bool LO = needs_lo(XT, WF16);
    constexpr int XW = x_words(XT);
    constexpr int NWB = 16;  // weight loads per wave issued up front (more: a second batch)
    extern __shared__ __attribute__((aligned(16))) uint8_t xs_lds[];
    const GemmArgs& a = sa.g;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t c = lane & 15u, g = lane >> 4, nt = wave & 3u, half = wave >> 2;
    const uint32_t n0 = blockIdx.x * 64u + 16u * nt, q = blockIdx.y;
    const uint32_t steps = a.k >> 5;
    const uint32_t q0 = q * steps / sa.S, q1 = (q + 1) * steps / sa.S, nq = q1 - q0;
    const uint32_t s0 = q0 + half * nq / 2u, s1 = q0 + (half + 1) * nq / 2u;
    const uint32_t m16 = sa.m16, chunks = 4u * nq;  // 8-element k chunks of the slice
    // LDS: operand (chunk ch, row r) at (ch * (m16 + 1) + r) * 16 bytes; the
    // padding row keeps both the staging stores (consecutive chunks of a
    // row) and the operand reads (consecutive rows of a chunk) free of bank
    // conflicts.
    const uint32_t rs = m16 + 1u;
    uint8_t* lo_base = xs_lds + static_cast<size_t>(chunks) * rs * 16u;
    // Order of the loads: the first XB items of the x slice, then the first
    // batch of weights, so x arrives first (a wave's loads return in order)
    // and is staged while the weights stream.
    constexpr int XB = 8;
    const uint32_t items = chunks * m16;  // item i: row i / chunks, chunk i % chunks (coalesced reads)
    uint32_t xv[XB][XW];
    auto load_items = [&](uint32_t i0) {
#pragma unroll
        for (int j = 0; j < XB; j++) {
            const uint32_t i = i0 + 512u * j + tid, r = i / chunks, ch = i - r * chunks;
            if (i < items && r < a.m) {
                load_x8<XT>(a.x, static_cast<uint64_t>(r) * a.k + 8u * (4u * q0 + ch), xv[j]);
            } else {
#pragma unroll
                for (int w = 0; w < XW; w++) xv[j][w] = 0u;
            }
        }
    };
    auto store_items = [&](uint32_t i0) {
#pragma unroll
        for (int j = 0; j < XB; j++) {
            const uint32_t i = i0 + 512u * j + tid, r = i / chunks, ch = i - r * chunks;
            if (i < items) {
                typename O::v8 hi, lo;
                x_operands<XT, WF16>(xv[j], hi, lo);
                const size_t off = (static_cast<size_t>(ch) * rs + r) * 16u;
                *reinterpret_cast<typename O::v8*>(xs_lds + off) = hi;
                if constexpr (LO) *reinterpret_cast<typename O::v8*>(lo_base + off) = lo;
            }
        }
    };
    load_items(0);
    const uint16_t* wrow = a.w + static_cast<uint64_t>(n0 + c) * a.k + 8u * g;
    u32x4 wv[NWB];
#pragma unroll
    for (int i = 0; i < NWB; i++)
        if (s0 + i < s1) wv[i] = ld_nt16(wrow + 32u * (s0 + i));
    store_items(0);
    for (uint32_t i0 = 512u * XB; i0 < items; i0 += 512u * XB) {  // more rows than fit one batch
        load_items(i0);
        store_items(i0);
    }
    __syncthreads();
    f32x4 d[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) d[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t sb = s0; sb < s1; sb += NWB) {
        if (sb != s0) {  // later batches (more than NWB steps per wave)
#pragma unroll
            for (int i = 0; i < NWB; i++)
                if (sb + i < s1) wv[i] = ld_nt16(wrow + 32u * (sb + i));
        }
#pragma unroll
        for (int i = 0; i < NWB; i++) {
            if (sb + i < s1) {
                const typename O::v8 A = __builtin_bit_cast(typename O::v8, wv[i]);
                const uint32_t ch = 4u * (sb + i - q0) + g;
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const size_t off = (static_cast<size_t>(ch) * rs + 16u * t + c) * 16u;
                    d[t] = O::mfma(A, *reinterpret_cast<const typename O::v8*>(xs_lds + off), d[t]);
                    if constexpr (LO)
                        d[t] = O::mfma(A, *reinterpret_cast<const typename O::v8*>(lo_base + off), d[t]);
                }
            }
        }
    }
    // The two halves of each n-tile add through LDS (half 0 + half 1), then
    // half 0 writes part[q][16 t + c][n0 + 4 g .. + 4].
    __syncthreads();
    f32x4* red = reinterpret_cast<f32x4*>(xs_lds);  // [4 n-tiles][MT][64]
    if (half == 1)
#pragma unroll
        for (int t = 0; t < MT; t++) red[(nt * MT + t) * 64u + lane] = d[t];
    __syncthreads();
    if (half == 0) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const uint32_t row = 16u * t + c;
            if (row < a.m) {
                const f32x4 s = d[t] + red[(nt * MT + t) * 64u + lane];
                publish4(sa.part + (static_cast<uint64_t>(q) * a.m + row) * a.n + n0 + 4u * g, s);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have completed
    __shared__ uint32_t s_arrived;
    __syncthreads();
    uint32_t* cnt = sa.cnt + blockIdx.x;
    if (tid == 0) s_arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived + 1u != sa.S) return;
    // The block's last slice: y[row][64 blockIdx.x + 4 u .. + 4] for every
    // row, 8 slices requested at once and added in slice order.
    const uint64_t mn = static_cast<uint64_t>(a.m) * a.n;
    for (uint32_t u = tid; u < a.m * 16u; u += 512u) {
        const uint32_t row = u >> 4;
        const uint64_t idx = static_cast<uint64_t>(row) * a.n + 64u * blockIdx.x + 4u * (u & 15u);
        f32x4* yp = reinterpret_cast<f32x4*>(a.y + idx);
        f32x4 acc = a.acc ? *yp : f32x4{0.f, 0.f, 0.f, 0.f};
        for (uint32_t q0 = 0; q0 < sa.S; q0 += 8) {
            f32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (q0 + j < sa.S) v[j] = coherent4(sa.part + (q0 + j) * mn + idx);
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (q0 + j < sa.S) acc += v[j];
        }
        *yp = acc;
    }
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// k-steps of 32 per slice of the split kernel (half that with a low part).
#ifndef THB_GEMM_SLICE_STEPS
#define THB_GEMM_SLICE_STEPS 32
#endif

// Library-owned partial sums of the split kernel, per device (the
// reference's backend keeps gemm_partial the same way, matmul.rs:9-18).
constexpr int kMaxDev = 64;
DevBuf g_part[kMaxDev];
DevBuf g_cnt[kMaxDev];  // split kernel's arrival counters (zero between launches)
std::mutex g_part_mu;

template <uint32_t XT, bool WF16>
void launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.m > 64) {
        const dim3 grid((a.n + kTile - 1) / kTile, (a.m + kTile - 1) / kTile);
        hipLaunchKernelGGL((gemm_tile<XT, WF16>), grid, dim3(256), 0, s, a);
        return;
    }
    constexpr int NB = XT == THB_DT_F32 ? 8 : 16;  // steps prefetched per batch
    if (a.m <= 16 || a.n % 64 != 0) {
        // Up to 16 rows (the gemv included), and widths that are not a
        // multiple of 64: one pass, every workgroup reading all of x.  At 16
        // rows and k = 4096 that is 128 KiB per workgroup from L2, cheaper
        // than the split kernel's partial round trip (Llama-3-8B o_proj,
        // kernel trace: 9.6 us one pass; 11.2 us split + 1.5-4 us merge).
        const dim3 grid(a.n / 16);
        if (a.m <= 16)
            hipLaunchKernelGGL((gemm_skinny<XT, WF16, 1, NB>), grid, dim3(512), 0, s, a);
        else if (a.m <= 32)
            hipLaunchKernelGGL((gemm_skinny<XT, WF16, 2, NB>), grid, dim3(512), 0, s, a);
        else if (a.m <= 48)
            hipLaunchKernelGGL((gemm_skinny<XT, WF16, 3, NB / 2>), grid, dim3(512), 0, s, a);
        else
            hipLaunchKernelGGL((gemm_skinny<XT, WF16, 4, NB / 2>), grid, dim3(512), 0, s, a);
        return;
    }
    // Slices of at most 1024 k (512 with a low part), so that x's slice for
    // 64 rows fits 128 KiB of LDS; a function of k and the types only, so a
    // row's sums do not depend on how many rows the call has.
    constexpr bool LO = needs_lo(XT, WF16);
    const uint32_t steps = a.k / 32, kq = LO ? THB_GEMM_SLICE_STEPS / 2 : THB_GEMM_SLICE_STEPS;
    const uint32_t S = std::max<uint32_t>(1, (steps + kq - 1) / kq);
    const uint32_t m16 = (a.m + 15) / 16 * 16;
    const uint32_t nq_max = (steps + S - 1) / S;
    const size_t lds = std::max<size_t>(static_cast<size_t>(4u * nq_max) * (m16 + 1) * 16u * (LO ? 2 : 1),
                                        4u * 4u * 64u * 16u);
    int dev = 0;
    THB_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDev) throw HipError{hipErrorInvalidDevice, "gemm partial buffer"};
    float* part;
    uint32_t* cnt;
    {
        std::lock_guard<std::mutex> lock(g_part_mu);
        part = static_cast<float*>(g_part[dev].reserve(static_cast<size_t>(S) * a.m * a.n * 4, false, s));
        cnt = static_cast<uint32_t*>(g_cnt[dev].reserve(static_cast<size_t>(a.n / 64) * 4, true, s));
    }
    SplitArgs sa;
    sa.g = a;
    sa.part = part;
    sa.cnt = cnt;
    sa.S = S;
    sa.m16 = m16;
    const dim3 grid(a.n / 64, S);
    if (a.m <= 16)
        hipLaunchKernelGGL((gemm_split<XT, WF16, 1>), grid, dim3(512), lds, s, sa);
    else if (a.m <= 32)
        hipLaunchKernelGGL((gemm_split<XT, WF16, 2>), grid, dim3(512), lds, s, sa);
    else if (a.m <= 48)
        hipLaunchKernelGGL((gemm_split<XT, WF16, 3>), grid, dim3(512), lds, s, sa);
    else
        hipLaunchKernelGGL((gemm_split<XT, WF16, 4>), grid, dim3(512), lds, s, sa);
    THB_HIP(hipGetLastError());
}

template <bool WF16>
void launch_w(uint32_t x_dt, const GemmArgs& a, hipStream_t s) {
    switch (x_dt) {
        case THB_DT_F32: launch_gemm<THB_DT_F32, WF16>(a, s); break;
        case THB_DT_F16: launch_gemm<THB_DT_F16, WF16>(a, s); break;
        default: launch_gemm<THB_DT_BF16, WF16>(a, s); break;
    }
}

}  // namespace
}  // namespace thb

using namespace thb;

extern "C" {

int thb_check_gemm_dims(uint32_t n, uint32_t k) {
    // ops::check_gemm_dims (crates/thuban_model/src/ops/gemm.rs:133-146)
    if (n % 16 != 0 || k % 64 != 0)
        return fail(THB_ERR_CONFIG, "dimension pair (N=" + std::to_string(n) + ", K=" + std::to_string(k) +
                                        ") does not satisfy N%16 and K%64");
    return THB_OK;
}

int thb_gemm_acc(const void* x, uint32_t x_dtype, const void* w, uint32_t w_dtype, float* y, uint32_t rows,
                 uint32_t n, uint32_t k, uint32_t acc, void* stream) {
    if (int rc = thb_check_gemm_dims(n, k)) return rc;
    if (rows == 0 || n == 0 || k == 0) return THB_OK;
    if (!x || !w || !y) return fail(THB_ERR_INVALID, "null x, w or y");
    if (x_dtype > THB_DT_BF16) return fail(THB_ERR_INVALID, "unknown x_dtype " + std::to_string(x_dtype));
    if (w_dtype != THB_DT_BF16 && w_dtype != THB_DT_F16)
        return fail(THB_ERR_INVALID, "weights must be THB_DT_BF16 or THB_DT_F16 (w_dtype " + std::to_string(w_dtype) +
                                         ")");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(y)) & 15u)
        return fail(THB_ERR_INVALID, "x, w and y must be 16-byte aligned");
    if (static_cast<uint64_t>(rows) * k >= (1ull << 40) || static_cast<uint64_t>(n) * k >= (1ull << 40))
        return fail(THB_ERR_INVALID, "gemm operands too large");
    return guarded([&]() -> int {
        GemmArgs a;
        a.x = x;
        a.w = static_cast<const uint16_t*>(w);
        a.y = y;
        a.m = rows;
        a.n = n;
        a.k = k;
        a.acc = acc ? 1u : 0u;
        hipStream_t s = as_stream(stream);
        if (w_dtype == THB_DT_F16)
            launch_w<true>(x_dtype, a, s);
        else
            launch_w<false>(x_dtype, a, s);
        THB_HIP(hipGetLastError());
        return THB_OK;
    });
}

}  // extern "C"
