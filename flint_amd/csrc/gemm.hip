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
//  * gemm_skinny (rows <= 64, decode): one workgroup per 16 output columns,
//    its 8 waves splitting the k-steps of 32.  Every wave issues the loads of
//    all its weight slices and x operands (a batch of up to NB steps) before
//    its first product, so a CU keeps 128 KiB of weights in flight; each
//    weight byte is read once (non-temporal), x comes from L2.  The 8 waves'
//    partial sums are added through LDS in wave order: one launch, no
//    atomics, deterministic.
//  * gemm_tile (rows > 64, prefill): 128 x 128 output tiles, 4 waves of
//    64 x 64, k-tiles of 64 staged in double-buffered LDS (rows of 144
//    bytes: conflict-free 16-byte operand reads), the next tile's loads in
//    flight during the products.
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
    const uint32_t s0 = wave * steps / 8u, s1 = (wave + 1) * steps / 8u;
    // A operand: weight row n0 + c, k = 32 s + 8 g .. + 8 (16 bytes).
    const uint16_t* wrow = a.w + static_cast<uint64_t>(n0 + c) * a.k + 8u * g;
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
    // waves' sums in wave order and write y[16 t + c][n0 + 4 g .. + 4].
    __shared__ f32x4 red[8][MT][64];
#pragma unroll
    for (int t = 0; t < MT; t++) red[wave][t][lane] = d[t];
    __syncthreads();
    if (wave < static_cast<uint32_t>(MT)) {
        f32x4 s = red[0][wave][lane];
#pragma unroll
        for (int q = 1; q < 8; q++) s += red[q][wave][lane];
        const uint32_t row = 16u * wave + c;
        if (row < a.m) {
            f32x4* yp = reinterpret_cast<f32x4*>(a.y + static_cast<uint64_t>(row) * a.n + n0 + 4u * g);
            if (a.acc) s += *yp;
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

template <uint32_t XT, bool WF16>
void launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.m > 64) {
        const dim3 grid((a.n + kTile - 1) / kTile, (a.m + kTile - 1) / kTile);
        hipLaunchKernelGGL((gemm_tile<XT, WF16>), grid, dim3(256), 0, s, a);
        return;
    }
    const dim3 grid(a.n / 16);
    // Steps prefetched per batch: all 16 of a wave at k = 4096 for up to 32
    // rows of 16-bit x; fewer where the operands take more registers.
    constexpr int NB2 = XT == THB_DT_F32 ? 8 : 16;
    constexpr int NB4 = XT == THB_DT_F32 ? 4 : 8;
    if (a.m <= 16)
        hipLaunchKernelGGL((gemm_skinny<XT, WF16, 1, NB2>), grid, dim3(512), 0, s, a);
    else if (a.m <= 32)
        hipLaunchKernelGGL((gemm_skinny<XT, WF16, 2, NB2>), grid, dim3(512), 0, s, a);
    else if (a.m <= 48)
        hipLaunchKernelGGL((gemm_skinny<XT, WF16, 3, NB4>), grid, dim3(512), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_skinny<XT, WF16, 4, NB4>), grid, dim3(512), 0, s, a);
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
