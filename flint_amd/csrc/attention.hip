// Paged attention: one launch per call over every row of the batch.
//
// Semantics follow the reference kernel attn.wgsl:53-365: per row i, key j
// is valid iff (!causal || j <= pos_i) && j >= window_start_i && j < kv_len,
// with kv_len and window_start exactly as attn.wgsl:78-88 (computed on the
// host into per-row [lo, hi) ranges).  Softmax in f32, base 2 internally.
//
// Work decomposition (MI355X):
//  * A "group" is a set of query vectors that read the same keys: R rows of
//    one sequence x H query heads of one KV head (GQA packing: every K/V
//    byte is read once for all NQ_PER_KV heads).  QV = R*H <= QVM.
//  * Keys are split into fixed logical partitions of part_len tokens
//    (split-K).  One workgroup (4 waves) handles one (group, partition, KV
//    head); each wave a quarter of the partition.  Partition boundaries are
//    fixed in logical token space, so the arithmetic of a row depends only on
//    that row: batch == solo and paged == contiguous hold bit-exactly.
//  * Inside a wave, DL lanes share one token: each lane loads 16 bytes per
//    token per 64*DL/8 dims (coalesced 128-byte segments), computes partial
//    dot products, and a DPP butterfly sums them across the DL lanes.
//  * f16 KV: q is rounded to f16 and QK^T uses v_dot2_f32_f16; PV packs two
//    tokens' probabilities into one f16x2 and uses v_dot2_f32_f16 as well.
//    bf16 KV (reference parity): plain f32 FMA after the exact bf16->f32 shift.
//  * Online softmax with a lazy rescale: the running max only moves when a
//    score exceeds it by more than 2^8 in probability space.
//  * The four waves' 4*T partial states are merged through LDS; with more
//    than one partition the workgroup writes (m, l, o) to scratch and the
//    last workgroup of the group (atomic arrival counter) merges all
//    partitions in partition order and writes y.  Counters reset themselves.
#include <algorithm>
#include <string>

#include "pool.hpp"

namespace thb {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr float kTau = 8.0f;          // lazy-rescale threshold (log2 units)
constexpr float kFloor = -1.0e30f;    // initial running max (finite on purpose)
constexpr uint32_t kGroupWords = 10;  // r0, R, h0, H, seq, lo, hi, n_parts, part0, item0
constexpr uint32_t kMaxPartPages = 256;
// Floats in the LDS o-buffer of every variant (SLOTS * QVM * HD == 16384).
constexpr uint32_t kMergeFloats = 16384;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

struct AttnArgs {
    const void* q;
    void* y;
    const uint32_t* groups;
    const uint32_t* items;
    const uint32_t* ranges;  // [m][2]: lo, hi
    const uint32_t* table;
    const uint16_t* k;
    const uint16_t* v;
    float* part_o;   // [n_items][n_kvh][QVM][hd]
    float* part_ml;  // [n_items][n_kvh][QVM][2]
    uint32_t* counters;  // [n_groups][n_kvh]
    uint64_t plane;  // elements per head plane
    uint32_t max_pages, page_shift, q_heads, nq_per_kv, head_dim, part_len, n_kvh;
    float qscale;  // scale * log2(e), or scale / softcap
    float cap2;    // softcap * log2(e), 0 = no soft-cap
    uint32_t q_f16, y_f16;
};

template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF,
                                                                     false));
}

// Sum over the DL consecutive lanes that share a token (DL in 8..64).
template <int DL>
__device__ __forceinline__ float group_sum(float x) {
    x = dpp_add<0xB1>(x);   // quad_perm [1,0,3,2]: xor 1
    x = dpp_add<0x4E>(x);   // quad_perm [2,3,0,1]: xor 2
    x = dpp_add<0x141>(x);  // row_half_mirror: sums 8 lanes
    if constexpr (DL >= 16) x = dpp_add<0x140>(x);  // row_mirror: 16 lanes
    if constexpr (DL >= 32) x += __shfl_xor(x, 16);
    if constexpr (DL >= 64) x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float tanh_approx(float x) {
    // tanh(x) = 1 - 2 / (exp(2x) + 1); saturates cleanly at +-1.
    const float e = fast_exp2(x * 2.8853900817779268f);  // 2 * log2(e)
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    half2_t h = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ uint32_t w4(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

template <int HD, int QVM, bool F16>
struct Cfg {
    static constexpr int DL = HD * QVM / 64;  // lanes per token
    static constexpr int T = 64 / DL;         // token slots per wave
    static constexpr int NR = HD / (8 * DL);  // 16-byte chunks per lane per token
    static constexpr int U = F16 ? 4 : 2;     // tokens per slot per iteration
    static constexpr int TPI = T * U;         // tokens per wave iteration
    static constexpr int SLOTS = kWaves * T;  // partial states per workgroup
    static_assert(NR * QVM == 8, "register budget: o holds 8*NR*QVM/8 floats per lane");
    static_assert(T * DL == 64, "wave64");
    static_assert(SLOTS * QVM * HD == kMergeFloats, "LDS o-buffer size");
};

template <int HD, int QVM, bool F16>
__global__ __launch_bounds__(kThreads, 2) void attn_splitk(AttnArgs a) {
    using C = Cfg<HD, QVM, F16>;
    constexpr int DL = C::DL, T = C::T, NR = C::NR, U = C::U, TPI = C::TPI, SLOTS = C::SLOTS;

    __shared__ float s_o[SLOTS * QVM * HD];
    __shared__ float s_m[SLOTS * QVM];
    __shared__ float s_l[SLOTS * QVM];
    __shared__ float s_w[SLOTS * QVM];
    __shared__ float s_red[2 * QVM];
    __shared__ uint32_t s_page[kMaxPartPages];
    __shared__ uint32_t s_last;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t slot = lane / DL, li = lane % DL;
    const uint32_t item = blockIdx.x, kvh = blockIdx.y;

    const uint32_t gi = a.items[item];
    const uint32_t* G = a.groups + gi * kGroupWords;
    const uint32_t r0 = G[0], R = G[1], h0 = G[2], H = G[3], seq = G[4];
    const uint32_t glo = G[5], ghi = G[6], n_parts = G[7], part0 = G[8], item0 = G[9];
    const uint32_t part = part0 + (item - item0);
    const uint32_t P = a.part_len;
    const uint32_t pbeg = part * P;
    const uint32_t tb = max(glo, pbeg), te = min(ghi, pbeg + P);
    const uint32_t QV = R * H;
    const uint32_t hd = a.head_dim;
    const uint32_t pmask = (1u << a.page_shift) - 1u;

    // Block-table entries of this partition (only pages that hold keys).
    {
        const uint32_t npg = P >> a.page_shift;
        const uint32_t lp0 = pbeg >> a.page_shift;
        const uint32_t* trow = a.table + static_cast<uint64_t>(seq) * a.max_pages;
        for (uint32_t i = tid; i < npg; i += kThreads) {
            const uint32_t lp = lp0 + i;
            const bool used = tb < te && (lp << a.page_shift) < te && ((lp + 1) << a.page_shift) > tb;
            s_page[i] = used ? trow[lp] : 0u;
        }
    }

    // Query vectors and row ranges of this lane's QV slots.
    uint32_t rlo[QVM], rhi[QVM];
    uint32_t qh[F16 ? QVM : 1][NR][4];
    float qf[F16 ? 1 : QVM][NR][8];
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) {
        const bool on = static_cast<uint32_t>(qv) < QV;
        const uint32_t rr = on ? static_cast<uint32_t>(qv) / H : 0u;
        const uint32_t hh = on ? static_cast<uint32_t>(qv) - rr * H : 0u;
        const uint32_t row = r0 + rr;
        rlo[qv] = on ? a.ranges[2 * row] : 0u;
        rhi[qv] = on ? a.ranges[2 * row + 1] : 0u;
        const uint32_t head = kvh * a.nq_per_kv + h0 + hh;
        const uint64_t qbase = (static_cast<uint64_t>(row) * a.q_heads + head) * hd;
#pragma unroll
        for (int c = 0; c < NR; c++) {
            const uint32_t d0 = 8u * li + 8u * DL * c;
            float x[8];
            if (on && d0 < hd) {
                if (a.q_f16) {
                    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qbase + d0);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        half2_t h2 = __builtin_bit_cast(half2_t, w4(w, j));
                        x[2 * j] = static_cast<float>(h2.x);
                        x[2 * j + 1] = static_cast<float>(h2.y);
                    }
                } else {
                    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.q) + qbase + d0);
                    const float4 u0 = p[0], u1 = p[1];
                    x[0] = u0.x; x[1] = u0.y; x[2] = u0.z; x[3] = u0.w;
                    x[4] = u1.x; x[5] = u1.y; x[6] = u1.z; x[7] = u1.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) x[j] = 0.0f;
            }
            if constexpr (F16) {
#pragma unroll
                for (int j = 0; j < 4; j++) qh[qv][c][j] = pack_f16(x[2 * j] * a.qscale, x[2 * j + 1] * a.qscale);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) qf[qv][c][j] = x[j] * a.qscale;
            }
        }
    }
    __syncthreads();

    float mq[QVM], lq[QVM], o[QVM][NR * 8];
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) {
        mq[qv] = kFloor;
        lq[qv] = 0.0f;
#pragma unroll
        for (int j = 0; j < NR * 8; j++) o[qv][j] = 0.0f;
    }

    // This wave's quarter of the partition, clipped to [tb, te).
    const uint32_t wq = P / kWaves;
    const uint32_t wbeg = pbeg + wave * wq, wend = wbeg + wq;
    const uint32_t lo_c = max(tb, wbeg), hi_c = min(te, wend);
    const uint32_t it_first = lo_c < hi_c ? (lo_c - wbeg) / TPI : 0u;
    const uint32_t it_end = lo_c < hi_c ? (hi_c - wbeg + TPI - 1) / TPI : 0u;
    const uint16_t* kplane = a.k + static_cast<uint64_t>(kvh) * a.plane;
    const uint16_t* vplane = a.v + static_cast<uint64_t>(kvh) * a.plane;

    for (uint32_t it = it_first; it < it_end; it++) {
        const uint32_t t0 = wbeg + it * TPI;
        uint4 kr[U][NR], vr[U][NR];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t tok = t0 + u * T + slot;
            const bool valid = tok >= tb && tok < te;
            const uint32_t page = s_page[(tok - pbeg) >> a.page_shift];
            const uint64_t base = ((static_cast<uint64_t>(page) << a.page_shift) | (tok & pmask)) * hd;
#pragma unroll
            for (int c = 0; c < NR; c++) {
                const uint32_t d0 = 8u * li + 8u * DL * c;
                if (valid && d0 < hd) {
                    kr[u][c] = *reinterpret_cast<const uint4*>(kplane + base + d0);
                    vr[u][c] = *reinterpret_cast<const uint4*>(vplane + base + d0);
                } else {
                    kr[u][c] = make_uint4(0, 0, 0, 0);
                    vr[u][c] = make_uint4(0, 0, 0, 0);
                }
            }
        }

        // Scores s[u][qv] (log2 domain), summed over the DL lanes of a token.
        float s[U][QVM];
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int qv = 0; qv < QVM; qv++) {
                float acc = 0.0f;
#pragma unroll
                for (int c = 0; c < NR; c++) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if constexpr (F16) {
                            acc = dot2(qh[qv][c][j], w4(kr[u][c], j), acc);
                        } else {
                            const uint32_t w = w4(kr[u][c], j);
                            acc = fmaf(qf[qv][c][2 * j], bf_lo(w), acc);
                            acc = fmaf(qf[qv][c][2 * j + 1], bf_hi(w), acc);
                        }
                    }
                }
                s[u][qv] = group_sum<DL>(acc);
            }
        }

        float p[U][QVM];
#pragma unroll
        for (int qv = 0; qv < QVM; qv++) {
            float mx = kFloor;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint32_t tok = t0 + u * T + slot;
                float x = s[u][qv];
                if (a.cap2 != 0.0f) x = a.cap2 * tanh_approx(x);
                const bool ok = tok >= rlo[qv] && tok < rhi[qv];
                x = ok ? x : -INFINITY;
                s[u][qv] = x;
                mx = fmaxf(mx, x);
            }
            if (mx > mq[qv] + kTau) {
                const float alpha = fast_exp2(mq[qv] - mx);
                lq[qv] *= alpha;
#pragma unroll
                for (int j = 0; j < NR * 8; j++) o[qv][j] *= alpha;
                mq[qv] = mx;
            }
#pragma unroll
            for (int u = 0; u < U; u++) p[u][qv] = fast_exp2(s[u][qv] - mq[qv]);
        }

        if constexpr (F16) {
#pragma unroll
            for (int pr = 0; pr < U / 2; pr++) {
                uint32_t pp[QVM];
#pragma unroll
                for (int qv = 0; qv < QVM; qv++) {
                    pp[qv] = pack_f16(p[2 * pr][qv], p[2 * pr + 1][qv]);
                    lq[qv] = dot2(pp[qv], 0x3C003C00u, lq[qv]);  // + both rounded weights
                }
#pragma unroll
                for (int c = 0; c < NR; c++) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t va = w4(vr[2 * pr][c], j), vb = w4(vr[2 * pr + 1][c], j);
                        const uint32_t vlo = __builtin_amdgcn_perm(vb, va, 0x05040100u);  // (va.lo, vb.lo)
                        const uint32_t vhi = __builtin_amdgcn_perm(vb, va, 0x07060302u);  // (va.hi, vb.hi)
#pragma unroll
                        for (int qv = 0; qv < QVM; qv++) {
                            o[qv][c * 8 + 2 * j] = dot2(pp[qv], vlo, o[qv][c * 8 + 2 * j]);
                            o[qv][c * 8 + 2 * j + 1] = dot2(pp[qv], vhi, o[qv][c * 8 + 2 * j + 1]);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++) {
#pragma unroll
                for (int qv = 0; qv < QVM; qv++) lq[qv] += p[u][qv];
#pragma unroll
                for (int c = 0; c < NR; c++) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t w = w4(vr[u][c], j);
                        const float v0 = bf_lo(w), v1 = bf_hi(w);
#pragma unroll
                        for (int qv = 0; qv < QVM; qv++) {
                            o[qv][c * 8 + 2 * j] = fmaf(p[u][qv], v0, o[qv][c * 8 + 2 * j]);
                            o[qv][c * 8 + 2 * j + 1] = fmaf(p[u][qv], v1, o[qv][c * 8 + 2 * j + 1]);
                        }
                    }
                }
            }
        }
    }

    // ---- merge the workgroup's SLOTS partial states through LDS ----------
    const uint32_t sidx = wave * T + slot;
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) {
        if (li == 0) {
            s_m[sidx * QVM + qv] = mq[qv];
            s_l[sidx * QVM + qv] = lq[qv];
        }
#pragma unroll
        for (int c = 0; c < NR; c++) {
            const uint32_t d0 = 8u * li + 8u * DL * c;
            float4* dst = reinterpret_cast<float4*>(s_o + (sidx * QVM + qv) * HD + d0);
            dst[0] = make_float4(o[qv][c * 8 + 0], o[qv][c * 8 + 1], o[qv][c * 8 + 2], o[qv][c * 8 + 3]);
            dst[1] = make_float4(o[qv][c * 8 + 4], o[qv][c * 8 + 5], o[qv][c * 8 + 6], o[qv][c * 8 + 7]);
        }
    }
    __syncthreads();
    if (tid < static_cast<uint32_t>(QVM)) {
        float M = kFloor;
        for (int sl = 0; sl < SLOTS; sl++) M = fmaxf(M, s_m[sl * QVM + tid]);
        float L = 0.0f;
        for (int sl = 0; sl < SLOTS; sl++) {
            const float w = fast_exp2(s_m[sl * QVM + tid] - M);
            s_w[sl * QVM + tid] = w;
            L += w * s_l[sl * QVM + tid];
        }
        s_red[2 * tid] = M;
        s_red[2 * tid + 1] = L;
    }
    __syncthreads();

    const uint32_t nout = QV * hd;
    if (n_parts == 1) {
        for (uint32_t idx = tid; idx < nout; idx += kThreads) {
            const uint32_t qv = idx / hd, d = idx - qv * hd;
            float acc = 0.0f;
            for (int sl = 0; sl < SLOTS; sl++) acc += s_w[sl * QVM + qv] * s_o[(sl * QVM + qv) * HD + d];
            const float yv = acc / s_red[2 * qv + 1];
            const uint32_t rr = qv / H, hh = qv - rr * H;
            const uint64_t yi = (static_cast<uint64_t>(r0 + rr) * a.q_heads + kvh * a.nq_per_kv + h0 + hh) * hd + d;
            if (a.y_f16)
                static_cast<_Float16*>(a.y)[yi] = static_cast<_Float16>(yv);
            else
                static_cast<float*>(a.y)[yi] = yv;
        }
        return;
    }

    // ---- several partitions: publish (m, l, o), last arrival merges -------
    const uint64_t pbase = (static_cast<uint64_t>(item) * a.n_kvh + kvh) * QVM;
    for (uint32_t idx = tid; idx < nout; idx += kThreads) {
        const uint32_t qv = idx / hd, d = idx - qv * hd;
        float acc = 0.0f;
        for (int sl = 0; sl < SLOTS; sl++) acc += s_w[sl * QVM + qv] * s_o[(sl * QVM + qv) * HD + d];
        a.part_o[(pbase + qv) * hd + d] = acc;
    }
    if (tid < QV) {
        a.part_ml[2 * (pbase + tid)] = s_red[2 * tid];
        a.part_ml[2 * (pbase + tid) + 1] = s_red[2 * tid + 1];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(a.counters + static_cast<uint64_t>(gi) * a.n_kvh + kvh, 1u);
        s_last = prev == n_parts - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // Merge every partition of the group in partition order.  Partition pi
    // is read by thread pi % 256; the max and the sum are reduced with a
    // fixed shuffle tree, so the result is deterministic.
    float* s_pw = s_o;                      // [n_parts][QVM] weights
    float* s_wr = s_o + kMergeFloats - kWaves * QVM;  // [kWaves][QVM]
    const uint64_t gbase = static_cast<uint64_t>(item0) * a.n_kvh;
    auto ml_at = [&](uint32_t pi, uint32_t qv) {
        return ((gbase + static_cast<uint64_t>(pi) * a.n_kvh + kvh) * QVM + qv) * 2;
    };
    float red[QVM];
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) red[qv] = kFloor;
    for (uint32_t pi = tid; pi < n_parts; pi += kThreads)
#pragma unroll
        for (int qv = 0; qv < QVM; qv++)
            if (static_cast<uint32_t>(qv) < QV) red[qv] = fmaxf(red[qv], __builtin_nontemporal_load(a.part_ml + ml_at(pi, qv)));
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) {
        float x = red[qv];
        for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
        if (lane == 0) s_wr[wave * QVM + qv] = x;
    }
    __syncthreads();
    float Mq[QVM];
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) {
        Mq[qv] = fmaxf(fmaxf(s_wr[qv], s_wr[QVM + qv]), fmaxf(s_wr[2 * QVM + qv], s_wr[3 * QVM + qv]));
        red[qv] = 0.0f;
    }
    __syncthreads();
    for (uint32_t pi = tid; pi < n_parts; pi += kThreads)
#pragma unroll
        for (int qv = 0; qv < QVM; qv++) {
            float w = 0.0f;
            if (static_cast<uint32_t>(qv) < QV) {
                const uint64_t b = ml_at(pi, qv);
                w = fast_exp2(__builtin_nontemporal_load(a.part_ml + b) - Mq[qv]);
                red[qv] += w * __builtin_nontemporal_load(a.part_ml + b + 1);
            }
            s_pw[pi * QVM + qv] = w;
        }
#pragma unroll
    for (int qv = 0; qv < QVM; qv++) {
        float x = red[qv];
        for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
        if (lane == 0) s_wr[wave * QVM + qv] = x;
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < nout; idx += kThreads) {
        const uint32_t qv = idx / hd, d = idx - qv * hd;
        const float L = ((s_wr[qv] + s_wr[QVM + qv]) + s_wr[2 * QVM + qv]) + s_wr[3 * QVM + qv];
        const float* src = a.part_o + (gbase * QVM + kvh * QVM + qv) * hd + d;
        const uint64_t step = static_cast<uint64_t>(a.n_kvh) * QVM * hd;
        float acc = 0.0f;
        uint32_t pi = 0;
        for (; pi + 8 <= n_parts; pi += 8) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = __builtin_nontemporal_load(src + (pi + j) * step);
#pragma unroll
            for (int j = 0; j < 8; j++) acc += s_pw[(pi + j) * QVM + qv] * x[j];
        }
        for (; pi < n_parts; pi++) acc += s_pw[pi * QVM + qv] * __builtin_nontemporal_load(src + pi * step);
        const float yv = acc / L;
        const uint32_t rr = qv / H, hh = qv - rr * H;
        const uint64_t yi = (static_cast<uint64_t>(r0 + rr) * a.q_heads + kvh * a.nq_per_kv + h0 + hh) * hd + d;
        if (a.y_f16)
            static_cast<_Float16*>(a.y)[yi] = static_cast<_Float16>(yv);
        else
            static_cast<float*>(a.y)[yi] = yv;
    }
    if (tid == 0) a.counters[static_cast<uint64_t>(gi) * a.n_kvh + kvh] = 0u;
}

// ------------------------------------------------------------ host side
struct Variant {
    uint32_t hd_t, qvm;
};

uint32_t template_hd(uint32_t hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : hd <= 256 ? 256 : 512; }

template <int HD, int QVM>
void launch_one(bool f16, dim3 grid, const AttnArgs& a, hipStream_t s) {
    if (f16)
        hipLaunchKernelGGL((attn_splitk<HD, QVM, true>), grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((attn_splitk<HD, QVM, false>), grid, dim3(kThreads), 0, s, a);
}

void launch(const Variant& v, bool f16, dim3 grid, const AttnArgs& a, hipStream_t s) {
    switch (v.hd_t * 16 + v.qvm) {
        case 64 * 16 + 8: launch_one<64, 8>(f16, grid, a, s); break;
        case 128 * 16 + 4: launch_one<128, 4>(f16, grid, a, s); break;
        case 128 * 16 + 8: launch_one<128, 8>(f16, grid, a, s); break;
        case 256 * 16 + 4: launch_one<256, 4>(f16, grid, a, s); break;
        case 256 * 16 + 8: launch_one<256, 8>(f16, grid, a, s); break;
        case 512 * 16 + 4: launch_one<512, 4>(f16, grid, a, s); break;
        default: launch_one<512, 8>(f16, grid, a, s); break;
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

int build_plan(thb_pool* pool, const thb_rows* rows, const thb_attn_spec& sp, uint32_t hd, AttnPlan& plan,
               hipStream_t stream) {
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

    // Variant: QVM = 4 when every group is a single decode row with G <= 4.
    const uint32_t hd_t = template_hd(hd);
    uint32_t max_chunk = 0;
    for (auto& c : rp.chunks) max_chunk = std::max(max_chunk, c.second - c.first);
    uint32_t qvm = (max_chunk == 1 && G <= 4 && hd_t >= 128) ? 4u : 8u;

    std::vector<uint32_t> groups, items;
    const uint32_t P = pool->part_len;
    uint32_t max_parts = 0;
    auto add_group = [&](uint32_t r0, uint32_t R, uint32_t h0, uint32_t H, uint32_t seq) {
        uint32_t lo = 0xFFFFFFFFu, hi = 0;
        for (uint32_t r = r0; r < r0 + R; r++) {
            if (rp.hi[r] <= rp.lo[r]) continue;
            lo = std::min(lo, rp.lo[r]);
            hi = std::max(hi, rp.hi[r]);
        }
        uint32_t part0, n_parts;
        if (hi <= lo || lo == 0xFFFFFFFFu) {
            lo = hi = 0;  // no keys: one empty partition, output 0/0 like the reference
            part0 = 0;
            n_parts = 1;
        } else {
            part0 = lo / P;
            n_parts = (hi - 1) / P - part0 + 1;
        }
        max_parts = std::max(max_parts, n_parts);
        const uint32_t gidx = static_cast<uint32_t>(groups.size() / kGroupWords);
        const uint32_t item0 = static_cast<uint32_t>(items.size());
        groups.insert(groups.end(), {r0, R, h0, H, seq, lo, hi, n_parts, part0, item0});
        for (uint32_t i = 0; i < n_parts; i++) items.push_back(gidx);
    };
    for (auto& c : rp.chunks) {
        const uint32_t seq = rp.seq[c.first];
        if (G <= qvm) {
            const uint32_t rg = qvm / G;
            for (uint32_t r = c.first; r < c.second; r += rg) add_group(r, std::min(rg, c.second - r), 0, G, seq);
        } else {
            for (uint32_t r = c.first; r < c.second; r++)
                for (uint32_t h0 = 0; h0 < G; h0 += qvm) add_group(r, 1, h0, std::min(qvm, G - h0), seq);
        }
    }
    const uint32_t n_groups = static_cast<uint32_t>(groups.size() / kGroupWords);
    const uint32_t n_items = static_cast<uint32_t>(items.size());
    if ((static_cast<uint64_t>(max_parts) + kWaves) * qvm > kMergeFloats)
        return fail(THB_ERR_CONFIG, "context of " + std::to_string(static_cast<uint64_t>(max_parts) * P) +
                                        " tokens exceeds the merge capacity of this part_len");

    std::vector<uint32_t> blob;
    blob.reserve(groups.size() + items.size() + 2 * m);
    blob.insert(blob.end(), groups.begin(), groups.end());
    blob.insert(blob.end(), items.begin(), items.end());
    for (uint32_t r = 0; r < m; r++) {
        blob.push_back(rp.lo[r]);
        blob.push_back(rp.hi[r]);
    }
    void* dev = plan.dev.reserve(blob.size() * 4, false);
    pool->stager.upload(dev, blob.data(), blob.size() * 4, stream);
    plan.n_groups = n_groups;
    plan.n_items = n_items;
    plan.qv_max = qvm;
    plan.variant = hd_t * 16 + qvm;
    return THB_OK;
}

}  // namespace
}  // namespace thb

using namespace thb;

extern "C" int thb_attn(thb_pool* pool, uint32_t layer, const void* q, void* y, const thb_attn_spec* spec,
                        const thb_rows* rows, void* stream) {
    if (!pool || !spec || !rows) return fail(THB_ERR_INVALID, "null pool, spec or rows");
    if (layer >= pool->layers)
        return fail(THB_ERR_INVALID, "layer " + std::to_string(layer) + " out of range (" +
                                         std::to_string(pool->layers) + " layers)");
    const thb_attn_spec& sp = *spec;
    if (sp.m == 0) return THB_OK;
    if (!q || !y) return fail(THB_ERR_INVALID, "null q or y");
    if (sp.q_heads == 0 || sp.q_heads % pool->kv_heads != 0)
        return fail(THB_ERR_CONFIG, "q_heads " + std::to_string(sp.q_heads) + " must be a positive multiple of kv_heads " +
                                        std::to_string(pool->kv_heads));
    if (sp.q_dtype > THB_DT_F16 || sp.y_dtype > THB_DT_F16)
        return fail(THB_ERR_INVALID, "q_dtype and y_dtype must be THB_DT_F32 or THB_DT_F16");
    if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(y) & 3u))
        return fail(THB_ERR_INVALID, "q must be 16-byte aligned and y 4-byte aligned");
    if (static_cast<uint64_t>(sp.row_off) + sp.m > rows->m)
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->m) + " rows, call needs " +
                                         std::to_string(static_cast<uint64_t>(sp.row_off) + sp.m));
    if (sp.seq != THB_SEQ_PER_ROW && sp.seq >= pool->arena.a.seqs())
        return fail(THB_ERR_INVALID, "sequence " + std::to_string(sp.seq) + " out of range");
    if (!(sp.softcap >= 0.0f)) return fail(THB_ERR_INVALID, "softcap must be >= 0");
    const uint32_t hd = pool->geom[layer].head_dim;
    if (pool->part_len >> pool->page_shift > kMaxPartPages)
        return fail(THB_ERR_CONFIG, "part_len / page_len must be at most " + std::to_string(kMaxPartPages));

    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        // Plan cache: one entry per (rows write, call shape, allocator state).
        const uint64_t av = pool->arena.a.version();
        AttnPlan* plan = nullptr;
        for (auto& p : pool->plans)
            if (p.rows == rows && p.rows_version == rows->version && p.arena_version == av && p.row_off == sp.row_off &&
                p.m == sp.m && p.seq == sp.seq && p.causal == sp.causal && p.window == sp.window &&
                p.q_heads == sp.q_heads && p.head_dim == hd) {
                plan = &p;
                break;
            }
        if (!plan) {
            plan = &pool->plans[0];
            for (auto& p : pool->plans)
                if (p.last_use < plan->last_use) plan = &p;
            plan->rows = nullptr;
            if (int rc = build_plan(pool, rows, sp, hd, *plan, s)) return rc;
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
        }
        plan->last_use = ++pool->plan_clock;

        const uint32_t qvm = plan->qv_max;
        const uint64_t n_part = static_cast<uint64_t>(plan->n_items) * pool->kv_heads * qvm;
        const uint64_t o_bytes = n_part * hd * 4, ml_bytes = n_part * 8;
        uint8_t* part = static_cast<uint8_t*>(pool->partials.reserve(o_bytes + ml_bytes + 256, false));
        uint32_t* cnt = static_cast<uint32_t*>(
            pool->counters.reserve(static_cast<uint64_t>(plan->n_groups) * pool->kv_heads * 4, true));

        const uint32_t* blob = static_cast<const uint32_t*>(plan->dev.get());
        const LayerGeom& g = pool->geom[layer];
        AttnArgs a;
        a.q = q;
        a.y = y;
        a.groups = blob;
        a.items = blob + static_cast<size_t>(plan->n_groups) * kGroupWords;
        a.ranges = a.items + plan->n_items;
        a.table = pool->table_dev;
        a.k = reinterpret_cast<const uint16_t*>(pool->mem + g.k_off);
        a.v = reinterpret_cast<const uint16_t*>(pool->mem + g.v_off);
        a.part_o = reinterpret_cast<float*>(part);
        a.part_ml = reinterpret_cast<float*>(part + ((o_bytes + 255) & ~uint64_t(255)));
        a.counters = cnt;
        a.plane = static_cast<uint64_t>(pool->arena.a.pages()) * pool->page_len * hd;
        a.max_pages = pool->arena.a.max_pages();
        a.page_shift = pool->page_shift;
        a.q_heads = sp.q_heads;
        a.nq_per_kv = sp.q_heads / pool->kv_heads;
        a.head_dim = hd;
        a.part_len = pool->part_len;
        a.n_kvh = pool->kv_heads;
        const float log2e = 1.4426950408889634f;
        if (sp.softcap > 0.0f) {
            a.qscale = sp.scale / sp.softcap;
            a.cap2 = sp.softcap * log2e;
        } else {
            a.qscale = sp.scale * log2e;
            a.cap2 = 0.0f;
        }
        a.q_f16 = sp.q_dtype == THB_DT_F16;
        a.y_f16 = sp.y_dtype == THB_DT_F16;
        Variant v{template_hd(hd), qvm};
        launch(v, pool->kv_dtype == THB_KV_F16_RNE, dim3(plan->n_items, pool->kv_heads), a, s);
        THB_HIP(hipGetLastError());
        return THB_OK;
    });
}
