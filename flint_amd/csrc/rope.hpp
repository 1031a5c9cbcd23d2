// Rotary position embedding and the RMSNorm that precedes it (rope.wgsl
// :16-40, norm.wgsl MODE 4), on f32 values.  Every product and sum is
// rounded on its own (no fused multiply-add), so the CPU restatement can
// reproduce the results bit for bit.
#pragma once

#include "codec.hpp"

namespace thb {

// Device view of a thb_rope for one operand (query or key).
struct RopeDev {
    const float* cos;  // [max_pos][half]
    const float* sin;
    const float* w;    // RMSNorm weight [head_dim], or null: rotation only
    uint32_t rot, half;
    float eps;
    uint32_t max_pos;  // table rows (> 0)
};

// The query (or key) view of a validated thb_rope.
inline RopeDev rope_dev(const thb_rope& r, bool query) {
    return RopeDev{r.cos_dev, r.sin_dev, query ? r.q_norm_dev : r.k_norm_dev, r.rot, r.rot / 2, r.eps, r.max_pos};
}

// x c - y s (the first half of the rotated dims).
__device__ inline float rope_lo(float x, float c, float y, float s) {
#pragma clang fp contract(off)
    return x * c - y * s;
}

// x c + y s (the second half).
__device__ inline float rope_hi(float x, float c, float y, float s) {
#pragma clang fp contract(off)
    return x * c + y * s;
}

// Sum of squares of 8 elements, in order.
__device__ inline float sumsq8(const float (&x)[8]) {
#pragma clang fp contract(off)
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) s = s + x[e] * x[e];
    return s;
}

// 1 / sqrt(ss / dim + eps), correctly rounded division and square root.
__device__ inline float rms_inv(float ss, uint32_t dim, float eps) {
    return 1.0f / __builtin_sqrtf(ss / static_cast<float>(dim) + eps);
}

// x = (x * inv) * w for 8 elements.
__device__ inline void norm8(float (&x)[8], float inv, const float* w) {
#pragma clang fp contract(off)
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(w), w1 = *reinterpret_cast<const f32x4*>(w + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        x[e] = (x[e] * inv) * w0[e];
        x[4 + e] = (x[4 + e] * inv) * w1[e];
    }
}

// Rotates the 8 elements x of dims [d0, d0 + 8) given their partners y
// (dims d0 +- half), at position pos.  d0 < rot, d0 % 8 == 0.  A position
// past the tables reads their last row: host calls refuse such rows, and
// a device-planned call gives them no keys (a NaN output) and reports them,
// so the clamp only keeps the read inside the tables.
__device__ inline void rotate8(float (&x)[8], const float (&y)[8], uint32_t d0, uint32_t pos, const RopeDev& r) {
    const bool lo = d0 < r.half;
    const uint32_t p = pos < r.max_pos ? pos : r.max_pos - 1u;
    const uint64_t t = static_cast<uint64_t>(p) * r.half + (lo ? d0 : d0 - r.half);
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(r.cos + t), c1 = *reinterpret_cast<const f32x4*>(r.cos + t + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(r.sin + t), s1 = *reinterpret_cast<const f32x4*>(r.sin + t + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        x[e] = lo ? rope_lo(x[e], c0[e], y[e], s0[e]) : rope_hi(x[e], c0[e], y[e], s0[e]);
        x[4 + e] = lo ? rope_lo(x[4 + e], c1[e], y[4 + e], s1[e]) : rope_hi(x[4 + e], c1[e], y[4 + e], s1[e]);
    }
}

// Loads 8 f32 or f16 elements at element index e as f32.
__device__ inline void load8_f32(uint32_t dtype, const void* src, uint64_t e, float (&x)[8]) {
    if (dtype == THB_DT_F32) {
        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + e);
        const f32x4 a = p[0], b = p[1];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[i] = a[i];
            x[4 + i] = b[i];
        }
    } else {
        const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + e);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[2 * i] = __uint_as_float(f16_to_f32_bits(ws[i] & 0xffffu));
            x[2 * i + 1] = __uint_as_float(f16_to_f32_bits(ws[i] >> 16));
        }
    }
}

// Head vectors in lane segments: the segment starting at lane seg_base
// holds one head, lane seg_base + u (u < cph) its dims [8u, 8u + 8) in x.
// Applies the RMSNorm (when r.w is set; the sum of squares runs over the
// chunks in order) and the rotation at position pos.  Every lane of the
// wavefront must call it (cross-lane reads); lanes with u >= cph carry no
// data and read none.
__device__ inline void rope_head_seg(float (&x)[8], uint32_t u, uint32_t cph, uint32_t seg_base, uint32_t pos,
                                     const RopeDev& r) {
    if (r.w) {
        const float s = u < cph ? sumsq8(x) : 0.0f;
        float ss = 0.0f;
        for (uint32_t i = 0; i < cph; i++) ss = ss + __shfl(s, static_cast<int>(seg_base + i));
        const float inv = rms_inv(ss, 8u * cph, r.eps);
        if (u < cph) norm8(x, inv, r.w + 8u * u);
    }
    const uint32_t hc = r.half >> 3;  // chunks per half
    const uint32_t partner = seg_base + (u < hc ? u + hc : u - hc);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = __shfl(x[e], static_cast<int>(partner & 63u));
    if (u < cph && 8u * u < r.rot) rotate8(x, y, 8u * u, pos, r);
}

// f32 -> f16 bits, round to nearest even (thuban_num::f32_to_f16).
__device__ inline uint32_t f32_to_f16_rne(float x) { return f32_to_f16_bits(__float_as_uint(x)); }

}  // namespace thb
