// Bit-exact KV encodings shared by the append path of every kernel.
//
// f16 follows crates/thuban_num/src/lib.rs:1-60 (round to nearest even,
// subnormals, saturation, NaN -> sign|0x7E00); bf16 is the reference's
// truncation (kv_store.wgsl:20-22, thuban_num/src/lib.rs:66-68).  Integer
// arithmetic only, so the bits do not depend on the floating-point mode.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/thuban_hip.h"

namespace thb {

// f32 -> f16 with round-to-nearest-even, subnormals, saturation to
// infinity and NaN -> sign|0x7E00, in integer ops so the bits match the
// reference codec (crates/thuban_num/src/lib.rs:25-60) for every input.
__device__ inline uint32_t f32_to_f16_bits(uint32_t bits) {
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exp = static_cast<int32_t>((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xff) return sign | (mant ? 0x7e00u : 0x7c00u);
    const int32_t he = exp - 112;
    if (he >= 31) return sign | 0x7c00u;
    if (he <= 0) {
        if (he < -10) return sign;
        const uint32_t m = mant | 0x800000u;
        const uint32_t shift = static_cast<uint32_t>(14 - he);
        const uint32_t sh = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        return sign | (sh + ((rem > half || (rem == half && (sh & 1u))) ? 1u : 0u));
    }
    const uint32_t frac = mant >> 13, rem = mant & 0x1fffu;
    uint32_t r = sign | (static_cast<uint32_t>(he) << 10) | frac;
    if (rem > 0x1000u || (rem == 0x1000u && (frac & 1u))) r += 1u;
    return r & 0xffffu;
}

// f16 -> f32 bits exactly as crates/thuban_num/src/lib.rs:1-23.
__device__ inline uint32_t f16_to_f32_bits(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (exp == 0) {
        if (mant == 0) return sign << 31;
        // normalise: leading one of the 10-bit mantissa
        const uint32_t lz = __builtin_clz(mant) - 22;  // zeros above bit 9
        const uint32_t m = (mant << (lz + 1)) & 0x3ffu;
        const uint32_t e = 113u - (lz + 1);
        return (sign << 31) | (e << 23) | (m << 13);
    }
    if (exp == 0x1f) return (sign << 31) | 0x7f800000u | (mant << 13);
    return (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
}

// Converts one 16-bit source word to the KV encoding.
template <uint32_t SRC, uint32_t KV>
__device__ inline uint32_t conv16(uint32_t w) {
    if constexpr (SRC == THB_DT_F16) {
        if constexpr (KV == THB_KV_F16_RNE) return w;
        return f16_to_f32_bits(w) >> 16;  // f16 -> f32 (exact) -> truncate
    } else {  // bf16
        if constexpr (KV == THB_KV_BF16_TRUNC) return w;
        return f32_to_f16_bits(w << 16);
    }
}

template <uint32_t KV>
__device__ inline uint32_t conv32(uint32_t bits) {
    if constexpr (KV == THB_KV_F16_RNE) return f32_to_f16_bits(bits);
    return bits >> 16;  // kv_store.wgsl:20-22
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (the source rows are read exactly once).
__device__ inline uint4 ld_stream16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads 8 source elements at element index e and returns them encoded.
template <uint32_t SRC, uint32_t KV>
__device__ inline uint4 load_encode8(const void* src, uint64_t e) {
    uint4 out;
    if constexpr (SRC == THB_DT_F32) {
        const float* p = static_cast<const float*>(src) + e;
        const uint4 a = ld_stream16(p), b = ld_stream16(p + 4);
        out.x = conv32<KV>(a.x) | (conv32<KV>(a.y) << 16);
        out.y = conv32<KV>(a.z) | (conv32<KV>(a.w) << 16);
        out.z = conv32<KV>(b.x) | (conv32<KV>(b.y) << 16);
        out.w = conv32<KV>(b.z) | (conv32<KV>(b.w) << 16);
    } else {
        const uint4 a = ld_stream16(static_cast<const uint16_t*>(src) + e);
        auto c2 = [](uint32_t w) { return conv16<SRC, KV>(w & 0xffffu) | (conv16<SRC, KV>(w >> 16) << 16); };
        out.x = c2(a.x);
        out.y = c2(a.y);
        out.z = c2(a.z);
        out.w = c2(a.w);
    }
    return out;
}

// 8 source elements as loaded (f32: 32 bytes in a, b; 16-bit types: 16
// bytes in a), so the load can be issued long before the encoding.
struct Raw8 {
    uint4 a, b;
};

__device__ inline Raw8 load_raw8_rt(uint32_t src_dtype, const void* src, uint64_t e) {
    Raw8 r{};
    if (src_dtype == THB_DT_F32) {
        const float* p = static_cast<const float*>(src) + e;
        r.a = ld_stream16(p);
        r.b = ld_stream16(p + 4);
    } else {
        r.a = ld_stream16(static_cast<const uint16_t*>(src) + e);
    }
    return r;
}

// The encoding of load_encode8 applied to loaded words.
template <uint32_t KV>
__device__ inline uint4 encode8_rt(uint32_t src_dtype, const Raw8& r) {
    uint4 out;
    if (src_dtype == THB_DT_F32) {
        out.x = conv32<KV>(r.a.x) | (conv32<KV>(r.a.y) << 16);
        out.y = conv32<KV>(r.a.z) | (conv32<KV>(r.a.w) << 16);
        out.z = conv32<KV>(r.b.x) | (conv32<KV>(r.b.y) << 16);
        out.w = conv32<KV>(r.b.z) | (conv32<KV>(r.b.w) << 16);
    } else if (src_dtype == THB_DT_F16) {
        auto c2 = [](uint32_t w) {
            return conv16<THB_DT_F16, KV>(w & 0xffffu) | (conv16<THB_DT_F16, KV>(w >> 16) << 16);
        };
        out = make_uint4(c2(r.a.x), c2(r.a.y), c2(r.a.z), c2(r.a.w));
    } else {
        auto c2 = [](uint32_t w) {
            return conv16<THB_DT_BF16, KV>(w & 0xffffu) | (conv16<THB_DT_BF16, KV>(w >> 16) << 16);
        };
        out = make_uint4(c2(r.a.x), c2(r.a.y), c2(r.a.z), c2(r.a.w));
    }
    return out;
}

// Runtime source type, compile-time KV encoding.
template <uint32_t KV>
__device__ inline uint4 load_encode8_rt(uint32_t src_dtype, const void* src, uint64_t e) {
    switch (src_dtype) {
        case THB_DT_F32: return load_encode8<THB_DT_F32, KV>(src, e);
        case THB_DT_F16: return load_encode8<THB_DT_F16, KV>(src, e);
        default: return load_encode8<THB_DT_BF16, KV>(src, e);
    }
}

}  // namespace thb
