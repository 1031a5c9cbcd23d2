// Element offsets inside one K or V page (THB_PAGE_LAYOUT_MFMA in
// include/thuban_hip.h).  A page holds P = 1 << shift slots of head_dim
// (hd) 16-bit elements and starts at (page * hd) << shift in its head plane.
//
// K: [ceil(hd / 32)][P][w], w = min(32, hd - 32 g): the 32-dimension group g
//    of slot j at 32 P g + w j.  One k-step operand load of the attention
//    kernel (16 slots x 32 dims) is 1 KiB of contiguous memory, and an
//    appended token touches one 64-byte piece per group.
// V: [P / 4][hd][4]: 4 consecutive slots of one dimension are 8 contiguous
//    bytes (the PV operand of one lane), and an appended token touches
//    hd * 8 contiguous bytes.
//
// Writing one token into pages dirties few cache lines (4 for K and 8 for V
// at head_dim 128), which is what the end-of-kernel write-back pays for.
#pragma once

#include <cstdint>

namespace thb {

// Width of the K group holding dimension d.
__host__ __device__ inline uint32_t k_group_width(uint32_t hd, uint32_t d) {
    const uint32_t g0 = d & ~31u;
    return hd - g0 < 32u ? hd - g0 : 32u;
}

// Offset of K element (slot j, dim d) in its page.
__host__ __device__ inline uint64_t k_off(uint32_t j, uint32_t d, uint32_t hd, uint32_t shift) {
    return (static_cast<uint64_t>(d & ~31u) << shift) + static_cast<uint64_t>(k_group_width(hd, d)) * j + (d & 31u);
}

// Offset of V element (slot j, dim d) in its page.
__host__ __device__ inline uint64_t v_off(uint32_t j, uint32_t d, uint32_t hd) {
    return (static_cast<uint64_t>(j >> 2) * hd + d) * 4u + (j & 3u);
}

}  // namespace thb
