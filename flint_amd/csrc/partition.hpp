// Split-K partitions of a key span, shared by the host planner and the
// device planner (and pinned on the CPU by tests/test_abi.py).
#pragma once

#include <cstdint>

namespace thb {

// Partitions of a key span (a function of the span only, so a group's
// arithmetic does not depend on the rest of the call): ceil(span / PL)
// rounded up to a power of two, as n_parts equal pieces of plen keys (a
// multiple of align), the last one shorter.  A span at most PL / 64 per
// piece over k * PL (k >= 2) counts as k pieces, each up to PL + PL / 64
// long: Gemma-2's global layers (8192 + 4 keys) then take 2 partitions
// instead of 4, one round of workgroups instead of two.  (k = 1 keeps two
// pieces: a span just over PL on one piece would leave half the CUs idle
// where a call holds few groups.)  Rounding down in general (pieces up to
// ~2 PL) measured faster on those layers and slower on the ragged Qwen3
// batch and the 131072-token Qwen2.5 contexts.
__host__ __device__ inline void part_split(uint64_t span, uint32_t PL, uint32_t align, uint32_t& n_parts,
                                           uint32_t& plen) {
    uint32_t n = static_cast<uint32_t>((span + PL - 1) / PL);
    const uint64_t k = span / PL;
    if (n > 2 && span - k * PL <= k * (PL / 64)) n = static_cast<uint32_t>(k);
    if (n > 1) n = 1u << (32 - __builtin_clz(n - 1));
    plen = static_cast<uint32_t>(((span + n - 1) / n + align - 1) / align * align);
    n_parts = static_cast<uint32_t>((span + plen - 1) / plen);
}

// part_split for 0 < span < 2^31 and a power-of-two align, in 32-bit
// arithmetic with shifts for the power-of-two divisors (n and align): the
// device planner's form (a 64-bit division is a long instruction sequence
// on the GPU).  Same results as part_split.
__host__ __device__ inline void part_split32(uint32_t span, uint32_t PL, uint32_t align, uint32_t& n_parts,
                                             uint32_t& plen) {
    const uint32_t k = span / PL;
    uint32_t n = k + (span - k * PL != 0 ? 1u : 0u);
    if (n > 2 && span - k * PL <= k * (PL / 64)) n = k;
    uint32_t sh = 0;
    if (n > 1) {
        sh = 32 - __builtin_clz(n - 1);
        n = 1u << sh;
    }
    plen = (((span + n - 1) >> sh) + align - 1) & ~(align - 1);
    n_parts = (span + plen - 1) / plen;
}

}  // namespace thb
