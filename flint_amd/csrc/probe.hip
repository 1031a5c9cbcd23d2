// Streaming probes of the device's achievable HBM rate (no reference
// counterpart: a measurement aid).  The roofline fractions of the paged-KV
// kernels are stated against the 8 TB/s specification and against what a
// plain linear stream of the same access kind reaches on the same device,
// measured by these kernels.
//
// Each workgroup streams its own contiguous slab with 16-byte non-temporal
// accesses (the attention and page-move kernels' access kind), U vectors per
// lane in flight.  Read mode folds every word into a register and writes one
// word per lane at the end (so the loads are not removed); copy mode writes
// every vector to the destination.
#include "common.hpp"
#include "codec.hpp"

namespace thb {
namespace {

constexpr uint32_t kProbeThreads = 512;
constexpr uint32_t kProbeUnroll = 8;

template <bool COPY>
__global__ __launch_bounds__(kProbeThreads) void hbm_stream_kernel(const uint4* src, uint4* dst, uint64_t vecs,
                                                                   uint32_t* sink) {
    const uint64_t per = (vecs + gridDim.x - 1) / gridDim.x;
    const uint64_t v0 = per * blockIdx.x, v1 = min(vecs, v0 + per);
    uint32_t acc = 0;
    for (uint64_t b = v0 + threadIdx.x; b < v1; b += static_cast<uint64_t>(kProbeUnroll) * kProbeThreads) {
        uint4 r[kProbeUnroll];
#pragma unroll
        for (uint32_t i = 0; i < kProbeUnroll; i++) {
            const uint64_t v = b + static_cast<uint64_t>(i) * kProbeThreads;
            if (v < v1) r[i] = ld_stream16(src + v);
        }
#pragma unroll
        for (uint32_t i = 0; i < kProbeUnroll; i++) {
            const uint64_t v = b + static_cast<uint64_t>(i) * kProbeThreads;
            if (v >= v1) continue;
            if constexpr (COPY)
                __builtin_nontemporal_store(u32x4{r[i].x, r[i].y, r[i].z, r[i].w}, reinterpret_cast<u32x4*>(dst + v));
            else
                acc ^= r[i].x ^ r[i].y ^ r[i].z ^ r[i].w;
        }
    }
    if constexpr (!COPY) sink[static_cast<uint64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

}  // namespace
}  // namespace thb

using namespace thb;

extern "C" int thb_hbm_stream(const void* src_dev, void* dst_dev, uint64_t bytes, uint32_t mode, uint32_t workgroups,
                              void* stream) {
    if (!src_dev || !dst_dev) return fail(THB_ERR_INVALID, "null buffer");
    if (mode > 1) return fail(THB_ERR_INVALID, "mode must be 0 (read) or 1 (copy)");
    if (workgroups == 0 || workgroups > 65536) return fail(THB_ERR_INVALID, "workgroups must be in [1, 65536]");
    if ((reinterpret_cast<uintptr_t>(src_dev) | reinterpret_cast<uintptr_t>(dst_dev)) & 15u || bytes % 16)
        return fail(THB_ERR_INVALID, "buffers and size must be 16-byte aligned");
    if (mode == 0 && static_cast<uint64_t>(workgroups) * kProbeThreads * 4 > bytes)
        return fail(THB_ERR_INVALID, "read mode writes 2 KiB per workgroup into dst: bytes too small");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        const auto* src = static_cast<const uint4*>(src_dev);
        auto* dst = static_cast<uint4*>(dst_dev);
        if (mode == 1)
            hipLaunchKernelGGL(hbm_stream_kernel<true>, dim3(workgroups), dim3(kProbeThreads), 0, s, src, dst,
                               bytes / 16, nullptr);
        else
            hipLaunchKernelGGL(hbm_stream_kernel<false>, dim3(workgroups), dim3(kProbeThreads), 0, s, src, dst,
                               bytes / 16, reinterpret_cast<uint32_t*>(dst_dev));
        THB_HIP(hipGetLastError());
        return THB_OK;
    });
}
