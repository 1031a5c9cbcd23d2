// Shared host-side helpers of the HIP backend: error state, HIP checks and
// the pinned staging ring used for every host-to-device upload.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/thuban_hip.h"

namespace thb {

// Sets the thread-local error message and returns `code`.
int fail(int code, const std::string& msg);
void clear_error();
// Process-wide monotonically increasing stamp (cache keys).
uint64_t next_version();

struct HipError {
    hipError_t err;
    std::string where;
};

#define THB_HIP(call)                                                              \
    do {                                                                           \
        hipError_t thb_e_ = (call);                                                \
        if (thb_e_ != hipSuccess) throw ::thb::HipError{thb_e_, #call};           \
    } while (0)

// Runs `body`, converting a HipError into THB_ERR_GPU with the HIP message.
template <class F>
int guarded(F&& body) {
    try {
        return body();
    } catch (const HipError& e) {
        return fail(THB_ERR_GPU, std::string("HIP error ") + hipGetErrorString(e.err) + " in " + e.where);
    } catch (const std::bad_alloc&) {
        return fail(THB_ERR_GPU, "host out of memory");
    }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Pinned host staging for host->device copies.  A ring of slots; a slot is
// reused only after the event recorded behind its last copy has completed,
// so the host never overwrites bytes a pending copy still reads.
class Stager {
public:
    Stager() = default;
    Stager(const Stager&) = delete;
    Stager& operator=(const Stager&) = delete;
    ~Stager();
    // Copies `bytes` from host `src` to device `dst` on `stream`.
    void upload(void* dst, const void* src, size_t bytes, hipStream_t stream);

private:
    struct Slot {
        void* host = nullptr;
        size_t cap = 0;
        hipEvent_t done = nullptr;
        bool pending = false;
    };
    static constexpr int kSlots = 8;
    Slot slots_[kSlots];
    int next_ = 0;
};

// Pinned host staging of a fixed size, allocated once (init) and never
// grown: two slots, each reused after the event behind its last copy.
// upload() allocates nothing.
class FixedStager {
public:
    FixedStager() = default;
    FixedStager(const FixedStager&) = delete;
    FixedStager& operator=(const FixedStager&) = delete;
    ~FixedStager();
    void init(size_t bytes);
    size_t capacity() const { return cap_; }
    // Copies `bytes` (at most capacity()) from host `src` to device `dst`.
    void upload(void* dst, const void* src, size_t bytes, hipStream_t stream);

private:
    static constexpr int kSlots = 2;
    void* host_[kSlots] = {nullptr, nullptr};
    hipEvent_t done_[kSlots] = {nullptr, nullptr};
    bool pending_[kSlots] = {false, false};
    size_t cap_ = 0;
    int next_ = 0;
};

// Device buffer that grows on demand (hipMalloc outside the hot path: only
// when a larger size than ever before is requested).
class DevBuf {
public:
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf();
    // Ensures capacity; newly grown memory is zero-filled when `zero`.
    void* reserve(size_t bytes, bool zero);
    void* get() const { return ptr_; }
    size_t size() const { return cap_; }

private:
    void* ptr_ = nullptr;
    size_t cap_ = 0;
};

}  // namespace thb
