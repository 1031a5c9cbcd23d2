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

// A call refused because its stream is capturing a graph and the call
// cannot be replayed correctly from a capture (THB_ERR_INVALID).
struct CaptureRefused {
    std::string what;
};

// True while `stream` captures a graph (also when the capture has been
// invalidated, or when another stream captures in global mode and `stream`
// is the legacy default stream).
bool capturing(hipStream_t stream);

// Writes `bytes` of host data to device `dst` inside the graph `stream` is
// capturing: the data travel in the arguments of copy kernels, so the graph
// owns them and every replay writes the same bytes.  Up to
// kGraphUploadMax bytes; more throws CaptureRefused.
constexpr size_t kGraphUploadMax = 256u << 10;
void upload_in_graph(void* dst, const void* src, size_t bytes, hipStream_t stream);

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
    } catch (const CaptureRefused& e) {
        return fail(THB_ERR_INVALID, "not capturable: " + e.what);
    } catch (const std::bad_alloc&) {
        return fail(THB_ERR_GPU, "host out of memory");
    }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Pinned host staging for host->device copies.  A ring of slots; a slot is
// reused only after the event recorded behind its last copy has completed,
// so the host never overwrites bytes a pending copy still reads.  On a
// capturing stream the bytes go into the graph instead (upload_in_graph): a
// captured copy from a slot would read the slot's contents at replay time.
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
// upload() allocates nothing; on a capturing stream it writes through
// upload_in_graph, which allocates nothing either.
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
// when a larger size than ever before is requested).  A buffer handed out
// while `stream` captures a graph may be read by every replay of that graph,
// so it is never freed before the DevBuf is destroyed: growth after a capture
// keeps the old allocation alive, and growth during a capture is refused.
class DevBuf {
public:
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf();
    // Ensures capacity for work queued on `stream`; newly grown memory is
    // zero-filled when `zero`.
    void* reserve(size_t bytes, bool zero, hipStream_t stream);
    // reserve() for a caller about to overwrite the contents from the host:
    // outside a capture, a buffer a graph has used is replaced by a new
    // allocation (the graph keeps reading the old contents).
    void* reserve_rewrite(size_t bytes, bool zero, hipStream_t stream);
    void* get() const { return ptr_; }
    size_t size() const { return cap_; }

private:
    void* ptr_ = nullptr;
    size_t cap_ = 0;
    bool captured_ = false;        // ptr_ was handed to a capture
    std::vector<void*> retired_;   // earlier allocations a graph may still read
};

}  // namespace thb
