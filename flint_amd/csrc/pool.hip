// C ABI of the host allocator, the device pool and the row metadata.
//
// Device layout: one allocation holds, for every layer, K then V, each
// [kv_heads, pages, <page>] 16-bit words: the elements of the reference's
// KvPool planes [kv_heads, pool_len, head_dim] (crates/thuban_model/src/
// pool.rs:131-153) with each page reordered for the attention kernel
// (layout.hpp): K in 32-dimension groups, [head_dim / 32][page_len][32]; V
// in 4-slot groups, [page_len / 4][head_dim][4].  Every plane is aligned to
// 256 bytes.
// The block table [seqs * max_pages] u32 lives in its own allocation and is
// shared by all layers.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <string>

#include "pool.hpp"

namespace thb {

static thread_local std::string g_error;
static std::atomic<uint64_t> g_version{0};

uint64_t next_version() { return ++g_version; }

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

void clear_error() { g_error.clear(); }

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &st);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return e == hipErrorStreamCaptureImplicit;
    }
    return st != hipStreamCaptureStatusNone;
}

namespace {

// Payload of one in-graph upload launch: 3968 bytes of data beside the
// destination and the word count (a 4 KiB kernel-argument block).
constexpr uint32_t kGraphChunkWords = 992;
struct GraphChunk {
    uint32_t* dst;
    uint32_t n;
    uint32_t w[kGraphChunkWords];
};

__global__ __launch_bounds__(256) void graph_upload_kernel(GraphChunk a) {
    for (uint32_t i = threadIdx.x; i < a.n; i += 256) a.dst[i] = a.w[i];
}

}  // namespace

void upload_in_graph(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return;
    if (bytes > kGraphUploadMax)
        throw CaptureRefused{"an upload of " + std::to_string(bytes) + " bytes under capture exceeds the " +
                             std::to_string(kGraphUploadMax) + " bytes a graph carries in kernel arguments"};
    if ((reinterpret_cast<uintptr_t>(dst) & 3u) || (bytes & 3u))
        throw CaptureRefused{"an upload under capture must be whole, aligned 32-bit words"};
    const uint32_t words = static_cast<uint32_t>(bytes / 4);
    const auto* from = static_cast<const uint32_t*>(src);
    for (uint32_t w0 = 0; w0 < words; w0 += kGraphChunkWords) {
        GraphChunk c;
        c.dst = static_cast<uint32_t*>(dst) + w0;
        c.n = std::min(kGraphChunkWords, words - w0);
        std::memcpy(c.w, from + w0, static_cast<size_t>(c.n) * 4);
        hipLaunchKernelGGL(graph_upload_kernel, dim3(1), dim3(256), 0, stream, c);
        THB_HIP(hipGetLastError());
    }
}

Stager::~Stager() {
    for (auto& s : slots_) {
        if (s.done) {
            (void)hipEventSynchronize(s.done);
            (void)hipEventDestroy(s.done);
        }
        if (s.host) (void)hipHostFree(s.host);
    }
}

void Stager::upload(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return;
    if (capturing(stream)) {
        upload_in_graph(dst, src, bytes, stream);
        return;
    }
    Slot& s = slots_[next_];
    next_ = (next_ + 1) % kSlots;
    if (s.pending) {
        THB_HIP(hipEventSynchronize(s.done));
        s.pending = false;
    }
    if (s.cap < bytes) {
        if (s.host) THB_HIP(hipHostFree(s.host));
        s.host = nullptr;
        size_t cap = std::max<size_t>(bytes, 4096);
        THB_HIP(hipHostMalloc(&s.host, cap, hipHostMallocDefault));
        s.cap = cap;
    }
    if (!s.done) THB_HIP(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
    std::memcpy(s.host, src, bytes);
    THB_HIP(hipMemcpyAsync(dst, s.host, bytes, hipMemcpyHostToDevice, stream));
    THB_HIP(hipEventRecord(s.done, stream));
    s.pending = true;
}

FixedStager::~FixedStager() {
    for (int i = 0; i < kSlots; i++) {
        if (done_[i]) {
            (void)hipEventSynchronize(done_[i]);
            (void)hipEventDestroy(done_[i]);
        }
        if (host_[i]) (void)hipHostFree(host_[i]);
    }
}

void FixedStager::init(size_t bytes) {
    for (int i = 0; i < kSlots; i++) {
        THB_HIP(hipHostMalloc(&host_[i], bytes, hipHostMallocDefault));
        THB_HIP(hipEventCreateWithFlags(&done_[i], hipEventDisableTiming));
    }
    cap_ = bytes;
}

void FixedStager::upload(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return;
    if (bytes > cap_) throw HipError{hipErrorInvalidValue, "fixed staging upload larger than its slots"};
    if (capturing(stream)) {
        upload_in_graph(dst, src, bytes, stream);
        return;
    }
    const int i = next_;
    next_ = (next_ + 1) % kSlots;
    if (pending_[i]) {
        THB_HIP(hipEventSynchronize(done_[i]));
        pending_[i] = false;
    }
    std::memcpy(host_[i], src, bytes);
    THB_HIP(hipMemcpyAsync(dst, host_[i], bytes, hipMemcpyHostToDevice, stream));
    THB_HIP(hipEventRecord(done_[i], stream));
    pending_[i] = true;
}

void* DevBuf::reserve_rewrite(size_t bytes, bool zero, hipStream_t stream) {
    if (captured_ && !capturing(stream)) {
        retired_.push_back(ptr_);
        ptr_ = nullptr;
        const size_t cap = std::max(bytes, cap_);
        cap_ = 0;
        captured_ = false;
        return reserve(cap, zero, stream);
    }
    return reserve(bytes, zero, stream);
}

DevBuf::~DevBuf() {
    if (ptr_ || !retired_.empty()) {
        (void)hipDeviceSynchronize();
        if (ptr_) (void)hipFree(ptr_);
        for (void* p : retired_) (void)hipFree(p);
    }
}

void* DevBuf::reserve(size_t bytes, bool zero, hipStream_t stream) {
    const bool cap_now = capturing(stream);
    if (bytes <= cap_) {
        captured_ = captured_ || cap_now;
        return ptr_;
    }
    if (cap_now)
        throw CaptureRefused{"a device buffer of the library must grow to " + std::to_string(bytes) +
                             " bytes (run the call once outside the capture first)"};
    size_t cap = std::max<size_t>(bytes, cap_ * 2);
    cap = (cap + 255) & ~size_t(255);
    if (ptr_) {
        if (captured_) {
            retired_.push_back(ptr_);  // a graph may still read it
        } else {
            // The old buffer may still be read by queued kernels.
            THB_HIP(hipDeviceSynchronize());
            THB_HIP(hipFree(ptr_));
        }
        ptr_ = nullptr;
        cap_ = 0;
        captured_ = false;
    }
    THB_HIP(hipMalloc(&ptr_, cap));
    if (zero) THB_HIP(hipMemset(ptr_, 0, cap));
    cap_ = cap;
    return ptr_;
}

}  // namespace thb

using namespace thb;

extern "C" {

const char* thb_last_error(void) { return g_error.c_str(); }

uint32_t thb_abi_version(void) { return THB_ABI_VERSION; }

int thb_check_head_dim(uint32_t head_dim) {
    // ops/attn.rs:83-90, exactly: any head_dim in [64, 512].
    if (head_dim < 64 || head_dim > 512)
        return fail(THB_ERR_CONFIG, "head_dim " + std::to_string(head_dim) + " outside [64, 512]");
    return THB_OK;
}

int thb_backend_head_dim(uint32_t head_dim) {
    if (int rc = thb_check_head_dim(head_dim)) return rc;
    if (head_dim % 8 != 0)
        return fail(THB_ERR_CONFIG, "head_dim " + std::to_string(head_dim) +
                                        " is not supported by the HIP backend: it must be a multiple of 8 "
                                        "(16-byte vector lanes)");
    return THB_OK;
}

// ---------------------------------------------------------------- arena
static int check_seq(const Arena& a, uint32_t seq) {
    if (seq >= a.seqs())
        return fail(THB_ERR_INVALID, "sequence " + std::to_string(seq) + " out of range (" +
                                         std::to_string(a.seqs()) + " sequences)");
    return THB_OK;
}

int thb_arena_create(const uint32_t* seq_lens, uint32_t seqs, int64_t pages, uint32_t page_len, thb_arena** out) {
    if (!out) return fail(THB_ERR_INVALID, "out is null");
    *out = nullptr;
    auto* h = new (std::nothrow) thb_arena;
    if (!h) return fail(THB_ERR_GPU, "host out of memory");
    std::string err = Arena::create(seq_lens, seqs, pages, page_len, h->a);
    if (!err.empty()) {
        delete h;
        return fail(THB_ERR_MODEL, err);
    }
    *out = h;
    return THB_OK;
}

void thb_arena_destroy(thb_arena* arena) { delete arena; }

int thb_arena_alloc(thb_arena* arena, uint32_t seq, uint32_t pos, uint32_t tokens) {
    if (!arena) return fail(THB_ERR_INVALID, "arena is null");
    if (int rc = check_seq(arena->a, seq)) return rc;
    std::string err = arena->a.alloc(seq, pos, tokens);
    return err.empty() ? THB_OK : fail(THB_ERR_MODEL, err);
}

int thb_arena_free_seq(thb_arena* arena, uint32_t seq) {
    if (!arena) return fail(THB_ERR_INVALID, "arena is null");
    if (int rc = check_seq(arena->a, seq)) return rc;
    arena->a.free_seq(seq);
    return THB_OK;
}

int thb_arena_truncate(thb_arena* arena, uint32_t seq, uint32_t keep_tokens) {
    if (!arena) return fail(THB_ERR_INVALID, "arena is null");
    if (int rc = check_seq(arena->a, seq)) return rc;
    arena->a.truncate(seq, keep_tokens);
    return THB_OK;
}

int thb_arena_covers(const thb_arena* arena, uint32_t seq, uint32_t tokens) {
    if (!arena) return fail(THB_ERR_INVALID, "arena is null");
    if (int rc = check_seq(arena->a, seq)) return rc;
    return arena->a.covers(seq, tokens) ? 1 : 0;
}

int thb_arena_fork(thb_arena* arena, uint32_t src, uint32_t dst, uint32_t tokens) {
    if (!arena) return fail(THB_ERR_INVALID, "arena is null");
    if (int rc = check_seq(arena->a, src)) return rc;
    if (int rc = check_seq(arena->a, dst)) return rc;
    if (src == dst) return fail(THB_ERR_INVALID, "fork source and target are the same sequence");
    std::string err = arena->a.fork(src, dst, tokens);
    return err.empty() ? THB_OK : fail(THB_ERR_MODEL, err);
}

int thb_arena_table(const thb_arena* arena, uint32_t* out, size_t n) {
    if (!arena || !out) return fail(THB_ERR_INVALID, "null argument");
    size_t want = static_cast<size_t>(arena->a.seqs()) * arena->a.max_pages();
    if (n != want)
        return fail(THB_ERR_INVALID, "block table must cover every sequence: " + std::to_string(n) +
                                         " != " + std::to_string(want));
    arena->a.table(out);
    return THB_OK;
}

int thb_arena_table_of(const thb_arena* arena, uint32_t seq, uint32_t* out, size_t cap, uint32_t* len) {
    if (!arena) return fail(THB_ERR_INVALID, "arena is null");
    if (int rc = check_seq(arena->a, seq)) return rc;
    const auto& t = arena->a.table_of(seq);
    if (len) *len = static_cast<uint32_t>(t.size());
    if (out) std::copy(t.begin(), t.begin() + std::min(cap, t.size()), out);
    return THB_OK;
}

int thb_arena_seq_len(const thb_arena* arena, uint32_t seq, uint32_t* len) {
    if (!arena || !len) return fail(THB_ERR_INVALID, "null argument");
    if (int rc = check_seq(arena->a, seq)) return rc;
    *len = arena->a.seq_len(seq);
    return THB_OK;
}

int thb_arena_info_get(const thb_arena* arena, thb_arena_info* info) {
    if (!arena || !info) return fail(THB_ERR_INVALID, "null argument");
    info->pages = arena->a.pages();
    info->used = arena->a.used();
    info->max_pages = arena->a.max_pages();
    info->seqs = arena->a.seqs();
    info->page_len = arena->a.page_len();
    info->pending_copies = static_cast<uint32_t>(const_cast<Arena&>(arena->a).copies().size());
    return THB_OK;
}

int thb_arena_take_copies(thb_arena* arena, uint32_t* triples, size_t cap, uint32_t* n) {
    if (!arena || !n) return fail(THB_ERR_INVALID, "null argument");
    auto& c = arena->a.copies();
    *n = static_cast<uint32_t>(c.size());
    if (c.size() > cap) return fail(THB_ERR_INVALID, "copy buffer holds " + std::to_string(cap) + " < " +
                                                         std::to_string(c.size()) + " triples");
    for (size_t i = 0; i < c.size(); i++) {
        triples[3 * i] = c[i].src;
        triples[3 * i + 1] = c[i].dst;
        triples[3 * i + 2] = c[i].tokens;
    }
    c.clear();
    return THB_OK;
}

int thb_arena_free_list(const thb_arena* arena, uint32_t* free_list, size_t cap, uint32_t* n) {
    if (!arena || !n) return fail(THB_ERR_INVALID, "null argument");
    const auto& f = arena->a.free_list();
    *n = static_cast<uint32_t>(f.size());
    if (free_list) {
        if (cap < f.size())
            return fail(THB_ERR_INVALID, "free list holds " + std::to_string(cap) + " < " + std::to_string(f.size()) +
                                             " pages");
        std::copy(f.begin(), f.end(), free_list);
    }
    return THB_OK;
}

int thb_arena_refs(const thb_arena* arena, uint32_t* refs, size_t cap) {
    if (!arena || !refs) return fail(THB_ERR_INVALID, "null argument");
    const auto& r = arena->a.refs();
    if (cap < r.size())
        return fail(THB_ERR_INVALID, "refs holds " + std::to_string(cap) + " < " + std::to_string(r.size()) + " pages");
    std::copy(r.begin(), r.end(), refs);
    return THB_OK;
}

// ----------------------------------------------------------------- pool
int thb_pool_create(const thb_pool_desc* d, thb_pool** out) {
    if (!d || !out) return fail(THB_ERR_INVALID, "null argument");
    *out = nullptr;
    if (d->layers == 0) return fail(THB_ERR_CONFIG, "pool needs at least one layer");
    if (d->kv_heads == 0) return fail(THB_ERR_CONFIG, "kv_heads must be positive");
    if (d->kv_dtype != THB_KV_BF16_TRUNC && d->kv_dtype != THB_KV_F16_RNE)
        return fail(THB_ERR_CONFIG, "unknown kv_dtype " + std::to_string(d->kv_dtype));
    if (d->page_len < 8 || d->page_len > 256 || (d->page_len & (d->page_len - 1)))
        return fail(THB_ERR_CONFIG, "page_len " + std::to_string(d->page_len) + " must be a power of two in [8, 256]");
    uint32_t part = d->part_len ? d->part_len : 4096;
    // At most 1008 pages: a partition may run part_len / 64 longer (a span a
    // few keys over a multiple of part_len), and the kernels stage at most
    // 1024 page numbers of one partition.
    if (part % 16 != 0 || part % d->page_len != 0 || part / d->page_len > 1008)
        return fail(THB_ERR_CONFIG, "part_len " + std::to_string(part) +
                                        " must be a multiple of 16 and of page_len, at most 1008 pages");
    for (uint32_t l = 0; l < d->layers; l++) {
        uint32_t hd = d->head_dims ? d->head_dims[l] : d->head_dim;
        if (int rc = thb_backend_head_dim(hd)) return rc;
    }
    return guarded([&]() -> int {
        auto p = std::make_unique<thb_pool>();
        std::string err = Arena::create(d->seq_lens, d->seqs, d->pages, d->page_len, p->arena.a);
        if (!err.empty()) return fail(THB_ERR_MODEL, err);
        p->layers = d->layers;
        p->kv_heads = d->kv_heads;
        p->page_len = d->page_len;
        p->page_shift = __builtin_ctz(d->page_len);
        p->kv_dtype = d->kv_dtype;
        p->part_len = part;
        const uint64_t pool_len = static_cast<uint64_t>(p->arena.a.pages()) * d->page_len;
        if (pool_len >= (1ull << 32)) return fail(THB_ERR_CONFIG, "pages * page_len must stay below 2^32 slots");
        uint64_t off = 0;
        for (uint32_t l = 0; l < d->layers; l++) {
            uint32_t hd = d->head_dims ? d->head_dims[l] : d->head_dim;
            // A decode tile of 16 tokens spans two pages at page_len 8, read
            // through one buffer resource with 32-bit offsets between them.
            if (d->page_len < 16 && pool_len * hd * 2 > 0xFFFF0000ull)
                return fail(THB_ERR_CONFIG, "page_len " + std::to_string(d->page_len) + " holds at most 4 GiB per KV-head plane (layer " +
                                                std::to_string(l) + " needs " + std::to_string(pool_len * hd * 2) +
                                                " bytes); use page_len >= 16");
            uint64_t plane = (static_cast<uint64_t>(d->kv_heads) * pool_len * hd * 2 + 255) & ~uint64_t(255);
            p->geom.push_back({hd, off, off + plane});
            off += 2 * plane;
        }
        p->mem_bytes = off;
        THB_HIP(hipGetDevice(&p->device));
        int cus = 0;
        THB_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device));
        if (cus > 0) p->cus = static_cast<uint32_t>(cus);
        if (d->arena_dev) {
            if (d->arena_bytes < off)
                return fail(THB_ERR_CONFIG, "external arena holds " + std::to_string(d->arena_bytes) +
                                                " bytes, pool needs " + std::to_string(off));
            if (reinterpret_cast<uintptr_t>(d->arena_dev) % 256 != 0)
                return fail(THB_ERR_CONFIG, "external arena must be 256-byte aligned");
            p->mem = static_cast<uint8_t*>(d->arena_dev);
            p->owns_mem = false;
        } else {
            hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->mem), off);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return fail(THB_ERR_GPU, "KV pool of " + std::to_string(off) + " bytes does not fit: " +
                                             hipGetErrorString(e));
            }
            p->owns_mem = true;
        }
        THB_HIP(hipMemset(p->mem, 0, off));
        const size_t tbl = static_cast<size_t>(p->arena.a.seqs()) * p->arena.a.max_pages();
        THB_HIP(hipMalloc(reinterpret_cast<void**>(&p->table_dev), tbl * 4));
        THB_HIP(hipMemset(p->table_dev, 0xFF, tbl * 4));
        init_page_state(p.get());
        p->fixed_stager.init(THB_NOALLOC_PLAN_BYTES);
        std::vector<DevLayer> dl;
        for (const auto& g : p->geom) dl.push_back({g.k_off, g.v_off, g.head_dim, 0});
        void* gd = p->geom_buf.reserve(dl.size() * sizeof(DevLayer), false, nullptr);
        THB_HIP(hipMemcpy(gd, dl.data(), dl.size() * sizeof(DevLayer), hipMemcpyHostToDevice));
        THB_HIP(hipDeviceSynchronize());
        *out = p.release();
        return THB_OK;
    });
}

void thb_pool_destroy(thb_pool* pool) {
    if (!pool) return;
    (void)hipDeviceSynchronize();
    if (pool->owns_mem && pool->mem) (void)hipFree(pool->mem);
    if (pool->table_dev) (void)hipFree(pool->table_dev);
    if (pool->state_dev) (void)hipFree(pool->state_dev);
    delete pool;
}

// Each page-API call runs on the host mirror (which reports errors as the
// reference does) and, when it changed the allocator, is queued for the
// device allocator; pool_flush replays the queue before the next kernel.
int thb_pool_alloc(thb_pool* pool, uint32_t seq, uint32_t pos, uint32_t tokens) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (int rc = sync_mirror(pool, nullptr)) return rc;
    const uint64_t v = pool->arena.a.version();
    const size_t c = pool->arena.a.copies().size();
    if (int rc = thb_arena_alloc(&pool->arena, seq, pos, tokens)) return rc;
    if (pool->arena.a.version() != v) queue_page_op(pool, kPageOpAlloc, seq, pos, tokens, c);
    return THB_OK;
}

int thb_pool_free_seq(thb_pool* pool, uint32_t seq) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (int rc = sync_mirror(pool, nullptr)) return rc;
    const uint64_t v = pool->arena.a.version();
    const size_t c = pool->arena.a.copies().size();
    if (int rc = thb_arena_free_seq(&pool->arena, seq)) return rc;
    if (pool->arena.a.version() != v) queue_page_op(pool, kPageOpFree, seq, 0, 0, c);
    return THB_OK;
}

int thb_pool_truncate(thb_pool* pool, uint32_t seq, uint32_t keep_tokens) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (int rc = sync_mirror(pool, nullptr)) return rc;
    const uint64_t v = pool->arena.a.version();
    const size_t c = pool->arena.a.copies().size();
    if (int rc = thb_arena_truncate(&pool->arena, seq, keep_tokens)) return rc;
    if (pool->arena.a.version() != v) queue_page_op(pool, kPageOpTruncate, seq, keep_tokens, 0, c);
    return THB_OK;
}

int thb_pool_fork(thb_pool* pool, uint32_t src, uint32_t dst, uint32_t tokens) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (int rc = sync_mirror(pool, nullptr)) return rc;
    const size_t c = pool->arena.a.copies().size();
    if (int rc = thb_arena_fork(&pool->arena, src, dst, tokens)) return rc;
    queue_page_op(pool, kPageOpFork, src, dst, tokens, c);
    return THB_OK;
}

int thb_pool_sync(thb_pool* pool, void* stream) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    return guarded([&]() -> int {
        pool_flush(pool, as_stream(stream));
        return THB_OK;
    });
}

const thb_arena* thb_pool_arena(const thb_pool* pool) { return pool ? &pool->arena : nullptr; }

int thb_pool_layer(const thb_pool* pool, uint32_t layer, void** k_dev, void** v_dev, thb_layer_info* info) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (layer >= pool->layers)
        return fail(THB_ERR_INVALID, "layer " + std::to_string(layer) + " out of range (" +
                                         std::to_string(pool->layers) + " layers)");
    const LayerGeom& g = pool->geom[layer];
    if (k_dev) *k_dev = pool->mem + g.k_off;
    if (v_dev) *v_dev = pool->mem + g.v_off;
    if (info) {
        info->kv_heads = pool->kv_heads;
        info->head_dim = g.head_dim;
        info->pool_len = pool->arena.a.pages() * pool->page_len;
        info->max_pages = pool->arena.a.max_pages();
        info->page_len = pool->page_len;
        info->kv_dtype = pool->kv_dtype;
        info->plane_elems = static_cast<uint64_t>(info->pool_len) * g.head_dim;
        info->page_layout = THB_PAGE_LAYOUT_MFMA;
    }
    return THB_OK;
}

int thb_pool_block_table(const thb_pool* pool, const uint32_t** table_dev) {
    if (!pool || !table_dev) return fail(THB_ERR_INVALID, "null argument");
    *table_dev = pool->table_dev;
    return THB_OK;
}

int thb_pool_memory(const thb_pool* pool, void** base_dev, uint64_t* bytes) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (base_dev) *base_dev = pool->mem;
    if (bytes) *bytes = pool->mem_bytes;
    return THB_OK;
}

// ----------------------------------------------------------------- rows
int thb_rows_create(uint32_t max_m, thb_rows** out) {
    if (!out) return fail(THB_ERR_INVALID, "out is null");
    *out = nullptr;
    if (max_m == 0) return fail(THB_ERR_INVALID, "max_m must be positive");
    return guarded([&]() -> int {
        auto r = std::make_unique<thb_rows>();
        r->max_m = max_m;
        THB_HIP(hipMalloc(reinterpret_cast<void**>(&r->dev), static_cast<size_t>(max_m) * 32));
        THB_HIP(hipMemset(r->dev, 0, static_cast<size_t>(max_m) * 32));
        r->host.assign(static_cast<size_t>(max_m) * 8, 0);
        *out = r.release();
        return THB_OK;
    });
}

void thb_rows_destroy(thb_rows* rows) {
    if (!rows) return;
    (void)hipDeviceSynchronize();
    if (rows->dev) (void)hipFree(rows->dev);
    delete rows;
}

int thb_rows_write(thb_rows* rows, const uint32_t* positions, const uint32_t* seqs, uint32_t m, void* stream) {
    // rows.rs:19-30
    if (!rows || (m && (!positions || !seqs))) return fail(THB_ERR_INVALID, "null argument");
    if (m > rows->max_m)
        return fail(THB_ERR_INVALID, "row meta arrays must cover the chunk size: " + std::to_string(m) + " > " +
                                         std::to_string(rows->max_m));
    return guarded([&]() -> int {
        std::fill(rows->host.begin(), rows->host.end(), 0u);
        for (uint32_t i = 0; i < m; i++) {
            rows->host[8 * i] = positions[i];
            rows->host[8 * i + 1] = seqs[i];
        }
        rows->m = m;
        rows->version = next_version();
        rows->stager.upload(rows->dev, rows->host.data(), static_cast<size_t>(std::max<uint32_t>(m, 1)) * 32,
                            as_stream(stream));
        return THB_OK;
    });
}

const uint32_t* thb_rows_device(const thb_rows* rows) { return rows ? rows->dev : nullptr; }

}  // extern "C"
