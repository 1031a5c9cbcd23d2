// Internal layout of the device pool and the row-meta object, shared by the
// translation units of the HIP backend.
#pragma once

#include <array>
#include <cstdint>
#include <memory>
#include <vector>

#include "arena.hpp"
#include "common.hpp"

namespace thb {

// Per-layer record the block-copy kernel reads on the device.
struct DevLayer {
    uint64_t k_off, v_off;  // byte offsets into the arena
    uint32_t head_dim, pad;
};

struct LayerGeom {
    uint32_t head_dim;
    uint64_t k_off;  // byte offsets into the arena
    uint64_t v_off;
};

// One cached attention launch plan (see attention.hip).
struct AttnPlan {
    // key
    const void* rows = nullptr;
    uint64_t rows_version = ~0ull;
    uint64_t arena_version = ~0ull;
    uint32_t row_off = 0, m = 0, seq = 0, causal = 0, window = 0, q_heads = 0, head_dim = 0;
    // value
    uint32_t n_groups = 0, n_items = 0;     // decode work items
    uint32_t n_blocks = 0, n_bitems = 0;    // prefill blocks and their work items
    uint32_t n_bpairs = 0;                  // pairs of work items (attn_prefill_wide)
    uint32_t n_slots = 0;                   // partial-result slots (all groups' partitions)
    uint32_t hd_t = 0;   // head_dim template of the kernel
    bool wide = false;   // prefill blocks run attn_prefill_wide (head_dim <= 128)
    bool mixed = false;  // decode items and prefill blocks run as one launch (attn_mixed)
    bool split = false;  // some group spans several partitions: merge kernel runs
    uint32_t n_merge = 0, merge_off = 0;  // groups of several partitions: count, blob offset (words)
    uint32_t n_merge_dec = 0;             // of those, decode groups (listed first)
    bool fusable = false;  // an append of the call's rows can run inside the launch
    std::vector<uint32_t> blob;  // [groups | items | row ranges | prefill items | pairs | order | merge list]
    DevBuf dev;                  // blob on the device, when uploaded
    bool uploaded = false;
    uint64_t last_use = 0;
};

// Page-API calls the device allocator replays (pages.hip).
enum : uint32_t { kPageOpAlloc = 1, kPageOpFree = 2, kPageOpTruncate = 3, kPageOpFork = 4, kPageOpAllocRows = 5 };
// Device allocator header: the status word (first failure since the last
// thb_pool_status, then 3 arguments), and the status a device-planned
// attention call records for a row its sequence's pages do not cover
// (arguments: sequence, slots held, keys the row reads), for a call whose
// append cannot run inside its attention launch (arguments: row, sequence,
// reason kNoFuse*) and for a row past the plan's position limit (arguments:
// position, limit).
constexpr uint32_t kPageHdrStatus = 1;
constexpr uint32_t kPageHdrCopies = 5;  // copy-on-write copies in the device list
constexpr uint32_t kPageStBadSeq = 5;
constexpr uint32_t kPageStCover = 6;
constexpr uint32_t kPageStNoFuse = 8;
constexpr uint32_t kPageStPosLimit = 9;
enum : uint32_t { kNoFuseChunk = 1, kNoFuseKeys = 2, kNoFuseSeq = 3, kNoFuseTwice = 4 };

// A page-API call queued for the device allocator (pages.hip): it has run on
// the host mirror and runs on the device before the pool's next kernel.
struct PageOp {
    uint32_t kind, a, b, c;
    uint32_t copy_begin, copy_end;  // its copy-on-write copies in the mirror's list
};

// Word offsets of the device page state (one allocation).
struct PageStateLayout {
    uint32_t free_off, refs_off, npages_off, lens_off, copies_off, keys_off;
    size_t words;
};

}  // namespace thb

struct thb_arena {
    thb::Arena a;
};

struct thb_rows {
    uint32_t max_m = 0;
    uint32_t m = 0;
    uint32_t* dev = nullptr;          // 8 * max_m u32
    std::vector<uint32_t> host;       // mirror of what was last uploaded
    uint64_t version = 0;
    thb::Stager stager;
};

struct thb_pool {
    thb_arena arena;
    uint32_t layers = 0, kv_heads = 0, page_len = 0, page_shift = 0, kv_dtype = 0, part_len = 4096;
    std::vector<thb::LayerGeom> geom;
    uint8_t* mem = nullptr;  // device arena
    uint64_t mem_bytes = 0;
    bool owns_mem = false;
    uint32_t* table_dev = nullptr;   // [seqs * max_pages]
    // Device page allocator: header, free stack, reference counts, page
    // counts, sequence budgets and the copy-on-write list (pages.hip).  The
    // host arena above mirrors it: every page-API call runs on both.
    uint32_t* state_dev = nullptr;
    thb::PageStateLayout state;
    std::vector<thb::PageOp> page_ops;  // queued for the device
    // Set for good once thb_pool_alloc_rows is captured in a graph: its
    // replays change the device allocator without the host, so every later
    // call that reads the host arena reloads it from the device first
    // (sync_mirror).
    bool graph_mode = false;
    thb::Stager stager;
    thb::FixedStager fixed_stager;   // plan uploads of thb_attn_noalloc (never grows)
    thb::DevBuf copy_buf;            // copy triples
    thb::DevBuf geom_buf;            // per-layer DevLayer records
    thb::DevBuf partials;            // split-K partial results
    thb::DevBuf merge_cnt;           // arrival counters of split decode groups (zero between launches)
    thb::DevBuf run_buf;             // append runs of the last row meta the append cut into runs
    thb::DevBuf range_buf;           // work items and range records of a batched gather / scatter
    std::vector<uint32_t> range_key; // what range_buf holds
    // Key of run_buf's contents: the model appends the same rows to every
    // layer, so the runs are cut and uploaded once per row-meta write.
    const void* runs_rows = nullptr;
    uint64_t runs_version = ~0ull;
    uint32_t runs_off = 0, runs_m = 0, runs_max = 0, runs_n = 0, runs_long = 0;
    std::array<thb::AttnPlan, 4> plans;
    uint64_t plan_clock = 0;
    int device = 0;
    uint32_t cus = 256;  // compute units of the device (orders mixed launches)
};

namespace thb {
// Runs the queued page-API calls on the device allocator (and their page
// copies) before the next kernel on `stream`.  Allocates nothing.
void pool_flush(thb_pool* p, hipStream_t stream);
// Queues a page-API call that has run on the host mirror (pages.hip).
void queue_page_op(thb_pool* p, uint32_t kind, uint32_t a, uint32_t b, uint32_t c, size_t copies_before);
// Allocates and initialises the device page state of a new pool.
void init_page_state(thb_pool* p);
// Launches the block-copy kernel over n triples already on the device.
void launch_block_copy_dev(thb_pool* p, const uint32_t* triples_dev, uint32_t n, uint32_t max_tokens,
                           hipStream_t stream);
// Launches the block-copy kernel over the triples of a device list whose
// length the kernel reads from count_dev when it runs: grid_x workgroups
// per plane walk the list (a launch whose size does not depend on host
// state, for graphs).
void launch_block_copy_counted(thb_pool* p, const uint32_t* triples_dev, const uint32_t* count_dev, uint32_t grid_x,
                               hipStream_t stream);
// In graph mode, waits for the device and reloads the host mirror from the
// device allocator (thb_pool_pull); otherwise nothing.  Call before reading
// the host arena; refuses (THB_ERR_INVALID) while `stream` captures.
int sync_mirror(thb_pool* p, hipStream_t stream);
// Validates a thb_rope for rows [row_off, row_off + m) of head_dim vectors.
int check_rope(const thb_rope* r, uint32_t head_dim, const thb_rows* rows, uint32_t row_off, uint32_t m);
// The checks of check_rope that do not read positions (tables, rot, alignment).
int check_rope_tables(const thb_rope* r, uint32_t head_dim);
// Launches the block-copy kernel for n non-chaining host triples (passed in
// the kernel arguments when few, else uploaded through the stager).
void launch_block_copy(thb_pool* p, const uint32_t* triples, uint32_t n, uint32_t max_tokens, hipStream_t stream);
}  // namespace thb
