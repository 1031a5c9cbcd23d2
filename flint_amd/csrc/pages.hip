// Device-side page allocator: the free stack, the per-page reference counts
// and each sequence's page count live in HBM next to the block table, and
// the kernels below change them.  Semantics are KvArena's (reference
// crates/thuban_model/src/pool.rs:47-79): pops come off the top of a LIFO
// stack initialised so that they yield pages 0, 1, 2, ...; freed pages are
// pushed back in table order; alloc(seq, pos, tokens) checks the context
// limit, then that enough pages are free, then appends pages to the
// sequence's table.  The extension for shared pages (fork, reference counts,
// copy-on-write) is the host Arena's (arena.cpp), step for step.
//
// The host Arena mirrors this state: every page-API call runs on the mirror
// first (which reports errors synchronously, as the reference does) and is
// then queued for the device, where one workgroup replays the queue before
// the pool's next kernel (pool_flush).  thb_pool_alloc_rows allocates the
// pages of a call's rows on the device directly from the row meta, the
// engine's per-plan alloc_pages loop (thuban_generate/src/engine.rs:197-200)
// without a block-table upload.  Both run the same deterministic algorithm on
// the same state, so they agree; thb_pool_pull reloads the mirror from the
// device after device-only changes (e.g. replays of a captured graph).
//
// Device state (u32 words, one allocation):
//   header [64]: free-stack top, status (first failure since the last
//                thb_pool_status: code + 3 arguments), copy count, epoch of
//                the last alloc-rows call
//   free [pages] | refs [pages] | npages [seqs] | budgets [seqs] |
//   copies [pages x 3]: (src page, dst page, tokens) of the copy-on-write
//   copies made since the list was last reset (a flush resets it per batch) |
//   keys [seqs] (64-bit, 8-byte aligned): per sequence, the epoch and first
//   row of the last alloc-rows call that saw it head a run of rows.
#include <algorithm>
#include <string>

#include "pool.hpp"

namespace thb {
namespace {

enum : uint32_t {
    kStOk = 0,
    kStLimit = 1,
    kStExhausted = 2,
    kStForkTarget = 3,
    kStForkCover = 4,
    kStBadSeq = kPageStBadSeq,
    kStCover = kPageStCover,
    kStDupSeq = 7,
    kStNoFuse = kPageStNoFuse,
    kStPosLimit = kPageStPosLimit
};
enum : uint32_t {
    kHdrTop = 0,
    kHdrStatus = 1,
    kHdrA = 2,
    kHdrB = 3,
    kHdrC = 4,
    kHdrCopies = kPageHdrCopies,
    kHdrEpoch = 6,
    kHdrWords = 64
};
static_assert(kHdrStatus == kPageHdrStatus, "status word shared with the attention planner");

constexpr uint32_t kOpsPerLaunch = 64;  // page ops passed in one launch's arguments
// Set on an alloc op that runs in one batch with the alloc op before it
// (consecutive allocs of distinct sequences in one launch).
constexpr uint32_t kOpBatched = 0x100u;
constexpr uint32_t kT = 1024;           // threads of the page-op workgroup
constexpr uint32_t kNone = 0xFFFFFFFFu;

struct PageOpArgs {
    uint32_t* state;
    uint32_t* table;       // [seqs * max_pages]
    const uint32_t* meta;  // row meta of an alloc-rows op (at its first row)
    uint32_t pages, seqs, max_pages, shift;
    uint32_t free_off, refs_off, npages_off, lens_off, copies_off, keys_off;
    uint32_t n_ops, reset_copies;
    uint32_t ops[4 * kOpsPerLaunch];  // (kind, a, b, c)
};

struct St {
    uint32_t* hdr;
    uint32_t* free;
    uint32_t* refs;
    uint32_t* npages;
    const uint32_t* lens;
    uint32_t* copies;
    unsigned long long* keys;
    uint32_t* table;
    uint32_t pages, seqs, mp, shift;
    __device__ uint32_t* row(uint32_t seq) const { return table + static_cast<uint64_t>(seq) * mp; }
};

// Per-chunk scratch of one round of allocations (a chunk = one
// KvArena::alloc call: seq, first position, tokens).
struct Lds {
    uint32_t seq[kT], pos[kT], tok[kT], have[kT], want[kT], code[kT];
    uint32_t cnt[kT], pre[kT], base[kT], nnew[kT];
    uint32_t red[kT / 64];
    uint32_t top, ncopy, first_fail, shared;
    uint32_t epoch, bad, reset;
};

// Inclusive scan (sum, or max when MAX) over the workgroup; *total gets the
// workgroup's result.  Every thread must call it.
template <bool MAX>
__device__ uint32_t block_scan(uint32_t v, Lds& L, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(v, d);
        if (lane >= d) v = MAX ? max(v, t) : v + t;
    }
    if (lane == 63) L.red[w] = v;
    __syncthreads();
    if (w == 0) {
        uint32_t x = lane < nw ? L.red[lane] : 0u;
#pragma unroll
        for (uint32_t d = 1; d < 64; d <<= 1) {
            const uint32_t t = __shfl_up(x, d);
            if (lane >= d) x = MAX ? max(x, t) : x + t;
        }
        if (lane < nw) L.red[lane] = x;
    }
    __syncthreads();
    if (w > 0) {
        const uint32_t p = L.red[w - 1];
        v = MAX ? max(v, p) : v + p;
    }
    *total = L.red[nw - 1];
    __syncthreads();
    return v;
}

// Smallest c < n with pre[c] > g (pre: inclusive prefix sums).
__device__ uint32_t find_chunk(const uint32_t* pre, uint32_t n, uint32_t g) {
    uint32_t lo = 0, hi = n - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (pre[mid] > g)
            hi = mid;
        else
            lo = mid + 1;
    }
    return lo;
}

// First failure since the status was last cleared (one thread).
__device__ void record(const St& st, uint32_t code, uint32_t a, uint32_t b, uint32_t c) {
    if (st.hdr[kHdrStatus] != kStOk) return;
    st.hdr[kHdrStatus] = code;
    st.hdr[kHdrA] = a;
    st.hdr[kHdrB] = b;
    st.hdr[kHdrC] = c;
}

// KvArena::alloc (pool.rs:47-65) with copy-on-write, for chunks [0, n) in
// L.{seq,pos,tok} in order, as if called one after another: a chunk fails on
// the context limit or on too few free pages, and the chunks after a failure
// are not run.  Returns true if a chunk failed.
//  * Without shared pages in any write range (the common case) the chunks
//    are independent: each needs want - have new pages, and an exclusive scan
//    of those counts gives the position of its first pop.
//  * Otherwise one thread walks the chunks in order with the host Arena's
//    copy-on-write step (a page shared by two chunks is copied only by the
//    first), recording each chunk's pop position; new pages are then
//    written in parallel either way.
__device__ bool alloc_chunks(const St& st, uint32_t n, Lds& L) {
    const uint32_t tid = threadIdx.x, P = 1u << st.shift;
    uint32_t total = 0;
    if (tid == 0) {
        L.first_fail = kNone;
        L.shared = 0;
    }
    if (tid < n) {
        const uint32_t seq = L.seq[tid], pos = L.pos[tid], tok = L.tok[tid];
        uint32_t code = kStOk, have = 0, want = 0, cnt = 0;
        if (seq >= st.seqs) {
            code = kStBadSeq;
        } else {
            have = st.npages[seq];
            const uint64_t end = static_cast<uint64_t>(pos) + tok;
            if (end > st.lens[seq]) {
                code = kStLimit;
            } else {
                want = static_cast<uint32_t>((end + P - 1) >> st.shift);
                const uint32_t r0 = pos >> st.shift, r1 = min(have, want);
                cnt = tok > 0 && r1 > r0 ? r1 - r0 : 0u;  // held pages the write range touches
            }
        }
        L.have[tid] = have;
        L.want[tid] = want;
        L.code[tid] = code;
        L.cnt[tid] = cnt;
    }
    // Is any page in a write range shared?  One (chunk, page) pair per lane.
    uint32_t incl = block_scan<false>(tid < n ? L.cnt[tid] : 0u, L, &total);
    if (tid < n) L.pre[tid] = incl;
    __syncthreads();
    for (uint32_t g = tid; g < total; g += blockDim.x) {
        const uint32_t c = find_chunk(L.pre, n, g);
        const uint32_t i = (L.pos[c] >> st.shift) + g - (L.pre[c] - L.cnt[c]);
        const uint32_t p = st.row(L.seq[c])[i];
        if (p < st.pages && st.refs[p] > 1) L.shared = 1;
    }
    __syncthreads();
    if (!L.shared) {
        const uint32_t nn = tid < n && L.code[tid] == kStOk && L.want[tid] > L.have[tid] ? L.want[tid] - L.have[tid] : 0u;
        incl = block_scan<false>(nn, L, &total);
        if (tid < n) {
            const uint32_t o = incl - nn;
            L.base[tid] = o;
            L.nnew[tid] = nn;
            if (L.code[tid] != kStOk || o + nn > L.top) atomicMin(&L.first_fail, tid);
        }
    } else if (tid == 0) {
        uint32_t o = 0;
        for (uint32_t c = 0; c < n; c++) {
            L.base[c] = o;
            if (L.code[c] != kStOk) {
                L.first_fail = c;
                break;
            }
            const uint32_t seq = L.seq[c], pos = L.pos[c], have = L.have[c], want = L.want[c];
            uint32_t* row = st.row(seq);
            const uint32_t r0 = pos >> st.shift, r1 = L.tok[c] > 0 ? min(have, want) : 0u;
            uint32_t cow = 0;
            for (uint32_t i = r0; i < r1; i++)
                if (row[i] < st.pages && st.refs[row[i]] > 1) cow++;
            const uint32_t nn = want > have ? want - have : 0u;
            if (o + nn + cow > L.top) {
                L.nnew[c] = nn + cow;  // the request the error reports
                L.first_fail = c;
                break;
            }
            for (uint32_t i = r0; i < r1; i++) {
                const uint32_t old = row[i];
                if (old >= st.pages || st.refs[old] <= 1) continue;
                const uint32_t fresh = st.free[L.top - 1 - o];
                o++;
                const uint64_t first = static_cast<uint64_t>(i) << st.shift;
                const uint32_t ntok = pos > first ? static_cast<uint32_t>(min<uint64_t>(P, pos - first)) : 0u;
                if (ntok && L.ncopy < st.pages) {
                    st.copies[3 * L.ncopy] = old;
                    st.copies[3 * L.ncopy + 1] = fresh;
                    st.copies[3 * L.ncopy + 2] = ntok;
                    L.ncopy++;
                }
                st.refs[old] -= 1;
                if (fresh < st.pages) st.refs[fresh] = 1;
                row[i] = fresh;
            }
            L.base[c] = o;
            L.nnew[c] = nn;
            o += nn;
        }
    }
    __syncthreads();
    const uint32_t ff = L.first_fail;  // kNone: every chunk succeeds
    const uint32_t done = ff == kNone ? n : ff;
    if (tid == ff) {
        const uint32_t code = L.code[tid], seq = L.seq[tid];
        if (code == kStBadSeq)
            record(st, kStBadSeq, seq, st.seqs, 0);
        else if (code == kStLimit)
            record(st, kStLimit, st.lens[seq], seq, 0);
        else
            record(st, kStExhausted, L.nnew[tid], L.top - L.base[tid], seq);
    }
    // New pages of the chunks that succeed: pop position base + j.
    const uint32_t mine = tid < done ? L.nnew[tid] : 0u;
    incl = block_scan<false>(mine, L, &total);
    if (tid < n) L.pre[tid] = incl;
    __syncthreads();
    for (uint32_t g = tid; g < total; g += blockDim.x) {
        const uint32_t c = find_chunk(L.pre, done, g);
        const uint32_t j = g - (L.pre[c] - L.nnew[c]);
        const uint32_t p = st.free[L.top - 1 - (L.base[c] + j)];
        st.row(L.seq[c])[L.have[c] + j] = p;
        if (p < st.pages) st.refs[p] = 1;
    }
    if (tid < done && L.want[tid] > L.have[tid]) st.npages[L.seq[tid]] = L.want[tid];
    __syncthreads();
    if (tid == 0) L.top -= ff == kNone ? L.base[n - 1] + L.nnew[n - 1] : L.base[ff];
    __syncthreads();
    return ff != kNone;
}

// Validates an alloc-rows call before anything is allocated, as the host
// does: every row's sequence in range, and no sequence heading two runs of
// rows (two runs allocated in one parallel round would write the same
// table slots).  The first offending row (in row order) is recorded and the
// call returns false.  A sequence's key (epoch << 32 inverted, | row) keeps,
// by atomicMin, the first row heading one of its runs in this call: older
// calls' epochs give larger keys.  When the epoch counter wraps, every key
// is reset first.
__device__ bool check_rows(const St& st, const uint32_t* meta, uint32_t m, Lds& L) {
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        uint32_t e = st.hdr[kHdrEpoch] + 1u;
        L.reset = e == 0u;
        if (e == 0u) e = 1u;
        st.hdr[kHdrEpoch] = e;
        L.epoch = e;
        L.bad = kNone;
    }
    __syncthreads();
    if (L.reset) {
        for (uint32_t s = tid; s < st.seqs; s += blockDim.x) st.keys[s] = ~0ull;
        __syncthreads();
    }
    const unsigned long long hi = static_cast<unsigned long long>(~L.epoch) << 32;
    for (uint32_t r = tid; r < m; r += blockDim.x) {
        const uint32_t seq = meta[8u * r + 1];
        if (seq >= st.seqs)
            atomicMin(&L.bad, r);
        else if (r == 0 || meta[8u * (r - 1) + 1] != seq)
            atomicMin(&st.keys[seq], hi | r);
    }
    __syncthreads();
    for (uint32_t r = tid; r < m; r += blockDim.x) {
        const uint32_t seq = meta[8u * r + 1];
        if (seq < st.seqs && (r == 0 || meta[8u * (r - 1) + 1] != seq)) {
            const unsigned long long k = atomicAdd(&st.keys[seq], 0ull);  // read at the cache the atomics used
            if (static_cast<uint32_t>(k) != r) atomicMin(&L.bad, r);
        }
    }
    __syncthreads();
    const uint32_t bad = L.bad;
    if (bad == kNone) return true;
    if (tid == 0) {
        const uint32_t seq = meta[8u * bad + 1];
        if (seq >= st.seqs)
            record(st, kStBadSeq, seq, st.seqs, 0);
        else
            record(st, kStDupSeq, seq, 0, 0);
    }
    __syncthreads();
    return false;
}

// Chunks of rows [0, m) of the row meta, in row order: maximal runs of rows
// of one sequence, each allocated as KvArena::alloc(seq, position of its
// first row, rows in the run), after check_rows.  Rows are read in tiles of one row per lane;
// the chunks that end in a tile are allocated before the next tile is read,
// and a failure ends the call.
__device__ void alloc_rows(const St& st, const uint32_t* meta, uint32_t m, Lds& L) {
    const uint32_t tid = threadIdx.x;
    if (!check_rows(st, meta, m, L)) return;
    uint32_t open = 0;  // 1 + first row of the chunk still open at the end of the last tile
    for (uint32_t t0 = 0; t0 < m; t0 += blockDim.x) {
        const uint32_t r = t0 + tid;
        const bool valid = r < m;
        const uint32_t seq = valid ? meta[8u * r + 1] : 0u;
        const bool first = valid && (r == 0 || meta[8u * (r - 1) + 1] != seq);
        const bool last = valid && (r + 1 == m || meta[8u * (r + 1) + 1] != seq);
        uint32_t tile_max = 0, n_last = 0;
        const uint32_t start = max(block_scan<true>(first ? r + 1 : 0u, L, &tile_max), open) - 1;
        const uint32_t idx = block_scan<false>(last ? 1u : 0u, L, &n_last);
        if (last) {
            L.seq[idx - 1] = seq;
            L.pos[idx - 1] = meta[8u * start];
            L.tok[idx - 1] = r - start + 1;
        }
        open = max(open, tile_max);
        __syncthreads();
        if (n_last && alloc_chunks(st, n_last, L)) return;
    }
}

// KvArena::free_seq (pool.rs:67-71) when keep == kNone, else truncate
// (pool.rs:73-79): pages [keep_pages, n) lose a reference; those left
// unreferenced are pushed in table order.
__device__ void release(const St& st, uint32_t seq, uint32_t keep, Lds& L) {
    const uint32_t tid = threadIdx.x;
    if (seq >= st.seqs) {
        if (tid == 0) record(st, kStBadSeq, seq, st.seqs, 0);
        return;
    }
    uint32_t* row = st.row(seq);
    const uint32_t n = st.npages[seq];
    uint32_t k = 0;
    if (keep != kNone) {
        const uint32_t kp = static_cast<uint32_t>((static_cast<uint64_t>(keep) + (1u << st.shift) - 1) >> st.shift);
        k = min(kp, n);
    }
    uint32_t top = L.top;
    for (uint32_t b = k; b < n; b += blockDim.x) {
        const uint32_t i = b + tid;
        uint32_t p = 0, flag = 0, total = 0;
        if (i < n) {
            p = row[i];
            if (p < st.pages) {
                const uint32_t r = st.refs[p] - 1;
                st.refs[p] = r;
                flag = r == 0;
            }
            row[i] = kNone;
        }
        const uint32_t incl = block_scan<false>(flag, L, &total);
        if (flag && top + incl - 1 < st.pages) st.free[top + incl - 1] = p;
        top += total;
    }
    if (tid == 0) {
        st.npages[seq] = k;
        L.top = top;
    }
    __syncthreads();
}

// Fork extension (arena.cpp Arena::fork): dst shares src's pages holding
// tokens [0, tokens); a partial last page is replaced by a fresh copy.
__device__ void fork(const St& st, uint32_t src, uint32_t dst, uint32_t tokens, Lds& L) {
    const uint32_t tid = threadIdx.x, P = 1u << st.shift;
    uint32_t code = kStOk, a = 0, b = 0;
    if (src >= st.seqs || dst >= st.seqs) {
        code = kStBadSeq;
        a = src >= st.seqs ? src : dst;
        b = st.seqs;
    } else if (st.npages[dst] != 0) {
        code = kStForkTarget;
        a = dst;
    } else if (tokens > st.lens[dst]) {
        code = kStLimit;
        a = st.lens[dst];
        b = dst;
    } else if ((static_cast<uint64_t>(st.npages[src]) << st.shift) < tokens) {
        code = kStForkCover;
        a = src;
        b = tokens;
    } else if ((tokens & (P - 1)) && L.top == 0) {
        code = kStExhausted;
        a = 1;
        b = 0;
    }
    if (code != kStOk) {
        if (tid == 0) record(st, code, a, b, dst);
        __syncthreads();
        return;
    }
    const uint32_t n = static_cast<uint32_t>((static_cast<uint64_t>(tokens) + P - 1) >> st.shift);
    const uint32_t* from = st.row(src);
    uint32_t* to = st.row(dst);
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const uint32_t p = from[i];
        to[i] = p;
        if (p < st.pages) st.refs[p] += 1;
    }
    __syncthreads();
    if (tid == 0) {
        const uint32_t partial = tokens & (P - 1);
        if (partial) {
            const uint32_t old = to[n - 1], fresh = st.free[L.top - 1];
            L.top -= 1;
            if (L.ncopy < st.pages) {
                st.copies[3 * L.ncopy] = old;
                st.copies[3 * L.ncopy + 1] = fresh;
                st.copies[3 * L.ncopy + 2] = partial;
                L.ncopy++;
            }
            if (old < st.pages) st.refs[old] -= 1;
            if (fresh < st.pages) st.refs[fresh] = 1;
            to[n - 1] = fresh;
        }
        st.npages[dst] = n;
    }
    __syncthreads();
}

// Runs a.n_ops page ops in order in one workgroup.
__global__ __launch_bounds__(kT) void page_ops_kernel(PageOpArgs a) {
    __shared__ Lds L;
    St st;
    st.hdr = a.state;
    st.free = a.state + a.free_off;
    st.refs = a.state + a.refs_off;
    st.npages = a.state + a.npages_off;
    st.lens = a.state + a.lens_off;
    st.copies = a.state + a.copies_off;
    st.keys = reinterpret_cast<unsigned long long*>(a.state + a.keys_off);
    st.table = a.table;
    st.pages = a.pages;
    st.seqs = a.seqs;
    st.mp = a.max_pages;
    st.shift = a.shift;
    if (threadIdx.x == 0) {
        L.top = st.hdr[kHdrTop];
        L.ncopy = a.reset_copies ? 0u : st.hdr[kHdrCopies];
    }
    __syncthreads();
    for (uint32_t o = 0; o < a.n_ops;) {
        const uint32_t kind = a.ops[4 * o] & 0xFFu, x = a.ops[4 * o + 1], y = a.ops[4 * o + 2], z = a.ops[4 * o + 3];
        uint32_t next = o + 1;
        switch (kind) {
            case kPageOpAlloc: {
                // A batch of allocs of distinct sequences: one alloc_chunks
                // over all of them, in order (the host mirror has run each
                // call already, so none of them fails).
                while (next < a.n_ops && (a.ops[4 * next] & kOpBatched)) next++;
                const uint32_t n = next - o, t = threadIdx.x;
                if (t < n) {
                    L.seq[t] = a.ops[4 * (o + t) + 1];
                    L.pos[t] = a.ops[4 * (o + t) + 2];
                    L.tok[t] = a.ops[4 * (o + t) + 3];
                }
                __syncthreads();
                alloc_chunks(st, n, L);
                break;
            }
            case kPageOpAllocRows: alloc_rows(st, a.meta, x, L); break;
            case kPageOpFree: release(st, x, kNone, L); break;
            case kPageOpTruncate: release(st, x, y, L); break;
            case kPageOpFork: fork(st, x, y, z, L); break;
            default: break;
        }
        __syncthreads();
        o = next;
    }
    if (threadIdx.x == 0) {
        st.hdr[kHdrTop] = L.top;
        st.hdr[kHdrCopies] = L.ncopy;
    }
}

PageOpArgs op_args(const thb_pool* p) {
    PageOpArgs a{};
    a.state = p->state_dev;
    a.table = p->table_dev;
    a.pages = p->arena.a.pages();
    a.seqs = p->arena.a.seqs();
    a.max_pages = p->arena.a.max_pages();
    a.shift = p->page_shift;
    a.free_off = p->state.free_off;
    a.refs_off = p->state.refs_off;
    a.npages_off = p->state.npages_off;
    a.lens_off = p->state.lens_off;
    a.copies_off = p->state.copies_off;
    a.keys_off = p->state.keys_off;
    return a;
}

void launch_ops(const PageOpArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(page_ops_kernel, dim3(1), dim3(kT), 0, s, a);
    THB_HIP(hipGetLastError());
}

// Launches the copy kernel over device copies [0, n) made since the last
// reset; max_tokens is the largest copy (the host mirror's record).
void run_device_copies(thb_pool* p, size_t c0, size_t c1, hipStream_t s) {
    if (c1 <= c0) return;
    const auto& copies = p->arena.a.copies();
    uint32_t max_tok = 0;
    for (size_t i = c0; i < c1; i++) max_tok = std::max(max_tok, copies[i].tokens);
    launch_block_copy_dev(p, p->state_dev + p->state.copies_off, static_cast<uint32_t>(c1 - c0), max_tok, s);
}

std::string status_message(const uint32_t* hdr) {
    const uint32_t a = hdr[kHdrA], b = hdr[kHdrB];
    switch (hdr[kHdrStatus]) {
        case kStLimit: return "context limit " + std::to_string(a) + " reached";
        case kStExhausted:
            return "KV arena exhausted: " + std::to_string(a) + " pages requested, " + std::to_string(b) + " free";
        case kStForkTarget: return "fork target " + std::to_string(a) + " is not empty";
        case kStForkCover:
            return "fork source " + std::to_string(a) + " does not cover " + std::to_string(b) + " tokens";
        case kStBadSeq: return "sequence " + std::to_string(a) + " out of range (" + std::to_string(b) + " sequences)";
        case kStDupSeq:
            return "sequence " + std::to_string(a) + " heads two runs of rows in one call (one run per sequence)";
        case kStCover:
            return "pages must cover the chunk: sequence " + std::to_string(a) + " holds " + std::to_string(b) +
                   " slots, a row reads " + std::to_string(hdr[kHdrC]);
        case kStPosLimit:
            return "row position " + std::to_string(a) + " outside the rope tables (" + std::to_string(b) +
                   " positions)";
        case kStNoFuse: {
            const uint32_t why = hdr[kHdrC];
            const char* reason = why == kNoFuseChunk   ? "its chunk holds more rows than one group"
                                 : why == kNoFuseKeys  ? "its keys do not end at its new token (position + 1), or "
                                                         "positions do not rise within its chunk"
                                 : why == kNoFuseSeq   ? "its sequence is not the call's fixed sequence"
                                 : why == kNoFuseTwice ? "its sequence heads an earlier chunk of the call too"
                                                       : "unknown reason";
            return "the append cannot run inside the attention launch: row " + std::to_string(a) + " (sequence " +
                   std::to_string(b) + "): " + reason + "; nothing was appended";
        }
        default: return "device page allocator status " + std::to_string(hdr[kHdrStatus]);
    }
}

}  // namespace

void init_page_state(thb_pool* p) {
    const Arena& ar = p->arena.a;
    const uint32_t pages = ar.pages(), seqs = ar.seqs();
    PageStateLayout& L = p->state;
    L.free_off = kHdrWords;
    L.refs_off = L.free_off + pages;
    L.npages_off = L.refs_off + pages;
    L.lens_off = L.npages_off + seqs;
    L.copies_off = L.lens_off + seqs;
    L.keys_off = (L.copies_off + 3u * pages + 1u) & ~1u;  // 8-byte aligned 64-bit keys
    L.words = static_cast<size_t>(L.keys_off) + 2ull * seqs;
    std::vector<uint32_t> h(L.words, 0u);
    std::fill(h.begin() + L.keys_off, h.end(), ~0u);
    h[kHdrTop] = pages;
    for (uint32_t i = 0; i < pages; i++) h[L.free_off + i] = ar.free_list()[i];
    for (uint32_t s = 0; s < seqs; s++) h[L.lens_off + s] = ar.seq_len(s);
    THB_HIP(hipMalloc(reinterpret_cast<void**>(&p->state_dev), L.words * 4));
    THB_HIP(hipMemcpy(p->state_dev, h.data(), L.words * 4, hipMemcpyHostToDevice));
}

void queue_page_op(thb_pool* p, uint32_t kind, uint32_t a, uint32_t b, uint32_t c, size_t copies_before) {
    p->page_ops.push_back({kind, a, b, c, static_cast<uint32_t>(copies_before),
                           static_cast<uint32_t>(p->arena.a.copies().size())});
}

// Replays the queued page ops on the device in batches whose copy-on-write
// copies touch distinct pages (a batch's copies run in parallel after its
// ops): one op launch per kOpsPerLaunch ops, passed in the kernel
// arguments, then one copy launch over the batch's device copy list.
void pool_flush(thb_pool* p, hipStream_t stream) {
    auto& ops = p->page_ops;
    if (ops.empty()) return;
    if (capturing(stream))
        throw CaptureRefused{"page-API calls queued on the host (thb_pool_alloc, _free_seq, _truncate, _fork) "
                             "must run before the capture starts (thb_pool_sync): a graph would repeat them on "
                             "every replay"};
    const auto& copies = p->arena.a.copies();
    auto emit = [&](size_t i0, size_t i1) {
        for (size_t k = i0; k < i1; k += kOpsPerLaunch) {
            PageOpArgs a = op_args(p);
            a.n_ops = static_cast<uint32_t>(std::min<size_t>(kOpsPerLaunch, i1 - k));
            a.reset_copies = k == i0;
            std::vector<uint32_t> batch;  // sequences of the alloc batch being formed
            for (uint32_t o = 0; o < a.n_ops; o++) {
                const PageOp& op = ops[k + o];
                uint32_t kind = op.kind;
                if (kind == kPageOpAlloc) {
                    if (!batch.empty() && std::find(batch.begin(), batch.end(), op.a) == batch.end())
                        kind |= kOpBatched;
                    else
                        batch.clear();
                    batch.push_back(op.a);
                } else {
                    batch.clear();
                }
                a.ops[4 * o] = kind;
                a.ops[4 * o + 1] = op.a;
                a.ops[4 * o + 2] = op.b;
                a.ops[4 * o + 3] = op.c;
            }
            launch_ops(a, stream);
        }
        run_device_copies(p, ops[i0].copy_begin, ops[i1 - 1].copy_end, stream);
    };
    std::vector<uint32_t> touched;
    size_t seg = 0;
    for (size_t i = 0; i < ops.size(); i++) {
        bool clash = false;
        for (uint32_t c = ops[i].copy_begin; c < ops[i].copy_end && !clash; c++)
            clash = std::find(touched.begin(), touched.end(), copies[c].src) != touched.end() ||
                    std::find(touched.begin(), touched.end(), copies[c].dst) != touched.end();
        if (clash) {
            emit(seg, i);
            seg = i;
            touched.clear();
        }
        for (uint32_t c = ops[i].copy_begin; c < ops[i].copy_end; c++) {
            touched.push_back(copies[c].src);
            touched.push_back(copies[c].dst);
        }
    }
    emit(seg, ops.size());
    ops.clear();
    p->arena.a.copies().clear();
}

int sync_mirror(thb_pool* p, hipStream_t stream) {
    if (!p->graph_mode) return THB_OK;
    return guarded([&]() -> int {
        if (capturing(stream) || capturing(nullptr))
            throw CaptureRefused{"in graph mode the host mirror is reloaded from the device first, which waits "
                                 "for the device"};
        THB_HIP(hipDeviceSynchronize());  // replays on any stream
        pool_flush(p, nullptr);
        THB_HIP(hipDeviceSynchronize());
        std::vector<uint32_t> h(p->state.words);
        THB_HIP(hipMemcpy(h.data(), p->state_dev, p->state.words * 4, hipMemcpyDeviceToHost));
        Arena& ar = p->arena.a;
        std::vector<uint32_t> table(static_cast<size_t>(ar.seqs()) * ar.max_pages());
        THB_HIP(hipMemcpy(table.data(), p->table_dev, table.size() * 4, hipMemcpyDeviceToHost));
        ar.load_state(h.data() + p->state.free_off, h[kHdrTop], h.data() + p->state.refs_off,
                      h.data() + p->state.npages_off, table.data());
        return THB_OK;
    });
}

}  // namespace thb

using namespace thb;

namespace {

// Reads the device page state into host arrays after the stream's work.
void read_state(thb_pool* p, hipStream_t s, std::vector<uint32_t>& h) {
    if (capturing(s)) throw CaptureRefused{"reading the device allocator's state waits for the stream"};
    pool_flush(p, s);
    THB_HIP(hipStreamSynchronize(s));
    h.resize(p->state.words);
    THB_HIP(hipMemcpy(h.data(), p->state_dev, p->state.words * 4, hipMemcpyDeviceToHost));
}

}  // namespace

extern "C" {

int thb_pool_alloc_rows(thb_pool* pool, const thb_rows* rows, uint32_t row_off, uint32_t m, void* stream) {
    if (!pool || !rows) return fail(THB_ERR_INVALID, "null pool or rows");
    if (m == 0) return THB_OK;
    hipStream_t s = as_stream(stream);
    if (capturing(s)) {
        // Under capture the call is the device allocator alone: replays read
        // the row meta of their own time, validate it (bad or repeated
        // sequences are recorded for thb_pool_status) and size the
        // copy-on-write launch from the device's own copy count.  The host
        // mirror cannot follow the replays: the pool enters graph mode.
        if (static_cast<uint64_t>(row_off) + m > rows->max_m)
            return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->max_m) + " rows, call needs " +
                                             std::to_string(static_cast<uint64_t>(row_off) + m));
        return guarded([&]() -> int {
            pool_flush(pool, s);  // refuses queued host page ops
            PageOpArgs a = op_args(pool);
            a.meta = rows->dev + 8 * static_cast<size_t>(row_off);
            a.n_ops = 1;
            a.reset_copies = 1;
            a.ops[0] = kPageOpAllocRows;
            a.ops[1] = m;
            launch_ops(a, s);
            // A run of t rows writes into at most t pages, so the call makes
            // at most m copies; 4 workgroups per plane walk them.
            launch_block_copy_counted(pool, pool->state_dev + pool->state.copies_off, pool->state_dev + kHdrCopies,
                                      std::min<uint32_t>(m, 4), s);
            pool->graph_mode = true;
            return THB_OK;
        });
    }
    if (int rc = sync_mirror(pool, s)) return rc;
    if (static_cast<uint64_t>(row_off) + m > rows->m)
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->m) + " rows, call needs " +
                                         std::to_string(static_cast<uint64_t>(row_off) + m));
    Arena& ar = pool->arena.a;
    const uint32_t* meta = rows->host.data() + 8 * static_cast<size_t>(row_off);
    // Chunks as the engine plans them: one run of rows per sequence.
    struct Chunk {
        uint32_t seq, pos, tokens;
    };
    std::vector<Chunk> chunks;
    std::vector<uint8_t> seen(ar.seqs(), 0);
    for (uint32_t r = 0; r < m; r++) {
        const uint32_t seq = meta[8 * r + 1];
        if (seq >= ar.seqs())
            return fail(THB_ERR_INVALID, "row " + std::to_string(r) + ": sequence " + std::to_string(seq) +
                                             " out of range (" + std::to_string(ar.seqs()) + " sequences)");
        if (r > 0 && meta[8 * (r - 1) + 1] == seq) {
            chunks.back().tokens++;
            continue;
        }
        if (seen[seq])
            return fail(THB_ERR_INVALID, "sequence " + std::to_string(seq) +
                                             " heads two runs of rows in one call (one run per sequence)");
        seen[seq] = 1;
        chunks.push_back({seq, meta[8 * r], 1});
    }
    return guarded([&]() -> int {
        pool_flush(pool, s);  // queued page ops first
        std::string err;
        for (const Chunk& c : chunks) {  // the host mirror, chunk by chunk
            err = ar.alloc(c.seq, c.pos, c.tokens);
            if (!err.empty()) break;
        }
        PageOpArgs a = op_args(pool);
        a.meta = rows->dev + 8 * static_cast<size_t>(row_off);
        a.n_ops = 1;
        a.reset_copies = 1;
        a.ops[0] = kPageOpAllocRows;
        a.ops[1] = m;
        launch_ops(a, s);
        run_device_copies(pool, 0, ar.copies().size(), s);
        ar.copies().clear();
        return err.empty() ? THB_OK : fail(THB_ERR_MODEL, err);
    });
}

int thb_pool_status(thb_pool* pool, void* stream) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    return guarded([&]() -> int {
        std::vector<uint32_t> h;
        hipStream_t s = as_stream(stream);
        read_state(pool, s, h);
        if (h[kHdrStatus] == kStOk) return THB_OK;
        const std::string msg = status_message(h.data());
        const uint32_t zero[4] = {0, 0, 0, 0};
        THB_HIP(hipMemcpy(pool->state_dev + kHdrStatus, zero, sizeof(zero), hipMemcpyHostToDevice));
        const uint32_t code = h[kHdrStatus];
        return fail(code == kStBadSeq || code == kStDupSeq || code == kStNoFuse ? THB_ERR_INVALID : THB_ERR_MODEL,
                    msg);
    });
}

int thb_pool_read_state(thb_pool* pool, void* stream, uint32_t* free_list, size_t free_cap, uint32_t* n_free,
                        uint32_t* refs, size_t refs_cap, uint32_t* table, size_t table_n) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    const Arena& ar = pool->arena.a;
    const size_t tn = static_cast<size_t>(ar.seqs()) * ar.max_pages();
    if (table && table_n != tn)
        return fail(THB_ERR_INVALID, "block table must cover every sequence: " + std::to_string(table_n) + " != " +
                                         std::to_string(tn));
    if (refs && refs_cap < ar.pages())
        return fail(THB_ERR_INVALID, "refs holds " + std::to_string(refs_cap) + " < " + std::to_string(ar.pages()) +
                                         " pages");
    return guarded([&]() -> int {
        std::vector<uint32_t> h;
        hipStream_t s = as_stream(stream);
        read_state(pool, s, h);
        const uint32_t top = h[kHdrTop];
        if (n_free) *n_free = top;
        if (free_list) {
            if (free_cap < top)
                return fail(THB_ERR_INVALID, "free list holds " + std::to_string(free_cap) + " < " +
                                                 std::to_string(top) + " pages");
            std::copy(h.begin() + pool->state.free_off, h.begin() + pool->state.free_off + top, free_list);
        }
        if (refs) std::copy(h.begin() + pool->state.refs_off, h.begin() + pool->state.refs_off + ar.pages(), refs);
        if (table) THB_HIP(hipMemcpy(table, pool->table_dev, tn * 4, hipMemcpyDeviceToHost));
        return THB_OK;
    });
}

int thb_pool_pull(thb_pool* pool, void* stream) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    return guarded([&]() -> int {
        std::vector<uint32_t> h;
        hipStream_t s = as_stream(stream);
        read_state(pool, s, h);
        Arena& ar = pool->arena.a;
        std::vector<uint32_t> table(static_cast<size_t>(ar.seqs()) * ar.max_pages());
        THB_HIP(hipMemcpy(table.data(), pool->table_dev, table.size() * 4, hipMemcpyDeviceToHost));
        ar.load_state(h.data() + pool->state.free_off, h[kHdrTop], h.data() + pool->state.refs_off,
                      h.data() + pool->state.npages_off, table.data());
        return THB_OK;
    });
}

}  // extern "C"
