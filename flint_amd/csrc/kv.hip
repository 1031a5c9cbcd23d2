// KV append/scatter (kv_store), gather, scatter and page copy kernels.
//
// One lane owns 8 consecutive head_dim elements of one token of one head.
// K pages are chunk-major ([head_dim / 8][page_len][8] per page), so a lane's
// 8 K elements are one 16-byte vector.  V pages are transposed ([head_dim]
// [page_len] per page, the operand layout of the attention kernel's PV
// product), so the lane's 8 V elements are 8 16-bit accesses page_len
// elements apart.  In both, element (slot s, dim d) of page p starts from
// the offset (p * head_dim + d) * page_len.
#include <string>

#include "codec.hpp"
#include "pool.hpp"

namespace thb {
namespace {

constexpr uint32_t kMaxGridY = 65535;

struct StoreArgs {
    const void* k_src;
    const void* v_src;
    uint16_t* k;
    uint16_t* v;
    const uint32_t* meta;   // row meta at the first row of the call
    const uint32_t* table;  // [seqs * max_pages]
    uint64_t plane;         // elements per head plane
    uint32_t max_pages, page_shift, head_dim, chunks;  // chunks = kv_heads * head_dim / 8
};

// kv_store.wgsl:24-46 with one lane per 8 elements.  Grid: (ceil(2 *
// chunks / 256), m); lanes [0, chunks) write K, [chunks, 2 * chunks) V.
template <uint32_t SRC, uint32_t KV>
__global__ __launch_bounds__(256) void kv_store_kernel(StoreArgs a) {
    uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= 2 * a.chunks) return;
    const uint32_t row = blockIdx.y;
    const bool is_v = c >= a.chunks;
    if (is_v) c -= a.chunks;
    const uint32_t pos = a.meta[8 * row], seq = a.meta[8 * row + 1];
    const uint32_t page = a.table[static_cast<uint64_t>(seq) * a.max_pages + (pos >> a.page_shift)];
    const uint64_t slot = (static_cast<uint64_t>(page) << a.page_shift) | (pos & ((1u << a.page_shift) - 1u));
    const uint32_t cph = a.head_dim >> 3;
    const uint32_t h = c / cph, d = (c - h * cph) << 3;
    const uint64_t src_e = (static_cast<uint64_t>(row) * a.chunks + c) << 3;
    const uint4 w = load_encode8<SRC, KV>(is_v ? a.v_src : a.k_src, src_e);
    if (!is_v) {
        *reinterpret_cast<uint4*>(a.k + h * a.plane + ((static_cast<uint64_t>(page) * a.head_dim + d) << a.page_shift) +
                                  ((pos & ((1u << a.page_shift) - 1u)) << 3)) = w;
        return;
    }
    // V^T: element (slot, d + e) of the page lives at (page * hd + d + e) *
    // page_len + slot % page_len.
    uint16_t* dst = a.v + h * a.plane + ((static_cast<uint64_t>(page) * a.head_dim + d) << a.page_shift) +
                    (pos & ((1u << a.page_shift) - 1u));
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t x = e == 0 ? w.x : e == 1 ? w.y : e == 2 ? w.z : w.w;
        dst[static_cast<uint64_t>(2 * e) << a.page_shift] = static_cast<uint16_t>(x & 0xffffu);
        dst[static_cast<uint64_t>(2 * e + 1) << a.page_shift] = static_cast<uint16_t>(x >> 16);
    }
}

struct RunArgs {
    const void* k_src;  // [m, kv_heads, head_dim] from the call's first row
    const void* v_src;
    uint16_t* k;
    uint16_t* v;
    const uint32_t* runs;   // [n_runs][4]: first row (call-relative), length, seq, first position
    const uint32_t* table;  // [seqs * max_pages]
    uint64_t plane;
    uint32_t max_pages, page_shift, head_dim, kv_heads;
};

constexpr uint32_t kMaxRun = 64;  // tokens of one run (LDS: kMaxRun * head_dim * 2 bytes)

// Append of runs: consecutive rows of one sequence whose positions are
// consecutive and inside one page (a prefill chunk).  One workgroup per
// (run, KV head).  K: the run's tokens of each chunk row are contiguous
// 16-byte units.  V: the encoded rows are staged in LDS as [token][dim] and
// written as the page's [dim][token] rows, 8 tokens (16 bytes) per store
// where a whole aligned group of 8 lies inside the run, 2 bytes at its ends.
template <uint32_t SRC, uint32_t KV>
__global__ __launch_bounds__(256) void kv_store_runs_kernel(RunArgs a) {
    __shared__ uint4 s_v[kMaxRun * 512 / 8];
    const uint32_t run = blockIdx.x / a.kv_heads, h = blockIdx.x - run * a.kv_heads;
    const uint32_t* R = a.runs + 4 * run;
    const uint32_t row0 = R[0], len = R[1], seq = R[2], pos0 = R[3];
    const uint32_t shift = a.page_shift, hd = a.head_dim, cph = hd >> 3;
    const uint32_t page = a.table[static_cast<uint64_t>(seq) * a.max_pages + (pos0 >> shift)];
    const uint32_t j0 = pos0 & ((1u << shift) - 1u);
    const uint64_t pbase = static_cast<uint64_t>(h) * a.plane + ((static_cast<uint64_t>(page) * hd) << shift);
    for (uint32_t u = threadIdx.x; u < len * cph; u += 256) {
        const uint32_t ch = u / len, t = u - ch * len;
        const uint64_t e = ((static_cast<uint64_t>(row0 + t)) * a.kv_heads + h) * hd + 8u * ch;
        *reinterpret_cast<uint4*>(a.k + pbase + (static_cast<uint64_t>(8u * ch) << shift) + ((j0 + t) << 3)) =
            load_encode8<SRC, KV>(a.k_src, e);
        s_v[t * cph + ch] = load_encode8<SRC, KV>(a.v_src, e);
    }
    __syncthreads();
    const uint16_t* sv = reinterpret_cast<const uint16_t*>(s_v);
    const uint32_t g0 = j0 >> 3, ng = ((j0 + len - 1) >> 3) - g0 + 1;
    for (uint32_t u = threadIdx.x; u < hd * ng; u += 256) {
        const uint32_t d = u / ng, jg = (g0 + (u - d * ng)) << 3;
        uint16_t* dst = a.v + pbase + (static_cast<uint64_t>(d) << shift) + jg;
        if (jg >= j0 && jg + 8 <= j0 + len) {
            uint32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                w[q] = static_cast<uint32_t>(sv[(jg - j0 + 2 * q) * hd + d]) |
                       (static_cast<uint32_t>(sv[(jg - j0 + 2 * q + 1) * hd + d]) << 16);
            *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (uint32_t e = 0; e < 8; e++) {
                const uint32_t j = jg + e;
                if (j >= j0 && j < j0 + len) dst[e] = sv[(j - j0) * hd + d];
            }
        }
    }
}

struct GatherArgs {
    uint16_t* k;
    uint16_t* v;
    uint16_t* k_flat;  // [kv_heads, n, head_dim]
    uint16_t* v_flat;
    const uint32_t* table_row;  // the sequence's block-table row
    uint64_t plane;
    uint32_t page_shift, head_dim, n, t0, cpt;  // cpt = chunks per token = kv_heads * head_dim / 8
};

// Gather (TO_FLAT) or scatter (!TO_FLAT) of tokens [t0, t0 + n) of one
// sequence.  Grid: (ceil(n * cpt / 256), 2); y selects K or V.
template <bool TO_FLAT>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
    const uint64_t c = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= static_cast<uint64_t>(a.n) * a.cpt) return;
    const uint32_t t = static_cast<uint32_t>(c / a.cpt);
    const uint32_t r = static_cast<uint32_t>(c - static_cast<uint64_t>(t) * a.cpt);
    const uint32_t cph = a.head_dim >> 3;
    const uint32_t h = r / cph, d = (r - h * cph) << 3;
    const uint32_t pos = a.t0 + t;
    const uint32_t page = a.table_row[pos >> a.page_shift];
    const uint32_t j = pos & ((1u << a.page_shift) - 1u);
    if (blockIdx.y == 0) {
        uint16_t* paged = a.k + h * a.plane + ((static_cast<uint64_t>(page) * a.head_dim + d) << a.page_shift) + (j << 3);
        uint16_t* flat = a.k_flat + (static_cast<uint64_t>(h) * a.n + t) * a.head_dim + d;
        if constexpr (TO_FLAT)
            *reinterpret_cast<uint4*>(flat) = *reinterpret_cast<const uint4*>(paged);
        else
            *reinterpret_cast<uint4*>(paged) = *reinterpret_cast<const uint4*>(flat);
        return;
    }
    uint16_t* paged = a.v + h * a.plane + ((static_cast<uint64_t>(page) * a.head_dim + d) << a.page_shift) + j;
    uint16_t* flat = a.v_flat + (static_cast<uint64_t>(h) * a.n + t) * a.head_dim + d;
    if constexpr (TO_FLAT) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            w[e] = static_cast<uint32_t>(paged[static_cast<uint64_t>(2 * e) << a.page_shift]) |
                   (static_cast<uint32_t>(paged[static_cast<uint64_t>(2 * e + 1) << a.page_shift]) << 16);
        *reinterpret_cast<uint4*>(flat) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        const uint4 v = *reinterpret_cast<const uint4*>(flat);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t x = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
            paged[static_cast<uint64_t>(2 * e) << a.page_shift] = static_cast<uint16_t>(x & 0xffffu);
            paged[static_cast<uint64_t>(2 * e + 1) << a.page_shift] = static_cast<uint16_t>(x >> 16);
        }
    }
}

struct CopyArgs {
    uint8_t* mem;
    const DevLayer* layers;
    const uint32_t* triples;  // (src_page, dst_page, tokens)
    uint64_t pool_len;
    uint32_t kv_heads, page_len;
};

// Copy of slots [0, ntok) of a page for every layer, K and V, every head.
// Grid: (ceil(page_len * max_head_dim / 256), n_triples, layers * 2 *
// kv_heads).  A whole page moves as contiguous 16-byte vectors; a partial K
// page as 16-byte chunks of its chunk rows; a partial V page element by
// element ([head_dim][page_len]).
__global__ __launch_bounds__(256) void block_copy_kernel(CopyArgs a) {
    const uint32_t z = blockIdx.z;
    const uint32_t h = z % a.kv_heads;
    const uint32_t which = (z / a.kv_heads) & 1u;
    const uint32_t layer = z / (2 * a.kv_heads);
    const DevLayer L = a.layers[layer];
    const uint32_t src = a.triples[3 * blockIdx.y], dst = a.triples[3 * blockIdx.y + 1];
    const uint32_t ntok = a.triples[3 * blockIdx.y + 2];
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    uint16_t* base = reinterpret_cast<uint16_t*>(a.mem + (which ? L.v_off : L.k_off)) +
                     static_cast<uint64_t>(h) * a.pool_len * L.head_dim;
    const uint64_t page_elems = static_cast<uint64_t>(a.page_len) * L.head_dim;
    const uint16_t* sp = base + static_cast<uint64_t>(src) * page_elems;
    uint16_t* dp = base + static_cast<uint64_t>(dst) * page_elems;
    if (ntok == a.page_len) {  // whole page, K or V: contiguous
        if (static_cast<uint64_t>(c) * 8 >= page_elems) return;
        const uint64_t off = static_cast<uint64_t>(c) * 8;
        *reinterpret_cast<uint4*>(dp + off) = *reinterpret_cast<const uint4*>(sp + off);
        return;
    }
    if (which == 0) {  // K: the first ntok 16-byte chunks of every chunk row
        const uint32_t rows = L.head_dim >> 3;
        if (c >= rows * ntok) return;
        const uint32_t r = c / ntok, j = c - r * ntok;
        const uint64_t off = (static_cast<uint64_t>(r) * a.page_len + j) * 8;
        *reinterpret_cast<uint4*>(dp + off) = *reinterpret_cast<const uint4*>(sp + off);
        return;
    }
    if (c >= ntok * L.head_dim) return;
    const uint32_t d = c / ntok, j = c - d * ntok;
    const uint64_t off = static_cast<uint64_t>(d) * a.page_len + j;
    dp[off] = sp[off];
}

template <uint32_t SRC>
void launch_store(uint32_t kv, dim3 grid, const StoreArgs& a, hipStream_t s) {
    if (kv == THB_KV_F16_RNE)
        hipLaunchKernelGGL((kv_store_kernel<SRC, THB_KV_F16_RNE>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((kv_store_kernel<SRC, THB_KV_BF16_TRUNC>), grid, dim3(256), 0, s, a);
}

template <uint32_t SRC>
void launch_runs(uint32_t kv, dim3 grid, const RunArgs& a, hipStream_t s) {
    if (kv == THB_KV_F16_RNE)
        hipLaunchKernelGGL((kv_store_runs_kernel<SRC, THB_KV_F16_RNE>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((kv_store_runs_kernel<SRC, THB_KV_BF16_TRUNC>), grid, dim3(256), 0, s, a);
}

// Cuts rows [0, m) of the call into runs (consecutive rows of one sequence,
// consecutive positions, one page, at most kMaxRun tokens).  Returns the
// number of rows in runs of 8 or more tokens.
uint32_t make_runs(const uint32_t* meta, uint32_t m, uint32_t page_shift, std::vector<uint32_t>& runs) {
    uint32_t long_rows = 0;
    uint32_t r = 0;
    while (r < m) {
        const uint32_t seq = meta[8 * r + 1], pos0 = meta[8 * r];
        uint32_t len = 1;
        while (r + len < m && len < kMaxRun && meta[8 * (r + len) + 1] == seq &&
               meta[8 * (r + len)] == pos0 + len && ((pos0 + len) >> page_shift) == (pos0 >> page_shift))
            len++;
        runs.insert(runs.end(), {r, len, seq, pos0});
        if (len >= 8) long_rows += len;
        r += len;
    }
    return long_rows;
}

int check_layer(const thb_pool* p, uint32_t layer) {
    if (layer >= p->layers)
        return fail(THB_ERR_INVALID, "layer " + std::to_string(layer) + " out of range (" +
                                         std::to_string(p->layers) + " layers)");
    return THB_OK;
}

// Host-side check that tokens [t0, t0 + n) of seq have pages.
int check_cover(const thb_pool* p, uint32_t seq, uint64_t end) {
    const Arena& a = p->arena.a;
    if (seq >= a.seqs())
        return fail(THB_ERR_INVALID, "sequence " + std::to_string(seq) + " out of range (" +
                                         std::to_string(a.seqs()) + " sequences)");
    if (!a.covers(seq, static_cast<uint32_t>(std::min<uint64_t>(end, 0xFFFFFFFFu))) || end > 0xFFFFFFFFull)
        return fail(THB_ERR_MODEL, "pages must cover the chunk: sequence " + std::to_string(seq) + " holds " +
                                       std::to_string(a.table_of(seq).size() * a.page_len()) + " slots, needs " +
                                       std::to_string(end));
    return THB_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void launch_block_copy(thb_pool* p, const uint32_t* triples_dev, uint32_t n, uint32_t max_tokens,
                       hipStream_t stream) {
    if (n == 0 || max_tokens == 0) return;
    uint32_t max_hd = 0;
    for (const auto& g : p->geom) max_hd = std::max(max_hd, g.head_dim);
    CopyArgs a{p->mem, static_cast<const DevLayer*>(p->geom_buf.get()), triples_dev,
               static_cast<uint64_t>(p->arena.a.pages()) * p->page_len, p->kv_heads, p->page_len};
    const uint32_t chunks = (max_tokens * max_hd + 255) / 256;
    const uint32_t planes = p->layers * 2 * p->kv_heads;
    if (planes > kMaxGridY) throw HipError{hipErrorInvalidConfiguration, "block copy: layers*2*kv_heads > 65535"};
    for (uint32_t i0 = 0; i0 < n; i0 += kMaxGridY) {
        CopyArgs b = a;
        b.triples = triples_dev + 3 * static_cast<size_t>(i0);
        hipLaunchKernelGGL(block_copy_kernel, dim3(chunks, std::min(kMaxGridY, n - i0), planes), dim3(256), 0, stream,
                           b);
        THB_HIP(hipGetLastError());
    }
}

}  // namespace thb

using namespace thb;

extern "C" {

int thb_kv_store(thb_pool* pool, uint32_t layer, const void* k_src, const void* v_src, uint32_t src_dtype,
                 const thb_rows* rows, uint32_t row_off, uint32_t m, void* stream) {
    if (!pool || !rows) return fail(THB_ERR_INVALID, "null pool or rows");
    if (int rc = check_layer(pool, layer)) return rc;
    if (m == 0) return THB_OK;
    if (!k_src || !v_src) return fail(THB_ERR_INVALID, "null source buffer");
    if (src_dtype > THB_DT_BF16) return fail(THB_ERR_INVALID, "unknown src_dtype " + std::to_string(src_dtype));
    if (!aligned16(k_src) || !aligned16(v_src)) return fail(THB_ERR_INVALID, "source buffers must be 16-byte aligned");
    if (static_cast<uint64_t>(row_off) + m > rows->m)
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->m) + " rows, call needs " +
                                         std::to_string(static_cast<uint64_t>(row_off) + m));
    for (uint32_t r = row_off; r < row_off + m; r++) {
        uint32_t pos = rows->host[8 * r], seq = rows->host[8 * r + 1];
        if (int rc = check_cover(pool, seq, static_cast<uint64_t>(pos) + 1)) return rc;
    }
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        const LayerGeom& g = pool->geom[layer];
        StoreArgs a;
        a.k_src = k_src;
        a.v_src = v_src;
        a.k = reinterpret_cast<uint16_t*>(pool->mem + g.k_off);
        a.v = reinterpret_cast<uint16_t*>(pool->mem + g.v_off);
        a.meta = rows->dev + 8 * static_cast<size_t>(row_off);
        a.table = pool->table_dev;
        a.plane = static_cast<uint64_t>(pool->arena.a.pages()) * pool->page_len * g.head_dim;
        a.max_pages = pool->arena.a.max_pages();
        a.page_shift = pool->page_shift;
        a.head_dim = g.head_dim;
        a.chunks = pool->kv_heads * g.head_dim / 8;
        const size_t esize = src_dtype == THB_DT_F32 ? 4 : 2;
        // Mostly long runs (prefill chunks): the run kernel writes whole V
        // page rows; otherwise (decode) one lane per 8 elements of a row.
        std::vector<uint32_t> runs;
        const uint32_t long_rows = make_runs(rows->host.data() + 8 * static_cast<size_t>(row_off), m,
                                             pool->page_shift, runs);
        if (2 * static_cast<uint64_t>(long_rows) >= m) {
            const uint32_t n_runs = static_cast<uint32_t>(runs.size() / 4);
            void* dev = pool->run_buf.reserve(runs.size() * 4, false);
            pool->stager.upload(dev, runs.data(), runs.size() * 4, s);
            RunArgs ra;
            ra.k_src = k_src;
            ra.v_src = v_src;
            ra.k = a.k;
            ra.v = a.v;
            ra.runs = static_cast<const uint32_t*>(dev);
            ra.table = a.table;
            ra.plane = a.plane;
            ra.max_pages = a.max_pages;
            ra.page_shift = a.page_shift;
            ra.head_dim = a.head_dim;
            ra.kv_heads = pool->kv_heads;
            const uint64_t n_wg = static_cast<uint64_t>(n_runs) * pool->kv_heads;
            if (n_wg > 0x7FFFFFFFull) throw HipError{hipErrorInvalidConfiguration, "append grid too large"};
            const dim3 grid(static_cast<uint32_t>(n_wg));
            switch (src_dtype) {
                case THB_DT_F32: launch_runs<THB_DT_F32>(pool->kv_dtype, grid, ra, s); break;
                case THB_DT_F16: launch_runs<THB_DT_F16>(pool->kv_dtype, grid, ra, s); break;
                default: launch_runs<THB_DT_BF16>(pool->kv_dtype, grid, ra, s); break;
            }
            THB_HIP(hipGetLastError());
            return THB_OK;
        }
        for (uint32_t r0 = 0; r0 < m; r0 += kMaxGridY) {  // grid.y limit
            const uint32_t n = std::min(kMaxGridY, m - r0);
            StoreArgs b = a;
            b.meta = a.meta + 8 * static_cast<size_t>(r0);
            b.k_src = static_cast<const uint8_t*>(k_src) + static_cast<size_t>(r0) * a.chunks * 8 * esize;
            b.v_src = static_cast<const uint8_t*>(v_src) + static_cast<size_t>(r0) * a.chunks * 8 * esize;
            dim3 grid((2 * a.chunks + 255) / 256, n);
            switch (src_dtype) {
                case THB_DT_F32: launch_store<THB_DT_F32>(pool->kv_dtype, grid, b, s); break;
                case THB_DT_F16: launch_store<THB_DT_F16>(pool->kv_dtype, grid, b, s); break;
                default: launch_store<THB_DT_BF16>(pool->kv_dtype, grid, b, s); break;
            }
            THB_HIP(hipGetLastError());
        }
        return THB_OK;
    });
}

static int gather_common(thb_pool* pool, uint32_t layer, uint32_t seq, uint32_t t0, uint32_t n, void* k, void* v,
                         void* stream, bool to_flat) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (int rc = check_layer(pool, layer)) return rc;
    if (n == 0) return THB_OK;
    if (!k || !v) return fail(THB_ERR_INVALID, "null buffer");
    if (!aligned16(k) || !aligned16(v)) return fail(THB_ERR_INVALID, "buffers must be 16-byte aligned");
    if (int rc = check_cover(pool, seq, static_cast<uint64_t>(t0) + n)) return rc;
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        const LayerGeom& g = pool->geom[layer];
        GatherArgs a;
        a.k = reinterpret_cast<uint16_t*>(pool->mem + g.k_off);
        a.v = reinterpret_cast<uint16_t*>(pool->mem + g.v_off);
        a.k_flat = static_cast<uint16_t*>(k);
        a.v_flat = static_cast<uint16_t*>(v);
        a.table_row = pool->table_dev + static_cast<size_t>(seq) * pool->arena.a.max_pages();
        a.plane = static_cast<uint64_t>(pool->arena.a.pages()) * pool->page_len * g.head_dim;
        a.page_shift = pool->page_shift;
        a.head_dim = g.head_dim;
        a.n = n;
        a.t0 = t0;
        a.cpt = pool->kv_heads * g.head_dim / 8;
        const uint64_t total = static_cast<uint64_t>(n) * a.cpt;
        dim3 grid(static_cast<uint32_t>((total + 255) / 256), 2);
        if (to_flat)
            hipLaunchKernelGGL(gather_kernel<true>, grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(gather_kernel<false>, grid, dim3(256), 0, s, a);
        THB_HIP(hipGetLastError());
        return THB_OK;
    });
}

int thb_kv_gather(thb_pool* pool, uint32_t layer, uint32_t seq, uint32_t t0, uint32_t n, void* k_dst, void* v_dst,
                  void* stream) {
    return gather_common(pool, layer, seq, t0, n, k_dst, v_dst, stream, true);
}

int thb_kv_scatter(thb_pool* pool, uint32_t layer, uint32_t seq, uint32_t t0, uint32_t n, const void* k_src,
                   const void* v_src, void* stream) {
    return gather_common(pool, layer, seq, t0, n, const_cast<void*>(k_src), const_cast<void*>(v_src), stream, false);
}

int thb_block_copy(thb_pool* pool, const uint32_t* triples, uint32_t n, void* stream) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (n == 0) return THB_OK;
    if (!triples) return fail(THB_ERR_INVALID, "triples is null");
    const uint32_t pages = pool->arena.a.pages();
    uint32_t max_tok = 0;
    std::vector<uint32_t> seen;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t s = triples[3 * i], d = triples[3 * i + 1], t = triples[3 * i + 2];
        if (s >= pages || d >= pages)
            return fail(THB_ERR_INVALID, "page copy " + std::to_string(s) + " -> " + std::to_string(d) +
                                             " outside the pool of " + std::to_string(pages) + " pages");
        if (t > pool->page_len)
            return fail(THB_ERR_INVALID, "page copy of " + std::to_string(t) + " tokens exceeds page_len " +
                                             std::to_string(pool->page_len));
        max_tok = std::max(max_tok, t);
        seen.push_back(s);
        seen.push_back(d);
    }
    std::vector<uint32_t> sorted = seen;
    std::sort(sorted.begin(), sorted.end());
    for (size_t i = 1; i < sorted.size(); i++)
        if (sorted[i] == sorted[i - 1])
            return fail(THB_ERR_INVALID, "page " + std::to_string(sorted[i]) + " appears twice in one block copy");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        void* dev = pool->copy_buf.reserve(static_cast<size_t>(n) * 12, false);
        pool->stager.upload(dev, triples, static_cast<size_t>(n) * 12, s);
        launch_block_copy(pool, static_cast<const uint32_t*>(dev), n, max_tok, s);
        return THB_OK;
    });
}

}  // extern "C"
