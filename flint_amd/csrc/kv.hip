// KV append/scatter (kv_store), gather, scatter and page copy kernels.
//
// One lane owns 8 consecutive head_dim elements of one token of one head.
// Pages follow layout.hpp: K in 32-dimension groups ([hd/32][P][32]), so a
// lane's 8 K elements are one 16-byte vector; V in 4-slot groups
// ([P/4][hd][4], the operand layout of the attention kernel's PV product),
// so the lane's 8 V elements are 8 16-bit accesses 8 bytes apart.
#include <algorithm>
#include <array>
#include <string>

#include "codec.hpp"
#include "layout.hpp"
#include "pool.hpp"
#include "rope.hpp"

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
    uint32_t pages, seqs;   // a row outside them, or on a page not held, stores nothing
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
    // The host checks every row's pages before an eager call; a captured
    // call replays with the row meta of its own time, so the device checks.
    if (seq >= a.seqs || (pos >> a.page_shift) >= a.max_pages) return;
    const uint32_t page = a.table[static_cast<uint64_t>(seq) * a.max_pages + (pos >> a.page_shift)];
    if (page >= a.pages) return;
    const uint32_t cph = a.head_dim >> 3;
    const uint32_t h = c / cph, d = (c - h * cph) << 3;
    const uint64_t src_e = (static_cast<uint64_t>(row) * a.chunks + c) << 3;
    const uint4 w = load_encode8<SRC, KV>(is_v ? a.v_src : a.k_src, src_e);
    const uint32_t j = pos & ((1u << a.page_shift) - 1u);
    const uint64_t pbase = h * a.plane + ((static_cast<uint64_t>(page) * a.head_dim) << a.page_shift);
    if (!is_v) {
        *reinterpret_cast<uint4*>(a.k + pbase + k_off(j, d, a.head_dim, a.page_shift)) = w;
        return;
    }
    // V: element (j, d + e) at v_off(j, d, hd) + 4 e.
    uint16_t* dst = a.v + pbase + v_off(j, d, a.head_dim);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t x = e == 0 ? w.x : e == 1 ? w.y : e == 2 ? w.z : w.w;
        dst[8 * e] = static_cast<uint16_t>(x & 0xffffu);
        dst[8 * e + 4] = static_cast<uint16_t>(x >> 16);
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
    uint32_t do_k;  // 0: V only (K is written by the rotary append kernel)
};

// Tokens per run.  A 4096-row prefill call at head_dim 128 (8 KV heads) took
// 11.1 / 9.8 / 8.2 / 9.8 us with runs of 64 / 32 / 16 / 8 tokens: 16 gives
// 2048 workgroups, enough to keep every CU's loads in flight.  Runs after a
// chunk's first start at multiples of kRunTokens positions, so only a
// chunk's first and last runs can cut a 4-slot V group.
constexpr uint32_t kRunTokens = 16;

// Lane l of a quad holds row l of a 4 x 4 matrix of words in a[0..3] and
// ends with column l (a[k] = the old a[l] of quad lane k): two exchanges of
// two words each, with lane l ^ 2 and then with lane l ^ 1 (DPP quad
// permutations; all 4 lanes of the quad must be active).
template <int CTRL>
__device__ inline uint32_t quad_perm(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), CTRL, 0xF, 0xF, false));
}
__device__ inline void quad_transpose(uint32_t (&a)[4], uint32_t l) {
    const bool b1 = (l & 2u) != 0, b0 = (l & 1u) != 0;
    {
        const uint32_t r0 = quad_perm<0x4E>(b1 ? a[0] : a[2]), r1 = quad_perm<0x4E>(b1 ? a[1] : a[3]);
        a[0] = b1 ? r0 : a[0];
        a[1] = b1 ? r1 : a[1];
        a[2] = b1 ? a[2] : r0;
        a[3] = b1 ? a[3] : r1;
    }
    {
        const uint32_t r0 = quad_perm<0xB1>(b0 ? a[0] : a[1]), r1 = quad_perm<0xB1>(b0 ? a[2] : a[3]);
        a[0] = b0 ? r0 : a[0];
        a[2] = b0 ? r1 : a[2];
        a[1] = b0 ? a[1] : r0;
        a[3] = b0 ? a[3] : r1;
    }
}

// The 4 lanes of a quad hold the V page units of dims 8c .. 8c + 7 of one
// 4-slot group (lane l: dims 8c + 2l and 8c + 2l + 1; element i of the unit
// is slot i % 4 of dim 8c + 2l + i / 4).  Returns slot l's 8 dims in order:
// lane l's row of the flat layout.
__device__ inline uint4 v_units_to_row(const uint4& w, uint32_t l) {
    // a[s]: (dim 8c + 2l, dim 8c + 2l + 1) of slot s
    uint32_t a[4] = {(w.x & 0xffffu) | (w.z << 16), (w.x >> 16) | (w.z & 0xffff0000u), (w.y & 0xffffu) | (w.w << 16),
                     (w.y >> 16) | (w.w & 0xffff0000u)};
    quad_transpose(a, l);  // a[k]: (dim 8c + 2k, dim 8c + 2k + 1) of slot l
    return make_uint4(a[0], a[1], a[2], a[3]);
}

// Inverse of v_units_to_row: lane l holds slot l's dims 8c .. 8c + 7 and
// gets the page unit of dims 8c + 2l, 8c + 2l + 1 over the group's 4 slots.
__device__ inline uint4 v_row_to_units(const uint4& r, uint32_t l) {
    uint32_t a[4] = {r.x, r.y, r.z, r.w};
    quad_transpose(a, l);  // a[s]: (dim 8c + 2l, dim 8c + 2l + 1) of slot s
    return make_uint4((a[0] & 0xffffu) | (a[1] << 16), (a[2] & 0xffffu) | (a[3] << 16),
                      (a[0] >> 16) | (a[1] & 0xffff0000u), (a[2] >> 16) | (a[3] & 0xffff0000u));
}

// Append of runs: consecutive rows of one sequence whose positions are
// consecutive (a prefill chunk), up to kRunTokens tokens, across pages.  One
// workgroup per (run, KV head); lane u moves (token u % len, 8-dimension
// chunk u / len).  The run record is the only load ahead of the others:
// every lane issues its source loads and its page's block-table entry
// together.  K: one 16-byte store per (token, chunk).  V:
// * a run of whole 4-slot groups (position and length multiples of 4): the
//   4 lanes of a quad hold one group's 4 tokens and trade their rows into the
//   group's 4 page units in registers, one 16-byte store each;
// * otherwise the encoded rows are staged in LDS as [token][dim] and written
//   as the pages' 4-slot groups, 16 bytes (2 dims x 4 slots) per store where
//   a whole group lies inside the run, 2 bytes at its ends.
template <uint32_t SRC, uint32_t KV>
__global__ __launch_bounds__(256) void kv_store_runs_kernel(RunArgs a) {
    extern __shared__ uint32_t s_run[];  // [len][head_dim + 2] 16-bit V slots
    const uint32_t run = blockIdx.x / a.kv_heads, h = blockIdx.x - run * a.kv_heads;
    const uint32_t* R = a.runs + 4 * run;
    const uint32_t row0 = R[0], len = R[1], seq = R[2], pos0 = R[3];
    const uint32_t shift = a.page_shift, hd = a.head_dim, cph = hd >> 3, mask = (1u << shift) - 1u;
    const uint32_t* trow = a.table + static_cast<uint64_t>(seq) * a.max_pages;
    const uint64_t hbase = static_cast<uint64_t>(h) * a.plane;
    auto page_base = [&](uint32_t page) { return hbase + ((static_cast<uint64_t>(page) * hd) << shift); };
    const bool whole_groups = ((pos0 | len) & 3u) == 0;  // then len * cph is a multiple of 4: whole quads
    const uint32_t rs = (hd + 2) >> 1;  // LDS row stride in 32-bit words
    // Up to two (token, chunk) units per lane at a time (71 VGPRs with four,
    // 7 waves per SIMD): all their loads are issued before the first store.
    const uint32_t units = len * cph;
    for (uint32_t u0 = threadIdx.x; u0 < units; u0 += 2 * 256) {
        uint4 kw[2], vw[2];
        uint32_t pg[2];
#pragma unroll
        for (uint32_t i = 0; i < 2; i++) {
            const uint32_t u = u0 + 256 * i;
            if (u >= units) continue;
            const uint32_t ch = u / len, t = u - ch * len;
            const uint64_t e = ((static_cast<uint64_t>(row0 + t)) * a.kv_heads + h) * hd + 8u * ch;
            if (a.do_k) kw[i] = load_encode8<SRC, KV>(a.k_src, e);
            vw[i] = load_encode8<SRC, KV>(a.v_src, e);
            pg[i] = trow[(pos0 + t) >> shift];
        }
#pragma unroll
        for (uint32_t i = 0; i < 2; i++) {
            const uint32_t u = u0 + 256 * i;
            if (u >= units) continue;
            const uint32_t ch = u / len, t = u - ch * len, pos = pos0 + t;
            const uint64_t pb = page_base(pg[i]);
            if (a.do_k) *reinterpret_cast<uint4*>(a.k + pb + k_off(pos & mask, 8u * ch, hd, shift)) = kw[i];
            if (whole_groups) {
                // a group never spans two pages (page_len is a multiple of 4)
                const uint32_t l = t & 3u;
                *reinterpret_cast<uint4*>(a.v + pb + v_off((pos & mask) & ~3u, 8u * ch + 2u * l, hd)) =
                    v_row_to_units(vw[i], l);
            } else {
                uint32_t* dst = s_run + t * rs + 4u * ch;
                dst[0] = vw[i].x;
                dst[1] = vw[i].y;
                dst[2] = vw[i].z;
                dst[3] = vw[i].w;
            }
        }
    }
    if (whole_groups) return;
    __syncthreads();
    const uint16_t* sv = reinterpret_cast<const uint16_t*>(s_run);
    const uint32_t S = hd + 2;                                               // LDS row stride (16-bit)
    const uint32_t Q0 = pos0 >> 2, nq = ((pos0 + len - 1) >> 2) - Q0 + 1;  // aligned 4-slot groups
    const uint32_t dpairs = hd >> 1;
    // One 16-byte unit per lane: dims (d, d + 1) x the 4 slots of a group;
    // consecutive lanes write consecutive units.
    for (uint32_t u = threadIdx.x; u < dpairs * nq; u += 256) {
        const uint32_t q = u / dpairs, d = 2u * (u - q * dpairs), p4 = (Q0 + q) << 2;
        uint16_t* dst = a.v + page_base(trow[p4 >> shift]) + v_off(p4 & mask, d, hd);
        if (p4 >= pos0 && p4 + 4 <= pos0 + len) {
            const uint32_t t = p4 - pos0;
            uint32_t w[4];
#pragma unroll
            for (int q2 = 0; q2 < 2; q2++)
#pragma unroll
                for (int h2 = 0; h2 < 2; h2++)
                    w[2 * q2 + h2] = static_cast<uint32_t>(sv[(t + 2 * h2) * S + d + q2]) |
                                     (static_cast<uint32_t>(sv[(t + 2 * h2 + 1) * S + d + q2]) << 16);
            *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (uint32_t e = 0; e < 4; e++) {
                const uint32_t p = p4 + e;
                if (p < pos0 || p >= pos0 + len) continue;
                dst[e] = sv[(p - pos0) * S + d];
                dst[4 + e] = sv[(p - pos0) * S + d + 1];
            }
        }
    }
}

struct RopeStoreArgs {
    const void* k_src;  // [m, kv_heads, head_dim], f32 or f16
    const void* v_src;
    uint16_t* k;
    uint16_t* v;
    const uint32_t* meta;
    const uint32_t* table;
    uint64_t plane;
    uint32_t max_pages, page_shift, head_dim, kv_heads, m;
    uint32_t seg_shift;  // log2 of the lanes per head (the power of two >= head_dim / 8)
    uint32_t do_v;       // 0: K only (V is written by the run kernel)
    RopeDev rope;
};

// Rotary append: each wavefront holds 64 >> seg_shift (row, KV head) pairs
// in lane segments, lane u of a segment holding dims [8u, 8u + 8).  K is
// normalised (with a weight), rotated at the row's position, rounded to the
// source type and encoded into its page chunk; V is stored as by
// kv_store_kernel.  Grid: ceil(pairs / (4 * heads per wave)) x 256.
template <uint32_t SRC, uint32_t KV>
__global__ __launch_bounds__(256) void kv_store_rope_kernel(RopeStoreArgs a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t seg = lane >> a.seg_shift, u = lane & ((1u << a.seg_shift) - 1u);
    const uint32_t pair = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (64u >> a.seg_shift) + seg;
    const uint32_t cph = a.head_dim >> 3;
    const bool act = pair < a.m * a.kv_heads && u < cph;
    const uint32_t row = act ? pair / a.kv_heads : 0u, h = act ? pair - row * a.kv_heads : 0u;
    const uint32_t pos = act ? a.meta[8 * row] : 0u;
    const uint64_t e = (static_cast<uint64_t>(row) * a.kv_heads + h) * a.head_dim + 8u * u;
    float x[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (act) load8_f32(SRC, a.k_src, e, x);
    rope_head_seg(x, act ? u : cph, cph, seg << a.seg_shift, pos, a.rope);
    if (!act) return;
    const uint32_t seq = a.meta[8 * row + 1];
    const uint32_t page = a.table[static_cast<uint64_t>(seq) * a.max_pages + (pos >> a.page_shift)];
    const uint32_t j = pos & ((1u << a.page_shift) - 1u);
    const uint64_t pbase = h * a.plane + ((static_cast<uint64_t>(page) * a.head_dim) << a.page_shift);
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if constexpr (SRC == THB_DT_F16)
            w[q] = conv16<THB_DT_F16, KV>(f32_to_f16_rne(x[2 * q])) |
                   (conv16<THB_DT_F16, KV>(f32_to_f16_rne(x[2 * q + 1])) << 16);
        else
            w[q] = conv32<KV>(__float_as_uint(x[2 * q])) | (conv32<KV>(__float_as_uint(x[2 * q + 1])) << 16);
    }
    *reinterpret_cast<uint4*>(a.k + pbase + k_off(j, 8u * u, a.head_dim, a.page_shift)) =
        make_uint4(w[0], w[1], w[2], w[3]);
    if (!a.do_v) return;
    const uint4 vw = load_encode8<SRC, KV>(a.v_src, e);
    uint16_t* dst = a.v + pbase + v_off(j, 8u * u, a.head_dim);
    const uint32_t vs[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        dst[8 * q] = static_cast<uint16_t>(vs[q] & 0xffffu);
        dst[8 * q + 4] = static_cast<uint16_t>(vs[q] >> 16);
    }
}

struct RopeRowsArgs {
    void* x;  // [m, heads, head_dim], f32 or f16, in place
    const uint32_t* meta;
    uint32_t m, heads, head_dim, seg_shift;
    RopeDev rope;
};

// ops::rope / ops::norm_rope in place: 64 >> seg_shift (row, head) vectors
// per wavefront, one per lane segment.
template <uint32_t DT>
__global__ __launch_bounds__(256) void rope_rows_kernel(RopeRowsArgs a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t seg = lane >> a.seg_shift, u = lane & ((1u << a.seg_shift) - 1u);
    const uint32_t vec = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (64u >> a.seg_shift) + seg;
    const uint32_t cph = a.head_dim >> 3;
    const bool act = vec < a.m * a.heads && u < cph;
    const uint32_t pos = act ? a.meta[8 * (vec / a.heads)] : 0u;
    const uint64_t e = static_cast<uint64_t>(vec) * a.head_dim + 8u * u;
    float x[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (act) load8_f32(DT, a.x, e, x);
    rope_head_seg(x, act ? u : cph, cph, seg << a.seg_shift, pos, a.rope);
    if (!act) return;
    if constexpr (DT == THB_DT_F16) {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) w[q] = f32_to_f16_rne(x[2 * q]) | (f32_to_f16_rne(x[2 * q + 1]) << 16);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.x) + e) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(a.x) + e);
        p[0] = f32x4{x[0], x[1], x[2], x[3]};
        p[1] = f32x4{x[4], x[5], x[6], x[7]};
    }
}

// log2 of the lanes a head of head_dim elements takes (8 per lane, a power
// of two).
inline uint32_t seg_shift_for(uint32_t head_dim) {
    uint32_t sh = 3;
    while ((1u << sh) < head_dim / 8) sh++;
    return sh;
}

struct GatherArgs {
    uint16_t* k;
    uint16_t* v;
    uint16_t* k_flat;  // [kv_heads, n, head_dim]
    uint16_t* v_flat;
    const uint32_t* table_row;  // the sequence's block-table row
    uint64_t plane;
    uint32_t page_shift, head_dim, n, t0;
    uint32_t pages;  // pages of the pool: a table entry outside them moves nothing
    uint32_t tile;   // tokens per LDS tile of V (min(page_len, 64))
    uint32_t heads;  // KV heads per workgroup
    // Batched calls (null otherwise): work item x = (range, page of the
    // range), and the range records, kRangeWords each: seq table row offset,
    // t0, n, pad, then K plane, V plane and flat element offsets (64 bits
    // each).  k / v / k_flat / v_flat are then the bases those offsets add to.
    const uint32_t* items;
    const uint32_t* ranges;
};

constexpr uint32_t kRangeWords = 10;

// Copies a 16-byte V unit (dims d, d + 1 x the 4 slots of a group; element
// i is slot i % 4 of dim d + i / 4) from `src` to `dst`, keeping the slots
// of `dst` outside [s0, s1) (a group that a range cuts).
__device__ inline void merge_v16(uint16_t* dst, const uint16_t* src, uint32_t s0, uint32_t s1) {
    if (s0 == 0 && s1 >= 4) {
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
        return;
    }
    uint4 o = *reinterpret_cast<const uint4*>(dst);
    const uint4 n = *reinterpret_cast<const uint4*>(src);
    uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
    const uint32_t* nw = reinterpret_cast<const uint32_t*>(&n);
#pragma unroll
    for (uint32_t e = 0; e < 8; e++) {
        if ((e & 3u) < s0 || (e & 3u) >= s1) continue;
        const uint32_t sh = 16u * (e & 1u), mask = 0xffffu << sh;
        ow[e >> 1] = (ow[e >> 1] & ~mask) | (nw[e >> 1] & mask);
    }
    *reinterpret_cast<uint4*>(dst) = o;
}

// Copies 16 bytes of K (8 dims of one slot) from `src` to `dst` when keep.
__device__ inline void copy16_if(uint16_t* dst, const uint16_t* src, bool keep) {
    if (keep) *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
}

// 16-byte store with the non-temporal hint (the destination is not read
// again by this kernel or soon after).
__device__ inline void st_stream16(void* p, const uint4& v) {
    __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, static_cast<u32x4*>(p));
}

// u / d without a division instruction: exact for u, d < 2^16 (the error
// term u * (m * d - 2^32) stays below 2^32).
struct DivSmall {
    uint64_t m;
    __device__ explicit DivSmall(uint32_t d) : m(0xFFFFFFFFull / d + 1u) {}
    __device__ uint32_t operator()(uint32_t u) const { return static_cast<uint32_t>((u * m) >> 32); }
};

// Gather (TO_FLAT) or scatter (!TO_FLAT) of tokens [t0, t0 + n) of one
// sequence.  One workgroup per (page of the range, group of `heads` KV
// heads).  K: a token's 8-dimension chunk is 16 contiguous bytes on both
// sides.  V, page side: 16-byte units (2 dims x the 4 slots of a group);
// flat side: 16-byte (slot, 8 dims) vectors.
// * A page the range covers whole: every lane moves one K vector (flat
//   order) and one V unit (page order) per round, two rounds in flight; the
//   4 lanes of a quad hold the 4 units of one group's 8 dims and trade them
//   into 4 flat rows in registers (no LDS, no barrier).
// * A page the range cuts: a tile of up to 64 slots of V goes through LDS as
//   [slot][dim] (rows of head_dim + 8 elements, 16-byte aligned), and a group
//   that the range cuts is merged into its 16 bytes by one lane.
template <bool TO_FLAT>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs args) {
    extern __shared__ uint4 s_tile[];
    GatherArgs a = args;
    uint32_t page = blockIdx.x;  // page of the range
    if (args.items) {  // batched: this workgroup's range
        const uint32_t r = args.items[2 * blockIdx.x];
        page = args.items[2 * blockIdx.x + 1];
        const uint32_t* R = args.ranges + static_cast<uint64_t>(r) * kRangeWords;
        auto off64 = [&](int w) { return static_cast<uint64_t>(R[w]) | (static_cast<uint64_t>(R[w + 1]) << 32); };
        a.table_row = args.table_row + R[0];
        a.t0 = R[1];
        a.n = R[2];
        a.k = args.k + off64(4);
        a.v = args.v + off64(6);
        a.k_flat = args.k_flat + off64(8);
        a.v_flat = args.v_flat + off64(8);
    }
    const uint32_t shift = a.page_shift, hd = a.head_dim, cph = hd >> 3, T = a.tile;
    const uint32_t RS = hd + 8;                // LDS row stride (16-bit elements)
    const uint32_t tile_elems = T * RS;
    uint16_t* tile16 = reinterpret_cast<uint16_t*>(s_tile);
    const uint32_t pi = (a.t0 >> shift) + page, h0 = blockIdx.y * a.heads;
    const uint32_t p0 = pi << shift;
    const uint32_t ja = max(a.t0, p0) - p0;
    const uint32_t jb = static_cast<uint32_t>(
        min(static_cast<uint64_t>(a.t0) + a.n, static_cast<uint64_t>(p0) + (1u << shift)) - p0);
    const uint32_t phys = a.table_row[pi];
    if (phys >= a.pages) return;  // whole workgroup: a page not held (a replay after the pages changed)
    const uint64_t pbase0 = (static_cast<uint64_t>(phys) * hd) << shift;
    auto pbase = [&](uint32_t hh) { return static_cast<uint64_t>(h0 + hh) * a.plane + pbase0; };
    // flat row of page slot j of head h: h * n + p0 + j - t0 (j >= ja keeps it >= h * n)
    auto flat_off = [&](uint32_t hh, uint32_t j, uint32_t c) {
        return (static_cast<uint64_t>(h0 + hh) * a.n + p0 - a.t0 + j) * hd + 8u * c;
    };
    auto k_paged = [&](uint32_t hh, uint32_t j, uint32_t c) { return a.k + pbase(hh) + k_off(j, 8u * c, hd, shift); };
    auto v_paged = [&](uint32_t hh, uint32_t j4, uint32_t d) { return a.v + pbase(hh) + v_off(j4, d, hd); };
    const DivSmall by_cph(cph), by_dp(hd >> 1);
    if (ja == 0 && jb == (1u << shift)) {
        // vectors per head plane: hd * page_len / 8, a multiple of 8, so the
        // bound below keeps whole quads active
        const uint32_t vecs = (hd << shift) >> 3, NV = a.heads * vecs, l = threadIdx.x & 3u;
        const DivSmall by_vecs(vecs);
        for (uint32_t u0 = threadIdx.x; u0 < NV; u0 += 512) {
            uint4 kr[2], vr[2];
#pragma unroll
            for (uint32_t i = 0; i < 2; i++) {
                const uint32_t u = u0 + 256 * i;
                if (u >= NV) continue;
                const uint32_t hh = by_vecs(u), r = u - hh * vecs;
                const uint32_t t = by_cph(r), c = r - t * cph;  // K: token t, chunk c
                const uint32_t q = by_dp(r), c8 = (r - q * (hd >> 1)) >> 2;  // V unit r: group q, dims 8 c8 + 2 l
                if constexpr (TO_FLAT) {
                    kr[i] = ld_stream16(k_paged(hh, t, c));
                    vr[i] = ld_stream16(a.v + pbase(hh) + 8u * r);
                } else {
                    kr[i] = ld_stream16(a.k_flat + flat_off(hh, t, c));
                    vr[i] = ld_stream16(a.v_flat + flat_off(hh, 4u * q + l, c8));
                }
            }
#pragma unroll
            for (uint32_t i = 0; i < 2; i++) {
                const uint32_t u = u0 + 256 * i;
                if (u >= NV) continue;
                const uint32_t hh = by_vecs(u), r = u - hh * vecs;
                const uint32_t t = by_cph(r), c = r - t * cph;
                const uint32_t q = by_dp(r), c8 = (r - q * (hd >> 1)) >> 2;
                if constexpr (TO_FLAT) {
                    st_stream16(a.k_flat + flat_off(hh, t, c), kr[i]);
                    st_stream16(a.v_flat + flat_off(hh, 4u * q + l, c8), v_units_to_row(vr[i], l));
                } else {
                    st_stream16(k_paged(hh, t, c), kr[i]);
                    st_stream16(a.v + pbase(hh) + 8u * r, v_row_to_units(vr[i], l));
                }
            }
        }
        return;
    }
    for (uint32_t tb = ja & ~(T - 1u); tb < jb; tb += T) {
        const uint32_t lo = max(ja, tb), hi = min(jb, tb + T);
        const uint32_t q_lo = (lo - tb) >> 2, q_hi = (hi - tb + 3u) >> 2;  // 4-slot groups the range touches
        const uint32_t nq = q_hi - q_lo;
        const uint32_t n_tok = (hi - lo) * cph;  // K (and flat V) vectors of the tile, per head
        const uint32_t n_grp = (hd >> 1) * nq;   // V page units of the tile, per head
        const DivSmall by_tok(n_tok), by_grp(n_grp);
        // vector u of the K (flat) side: head hh, token lo + t, chunk c
        auto split_tok = [&](uint32_t u, uint32_t& hh, uint32_t& t, uint32_t& c) {
            hh = by_tok(u);
            const uint32_t r = u - hh * n_tok;
            t = by_cph(r);
            c = r - t * cph;
        };
        // unit u of the V page side: head hh, group q (slots tb + 4q ..), dims d, d + 1
        auto split_grp = [&](uint32_t u, uint32_t& hh, uint32_t& q, uint32_t& d) {
            hh = by_grp(u);
            const uint32_t r = u - hh * n_grp;
            const uint32_t qq = by_dp(r);
            q = q_lo + qq;
            d = 2u * (r - qq * (hd >> 1));
        };
        const uint32_t NT = a.heads * n_tok, NG = a.heads * n_grp;
        if constexpr (TO_FLAT) {
            for (uint32_t u0 = threadIdx.x; u0 < max(NT, NG); u0 += 512) {
                uint4 kr[2], vr[2];
#pragma unroll
                for (uint32_t i = 0; i < 2; i++) {
                    const uint32_t u = u0 + 256 * i;
                    uint32_t hh, t, c, q, d;
                    split_tok(u, hh, t, c);
                    if (u < NT) kr[i] = ld_stream16(k_paged(hh, lo + t, c));
                    split_grp(u, hh, q, d);
                    if (u < NG) vr[i] = ld_stream16(v_paged(hh, tb + 4u * q, d));
                }
#pragma unroll
                for (uint32_t i = 0; i < 2; i++) {
                    const uint32_t u = u0 + 256 * i;
                    uint32_t hh, t, c, q, d;
                    split_tok(u, hh, t, c);
                    if (u < NT) st_stream16(a.k_flat + flat_off(hh, lo + t, c), kr[i]);
                    split_grp(u, hh, q, d);
                    if (u < NG) {
                        uint16_t* tl = tile16 + hh * tile_elems;
                        const uint32_t w[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
                        for (uint32_t e = 0; e < 8; e++)  // element e: slot e % 4 of dim d + e / 4
                            tl[(4u * q + (e & 3u)) * RS + d + (e >> 2)] =
                                static_cast<uint16_t>(w[e >> 1] >> (16u * (e & 1u)));
                    }
                }
            }
            __syncthreads();
            for (uint32_t u = threadIdx.x; u < NT; u += 256) {
                uint32_t hh, t, c;
                split_tok(u, hh, t, c);
                const uint32_t jj = lo - tb + t;
                st_stream16(a.v_flat + flat_off(hh, tb + jj, c),
                            *reinterpret_cast<const uint4*>(tile16 + hh * tile_elems + jj * RS + 8u * c));
            }
        } else {
            for (uint32_t u0 = threadIdx.x; u0 < NT; u0 += 512) {
                uint4 kr[2], vr[2];
#pragma unroll
                for (uint32_t i = 0; i < 2; i++) {
                    const uint32_t u = u0 + 256 * i;
                    uint32_t hh, t, c;
                    split_tok(u, hh, t, c);
                    if (u < NT) {
                        kr[i] = ld_stream16(a.k_flat + flat_off(hh, lo + t, c));
                        vr[i] = ld_stream16(a.v_flat + flat_off(hh, lo + t, c));
                    }
                }
#pragma unroll
                for (uint32_t i = 0; i < 2; i++) {
                    const uint32_t u = u0 + 256 * i;
                    if (u >= NT) continue;
                    uint32_t hh, t, c;
                    split_tok(u, hh, t, c);
                    st_stream16(k_paged(hh, lo + t, c), kr[i]);
                    *reinterpret_cast<uint4*>(tile16 + hh * tile_elems + (lo - tb + t) * RS + 8u * c) = vr[i];
                }
            }
            __syncthreads();
            for (uint32_t u = threadIdx.x; u < NG; u += 256) {
                uint32_t hh, q, d;
                split_grp(u, hh, q, d);
                const uint32_t j4 = tb + 4u * q;
                const uint16_t* tl = tile16 + hh * tile_elems;
                uint32_t w[4];
#pragma unroll
                for (uint32_t e2 = 0; e2 < 4; e2++) {  // words: (slot 2(e2%2), +1) of dim d + e2 / 2
                    const uint32_t sl = 4u * q + 2u * (e2 & 1u), dd = d + (e2 >> 1);
                    w[e2] = static_cast<uint32_t>(tl[sl * RS + dd]) | (static_cast<uint32_t>(tl[(sl + 1u) * RS + dd]) << 16);
                }
                const uint4 unit = make_uint4(w[0], w[1], w[2], w[3]);
                merge_v16(v_paged(hh, j4, d), reinterpret_cast<const uint16_t*>(&unit), max(lo, j4) - j4,
                          min(hi, j4 + 4u) - j4);
            }
        }
        __syncthreads();
    }
}

constexpr uint32_t kInlineCopies = 32;  // page copies passed in the kernel arguments

struct CopyArgs {
    uint8_t* mem;
    const DevLayer* layers;
    const uint32_t* triples;  // device (src_page, dst_page, tokens) list, or null: the inline list
    const uint32_t* count;    // device length of `triples` (workgroups walk it), or null: one triple per x
    uint64_t pool_len;
    uint32_t kv_heads, page_shift;
    uint32_t inl[3 * kInlineCopies];
};

// Copy of slots [0, ntok) of one (page, head, K or V) plane of one layer.
// Every access is a 16-byte vector: a whole page is one contiguous run (4
// vectors in flight per lane); of a partial page, each K group moves the
// 16-byte pieces of its first ntok slots, and V its first ceil(ntok / 4)
// 4-slot groups, the group that ntok cuts merged slot by slot.
__device__ void copy_page_plane(const CopyArgs& a, const DevLayer& L, uint32_t which, uint32_t h, uint32_t src,
                                uint32_t dst, uint32_t ntok) {
    const uint32_t shift = a.page_shift, P = 1u << shift, hd = L.head_dim;
    const uint32_t vecs = (hd << shift) >> 3;  // 16-byte vectors per page plane
    const uint64_t page_elems = static_cast<uint64_t>(L.head_dim) << shift;
    const uint16_t* base = reinterpret_cast<const uint16_t*>(a.mem + (which ? L.v_off : L.k_off)) +
                           static_cast<uint64_t>(h) * a.pool_len * L.head_dim;
    const uint16_t* sp = base + src * page_elems;
    uint16_t* dp = const_cast<uint16_t*>(base) + dst * page_elems;
    if (ntok == P) {
        for (uint32_t b = threadIdx.x; b < vecs; b += 4 * 256) {
            uint4 r[4];
#pragma unroll
            for (uint32_t i = 0; i < 4; i++)
                if (b + 256 * i < vecs) r[i] = ld_stream16(sp + 8u * (b + 256 * i));
#pragma unroll
            for (uint32_t i = 0; i < 4; i++)
                if (b + 256 * i < vecs) st_stream16(dp + 8u * (b + 256 * i), r[i]);
        }
        return;
    }
    for (uint32_t u = threadIdx.x; u < vecs; u += 256) {
        const uint32_t e = 8u * u;
        if (which == 0) {  // K: element e of group g (32 P elements before it), slot (e - 32 P g) / width
            const uint32_t g = e / (32u * P);
            const uint32_t j = (e - 32u * P * g) / k_group_width(hd, 32u * g);
            copy16_if(dp + e, sp + e, j < ntok);
        } else {  // V: the unit's 4-slot group q (4 hd elements per group)
            const uint32_t q = e / (4u * hd);
            if (4u * q < ntok) merge_v16(dp + e, sp + e, 0, ntok - 4u * q);
        }
    }
}

// Grid: (x, layers * 2 * kv_heads), plane fastest.  Without a count,
// workgroup x copies triple x; with one, the x workgroups of a plane walk
// the *count triples of the device list (a launch sized without the host).
__global__ __launch_bounds__(256) void block_copy_kernel(CopyArgs a) {
    const uint32_t planes = 2 * a.kv_heads;
    const uint32_t layer = blockIdx.y / planes, plane = blockIdx.y - layer * planes;
    const uint32_t which = plane >= a.kv_heads, h = plane - which * a.kv_heads;
    const DevLayer L = a.layers[layer];
    if (a.count) {
        const uint32_t n = *a.count;
        for (uint32_t t = blockIdx.x; t < n; t += gridDim.x)
            copy_page_plane(a, L, which, h, a.triples[3 * t], a.triples[3 * t + 1], a.triples[3 * t + 2]);
        return;
    }
    if (a.triples)
        copy_page_plane(a, L, which, h, a.triples[3 * blockIdx.x], a.triples[3 * blockIdx.x + 1],
                        a.triples[3 * blockIdx.x + 2]);
    else
        copy_page_plane(a, L, which, h, a.inl[3 * blockIdx.x], a.inl[3 * blockIdx.x + 1], a.inl[3 * blockIdx.x + 2]);
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
    const size_t lds = static_cast<size_t>(kRunTokens) * (a.head_dim + 2) * 2;
    if (kv == THB_KV_F16_RNE)
        hipLaunchKernelGGL((kv_store_runs_kernel<SRC, THB_KV_F16_RNE>), grid, dim3(256), lds, s, a);
    else
        hipLaunchKernelGGL((kv_store_runs_kernel<SRC, THB_KV_BF16_TRUNC>), grid, dim3(256), lds, s, a);
}

// Cuts rows [0, m) of the call into runs: chunks of consecutive rows of one
// sequence at consecutive positions, cut where a position is a multiple of
// max_run (so every run but a chunk's first and last covers whole 4-slot
// groups).  Returns the number of rows in chunks of 8 or more tokens.
uint32_t make_runs(const uint32_t* meta, uint32_t m, uint32_t max_run, std::vector<uint32_t>& runs) {
    uint32_t long_rows = 0;
    uint32_t r = 0;
    while (r < m) {
        const uint32_t seq = meta[8 * r + 1], pos0 = meta[8 * r];
        uint32_t len = 1;
        while (r + len < m && meta[8 * (r + len) + 1] == seq && meta[8 * (r + len)] == pos0 + len) len++;
        if (len >= 8) long_rows += len;
        for (uint32_t t = 0; t < len;) {
            const uint32_t n = std::min(len - t, max_run - (pos0 + t) % max_run);
            runs.insert(runs.end(), {r + t, n, seq, pos0 + t});
            t += n;
        }
        r += len;
    }
    return long_rows;
}

// The runs of rows [row_off, row_off + m) on the device (cut and uploaded
// once per row-meta write).  Sets *n_runs; returns null when fewer than half
// of the rows lie in runs of 8 or more (decode-shaped calls), which use the
// row kernel instead.
const uint32_t* device_runs(thb_pool* p, const thb_rows* rows, uint32_t row_off, uint32_t m, uint32_t max_run,
                            hipStream_t s, uint32_t* n_runs) {
    // Under capture a new cut is uploaded inside the graph and not kept as
    // the cache (the buffer holds it only once the graph has run); a cached
    // cut that a capture uses stays in its buffer (reserve_rewrite moves
    // later uploads to a new one).
    const bool cap = capturing(s);
    if (p->runs_rows != rows || p->runs_version != rows->version || p->runs_off != row_off || p->runs_m != m ||
        p->runs_max != max_run) {
        std::vector<uint32_t> runs;
        p->runs_long = make_runs(rows->host.data() + 8 * static_cast<size_t>(row_off), m, max_run, runs);
        p->runs_n = static_cast<uint32_t>(runs.size() / 4);
        p->runs_rows = nullptr;  // invalid until the upload below is queued
        if (2 * static_cast<uint64_t>(p->runs_long) >= m) {
            void* dev = cap ? p->run_buf.reserve(runs.size() * 4, false, s)
                            : p->run_buf.reserve_rewrite(runs.size() * 4, false, s);
            p->stager.upload(dev, runs.data(), runs.size() * 4, s);
        }
        if (!cap) {
            p->runs_rows = rows;
            p->runs_version = rows->version;
            p->runs_off = row_off;
            p->runs_m = m;
            p->runs_max = max_run;
        }
    } else if (2 * static_cast<uint64_t>(p->runs_long) >= m) {
        p->run_buf.reserve(static_cast<size_t>(p->runs_n) * 16, false, s);  // marks it as used by a capture
    }
    *n_runs = p->runs_n;
    return 2 * static_cast<uint64_t>(p->runs_long) >= m ? static_cast<const uint32_t*>(p->run_buf.get()) : nullptr;
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

template <uint32_t SRC>
void launch_store_rope(uint32_t kv, dim3 grid, const RopeStoreArgs& a, hipStream_t s) {
    if (kv == THB_KV_F16_RNE)
        hipLaunchKernelGGL((kv_store_rope_kernel<SRC, THB_KV_F16_RNE>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((kv_store_rope_kernel<SRC, THB_KV_BF16_TRUNC>), grid, dim3(256), 0, s, a);
}

}  // namespace

int check_rope_tables(const thb_rope* r, uint32_t head_dim) {
    if (!r || !r->cos_dev || !r->sin_dev) return fail(THB_ERR_INVALID, "null rope tables");
    if (r->rot == 0 || r->rot % 16 != 0 || r->rot > head_dim)
        return fail(THB_ERR_CONFIG, "rope rot " + std::to_string(r->rot) +
                                        " must be a positive multiple of 16 not above head_dim " +
                                        std::to_string(head_dim));
    if (!aligned16(r->cos_dev) || !aligned16(r->sin_dev) || !aligned16(r->q_norm_dev) || !aligned16(r->k_norm_dev))
        return fail(THB_ERR_INVALID, "rope tables and norm weights must be 16-byte aligned");
    return THB_OK;
}

int check_rope(const thb_rope* r, uint32_t head_dim, const thb_rows* rows, uint32_t row_off, uint32_t m) {
    if (int rc = check_rope_tables(r, head_dim)) return rc;
    if (static_cast<uint64_t>(row_off) + m > rows->m)
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(rows->m) + " rows, call needs " +
                                         std::to_string(static_cast<uint64_t>(row_off) + m));
    for (uint32_t i = row_off; i < row_off + m; i++)
        if (rows->host[8 * i] >= r->max_pos)
            return fail(THB_ERR_MODEL, "row position " + std::to_string(rows->host[8 * i]) +
                                           " outside the rope tables (" + std::to_string(r->max_pos) + " positions)");
    return THB_OK;
}

namespace {
// Copy arguments of pool p; the triples are set by the caller.
CopyArgs copy_args(const thb_pool* p) {
    CopyArgs a{};
    a.mem = p->mem;
    a.layers = static_cast<const DevLayer*>(p->geom_buf.get());
    a.pool_len = static_cast<uint64_t>(p->arena.a.pages()) * p->page_len;
    a.kv_heads = p->kv_heads;
    a.page_shift = p->page_shift;
    return a;
}

// Launches block_copy_kernel over n triples (a.triples on the device, or
// a.inl), one workgroup per (triple, plane).
void launch_copy_grid(const CopyArgs& a, uint32_t n, uint32_t layers, hipStream_t stream) {
    const uint64_t planes = static_cast<uint64_t>(layers) * 2 * a.kv_heads;
    if (planes > kMaxGridY) throw HipError{hipErrorInvalidConfiguration, "block copy: layers*2*kv_heads > 65535"};
    constexpr uint32_t kMaxGridX = 1u << 30;
    for (uint32_t i0 = 0; i0 < n; i0 += kMaxGridX) {
        CopyArgs b = a;
        if (a.triples) b.triples = a.triples + 3 * static_cast<size_t>(i0);
        hipLaunchKernelGGL(block_copy_kernel, dim3(std::min(kMaxGridX, n - i0), static_cast<uint32_t>(planes)),
                           dim3(256), 0, stream, b);
        THB_HIP(hipGetLastError());
    }
}
}  // namespace

void launch_block_copy(thb_pool* p, const uint32_t* triples, uint32_t n, uint32_t max_tokens, hipStream_t stream) {
    if (n == 0 || max_tokens == 0) return;
    CopyArgs a = copy_args(p);
    if (n <= kInlineCopies) {  // a fork's or rollback's few copies: no upload
        std::copy(triples, triples + 3 * static_cast<size_t>(n), a.inl);
        a.triples = nullptr;
    } else {
        void* dev = p->copy_buf.reserve_rewrite(static_cast<size_t>(n) * 12, false, stream);
        p->stager.upload(dev, triples, static_cast<size_t>(n) * 12, stream);
        a.triples = static_cast<const uint32_t*>(dev);
    }
    launch_copy_grid(a, n, p->layers, stream);
}

void launch_block_copy_dev(thb_pool* p, const uint32_t* triples_dev, uint32_t n, uint32_t max_tokens,
                           hipStream_t stream) {
    if (n == 0 || max_tokens == 0) return;
    CopyArgs a = copy_args(p);
    a.triples = triples_dev;
    launch_copy_grid(a, n, p->layers, stream);
}

void launch_block_copy_counted(thb_pool* p, const uint32_t* triples_dev, const uint32_t* count_dev, uint32_t grid_x,
                               hipStream_t stream) {
    CopyArgs a = copy_args(p);
    a.triples = triples_dev;
    a.count = count_dev;
    launch_copy_grid(a, std::max<uint32_t>(grid_x, 1), p->layers, stream);
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
    // Under capture in graph mode (after a captured thb_pool_alloc_rows) the
    // call follows the row meta of each replay on the row kernel, its pages
    // checked on the device: the host mirror cannot know them.
    const bool cap = capturing(as_stream(stream));
    const bool follow = cap && pool->graph_mode;
    if (static_cast<uint64_t>(row_off) + m > (follow ? rows->max_m : rows->m))
        return fail(THB_ERR_INVALID, "row meta holds " + std::to_string(follow ? rows->max_m : rows->m) +
                                         " rows, call needs " + std::to_string(static_cast<uint64_t>(row_off) + m));
    if (!follow) {
        if (!cap)
            if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
        for (uint32_t r = row_off; r < row_off + m; r++) {
            uint32_t pos = rows->host[8 * r], seq = rows->host[8 * r + 1];
            if (int rc = check_cover(pool, seq, static_cast<uint64_t>(pos) + 1)) return rc;
        }
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
        a.pages = pool->arena.a.pages();
        a.seqs = pool->arena.a.seqs();
        const size_t esize = src_dtype == THB_DT_F32 ? 4 : 2;
        // Mostly long runs (prefill chunks): the run kernel writes whole V
        // page rows; otherwise (decode) one lane per 8 elements of a row.
        // The runs are cut on the host from the row meta's host mirror, so
        // a call that follows the replays' rows never takes them (a captured
        // call outside graph mode replays the captured runs).
        uint32_t n_runs = 0;
        if (const uint32_t* dev = follow ? nullptr : device_runs(pool, rows, row_off, m, kRunTokens, s, &n_runs)) {
            RunArgs ra;
            ra.k_src = k_src;
            ra.v_src = v_src;
            ra.k = a.k;
            ra.v = a.v;
            ra.runs = dev;
            ra.table = a.table;
            ra.plane = a.plane;
            ra.max_pages = a.max_pages;
            ra.page_shift = a.page_shift;
            ra.head_dim = a.head_dim;
            ra.kv_heads = pool->kv_heads;
            ra.do_k = 1;
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

// A scatter writes in place: a page another sequence also holds (a fork's
// shared prefix) would change under it.
static int check_unshared(const thb_pool* pool, uint32_t seq, uint32_t t0, uint32_t n) {
    const Arena& ar = pool->arena.a;
    const auto& tbl = ar.table_of(seq);
    const uint32_t p0 = t0 >> pool->page_shift;
    const uint32_t p1 = static_cast<uint32_t>((static_cast<uint64_t>(t0) + n - 1) >> pool->page_shift);
    for (uint32_t i = p0; i <= p1; i++)
        if (ar.refs()[tbl[i]] > 1)
            return fail(THB_ERR_MODEL, "scatter into page " + std::to_string(tbl[i]) + " of sequence " +
                                           std::to_string(seq) + ", which is shared with another sequence");
    return THB_OK;
}

// Launch shape of the gather kernel at one head_dim: LDS tile of V and KV
// heads per workgroup.  V tile: up to 64 slots x (head_dim + 8) elements,
// at most 32 KiB of LDS per head.  Heads per workgroup: enough for 4 KiB of
// K per page (small pages), at most 4, within 64 KiB of LDS.  More heads
// per workgroup serialise load rounds and measured slower at 4 KiB pages.
static void gather_shape(const thb_pool* pool, uint32_t hd, GatherArgs& a, size_t& lds) {
    uint32_t tile = std::min(pool->page_len, 64u);
    while (tile > 4 && tile * (hd + 8) * 2 > 32768) tile >>= 1;
    a.tile = tile;
    const size_t tile_bytes = static_cast<size_t>(tile) * (hd + 8) * 2;
    const uint32_t want = std::min<uint32_t>(4, std::max<uint32_t>(1, 2048 / (pool->page_len * hd)));
    uint32_t heads = 1;
    for (uint32_t hpw = want; hpw > 1; hpw--)
        if (pool->kv_heads % hpw == 0 && hpw * tile_bytes <= 65536) {
            heads = hpw;
            break;
        }
    a.heads = heads;
    lds = heads * tile_bytes;
}

static int gather_common(thb_pool* pool, uint32_t layer, uint32_t seq, uint32_t t0, uint32_t n, void* k, void* v,
                         void* stream, bool to_flat) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (int rc = check_layer(pool, layer)) return rc;
    if (n == 0) return THB_OK;
    if (!k || !v) return fail(THB_ERR_INVALID, "null buffer");
    if (!aligned16(k) || !aligned16(v)) return fail(THB_ERR_INVALID, "buffers must be 16-byte aligned");
    if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
    if (int rc = check_cover(pool, seq, static_cast<uint64_t>(t0) + n)) return rc;
    if (!to_flat)
        if (int rc = check_unshared(pool, seq, t0, n)) return rc;
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        const LayerGeom& g = pool->geom[layer];
        GatherArgs a{};
        a.k = reinterpret_cast<uint16_t*>(pool->mem + g.k_off);
        a.v = reinterpret_cast<uint16_t*>(pool->mem + g.v_off);
        a.k_flat = static_cast<uint16_t*>(k);
        a.v_flat = static_cast<uint16_t*>(v);
        a.table_row = pool->table_dev + static_cast<size_t>(seq) * pool->arena.a.max_pages();
        a.plane = static_cast<uint64_t>(pool->arena.a.pages()) * pool->page_len * g.head_dim;
        a.page_shift = pool->page_shift;
        a.head_dim = g.head_dim;
        a.pages = pool->arena.a.pages();
        a.n = n;
        a.t0 = t0;
        size_t lds = 0;
        gather_shape(pool, g.head_dim, a, lds);
        const uint32_t pages = static_cast<uint32_t>(((static_cast<uint64_t>(t0) + n - 1) >> pool->page_shift) -
                                                     (t0 >> pool->page_shift) + 1);
        dim3 grid(pages, pool->kv_heads / a.heads);
        if (to_flat)
            hipLaunchKernelGGL(gather_kernel<true>, grid, dim3(256), lds, s, a);
        else
            hipLaunchKernelGGL(gather_kernel<false>, grid, dim3(256), lds, s, a);
        THB_HIP(hipGetLastError());
        return THB_OK;
    });
}

// One launch over many ranges: range i moves to / from [kv_heads, n_i,
// head_dim] at element offset sum_{j < i} kv_heads * n_j * head_dim.
static int gather_batch(thb_pool* pool, const thb_kv_range* ranges, uint32_t count, void* k, void* v, void* stream,
                        bool to_flat) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (count == 0) return THB_OK;
    if (!ranges) return fail(THB_ERR_INVALID, "ranges is null");
    if (!k || !v) return fail(THB_ERR_INVALID, "null buffer");
    if (!aligned16(k) || !aligned16(v)) return fail(THB_ERR_INVALID, "buffers must be 16-byte aligned");
    if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
    uint32_t hd = 0;
    for (uint32_t i = 0; i < count; i++) {
        const thb_kv_range& r = ranges[i];
        if (int rc = check_layer(pool, r.layer)) return rc;
        if (r.n == 0) continue;
        if (hd == 0) hd = pool->geom[r.layer].head_dim;
        if (pool->geom[r.layer].head_dim != hd)
            return fail(THB_ERR_INVALID, "the ranges of one batched call must share a head_dim");
        if (int rc = check_cover(pool, r.seq, static_cast<uint64_t>(r.t0) + r.n)) return rc;
        if (!to_flat)
            if (int rc = check_unshared(pool, r.seq, r.t0, r.n)) return rc;
    }
    if (hd == 0) return THB_OK;
    if (!to_flat) {  // two ranges writing one token would race
        std::vector<std::array<uint64_t, 3>> spans;
        for (uint32_t i = 0; i < count; i++)
            if (ranges[i].n)
                spans.push_back({(static_cast<uint64_t>(ranges[i].layer) << 32) | ranges[i].seq, ranges[i].t0,
                                 static_cast<uint64_t>(ranges[i].t0) + ranges[i].n});
        std::sort(spans.begin(), spans.end());
        for (size_t i = 1; i < spans.size(); i++)
            if (spans[i][0] == spans[i - 1][0] && spans[i][1] < spans[i - 1][2])
                return fail(THB_ERR_INVALID, "scatter ranges of one sequence and layer overlap");
    }
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        const uint32_t mp = pool->arena.a.max_pages();
        std::vector<uint32_t> blob;  // items (2 words each), then the range records
        std::vector<uint32_t> recs;
        uint64_t flat = 0;
        for (uint32_t i = 0; i < count; i++) {
            const thb_kv_range& r = ranges[i];
            const uint32_t rec = static_cast<uint32_t>(recs.size() / kRangeWords);
            if (r.n) {
                const uint32_t pages = static_cast<uint32_t>(
                    ((static_cast<uint64_t>(r.t0) + r.n - 1) >> pool->page_shift) - (r.t0 >> pool->page_shift) + 1);
                for (uint32_t p = 0; p < pages; p++) blob.insert(blob.end(), {rec, p});
                const LayerGeom& g = pool->geom[r.layer];
                const uint64_t ko = g.k_off / 2, vo = g.v_off / 2;  // 16-bit elements from the arena base
                recs.insert(recs.end(), {r.seq * mp, r.t0, r.n, 0u, static_cast<uint32_t>(ko),
                                         static_cast<uint32_t>(ko >> 32), static_cast<uint32_t>(vo),
                                         static_cast<uint32_t>(vo >> 32), static_cast<uint32_t>(flat),
                                         static_cast<uint32_t>(flat >> 32)});
            }
            flat += static_cast<uint64_t>(pool->kv_heads) * r.n * hd;
        }
        const uint32_t n_items = static_cast<uint32_t>(blob.size() / 2);
        if (n_items > 0x7FFFFFFFu) throw HipError{hipErrorInvalidConfiguration, "batched gather too large"};
        const size_t items_words = blob.size();
        blob.insert(blob.end(), recs.begin(), recs.end());
        // Uploaded only when the ranges change: repeating a call (or
        // capturing it in a graph after a first call) moves nothing.  Under
        // capture a new list is uploaded inside the graph and not kept as
        // the cache; a cached list that a capture uses stays in its buffer.
        const bool cap = capturing(s);
        if (blob != pool->range_key) {
            void* d = cap ? pool->range_buf.reserve(blob.size() * 4, false, s)
                          : pool->range_buf.reserve_rewrite(blob.size() * 4, false, s);
            pool->stager.upload(d, blob.data(), blob.size() * 4, s);
            if (cap)
                pool->range_key.clear();
            else
                pool->range_key.swap(blob);
        } else {
            pool->range_buf.reserve(blob.size() * 4, false, s);  // marks it as used by a capture
        }
        const uint32_t* dev = static_cast<const uint32_t*>(pool->range_buf.get());
        GatherArgs a{};
        a.k = reinterpret_cast<uint16_t*>(pool->mem);
        a.v = reinterpret_cast<uint16_t*>(pool->mem);
        a.k_flat = static_cast<uint16_t*>(k);
        a.v_flat = static_cast<uint16_t*>(v);
        a.table_row = pool->table_dev;
        a.plane = static_cast<uint64_t>(pool->arena.a.pages()) * pool->page_len * hd;
        a.page_shift = pool->page_shift;
        a.head_dim = hd;
        a.pages = pool->arena.a.pages();
        a.items = dev;
        a.ranges = dev + items_words;
        size_t lds = 0;
        gather_shape(pool, hd, a, lds);
        dim3 grid(n_items, pool->kv_heads / a.heads);
        if (to_flat)
            hipLaunchKernelGGL(gather_kernel<true>, grid, dim3(256), lds, s, a);
        else
            hipLaunchKernelGGL(gather_kernel<false>, grid, dim3(256), lds, s, a);
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

int thb_kv_gather_batch(thb_pool* pool, const thb_kv_range* ranges, uint32_t count, void* k_dst, void* v_dst,
                        void* stream) {
    return gather_batch(pool, ranges, count, k_dst, v_dst, stream, true);
}

int thb_kv_scatter_batch(thb_pool* pool, const thb_kv_range* ranges, uint32_t count, const void* k_src,
                         const void* v_src, void* stream) {
    return gather_batch(pool, ranges, count, const_cast<void*>(k_src), const_cast<void*>(v_src), stream, false);
}

int thb_block_copy(thb_pool* pool, const uint32_t* triples, uint32_t n, void* stream) {
    if (!pool) return fail(THB_ERR_INVALID, "pool is null");
    if (n == 0) return THB_OK;
    if (!triples) return fail(THB_ERR_INVALID, "triples is null");
    if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
    const uint32_t pages = pool->arena.a.pages();
    uint32_t max_tok = 0;
    std::vector<uint32_t> srcs, dsts;
    for (uint32_t i = 0; i < n; i++) {
        uint32_t s = triples[3 * i], d = triples[3 * i + 1], t = triples[3 * i + 2];
        if (s >= pages || d >= pages)
            return fail(THB_ERR_INVALID, "page copy " + std::to_string(s) + " -> " + std::to_string(d) +
                                             " outside the pool of " + std::to_string(pages) + " pages");
        if (t > pool->page_len)
            return fail(THB_ERR_INVALID, "page copy of " + std::to_string(t) + " tokens exceeds page_len " +
                                             std::to_string(pool->page_len));
        max_tok = std::max(max_tok, t);
        srcs.push_back(s);
        dsts.push_back(d);
    }
    // The copies run in parallel: a destination written twice, or a page
    // both read and written, would race.  One source may feed many copies.
    std::sort(srcs.begin(), srcs.end());
    std::sort(dsts.begin(), dsts.end());
    for (size_t i = 1; i < dsts.size(); i++)
        if (dsts[i] == dsts[i - 1])
            return fail(THB_ERR_INVALID, "page " + std::to_string(dsts[i]) + " is the destination of two copies");
    for (uint32_t d : dsts)
        if (std::binary_search(srcs.begin(), srcs.end(), d))
            return fail(THB_ERR_INVALID, "page " + std::to_string(d) + " is both a source and a destination");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        launch_block_copy(pool, triples, n, max_tok, s);
        return THB_OK;
    });
}

int thb_rope_rows(void* x, uint32_t dtype, uint32_t m, uint32_t heads, uint32_t head_dim, const float* norm_w,
                  const thb_rope* rope, const thb_rows* rows, uint32_t row_off, void* stream) {
    if (!rows) return fail(THB_ERR_INVALID, "null rows");
    if (m == 0 || heads == 0) return THB_OK;
    if (!x || !aligned16(x)) return fail(THB_ERR_INVALID, "x must be a 16-byte aligned device buffer");
    if (dtype != THB_DT_F32 && dtype != THB_DT_F16)
        return fail(THB_ERR_INVALID, "rope rows take f32 or f16 (dtype " + std::to_string(dtype) + ")");
    if (int rc = thb_backend_head_dim(head_dim)) return rc;
    if (capturing(as_stream(stream)))
        return fail(THB_ERR_INVALID, "not capturable: thb_rope_rows checks the rows' positions against the rotary "
                                     "tables on the host");
    if (int rc = check_rope(rope, head_dim, rows, row_off, m)) return rc;
    if (!aligned16(norm_w)) return fail(THB_ERR_INVALID, "norm weight must be 16-byte aligned");
    const uint64_t waves = static_cast<uint64_t>(m) * heads;
    if (waves > 0x7FFFFFFFull) return fail(THB_ERR_INVALID, "rope rows: m * heads too large");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        RopeRowsArgs a;
        a.x = x;
        a.meta = rows->dev + 8 * static_cast<size_t>(row_off);
        a.m = m;
        a.heads = heads;
        a.head_dim = head_dim;
        a.rope = rope_dev(*rope, true);
        a.rope.w = norm_w;
        a.seg_shift = seg_shift_for(head_dim);
        const uint64_t per_block = 4ull * (64u >> a.seg_shift);
        const dim3 grid(static_cast<uint32_t>((waves + per_block - 1) / per_block));
        if (dtype == THB_DT_F16)
            hipLaunchKernelGGL(rope_rows_kernel<THB_DT_F16>, grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(rope_rows_kernel<THB_DT_F32>, grid, dim3(256), 0, s, a);
        THB_HIP(hipGetLastError());
        return THB_OK;
    });
}

int thb_kv_store_rope(thb_pool* pool, uint32_t layer, const void* k_src, const void* v_src, uint32_t src_dtype,
                      const thb_rope* rope, const thb_rows* rows, uint32_t row_off, uint32_t m, void* stream) {
    if (!pool || !rows) return fail(THB_ERR_INVALID, "null pool or rows");
    if (int rc = check_layer(pool, layer)) return rc;
    if (m == 0) return THB_OK;
    if (!k_src || !v_src) return fail(THB_ERR_INVALID, "null source buffer");
    if (src_dtype != THB_DT_F32 && src_dtype != THB_DT_F16)
        return fail(THB_ERR_INVALID, "rotary append takes f32 or f16 sources (src_dtype " +
                                         std::to_string(src_dtype) + ")");
    if (!aligned16(k_src) || !aligned16(v_src)) return fail(THB_ERR_INVALID, "source buffers must be 16-byte aligned");
    if (capturing(as_stream(stream)))
        return fail(THB_ERR_INVALID, "not capturable: thb_kv_store_rope checks the rows' positions against the "
                                     "rotary tables on the host");
    if (int rc = sync_mirror(pool, as_stream(stream))) return rc;
    if (int rc = check_rope(rope, pool->geom[layer].head_dim, rows, row_off, m)) return rc;
    for (uint32_t r = row_off; r < row_off + m; r++) {
        uint32_t pos = rows->host[8 * r], seq = rows->host[8 * r + 1];
        if (int rc = check_cover(pool, seq, static_cast<uint64_t>(pos) + 1)) return rc;
    }
    const uint64_t waves = static_cast<uint64_t>(m) * pool->kv_heads;
    if (waves > 0x7FFFFFFFull) return fail(THB_ERR_INVALID, "rotary append: m * kv_heads too large");
    return guarded([&]() -> int {
        hipStream_t s = as_stream(stream);
        pool_flush(pool, s);
        const LayerGeom& g = pool->geom[layer];
        RopeStoreArgs a;
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
        a.kv_heads = pool->kv_heads;
        a.m = m;
        a.rope = rope_dev(*rope, false);
        // Prefill chunks: V goes through the run kernel (whole page rows).
        uint32_t n_runs = 0;
        const uint32_t* run_dev = device_runs(pool, rows, row_off, m, kRunTokens, s, &n_runs);
        const bool by_runs = run_dev != nullptr;
        a.do_v = by_runs ? 0u : 1u;
        a.seg_shift = seg_shift_for(g.head_dim);
        const uint64_t per_block = 4ull * (64u >> a.seg_shift);
        const dim3 grid(static_cast<uint32_t>((waves + per_block - 1) / per_block));
        if (src_dtype == THB_DT_F16)
            launch_store_rope<THB_DT_F16>(pool->kv_dtype, grid, a, s);
        else
            launch_store_rope<THB_DT_F32>(pool->kv_dtype, grid, a, s);
        THB_HIP(hipGetLastError());
        if (by_runs) {
            RunArgs ra;
            ra.k_src = k_src;
            ra.v_src = v_src;
            ra.k = a.k;
            ra.v = a.v;
            ra.runs = run_dev;
            ra.table = a.table;
            ra.plane = a.plane;
            ra.max_pages = a.max_pages;
            ra.page_shift = a.page_shift;
            ra.head_dim = a.head_dim;
            ra.kv_heads = pool->kv_heads;
            ra.do_k = 0;
            const uint64_t n_wg = static_cast<uint64_t>(n_runs) * pool->kv_heads;
            if (n_wg > 0x7FFFFFFFull) throw HipError{hipErrorInvalidConfiguration, "append grid too large"};
            if (src_dtype == THB_DT_F16)
                launch_runs<THB_DT_F16>(pool->kv_dtype, dim3(static_cast<uint32_t>(n_wg)), ra, s);
            else
                launch_runs<THB_DT_F32>(pool->kv_dtype, dim3(static_cast<uint32_t>(n_wg)), ra, s);
            THB_HIP(hipGetLastError());
        }
        return THB_OK;
    });
}

}  // extern "C"
