// Host page allocator.  Semantics follow KvArena in the reference
// (crates/thuban_model/src/pool.rs:11-118): a LIFO free list initialised so
// that pops yield pages 0, 1, 2, ...; pages return in table order.  The
// extension for shared pages keeps a reference count per page: a page goes
// back to the free list when its last holder drops it.
#include "arena.hpp"

#include <algorithm>

namespace thb {

static uint32_t div_ceil(uint64_t a, uint32_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

std::string Arena::create(const uint32_t* seq_lens, uint32_t seqs, int64_t pages, uint32_t page_len,
                          Arena& out) {
    if (page_len == 0 || page_len > 256 || (page_len & (page_len - 1)) != 0)
        return "page_len " + std::to_string(page_len) + " must be a power of two in [1, 256]";
    if (seqs == 0 || seq_lens == nullptr) return "sequence budgets must be non-empty and positive";
    for (uint32_t i = 0; i < seqs; i++)
        if (seq_lens[i] == 0) return "sequence budgets must be non-empty and positive";
    Arena a;
    a.page_len_ = page_len;
    a.seq_lens_.assign(seq_lens, seq_lens + seqs);
    uint64_t total = 0;
    for (uint32_t l : a.seq_lens_) {
        uint32_t p = div_ceil(l, page_len);
        a.max_pages_ = std::max(a.max_pages_, p);
        total += p;
    }
    uint64_t n = pages >= 0 ? static_cast<uint64_t>(pages) : total;
    if (n == 0) return "KV arena needs at least one page";
    if (n >= 0xFFFFFFFFull) return "KV arena page count exceeds u32";
    a.pages_ = static_cast<uint32_t>(n);
    a.tables_.assign(seqs, {});
    a.free_.resize(a.pages_);
    for (uint32_t i = 0; i < a.pages_; i++) a.free_[i] = a.pages_ - 1 - i;
    a.refs_.assign(a.pages_, 0);
    a.dirty_.assign(seqs, 1);
    a.any_dirty_ = true;
    out = std::move(a);
    return {};
}

void Arena::touch(uint32_t seq) {
    dirty_[seq] = 1;
    any_dirty_ = true;
    version_++;
}

void Arena::clear_dirty() {
    std::fill(dirty_.begin(), dirty_.end(), 0);
    any_dirty_ = false;
}

void Arena::release(uint32_t page) {
    if (--refs_[page] == 0) free_.push_back(page);
}

std::string Arena::alloc(uint32_t seq, uint32_t pos, uint32_t tokens) {
    uint32_t limit = seq_lens_[seq];
    if (static_cast<uint64_t>(pos) + tokens > limit) return "context limit " + std::to_string(limit) + " reached";
    auto& table = tables_[seq];
    uint32_t want = div_ceil(static_cast<uint64_t>(pos) + tokens, page_len_);
    uint32_t have = static_cast<uint32_t>(table.size());
    // Shared pages inside the write range must be copied before the write.
    std::vector<uint32_t> cow;
    if (tokens > 0)
        for (uint32_t i = pos / page_len_; i < std::min(have, want); i++)
            if (refs_[table[i]] > 1) cow.push_back(i);
    uint32_t need = (want > have ? want - have : 0) + static_cast<uint32_t>(cow.size());
    if (need > free_.size())
        return "KV arena exhausted: " + std::to_string(need) + " pages requested, " + std::to_string(free_.size()) +
               " free";
    for (uint32_t i : cow) {
        uint32_t old = table[i];
        uint32_t fresh = free_.back();
        free_.pop_back();
        uint64_t first = static_cast<uint64_t>(i) * page_len_;
        uint32_t ntok = pos > first ? static_cast<uint32_t>(std::min<uint64_t>(page_len_, pos - first)) : 0;
        if (ntok) copies_.push_back({old, fresh, ntok});
        refs_[old]--;
        refs_[fresh] = 1;
        table[i] = fresh;
    }
    while (table.size() < want) {
        uint32_t p = free_.back();
        free_.pop_back();
        refs_[p] = 1;
        table.push_back(p);
    }
    if (need) touch(seq);
    return {};
}

void Arena::free_seq(uint32_t seq) {
    for (uint32_t p : tables_[seq]) release(p);
    if (!tables_[seq].empty()) touch(seq);
    tables_[seq].clear();
}

void Arena::truncate(uint32_t seq, uint32_t keep_tokens) {
    auto& table = tables_[seq];
    size_t keep = std::min<size_t>(div_ceil(keep_tokens, page_len_), table.size());
    if (keep == table.size()) return;
    for (size_t i = keep; i < table.size(); i++) release(table[i]);
    table.resize(keep);
    touch(seq);
}

bool Arena::covers(uint32_t seq, uint32_t tokens) const {
    return static_cast<uint64_t>(tables_[seq].size()) * page_len_ >= tokens;
}

std::string Arena::fork(uint32_t src, uint32_t dst, uint32_t tokens) {
    if (!tables_[dst].empty()) return "fork target " + std::to_string(dst) + " is not empty";
    if (tokens > seq_lens_[dst]) return "context limit " + std::to_string(seq_lens_[dst]) + " reached";
    if (!covers(src, tokens))
        return "fork source " + std::to_string(src) + " does not cover " + std::to_string(tokens) + " tokens";
    uint32_t n = div_ceil(tokens, page_len_);
    uint32_t partial = tokens % page_len_;
    if (partial && free_.empty())
        return "KV arena exhausted: 1 pages requested, " + std::to_string(free_.size()) + " free";
    auto& out = tables_[dst];
    out.assign(tables_[src].begin(), tables_[src].begin() + n);
    for (uint32_t p : out) refs_[p]++;
    if (partial) {
        uint32_t old = out.back();
        uint32_t fresh = free_.back();
        free_.pop_back();
        copies_.push_back({old, fresh, partial});
        refs_[old]--;
        refs_[fresh] = 1;
        out.back() = fresh;
    }
    touch(dst);
    return {};
}

void Arena::load_state(const uint32_t* free_stack, uint32_t n_free, const uint32_t* refs, const uint32_t* npages,
                       const uint32_t* table) {
    free_.assign(free_stack, free_stack + n_free);
    refs_.assign(refs, refs + pages_);
    for (size_t s = 0; s < tables_.size(); s++) {
        const uint32_t* row = table + s * max_pages_;
        tables_[s].assign(row, row + std::min(npages[s], max_pages_));
        touch(static_cast<uint32_t>(s));
    }
    copies_.clear();
}

void Arena::table(uint32_t* out) const {
    std::fill(out, out + static_cast<size_t>(tables_.size()) * max_pages_, 0xFFFFFFFFu);
    for (size_t s = 0; s < tables_.size(); s++)
        std::copy(tables_[s].begin(), tables_[s].end(), out + s * max_pages_);
}

}  // namespace thb
