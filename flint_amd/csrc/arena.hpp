// Host page allocator: KvArena (reference crates/thuban_model/src/pool.rs
// :11-118) with a runtime page length and reference-counted page sharing.
// Pure C++ (no HIP), so it is usable and testable without a GPU.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace thb {

struct PageCopy {
    uint32_t src, dst, tokens;
};

class Arena {
public:
    // KvArena::new (pool.rs:20-45).  pages < 0 == ArenaSpec.pages = None.
    // Returns an empty string on success, else the error message.
    static std::string create(const uint32_t* seq_lens, uint32_t seqs, int64_t pages, uint32_t page_len,
                              Arena& out);

    // KvArena::alloc (pool.rs:47-65) + copy-on-write of shared pages that the
    // write range [pos, pos + tokens) touches.
    std::string alloc(uint32_t seq, uint32_t pos, uint32_t tokens);
    void free_seq(uint32_t seq);                        // pool.rs:67-71
    void truncate(uint32_t seq, uint32_t keep_tokens);  // pool.rs:73-79
    bool covers(uint32_t seq, uint32_t tokens) const;   // pool.rs:81-83
    std::string fork(uint32_t src, uint32_t dst, uint32_t tokens);

    void table(uint32_t* out) const;  // pool.rs:85-93
    const std::vector<uint32_t>& table_of(uint32_t seq) const { return tables_[seq]; }

    uint32_t pages() const { return pages_; }
    uint32_t used() const { return pages_ - static_cast<uint32_t>(free_.size()); }
    uint32_t max_pages() const { return max_pages_; }
    uint32_t seqs() const { return static_cast<uint32_t>(tables_.size()); }
    uint32_t page_len() const { return page_len_; }
    uint32_t seq_len(uint32_t seq) const { return seq_lens_[seq]; }

    // Free stack (back() is the next page handed out) and reference counts.
    const std::vector<uint32_t>& free_list() const { return free_; }
    const std::vector<uint32_t>& refs() const { return refs_; }
    // Replaces the allocator state with a device allocator's: free stack
    // [n_free], reference counts [pages], page counts [seqs] and the
    // flattened table [seqs * max_pages].  Pending copies are dropped.
    void load_state(const uint32_t* free_stack, uint32_t n_free, const uint32_t* refs, const uint32_t* npages,
                    const uint32_t* table);

    // Copies recorded by fork / copy-on-write, not yet executed on a device.
    std::vector<PageCopy>& copies() { return copies_; }
    // Rows of the flattened table changed since the last clear_dirty().
    const std::vector<uint8_t>& dirty() const { return dirty_; }
    bool any_dirty() const { return any_dirty_; }
    void clear_dirty();
    // Bumped by every mutation (lets callers cache derived state).
    uint64_t version() const { return version_; }

private:
    void release(uint32_t page);
    void touch(uint32_t seq);

    std::vector<uint32_t> seq_lens_;
    uint32_t max_pages_ = 0;
    uint32_t pages_ = 0;
    uint32_t page_len_ = 32;
    std::vector<std::vector<uint32_t>> tables_;
    std::vector<uint32_t> free_;  // stack; back() is the next page handed out
    std::vector<uint32_t> refs_;
    std::vector<PageCopy> copies_;
    std::vector<uint8_t> dirty_;
    bool any_dirty_ = false;
    uint64_t version_ = 0;
};

}  // namespace thb
