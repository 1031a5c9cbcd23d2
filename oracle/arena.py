"""Host page-allocator oracle -- TEST INFRASTRUCTURE ONLY.

Restates ``KvArena`` (reference ``crates/thuban_model/src/pool.rs:11-118``)
and adds the fork / copy-on-write extension that the reference lacks.

Pinned by: the reference's own arena tests
(``crates/thuban_model/tests/pool.rs:3-109``, transcribed as
``tests/golden/arena_cases.json``) for the reference semantics; by the
conservation invariants in ``check_invariants`` (every page is free xor
referenced, refcount == number of tables holding the page, no page twice in
the free list) for the fork / CoW extension, whose parity against the
reference is otherwise unpinned (the reference has no fork).
"""

from __future__ import annotations

U32_MAX = 0xFFFFFFFF


class ArenaError(Exception):
    """Mirrors thuban_error::Error::Model(String) raised by KvArena."""


class KvArena:
    """pool.rs:11-118, with the page length as a parameter (the reference
    hard-codes PAGE_LEN = 32 at thuban_kernel/src/lib.rs:9)."""

    def __init__(self, seq_lens, pages=None, page_len=32):
        # pool.rs:20-45
        if len(seq_lens) == 0 or any(l == 0 for l in seq_lens):
            raise ArenaError("sequence budgets must be non-empty and positive")
        self.page_len = page_len
        self.seq_lens = list(seq_lens)
        self.max_pages = max(-(-l // page_len) for l in seq_lens)
        self.pages = pages if pages is not None else sum(-(-l // page_len) for l in seq_lens)
        if self.pages == 0:
            raise ArenaError("KV arena needs at least one page")
        self.tables = [[] for _ in seq_lens]
        self.free = list(range(self.pages - 1, -1, -1))  # pops yield 0, 1, 2, ...
        self.refs = [0] * self.pages
        self.copies = []  # pending (src_page, dst_page, ntok) device copies

    # -- reference API -------------------------------------------------
    def alloc(self, seq, pos, tokens):
        """pool.rs:47-65.  Extension: a shared page that the write range
        [pos, pos+tokens) would touch is first copied (copy-on-write), in
        table order, before new pages are popped."""
        limit = self.seq_lens[seq]
        if pos + tokens > limit:
            raise ArenaError(f"context limit {limit} reached")
        pl = self.page_len
        want = -(-(pos + tokens) // pl)
        table = self.tables[seq]
        first = pos // pl
        cow = [i for i in range(first, min(len(table), want)) if self.refs[table[i]] > 1] if tokens else []
        need = max(0, want - len(table)) + len(cow)
        if need > len(self.free):
            raise ArenaError(f"KV arena exhausted: {need} pages requested, {len(self.free)} free")
        for i in cow:
            old = table[i]
            new = self.free.pop()
            ntok = min(pl, max(0, pos - i * pl))
            if ntok:
                self.copies.append((old, new, ntok))
            self.refs[old] -= 1
            self.refs[new] = 1
            table[i] = new
        for _ in range(max(0, want - len(table))):
            p = self.free.pop()
            self.refs[p] = 1
            table.append(p)

    def alloc_rows(self, positions, seqs):
        """The engine's per-plan allocation driven from row meta: Engine::step
        calls alloc_pages(seq, tokens) once per plan (thuban_generate/src/
        engine.rs:197-200), which is alloc(seq, pos, tokens) at the
        sequence's position (transformer/forward.rs:534-538).  Here a plan is
        a maximal run of rows of one sequence (its first row's position, its
        row count), in row order; the first failure propagates and the runs
        before it keep their pages, as the engine's `?` leaves them."""
        runs, r, m = [], 0, len(seqs)
        while r < m:
            e = r + 1
            while e < m and seqs[e] == seqs[r]:
                e += 1
            runs.append((seqs[r], positions[r], e - r))
            r = e
        for seq, pos, n in runs:
            self.alloc(seq, pos, n)

    def free_seq(self, seq):
        """pool.rs:67-71 (pages return in table order once unreferenced)."""
        for p in self.tables[seq]:
            self._release(p)
        self.tables[seq] = []

    def truncate(self, seq, keep_tokens):
        """pool.rs:73-79."""
        table = self.tables[seq]
        keep = min(-(-keep_tokens // self.page_len), len(table))
        for p in table[keep:]:
            self._release(p)
        del table[keep:]

    def covers(self, seq, tokens):
        """pool.rs:81-83."""
        return len(self.tables[seq]) * self.page_len >= tokens

    def table(self):
        """pool.rs:85-93."""
        flat = [U32_MAX] * (len(self.tables) * self.max_pages)
        for s, t in enumerate(self.tables):
            for i, p in enumerate(t):
                flat[s * self.max_pages + i] = p
        return flat

    def used(self):
        return self.pages - len(self.free)

    def table_of(self, seq):
        return list(self.tables[seq])

    # -- extension -------------------------------------------------------
    def fork(self, src, dst, tokens):
        """dst shares src's pages that hold tokens [0, tokens); a partial last
        page is copied (copy-on-write) so that both sequences can append."""
        if self.tables[dst]:
            raise ArenaError(f"fork target {dst} is not empty")
        if tokens > self.seq_lens[dst]:
            raise ArenaError(f"context limit {self.seq_lens[dst]} reached")
        if not self.covers(src, tokens):
            raise ArenaError(f"fork source {src} does not cover {tokens} tokens")
        pl = self.page_len
        n = -(-tokens // pl)
        partial = tokens % pl
        if partial and not self.free:
            raise ArenaError(f"KV arena exhausted: 1 pages requested, {len(self.free)} free")
        shared = self.tables[src][:n]
        for p in shared:
            self.refs[p] += 1
        self.tables[dst] = list(shared)
        if partial:
            old = shared[-1]
            new = self.free.pop()
            self.copies.append((old, new, partial))
            self.refs[old] -= 1
            self.refs[new] = 1
            self.tables[dst][-1] = new

    def take_copies(self):
        c, self.copies = self.copies, []
        return c

    def _release(self, p):
        self.refs[p] -= 1
        if self.refs[p] == 0:
            self.free.append(p)

    def check_invariants(self):
        held = {}
        for t in self.tables:
            for p in t:
                held[p] = held.get(p, 0) + 1
        assert len(set(self.free)) == len(self.free), "page twice in the free list"
        for p in range(self.pages):
            assert self.refs[p] == held.get(p, 0), f"page {p}: refcount {self.refs[p]} != holders {held.get(p, 0)}"
            assert (p in held) != (p in set(self.free)), f"page {p} must be free xor held"
