"""Host page allocator: the reference's arena tests (tests/pool.rs) against
both the oracle restatement and the product allocator in libthuban_hip.so
(host-only entry points, no GPU), then a differential random walk."""

import random

import pytest

from oracle.arena import ArenaError, KvArena as OracleArena

U32_MAX = 0xFFFFFFFF


def _product_arena(seq_lens, pages, page_len):
    from flint_amd.pool import ArenaSpec, KvArena

    return KvArena(ArenaSpec(list(seq_lens), pages), page_len=page_len)


def _run_case(case, make, err_type):
    a = make(case["seq_lens"], case["pages"], 32)
    for st in case["steps"]:
        if "op" in st:
            fn = getattr(a, st["op"])
            if "error" in st:
                with pytest.raises(err_type) as e:
                    fn(*st["args"])
                assert st["error"] in str(e.value), (case["name"], str(e.value))
            else:
                fn(*st["args"])
        exp = st.get("expect", {})
        if "pages" in exp:
            assert (a.pages() if callable(a.pages) else a.pages) == exp["pages"]
        if "used" in exp:
            assert a.used() == exp["used"], case["name"]
        if "table_of" in exp:
            s, t = exp["table_of"]
            assert list(a.table_of(s)) == t
        if "table_len" in exp:
            s, n = exp["table_len"]
            assert len(a.table_of(s)) == n
        tab = list(a.table())
        if "table_size" in exp:
            assert len(tab) == exp["table_size"]
        for i, v in exp.get("table_eq", []):
            assert tab[i] == v
        for i, v in exp.get("table_ne", []):
            assert tab[i] != v
        for i, j in exp.get("table_ne_idx", []):
            assert tab[i] != tab[j]


def test_reference_arena_cases_on_oracle(golden):
    for case in golden("arena_cases.json"):
        _run_case(case, lambda sl, p, pl: OracleArena(sl, p, pl), ArenaError)


def test_reference_arena_cases_on_product(golden):
    from flint_amd import ThubanError

    for case in golden("arena_cases.json"):
        _run_case(case, _product_arena, ThubanError)


def test_error_messages_match_reference_text():
    from flint_amd import ThubanError

    a = _product_arena([64], 1, 32)
    with pytest.raises(ThubanError) as e:
        a.alloc(0, 0, 64)
    assert str(e.value) == "KV arena exhausted: 2 pages requested, 1 free"  # pool.rs:55-59
    assert e.value.kind == "Model"
    with pytest.raises(ThubanError) as e:
        a.alloc(0, 60, 5)
    assert str(e.value) == "context limit 64 reached"  # pool.rs:49-51
    with pytest.raises(ThubanError) as e:
        _product_arena([], None, 32)
    assert "non-empty and positive" in str(e.value)  # pool.rs:21-25
    with pytest.raises(ThubanError):
        _product_arena([0, 5], None, 32)


def test_pop_order_and_sentinels():
    a = _product_arena([40, 100], None, 16)
    assert a.pages() == 3 + 7 and a.max_pages() == 7
    a.alloc(1, 0, 33)
    a.alloc(0, 0, 1)
    assert a.table_of(1) == [0, 1, 2] and a.table_of(0) == [3]
    t = a.table()
    assert t[:7] == [3] + [U32_MAX] * 6
    assert t[7:] == [0, 1, 2] + [U32_MAX] * 4
    a.free_seq(1)  # returned in table order, popped LIFO
    a.alloc(0, 1, 39)
    assert a.table_of(0) == [3, 2, 1]


def _apply(a, op, args):
    try:
        getattr(a, op)(*args)
        return None
    except Exception as e:  # both error types carry the reference message
        return str(e)


@pytest.mark.parametrize("seed", range(6))
def test_differential_random_walk(seed):
    """Random alloc/free/truncate/fork sequences: the product allocator and
    the oracle agree on every table, every error and every CoW copy."""
    rng = random.Random(seed)
    page_len = rng.choice([8, 16, 32])
    seqs = rng.randint(2, 6)
    seq_lens = [rng.randint(1, 200) for _ in range(seqs)]
    pages = rng.choice([None, rng.randint(4, 40)])
    o = OracleArena(seq_lens, pages, page_len)
    p = _product_arena(seq_lens, pages, page_len)
    pos = [0] * seqs
    for _ in range(300):
        s = rng.randrange(seqs)
        r = rng.random()
        if r < 0.45:
            n = rng.randint(0, 40)
            op, args = "alloc", (s, pos[s], n)
        elif r < 0.6:
            op, args = "free_seq", (s,)
        elif r < 0.8:
            op, args = "truncate", (s, rng.randint(0, pos[s] + 5))
        else:
            d = rng.randrange(seqs)
            op, args = "fork", (s, d, rng.randint(0, pos[s] + 3))
            if d == s:
                continue
        eo, ep = _apply(o, op, args), _apply(p, op, args)
        assert eo == ep, (op, args, eo, ep)
        if eo is None:
            if op == "alloc":
                pos[s] = args[1] + args[2]
            elif op == "free_seq":
                pos[s] = 0
            elif op == "truncate":
                pos[s] = min(pos[s], args[1])
            elif op == "fork":
                pos[args[1]] = args[2]
        o.check_invariants()
        assert list(p.table()) == o.table()
        assert p.used() == o.used()
        assert p.take_copies() == o.take_copies()


def test_fork_shares_full_pages_and_copies_the_partial_one():
    a = _product_arena([100, 100, 100], 12, 16)
    a.alloc(0, 0, 40)  # pages 0, 1, 2 (last holds 8 tokens)
    a.fork(0, 1, 40)
    t0, t1 = a.table_of(0), a.table_of(1)
    assert t1[:2] == t0[:2] and t1[2] != t0[2]
    assert a.take_copies() == [(t0[2], t1[2], 8)]
    assert a.used() == 4
    # appending to seq 1 writes into its own page 2; a truncate into a shared
    # page followed by alloc copies that page first (copy-on-write)
    a.truncate(1, 20)
    a.alloc(1, 20, 1)
    t1b = a.table_of(1)
    assert t1b[0] == t0[0] and t1b[1] not in t0
    assert a.take_copies() == [(t0[1], t1b[1], 4)]
    a.free_seq(0)
    a.free_seq(1)
    assert a.used() == 0
