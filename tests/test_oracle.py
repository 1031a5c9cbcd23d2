"""Pins the CPU oracle (oracle/) against the reference's own known answers
and against closed forms.  CPU only."""

import math
import struct

import numpy as np
import pytest


def f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def bits32(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ------------------------------------------------------------------ codecs
def test_codec_known_answers(orc, golden):
    g = golden("codec_cases.json")
    L = orc.lib()
    for h, fb in g["f16_to_f32"]:
        assert bits32(L.orc_f16_to_f32(h)) == fb, hex(h)
    for fb, h in g["f32_to_f16"]:
        assert L.orc_f32_to_f16(f32(fb)) == h, (hex(fb), hex(h))
    for fb in g["f16_round_trip"]:
        assert bits32(L.orc_f16_to_f32(L.orc_f32_to_f16(f32(fb)))) == fb
    for fb in g["bf16_round_trip"]:
        assert bits32(L.orc_bf16_to_f32(L.orc_f32_to_bf16(f32(fb)))) == fb


def test_f16_decode_exhaustive_matches_ieee(orc):
    h = np.arange(65536, dtype=np.uint16)
    ours = orc.f16_to_f32(h).view(np.uint32)
    ieee = h.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(ours, ieee)


def special_f32_bits():
    """Every sign/exponent/top-10-mantissa pattern crossed with the low-13-bit
    patterns that decide rounding (tie, just below, just above, ...)."""
    hi = np.arange(1 << 19, dtype=np.uint32) << np.uint32(13)
    low = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x0800, 0x1800], dtype=np.uint32)
    return (hi[:, None] | low[None, :]).reshape(-1)


def test_f16_encode_matches_ieee_rne(orc):
    # f32 -> f16 RNE is the IEEE conversion numpy implements, except that the
    # reference turns every NaN into sign|0x7E00 (thuban_num lib.rs:30-35).
    b = special_f32_bits()
    ours = orc.f32_to_f16(b.view(np.float32))
    x = b.view(np.float32)
    nan = np.isnan(x)
    with np.errstate(over="ignore"):
        ieee = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours[~nan], ieee[~nan])
    sign = ((b[nan] >> 16) & 0x8000).astype(np.uint16)
    assert np.array_equal(ours[nan], sign | np.uint16(0x7E00))


def test_bf16_is_truncation(orc):
    b = special_f32_bits()
    assert np.array_equal(orc.f32_to_bf16(b.view(np.float32)), (b >> 16).astype(np.uint16))


# --------------------------------------------------------------- kv_store
def _identity_layer(orc, case, page_len):
    # cpu_ref's contiguous cache [kv_heads, max_seq, hd] equals a paged pool
    # whose pages are laid out in order (identity block table).
    pages = case["max_seq"] // page_len
    return orc.Layer(case["kv_heads"], case["head_dim"], pages, page_len, np.arange(pages, dtype=np.uint32),
                     pages, orc.KV_BF16)


@pytest.mark.parametrize("page_len", [1, 2])
def test_kv_store_reference_vectors(orc, golden, page_len):
    for case in golden("kv_store_cases.json"):
        L = _identity_layer(orc, case, page_len)
        m = case["m"]
        args = orc.row_meta([case["pos"] + i for i in range(m)], [0] * m)
        k = np.array(case["k_src"], np.uint32).view(np.float32)
        v = np.array(case["v_src"], np.uint32).view(np.float32)
        L.kv_store(k, v, args, m)
        assert np.array_equal(L.k.reshape(-1), np.array(case["expect_k"], np.uint16)), case["name"]
        assert np.array_equal(L.v.reshape(-1), np.array(case["expect_v"], np.uint16)), case["name"]


def test_kv_store_scatters_through_block_table(orc):
    rng = np.random.default_rng(7)
    nkv, hd, page_len, pages = 2, 8, 4, 6
    perm = rng.permutation(pages).astype(np.uint32)
    bt = perm.reshape(2, 3)  # 2 sequences x 3 pages
    L = orc.Layer(nkv, hd, pages, page_len, bt.reshape(-1), 3, orc.KV_F16)
    pos = [5, 0, 11]
    seqs = [1, 0, 0]
    src = rng.standard_normal((3, nkv, hd)).astype(np.float32)
    L.kv_store(src, -src, orc.row_meta(pos, seqs), 3)
    for r in range(3):
        slot = bt[seqs[r], pos[r] // page_len] * page_len + pos[r] % page_len
        assert np.array_equal(L.k[:, slot, :], orc.f32_to_f16(src[r]))
        assert np.array_equal(L.v[:, slot, :], orc.f32_to_f16(-src[r]))
    assert np.count_nonzero(L.k.reshape(-1, hd).any(axis=1)) == 3 * nkv


# ------------------------------------------------------------------- attn
def test_attn_reference_anchors(orc, golden):
    for case in golden("attn_cases.json"):
        L = orc.Layer(1, 2, 1, 2, np.array([0], np.uint32), 1, orc.KV_BF16)
        L.k[:] = orc.f32_to_bf16(np.array(case["k"], np.float32)).reshape(L.k.shape)
        L.v[:] = orc.f32_to_bf16(np.array(case["v"], np.float32)).reshape(L.v.shape)
        y = L.attn(np.array(case["q"], np.float32), orc.row_meta([case["pos"]], [0]), 1, 1,
                   1.0 / math.sqrt(case["head_dim"]), window=case["window"], causal=case["causal"], seq=0)
        assert np.allclose(y.reshape(-1), case["expect"], atol=case["tol"]), case["name"]


def _random_pool(orc, rng, nkv=2, hd=16, page_len=4, seqs=3, max_pages=8, kv=None, extra_pages=5):
    kv = orc.KV_F16 if kv is None else kv
    pages = seqs * max_pages + extra_pages
    perm = rng.permutation(pages)[: seqs * max_pages].astype(np.uint32)
    L = orc.Layer(nkv, hd, pages, page_len, perm, max_pages, kv)
    L.k[:] = orc.encode_kv(rng.standard_normal(L.k.shape).astype(np.float32), kv)
    L.v[:] = orc.encode_kv(rng.standard_normal(L.v.shape).astype(np.float32), kv)
    return L


def test_attn_ranges_follow_wgsl(orc):
    # 10 rows of one sequence at positions 20..29, causal, window 4:
    # kv_len of rows 0-7 is pos[7]+1 = 28, of rows 8-9 pos[9]+1 = 30.
    args = orc.row_meta(list(range(20, 30)), [0] * 10)
    lo, hi, _ = orc.attn_ranges(args, 10, seq=0, causal=True, window=4)
    assert list(lo) == [p + 1 - 4 for p in range(20, 30)]
    assert list(hi) == [p + 1 for p in range(20, 30)]
    lo, hi, _ = orc.attn_ranges(args, 10, seq=0, causal=False, window=4)
    assert list(lo) == [0] * 10 and list(hi) == [30] * 10  # window needs causal (attn.wgsl:80)
    # non-monotonic positions: the 8-row block's last row caps kv_len
    args = orc.row_meta([9, 3, 1], [0, 0, 0])
    lo, hi, _ = orc.attn_ranges(args, 3, seq=0, causal=True, window=0)
    assert list(hi) == [2, 2, 2]


def test_attn_single_key_returns_its_value(orc):
    rng = np.random.default_rng(1)
    L = _random_pool(orc, rng)
    q = rng.standard_normal((1, 4, 16)).astype(np.float32)
    y = L.attn(q, orc.row_meta([9], [1]), 1, 4, 0.25, window=1, causal=True)
    slot = L.block_table[1 * L.max_pages + 9 // 4] * 4 + 9 % 4
    for h in range(4):
        assert np.array_equal(y[0, h], orc.decode_kv(L.v[h // 2, slot], L.kv_dtype).astype(np.float64))


def test_attn_zero_query_averages_values(orc):
    rng = np.random.default_rng(2)
    L = _random_pool(orc, rng)
    q = np.zeros((1, 2, 16), np.float32)
    y = L.attn(q, orc.row_meta([13], [2]), 1, 2, 0.25, window=6, causal=True)
    vals = []
    for j in range(13 + 1 - 6, 14):
        slot = L.block_table[2 * L.max_pages + j // 4] * 4 + j % 4
        vals.append(orc.decode_kv(L.v[:, slot], L.kv_dtype))
    mean = np.mean(np.array(vals, np.float64), axis=0)
    assert np.allclose(y[0], mean, atol=1e-12)


def test_attn_paged_equals_contiguous(orc):
    # batch.rs:302-347 invariant, here exactly (same arithmetic, other pages).
    rng = np.random.default_rng(3)
    L = _random_pool(orc, rng, seqs=2)
    perm2 = rng.permutation(L.pool_len // L.page_len)[: 2 * L.max_pages].astype(np.uint32)
    L2 = orc.Layer(L.kv_heads, L.head_dim, L.pool_len // L.page_len, L.page_len, perm2, L.max_pages, L.kv_dtype)
    for s in range(2):
        for j in range(L.max_pages * L.page_len):
            a = L.block_table[s * L.max_pages + j // 4] * 4 + j % 4
            b = perm2[s * L.max_pages + j // 4] * 4 + j % 4
            L2.k[:, b] = L.k[:, a]
            L2.v[:, b] = L.v[:, a]
    q = rng.standard_normal((3, 4, 16)).astype(np.float32)
    args = orc.row_meta([5, 30, 31], [0, 1, 1])
    assert np.array_equal(L.attn(q, args, 3, 4, 0.25), L2.attn(q, args, 3, 4, 0.25))


def test_attn_window_beyond_context_is_no_window(orc):
    rng = np.random.default_rng(4)
    L = _random_pool(orc, rng)
    q = rng.standard_normal((2, 2, 16)).astype(np.float32)
    args = orc.row_meta([17, 18], [0, 0])
    assert np.array_equal(L.attn(q, args, 2, 2, 0.3, window=0, seq=0), L.attn(q, args, 2, 2, 0.3, window=19, seq=0))
    assert not np.array_equal(L.attn(q, args, 2, 2, 0.3, window=0, seq=0),
                              L.attn(q, args, 2, 2, 0.3, window=18, seq=0))


def test_attn_softcap_closed_form(orc):
    # one row, two keys: weights are softmax of cap*tanh(s/cap)
    L = orc.Layer(1, 8, 1, 8, np.array([0], np.uint32), 1, orc.KV_F16)
    k = np.zeros((2, 8), np.float32)
    k[0, 0], k[1, 1] = 3.0, -2.0
    v = np.eye(2, 8, dtype=np.float32)
    L.k[0, :2] = orc.f32_to_f16(k)
    L.v[0, :2] = orc.f32_to_f16(v)
    q = np.zeros((1, 1, 8), np.float32)
    q[0, 0, :2] = [10.0, 10.0]
    cap = 5.0
    y = L.attn(q, orc.row_meta([1], [0]), 1, 1, 0.5, softcap=cap)
    s = cap * np.tanh(np.array([30.0 * 0.5, -20.0 * 0.5]) / cap)
    w = np.exp(s - s.max())
    w /= w.sum()
    assert np.allclose(y[0, 0, :2], w, atol=1e-12)


def test_attn_f32_mode_matches_double(orc):
    rng = np.random.default_rng(5)
    L = _random_pool(orc, rng, hd=64, page_len=8, max_pages=40, kv=orc.KV_BF16)
    q = rng.standard_normal((4, 4, 64)).astype(np.float32)
    args = orc.row_meta([300, 301, 40, 250], [0, 0, 1, 2])
    y64 = L.attn(q, args, 4, 4, 0.125, window=128)
    y32 = L.attn(q, args, 4, 4, 0.125, window=128, precision=1)
    assert np.max(np.abs(y64 - y32)) < 1e-5


def test_gather_and_block_copy_closed_form(orc):
    rng = np.random.default_rng(6)
    L = _random_pool(orc, rng)
    k, v = L.gather(1, 3, 9)
    for t in range(9):
        j = 3 + t
        slot = L.block_table[L.max_pages + j // 4] * 4 + j % 4
        assert np.array_equal(k[:, t], L.k[:, slot]) and np.array_equal(v[:, t], L.v[:, slot])
    before = L.k.copy()
    L.block_copy([[2, 5, 3]])
    assert np.array_equal(L.k[:, 20:23], before[:, 8:11])
    assert np.array_equal(L.k[:, 23], before[:, 23])


# ------------------------------------------------------------------ rope
def _tables(max_pos, rot, theta=10000.0):
    half = rot // 2
    inv = 1.0 / theta ** (2.0 * np.arange(half) / rot)
    a = np.arange(max_pos)[:, None] * inv[None, :]
    return np.cos(a).astype(np.float32), np.sin(a).astype(np.float32)


def test_rope_reference_cases(orc, golden):
    """rope_case and anchor_rope of the reference's kernel tests, with the
    reference's tolerance (kernels.rs:132-147: |got - want| <= rel |want| + abs)."""
    for case in golden("rope_cases.json"):
        m, heads, hd, rot = case["m"], case["heads"], case["head_dim"], case["rot"]
        half = rot // 2
        x = np.array(case["x"], np.float32).reshape(m, heads, hd)
        cos = np.array(case["cos"], np.float32).reshape(-1, half)
        sin = np.array(case["sin"], np.float32).reshape(-1, half)
        got = orc.rope_rows(x, case["pos"], rot, cos, sin).reshape(-1).astype(np.float64)
        want = np.array(case["expect"], np.float64)
        assert np.all(np.abs(got - want) <= case["rel"] * np.abs(want) + case["abs"]), case["cite"]


def test_rope_closed_forms(orc):
    """Position 0 is the identity; dims >= rot pass through bit for bit; each
    rotated pair keeps its norm; dot products of rotated vectors depend only
    on the position difference (the defining property of RoPE)."""
    rng = np.random.default_rng(3)
    hd, rot, heads = 64, 32, 3
    cos, sin = _tables(40, rot)
    x = rng.standard_normal((4, heads, hd)).astype(np.float32)
    same = orc.rope_rows(x, [0, 0, 0, 0], rot, cos, sin)
    assert np.array_equal(same, x)
    y = orc.rope_rows(x, [5, 9, 17, 33], rot, cos, sin)
    assert np.array_equal(y[..., rot:], x[..., rot:])
    half = rot // 2
    n_in = x[..., :half].astype(np.float64) ** 2 + x[..., half:rot].astype(np.float64) ** 2
    n_out = y[..., :half].astype(np.float64) ** 2 + y[..., half:rot].astype(np.float64) ** 2
    assert np.allclose(n_out, n_in, rtol=1e-5, atol=1e-6)
    q = rng.standard_normal((1, 1, hd)).astype(np.float32)
    k = rng.standard_normal((1, 1, hd)).astype(np.float32)
    dots = []
    for a, b in [(7, 3), (11, 7), (30, 26)]:
        qa = orc.rope_rows(q, [a], rot, cos, sin).astype(np.float64)
        kb = orc.rope_rows(k, [b], rot, cos, sin).astype(np.float64)
        dots.append(float(np.sum(qa * kb)))
    assert max(dots) - min(dots) < 1e-4 * (1 + abs(dots[0]))
    # a plausible slip (partner from the wrong half) breaks the property
    assert not np.allclose(y[..., :half], x[..., :half] * cos[[5, 9, 17, 33]][:, None, :]
                           + x[..., half:rot] * sin[[5, 9, 17, 33]][:, None, :], atol=1e-3)


def test_rope_rmsnorm_matches_double(orc):
    """norm.wgsl MODE 4: y = x / sqrt(mean(x^2) + eps) * w, then the rotation;
    against a double-precision evaluation."""
    rng = np.random.default_rng(4)
    hd, rot, eps = 128, 64, 1e-6
    cos, sin = _tables(16, rot)
    x = (rng.standard_normal((2, 4, hd)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    got = orc.rope_rows(x, [3, 12], rot, cos, sin, w=w, eps=eps).astype(np.float64)
    xd = x.astype(np.float64)
    t = xd / np.sqrt(np.mean(xd * xd, axis=-1, keepdims=True) + eps) * w.astype(np.float64)
    half = rot // 2
    want = t.copy()
    for r, p in enumerate([3, 12]):
        c, s = cos[p].astype(np.float64), sin[p].astype(np.float64)
        want[r, :, :half] = t[r, :, :half] * c - t[r, :, half:rot] * s
        want[r, :, half:rot] = t[r, :, half:rot] * c + t[r, :, :half] * s
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    # no rotation (rot 0) leaves only the norm
    only = orc.rope_rows(x, [3, 12], 0, cos, sin, w=w, eps=eps).astype(np.float64)
    assert np.allclose(only, t, rtol=1e-6, atol=1e-7)
    with pytest.raises(ValueError):
        orc.rope_rows(x, [3, 16], rot, cos, sin)  # position outside the tables


def test_lcg_reproduces_the_reference_vector(orc, golden):
    """oracle.lcg_fill restates the reference tests' Rng (kernels.rs
    :112-124): Rng(111) draws the k_src then v_src of kv_store_writes_both_caches
    (kernels.rs:1271-1273), transcribed bit by bit in kv_store_cases.json."""
    case = [c for c in golden("kv_store_cases.json") if c["name"] == "kv_store_writes_both_caches"][0]
    n = len(case["k_src"])
    draws = orc.lcg_fill(111, 2 * n).view(np.uint32)
    assert draws[:n].tolist() == case["k_src"] and draws[n:].tolist() == case["v_src"]


def test_gemm_matches_float64_within_the_f32_bound(orc):
    """cpu_ref::gemm's f32 sums in k order (cpu_ref.rs:11-25) against numpy's
    float64 matmul: |f32 sum - exact| <= k * 2^-24 * sum |x w| (the textbook
    bound of a sequential sum), and the double mode within one rounding."""
    rng = np.random.default_rng(5)
    for m, n, k in ((1, 32, 128), (7, 48, 256), (33, 16, 1024)):
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = rng.standard_normal((n, k)).astype(np.float32)
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        bound = k * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
        got = orc.gemm(x, w, m, n, k)
        assert np.all(np.abs(got - exact) <= bound + 1e-30)
        ex = orc.gemm(x, w, m, n, k, exact=True)
        assert np.all(np.abs(ex - exact) <= np.abs(exact) * 2.0 ** -24 + 1e-30)
        y0 = rng.standard_normal((m, n)).astype(np.float32)
        acc = orc.gemm(x, w, m, n, k, y0=y0, exact=True)
        assert np.all(np.abs(acc - (exact + y0)) <= np.abs(exact + y0) * 2.0 ** -24 + 1e-30)


def test_gemm_closed_forms(orc):
    """Identity weights give y = x exactly (+ y0 with one rounding); a
    single row equals cpu_ref::gemv, the same loop (cpu_ref.rs:27-35); a
    transposed-operand mistake would break the rectangular case."""
    rng = np.random.default_rng(6)
    k = 64
    x = rng.standard_normal((5, k)).astype(np.float32)
    eye = np.eye(k, dtype=np.float32)
    assert np.array_equal(orc.gemm(x, eye, 5, k, k), x)
    y0 = rng.standard_normal((5, k)).astype(np.float32)
    assert np.array_equal(orc.gemm(x, eye, 5, k, k, y0=y0), x + y0)
    w = rng.standard_normal((16, k)).astype(np.float32)
    full = orc.gemm(x, w, 5, 16, k)
    for r in range(5):
        assert np.array_equal(orc.gemm(x[r:r + 1], w, 1, 16, k), full[r:r + 1])
    sel = np.zeros((3, k), np.float32)
    sel[0, 2], sel[1, 7], sel[2, 63] = 1.0, 2.0, -1.0  # picks columns of x
    assert np.array_equal(orc.gemm(x, sel, 5, 3, k), np.stack([x[:, 2], 2 * x[:, 7], -x[:, 63]], 1))
