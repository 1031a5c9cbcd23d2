"""GPU parity of append (kv_store), gather, scatter, block copy and fork:
bit-exact against the CPU oracle on identical inputs."""

import random

import numpy as np
import pytest

import oracle
from gpu_util import fill, make_pool, oracle_layer, say, scattered_alloc

pytestmark = pytest.mark.gpu

SRC = {"f32": oracle.SRC_F32, "f16": oracle.SRC_F16, "bf16": oracle.SRC_BF16}


def _src_words(torch, t):
    if t.dtype == torch.float32:
        return t.cpu().numpy()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("kv", ["bf16", "f16"])
@pytest.mark.parametrize("src", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("page_len", [16, 32])
def test_kv_store_bit_exact(torch_cuda, kv, src, page_len):
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    say("kv_store", kv, src, page_len)
    rng = random.Random(11)
    lens = [70, 33, 129]
    pool = make_pool(lens, kv_heads=4, head_dim=128, page_len=page_len, kv_dtype=kv, extra_pages=3)
    scattered_alloc(pool, lens, rng, page_len)
    ref = oracle_layer(torch, pool)  # zero pool + the table
    rows = RowMeta(64)
    pairs = [(p, s) for s, n in enumerate(lens) for p in range(n)]
    rng.shuffle(pairs)
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[src]
    for i in range(0, len(pairs), 64):
        chunk = pairs[i: i + 64]
        m = len(chunk)
        pos, seqs = [p for p, _ in chunk], [s for _, s in chunk]
        rows.write(pos, seqs, m)
        k = torch.randn(m, 4, 128, device="cuda").to(dt)
        v = (torch.randn(m, 4, 128, device="cuda") * 1e3).to(dt)
        ops.kv_store(k, v, pool, 0, m, rows)
        ref.kv_store(_src_words(torch, k), _src_words(torch, v), oracle.row_meta(pos, seqs), m, SRC[src])
    got = oracle_layer(torch, pool)
    assert np.array_equal(got.k, ref.k)
    assert np.array_equal(got.v, ref.v)


def test_kv_store_special_values_bit_exact(torch_cuda):
    """Every sign/exponent/top-10-mantissa pattern x rounding-relevant low
    bits (incl. NaN, inf, subnormals, ties) through f32 -> f16 and -> bf16."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    hi = np.arange(1 << 19, dtype=np.uint32) << np.uint32(13)
    low = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x0800, 0x1800], dtype=np.uint32)
    bits = (hi[:, None] | low[None, :]).reshape(-1)  # 4 Mi values
    nkv, hd = 8, 128
    m = bits.size // (nkv * hd)  # 4096 rows
    for kv in ("f16", "bf16"):
        say("special values", kv)
        pool = make_pool([m], kv_heads=nkv, head_dim=hd, page_len=32, kv_dtype=kv)
        pool.alloc(0, 0, m)
        rows = RowMeta(m)
        rows.write(list(range(m)), [0] * m, m)
        src = torch.from_numpy(bits.view(np.float32).reshape(m, nkv, hd).copy()).cuda()
        ops.kv_store(src, src, pool, 0, m, rows)
        k, v = pool.read_layer(0)
        table = np.array(pool.arena.table_of(0))
        # slot of token t = table[t // 32] * 32 + t % 32; gather back in token order
        slots = (table[np.arange(m) // 32] * 32 + np.arange(m) % 32)
        got = k[:, slots, :].transpose(1, 0, 2).reshape(-1)
        want = (oracle.f32_to_f16 if kv == "f16" else oracle.f32_to_bf16)(bits.view(np.float32))
        assert np.array_equal(got, want)
        gotv = v[:, slots, :].transpose(1, 0, 2).reshape(-1)
        assert np.array_equal(gotv, want)


def test_kv_store_reference_lcg_vector(torch_cuda, golden):
    """kv_store_writes_both_caches (kernels.rs:1266-1308) embedded in the
    first 4 dims of a head_dim-64 pool (the product needs head_dim >= 64)."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    case = [c for c in golden("kv_store_cases.json") if c["name"] == "kv_store_writes_both_caches"][0]
    m, nkv, hd, pos = case["m"], case["kv_heads"], case["head_dim"], case["pos"]
    say("reference kv_store vector")
    pool = make_pool([case["max_seq"]], kv_heads=nkv, head_dim=64, page_len=8, kv_dtype="bf16")
    pool.alloc(0, 0, case["max_seq"])
    rows = RowMeta(8)
    rows.write([pos + i for i in range(m)], [0] * m, m)
    ks = np.zeros((m, nkv, 64), np.float32)
    vs = np.zeros((m, nkv, 64), np.float32)
    ks[:, :, :hd] = np.array(case["k_src"], np.uint32).view(np.float32).reshape(m, nkv, hd)
    vs[:, :, :hd] = np.array(case["v_src"], np.uint32).view(np.float32).reshape(m, nkv, hd)
    ops.kv_store(torch.from_numpy(ks).cuda(), torch.from_numpy(vs).cuda(), pool, 0, m, rows)
    k, v = pool.read_layer(0)
    got_k = k[:, :, :hd].reshape(-1)
    got_v = v[:, :, :hd].reshape(-1)
    assert np.array_equal(got_k, np.array(case["expect_k"], np.uint16))
    assert np.array_equal(got_v, np.array(case["expect_v"], np.uint16))


@pytest.mark.parametrize("hd,pl", [(64, 16), (128, 16), (256, 16), (80, 8), (128, 32), (96, 64)])
def test_gather_scatter_round_trip(torch_cuda, hd, pl):
    """Gather and scatter over ranges that cut a page at both ends and cover
    whole pages between (the whole pages take the register-transpose path,
    the cut ones the LDS path); head_dim 80 and 96 end K in a group narrower
    than 32 dims, head_dim 64 at page 16 and 80 at page 8 put several KV
    heads in one workgroup."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    say("gather/scatter", hd, pl)
    rng = random.Random(hd * 1000 + pl)
    lens = [6 * pl + 4, 3 * pl + 4]
    pool = make_pool(lens, kv_heads=2, head_dim=hd, page_len=pl, kv_dtype="f16", layers=2, extra_pages=4)
    scattered_alloc(pool, lens, rng, pl)
    rows = RowMeta(128)
    fill(torch, pool, rows, lens, layer=1, seed=3)
    ref = oracle_layer(torch, pool, layer=1)
    g0, gn = pl + 3, 4 * pl + 4  # pages 1 (cut), 2..4 (whole), 5 (cut)
    kd = torch.empty(2, gn, hd, dtype=torch.int16, device="cuda")
    vd = torch.empty_like(kd)
    ops.kv_gather(pool, 1, 0, g0, gn, kd, vd)
    torch.cuda.synchronize()
    rk, rv = ref.gather(0, g0, gn)
    assert np.array_equal(kd.cpu().numpy().view(np.uint16), rk)
    assert np.array_equal(vd.cpu().numpy().view(np.uint16), rv)
    # scatter new words into seq 1 tokens [5, 2 pl + 8): pages 0 (cut), 1 (whole), 2 (cut)
    s0, sn = 5, 2 * pl + 3
    nk = torch.randint(-30000, 30000, (2, sn, hd), dtype=torch.int16, device="cuda")
    nv = torch.randint(-30000, 30000, (2, sn, hd), dtype=torch.int16, device="cuda")
    ops.kv_scatter(pool, 1, 1, s0, sn, nk, nv)
    k2 = torch.empty(2, sn, hd, dtype=torch.int16, device="cuda")
    v2 = torch.empty_like(k2)
    ops.kv_gather(pool, 1, 1, s0, sn, k2, v2)
    torch.cuda.synchronize()
    assert torch.equal(k2, nk) and torch.equal(v2, nv)
    # the scatter left every other token of the layer as it was
    after = oracle_layer(torch, pool, layer=1)
    table = pool.arena.table_of(1)
    slots = [table[t // pl] * pl + t % pl for t in range(s0, s0 + sn)]
    ref.k[:, slots, :] = nk.cpu().numpy().view(np.uint16)
    ref.v[:, slots, :] = nv.cpu().numpy().view(np.uint16)
    assert np.array_equal(after.k, ref.k) and np.array_equal(after.v, ref.v)
    # layer 0 untouched by layer-1 traffic
    k0, _ = pool.layer_tensors(0)
    assert int(k0.abs().sum()) == 0


def test_block_copy_and_fork_copy_on_write(torch_cuda):
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    say("block copy / fork")
    rng = random.Random(5)
    lens = [90, 0, 0]
    pool = make_pool(lens, kv_heads=2, head_dim=128, page_len=16, kv_dtype="bf16", layers=3, extra_pages=20,
                     seq_lens=[200, 200, 200])
    scattered_alloc(pool, [90], rng, 16)
    rows = RowMeta(128)
    for layer in range(3):
        fill(torch, pool, rows, [90], layer=layer, seed=layer)
    before = [oracle_layer(torch, pool, layer) for layer in range(3)]
    pool.fork(0, 1, 90)  # 5 full pages shared, page 5 (10 tokens) copied
    t0, t1 = pool.arena.table_of(0), pool.arena.table_of(1)
    assert t1[:5] == t0[:5] and t1[5] != t0[5]
    pool.sync()
    for layer in range(3):
        after = oracle_layer(torch, pool, layer)
        want = before[layer]
        want.block_copy([[t0[5], t1[5], 10]])
        assert np.array_equal(after.k, want.k) and np.array_equal(after.v, want.v)
        ka, va = after.gather(0, 0, 90)
        kb, vb = after.gather(1, 0, 90)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # explicit block copy: page of seq 0 -> a free page, all layers
    free_page = [p for p in range(pool.arena.pages()) if p not in t0 + t1][0]
    ops.block_copy(pool, [[t0[1], free_page, 16]])
    pool.sync()
    for layer in range(3):
        after = oracle_layer(torch, pool, layer)
        assert np.array_equal(after.k[:, free_page * 16:(free_page + 1) * 16], after.k[:, t0[1] * 16:(t0[1] + 1) * 16])


def test_kv_store_errors(torch_cuda):
    torch = torch_cuda
    from flint_amd import ThubanError, ops
    from flint_amd.pool import RowMeta

    pool = make_pool([40], kv_heads=2, head_dim=64, page_len=16)
    pool.alloc(0, 0, 16)
    rows = RowMeta(4)
    rows.write([20], [0], 1)
    k = torch.zeros(1, 2, 64, device="cuda")
    with pytest.raises(ThubanError) as e:
        ops.kv_store(k, k, pool, 0, 1, rows)
    assert "pages must cover" in str(e.value) and e.value.kind == "Model"
    rows.write([3], [0], 1)
    ops.kv_store(k, k, pool, 0, 0, rows)  # m == 0 is a no-op
    with pytest.raises(ThubanError):
        ops.kv_store(k, k, pool, 1, 1, rows)  # no layer 1
    torch.cuda.synchronize()


@pytest.mark.parametrize("page_len,hd", [(16, 128), (32, 64), (8, 256)])
def test_page_layout_matches_header(torch_cuda, page_len, hd):
    """Words written in the reference layout [kv_heads, pool_len, head_dim]
    through KvPool.write_layer come back unchanged through read_layer and,
    token by token, through the gather kernel (which addresses the device
    page layout documented in include/thuban_hip.h)."""
    torch = torch_cuda
    from flint_amd import ops

    say("page layout", page_len, hd)
    rng = np.random.default_rng(page_len * hd)
    lens = [3 * page_len + 5, 2 * page_len]
    pool = make_pool(lens, kv_heads=3, head_dim=hd, page_len=page_len, kv_dtype="f16", extra_pages=2)
    scattered_alloc(pool, lens, random.Random(7), page_len)
    info = pool.layer_info(0)
    k = rng.integers(0, 1 << 16, size=(3, info.pool_len, hd), dtype=np.uint16)
    v = rng.integers(0, 1 << 16, size=(3, info.pool_len, hd), dtype=np.uint16)
    pool.write_layer(0, k, v)
    k2, v2 = pool.read_layer(0)
    assert np.array_equal(k2, k) and np.array_equal(v2, v)
    ref = oracle.Layer(3, hd, pool.arena.pages(), page_len, np.array(pool.arena.table(), np.uint32),
                       pool.arena.max_pages(), oracle.KV_F16, k=k, v=v)
    for s, n in enumerate(lens):
        kd = torch.empty(3, n, hd, dtype=torch.int16, device="cuda")
        vd = torch.empty_like(kd)
        ops.kv_gather(pool, 0, s, 0, n, kd, vd)
        torch.cuda.synchronize()
        rk, rv = ref.gather(s, 0, n)
        assert np.array_equal(kd.cpu().numpy().view(np.uint16), rk)
        assert np.array_equal(vd.cpu().numpy().view(np.uint16), rv)


@pytest.mark.parametrize("page_len,hd,src", [(16, 128, "f16"), (8, 64, "f32"), (32, 256, "bf16"),
                                             (64, 512, "f32"), (16, 80, "f16")])
@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_kv_store_prefill_runs_bit_exact(torch_cuda, page_len, hd, src, kv):
    """Prefill-like appends (consecutive positions of one sequence, starting
    mid-page, several sequences interleaved in one call, plus a few decode
    rows) take the run kernel; the pool must equal the oracle's appends."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta

    say("kv_store runs", page_len, hd, src, kv)
    lens = [300, 137, 90]
    pool = make_pool(lens, kv_heads=3, head_dim=hd, page_len=page_len, kv_dtype=kv, extra_pages=2)
    scattered_alloc(pool, lens, random.Random(page_len + hd), page_len)
    ref = oracle_layer(torch, pool)
    rows = RowMeta(512)
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[src]
    g = torch.Generator(device="cuda")
    g.manual_seed(hd)
    # call 1: seq 0 tokens [5, 205) + seq 1 tokens [3, 100) + decode rows of seq 2
    # call 2: the rest of every sequence
    calls = [[(0, p) for p in range(5, 205)] + [(1, p) for p in range(3, 100)] + [(2, 7), (2, 8)],
             [(0, p) for p in list(range(0, 5)) + list(range(205, 300))] + [(1, p) for p in list(range(0, 3)) +
                                                                             list(range(100, 137))] +
             [(2, p) for p in range(90) if p not in (7, 8)]]
    for chunk in calls:
        m = len(chunk)
        pos, seqs = [p for _, p in chunk], [s for s, _ in chunk]
        rows.write(pos, seqs, m)
        k = (torch.randn(m, 3, hd, device="cuda", generator=g) * 3).to(dt)
        v = (torch.randn(m, 3, hd, device="cuda", generator=g) * 100).to(dt)
        ops.kv_store(k, v, pool, 0, m, rows)
        ref.kv_store(_src_words(torch, k), _src_words(torch, v), oracle.row_meta(pos, seqs), m, SRC[src])
    got = oracle_layer(torch, pool)
    assert np.array_equal(got.k, ref.k)
    assert np.array_equal(got.v, ref.v)


@pytest.mark.parametrize("page_len,hd", [(8, 64), (16, 128), (32, 80), (64, 512), (256, 128)])
def test_gather_scatter_unaligned_ranges_bit_exact(torch_cuda, page_len, hd):
    """Gather and scatter over ranges that start and end inside pages and
    inside 8-token groups of the transposed V page.  Gather matches the
    oracle; after a scatter the whole layer equals the closed form (the
    range replaced, every other slot, including the rest of a cut group,
    unchanged)."""
    torch = torch_cuda
    from flint_amd import ops

    say("gather/scatter unaligned", page_len, hd)
    P = page_len
    lens = [4 * P + 3, 2 * P + 1]
    pool = make_pool(lens, kv_heads=2, head_dim=hd, page_len=P, kv_dtype="f16", extra_pages=3)
    scattered_alloc(pool, lens, random.Random(P + hd), P)
    info = pool.layer_info(0)
    rng = np.random.default_rng(P * hd)
    k = rng.integers(0, 1 << 16, size=(2, info.pool_len, hd), dtype=np.uint16)
    v = rng.integers(0, 1 << 16, size=(2, info.pool_len, hd), dtype=np.uint16)
    pool.write_layer(0, k, v)
    ranges = [(0, 0, lens[0]), (0, 3, P), (0, P - 1, 2), (0, 5, 2 * P + 3), (1, P + 1, P), (1, 2 * P, 1),
              (0, 1, 6), (1, 0, lens[1])]
    for seq, t0, n in ranges:
        table = pool.arena.table_of(seq)
        ref = oracle.Layer(2, hd, pool.arena.pages(), P, np.array(pool.arena.table(), np.uint32),
                           pool.arena.max_pages(), oracle.KV_F16, k=k, v=v)
        kd = torch.empty(2, n, hd, dtype=torch.int16, device="cuda")
        vd = torch.empty_like(kd)
        ops.kv_gather(pool, 0, seq, t0, n, kd, vd)
        torch.cuda.synchronize()
        rk, rv = ref.gather(seq, t0, n)
        assert np.array_equal(kd.cpu().numpy().view(np.uint16), rk), (seq, t0, n)
        assert np.array_equal(vd.cpu().numpy().view(np.uint16), rv), (seq, t0, n)
        nk = rng.integers(0, 1 << 16, size=(2, n, hd), dtype=np.uint16)
        nv = rng.integers(0, 1 << 16, size=(2, n, hd), dtype=np.uint16)
        ops.kv_scatter(pool, 0, seq, t0, n, torch.from_numpy(nk.view(np.int16)).cuda(),
                       torch.from_numpy(nv.view(np.int16)).cuda())
        torch.cuda.synchronize()
        slots = [table[t // P] * P + t % P for t in range(t0, t0 + n)]
        k[:, slots] = nk
        v[:, slots] = nv
        k2, v2 = pool.read_layer(0)
        assert np.array_equal(k2, k) and np.array_equal(v2, v), (seq, t0, n)


@pytest.mark.parametrize("page_len", [8, 16, 64])
def test_block_copy_partial_pages_bit_exact(torch_cuda, page_len):
    """Block copies of 1 .. page_len tokens (cutting 8-token V groups) in a
    pool whose layers have different head dims; every layer matches the
    oracle's copy of slots [0, tokens)."""
    torch = torch_cuda
    from flint_amd import ops

    say("block copy partial", page_len)
    P = page_len
    hds = [64, 80, 128]
    pool = make_pool([P * 8], kv_heads=3, head_dim=128, page_len=P, kv_dtype="bf16", layers=3, extra_pages=8,
                     head_dims=hds)
    rng = np.random.default_rng(P)
    want = []
    for layer, hd in enumerate(hds):
        info = pool.layer_info(layer)
        k = rng.integers(0, 1 << 16, size=(3, info.pool_len, hd), dtype=np.uint16)
        v = rng.integers(0, 1 << 16, size=(3, info.pool_len, hd), dtype=np.uint16)
        pool.write_layer(layer, k, v)
        want.append(oracle.Layer(3, hd, pool.arena.pages(), P, np.array(pool.arena.table(), np.uint32),
                                 pool.arena.max_pages(), oracle.KV_BF16, k=k, v=v))
    counts = sorted({1, 7, 8, 9, P - 1, P} & set(range(1, P + 1)))
    pages = list(range(pool.arena.pages()))
    random.Random(P).shuffle(pages)
    triples = [[pages[2 * i], pages[2 * i + 1], c] for i, c in enumerate(counts)]
    ops.block_copy(pool, triples)
    torch.cuda.synchronize()
    for layer in range(3):
        want[layer].block_copy(triples)
        k2, v2 = pool.read_layer(layer)
        assert np.array_equal(k2, want[layer].k) and np.array_equal(v2, want[layer].v), layer


@pytest.mark.parametrize("page_len,hd", [(16, 128), (8, 64), (32, 80)])
def test_batched_gather_and_scatter(torch_cuda, page_len, hd):
    """thb_kv_gather_batch over ranges of several sequences and layers (whole
    pages and ranges cut at both ends, one empty range) equals the oracle's
    gathers laid back to back; thb_kv_scatter_batch writes them back so the
    pool is unchanged, and new words land exactly in the scattered ranges.
    Overlapping scatter ranges and pages shared with a fork are refused."""
    torch = torch_cuda
    from flint_amd import ThubanError, ops

    say("batched gather", page_len, hd)
    rng = np.random.default_rng(7 * page_len + hd)
    lens = [5 * page_len + 3, 2 * page_len, 7 * page_len - 1, 40]
    pool = make_pool(lens, kv_heads=2, head_dim=hd, page_len=page_len, kv_dtype="f16", layers=2, extra_pages=8)
    scattered_alloc(pool, lens, random.Random(page_len), page_len)
    info = pool.layer_info(0)
    refs = []
    for layer in range(2):
        k = rng.integers(0, 1 << 16, size=(2, info.pool_len, hd), dtype=np.uint16)
        v = rng.integers(0, 1 << 16, size=(2, info.pool_len, hd), dtype=np.uint16)
        pool.write_layer(layer, k, v)
        refs.append(oracle.Layer(2, hd, pool.arena.pages(), page_len, np.array(pool.arena.table(), np.uint32),
                                 pool.arena.max_pages(), oracle.KV_F16, k=k, v=v))
    ranges = [(0, 0, 0, lens[0]), (2, 1, 3, lens[2] - 5), (1, 1, page_len - 2, 5), (3, 0, 7, 0), (3, 1, 0, 40),
              (2, 0, page_len, page_len)]
    total = sum(n for *_, n in ranges) * 2 * hd
    kd = torch.empty(total, dtype=torch.int16, device="cuda")
    vd = torch.empty_like(kd)
    ops.kv_gather_batch(pool, ranges, kd, vd)
    torch.cuda.synchronize()
    kh, vh = kd.cpu().numpy().view(np.uint16), vd.cpu().numpy().view(np.uint16)
    off = 0
    for seq, layer, t0, n in ranges:
        rk, rv = refs[layer].gather(seq, t0, n)
        assert np.array_equal(kh[off:off + rk.size].reshape(rk.shape), rk), (seq, layer, t0, n)
        assert np.array_equal(vh[off:off + rv.size].reshape(rv.shape), rv), (seq, layer, t0, n)
        off += rk.size
    # scatter new words into the ranges (the empty and the overlapping-free set)
    new_k = torch.from_numpy(rng.integers(0, 1 << 16, size=total, dtype=np.uint16).view(np.int16)).cuda()
    new_v = torch.from_numpy(rng.integers(0, 1 << 16, size=total, dtype=np.uint16).view(np.int16)).cuda()
    ops.kv_scatter_batch(pool, ranges, new_k, new_v)
    k2 = torch.empty_like(kd)
    v2 = torch.empty_like(vd)
    ops.kv_gather_batch(pool, ranges, k2, v2)
    torch.cuda.synchronize()
    assert torch.equal(k2, new_k) and torch.equal(v2, new_v)
    # tokens outside the ranges are untouched: seq 1 token 0 of layer 1
    k1 = torch.empty(2, 1, hd, dtype=torch.int16, device="cuda")
    v1 = torch.empty_like(k1)
    ops.kv_gather(pool, 1, 1, 0, 1, k1, v1)
    torch.cuda.synchronize()
    assert np.array_equal(k1.cpu().numpy().view(np.uint16), refs[1].gather(1, 0, 1)[0])
    with pytest.raises(ThubanError) as e:
        ops.kv_scatter_batch(pool, [(0, 0, 0, 10), (0, 0, 5, 10)], new_k, new_v)
    assert "overlap" in str(e.value)
