"""GPU parity of the rotary path: ops::rope / norm_rope (thb_rope_rows),
the rotary append (thb_kv_store_rope) and rope fused into attention
(thb_attn_rope, thb_attn_append_rope), against the CPU oracle.  Rotation
and append are bit-exact; attention within 2e-3 of the exact softmax over
the oracle's rotated queries and keys."""

import math
import random
import zlib

import numpy as np
import pytest

import oracle
from gpu_util import fill, make_pool, oracle_layer, say, scattered_alloc

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _tables(max_pos, rot, theta=1e6):
    from flint_amd.rope import rope_tables

    return rope_tables(max_pos, rot, rot, theta)


def _rope(torch, hd, rot, norm, max_pos=20000, seed=0):
    from flint_amd.rope import Rope

    cos, sin = _tables(max_pos, rot)
    rng = np.random.default_rng(seed)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    return Rope(cos, sin, rot, q_norm=qn, k_norm=kn, eps=1e-6), cos, sin, qn, kn


def _oracle_rope(x, pos, rot, cos, sin, w):
    """x: torch tensor [m, heads, hd] (f32 or f16) -> numpy after the oracle rope."""
    return oracle.rope_rows(x.cpu().numpy(), pos, rot, cos, sin, w=w)


ROWS_CASES = [
    # name, heads, hd, rot, dtype, norm
    ("llama-f32", 32, 128, 128, "f32", False),
    ("partial-f16", 8, 128, 64, "f16", False),
    ("qwen3-norm-f32", 8, 128, 128, "f32", True),
    ("hd80-norm-f16", 5, 80, 80, "f16", True),
    ("hd512-norm-partial", 2, 512, 128, "f32", True),
]


@pytest.mark.parametrize("case", ROWS_CASES, ids=[c[0] for c in ROWS_CASES])
def test_rope_rows_bit_exact(torch_cuda, case):
    torch = torch_cuda
    from flint_amd.pool import RowMeta
    from flint_amd.rope import rope_rows

    name, heads, hd, rot, dt, norm = case
    say("rope rows", name)
    rope, cos, sin, qn, _ = _rope(torch, hd, rot, norm, seed=zlib.crc32(name.encode()))
    m = 37
    pos = [int(p) for p in np.random.default_rng(1).integers(0, rope.max_pos, m)]
    rows = RowMeta(64)
    rows.write(pos, [0] * m, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    x = (torch.randn(m, heads, hd, device="cuda", generator=g) * 2).to(torch.float16 if dt == "f16" else torch.float32)
    want = _oracle_rope(x, pos, rot, cos, sin, qn)
    rope_rows(x, heads, rope, rows, m, norm_w=rope.q_norm if norm else None)
    torch.cuda.synchronize()
    got = x.cpu().numpy()
    assert np.array_equal(got.view(np.uint16 if dt == "f16" else np.uint32),
                          want.view(np.uint16 if dt == "f16" else np.uint32)), name


def _append_oracle(torch, pool, layer, k, v, pos, seqs, rot, cos, sin, kn):
    """The oracle's expectation of a rotary append: rope(k) in the source
    type, then kv_store."""
    ref = oracle_layer(torch, pool, layer)
    kr = _oracle_rope(k, pos, rot, cos, sin, kn)
    src = oracle.SRC_F16 if k.dtype == torch.float16 else oracle.SRC_F32
    kw = kr.view(np.uint16) if src == oracle.SRC_F16 else kr
    vw = v.cpu().numpy()
    vw = vw.view(np.uint16) if src == oracle.SRC_F16 else vw
    ref.kv_store(np.ascontiguousarray(kw), np.ascontiguousarray(vw), oracle.row_meta(pos, seqs), len(pos), src)
    return ref


APPEND_CASES = [
    # name, nkv, hd, rot, src, kv, norm, shape ("decode" | "prefill")
    ("decode-f32-f16", 8, 128, 128, "f32", "f16", False, "decode"),
    ("decode-f16-bf16-norm", 8, 128, 128, "f16", "bf16", True, "decode"),
    ("prefill-f32-f16-norm", 4, 128, 64, "f32", "f16", True, "prefill"),
    ("prefill-f16-f16", 2, 256, 256, "f16", "f16", False, "prefill"),
    ("decode-hd80-bf16", 2, 80, 48, "f32", "bf16", True, "decode"),
]


@pytest.mark.parametrize("case", APPEND_CASES, ids=[c[0] for c in APPEND_CASES])
def test_kv_store_rope_bit_exact(torch_cuda, case):
    torch = torch_cuda
    from flint_amd.pool import RowMeta
    from flint_amd.rope import kv_store_rope

    name, nkv, hd, rot, src, kv, norm, shape = case
    say("rotary append", name)
    rope, cos, sin, _, kn = _rope(torch, hd, rot, norm, seed=zlib.crc32(name.encode()))
    if shape == "decode":
        lens = [300, 17, 1000, 64]
        pos = [n - 1 for n in lens]
        seqs = list(range(len(lens)))
    else:
        lens = [5 + 200, 90]
        pos = list(range(5, 205)) + list(range(0, 90))
        seqs = [0] * 200 + [1] * 90
    pool = make_pool(lens, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=2)
    scattered_alloc(pool, lens, random.Random(3), 16)
    m = len(pos)
    rows = RowMeta(m)
    rows.write(pos, seqs, m)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    dt = torch.float16 if src == "f16" else torch.float32
    k = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    v = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    want = _append_oracle(torch, pool, 0, k, v, pos, seqs, rot, cos, sin, kn)
    kv_store_rope(k, v, pool, 0, m, rows, rope)
    torch.cuda.synchronize()
    gk, gv = pool.read_layer(0)
    assert np.array_equal(gk, want.k) and np.array_equal(gv, want.v), name


FUSED_CASES = [
    # name, nq, nkv, hd, rot, src, kv, norm, rows per seq
    ("llama-decode", 32, 8, 128, 128, "f16", "f16", False, 1),
    ("qwen3-decode-norm", 32, 8, 128, 128, "f32", "f16", True, 1),
    ("verify4-partial-bf16", 16, 8, 128, 64, "f16", "bf16", True, 4),
    ("gemma-hd256", 16, 8, 256, 256, "f32", "f16", False, 1),
    # 32 query heads per KV head: each row's two query groups run in two
    # workgroups, and both rotate and store the row's key (the same bytes)
    ("mqa32-two-groups-norm", 32, 1, 128, 128, "f16", "f16", True, 1),
    ("prefill-fallback", 8, 2, 128, 128, "f32", "f16", True, 40),
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=[c[0] for c in FUSED_CASES])
def test_attn_append_rope(torch_cuda, case):
    """kv_store_attn_rope (one launch where it fuses) == kv_store_rope then
    attn_rope, bit for bit (outputs and pool); the pool equals the oracle's
    rotary append and the output the exact softmax over rotated queries."""
    torch = torch_cuda
    from flint_amd import ops
    from flint_amd.pool import RowMeta
    from flint_amd.rope import attn_rope, kv_store_attn_rope, kv_store_rope

    name, nq, nkv, hd, rot, src, kv, norm, rps = case
    say("rope fused", name)
    rope, cos, sin, qn, kn = _rope(torch, hd, rot, norm, seed=zlib.crc32(name.encode()))
    lens = [700, 1500, 33]
    budget = [n + rps for n in lens]
    pools = []
    for _ in range(2):
        P = make_pool(budget, kv_heads=nkv, head_dim=hd, page_len=16, kv_dtype=kv, extra_pages=3)
        scattered_alloc(P, budget, random.Random(zlib.crc32(name.encode())), 16)
        pools.append(P)
    rows = RowMeta(256)
    for P in pools:
        fill(torch, P, rows, lens, seed=7)
    positions, seqs = [], []
    for s, n in enumerate(lens):
        positions += list(range(n, n + rps))
        seqs += [s] * rps
    m = len(seqs)
    dt = torch.float16 if src == "f16" else torch.float32
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    k_new = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    v_new = torch.randn(m, nkv, hd, device="cuda", generator=g).to(dt)
    q = torch.randn(m, nq, hd, device="cuda", generator=g)
    rows.write(positions, seqs, m)
    want_pool = _append_oracle(torch, pools[0], 0, k_new, v_new, positions, seqs, rot, cos, sin, kn)
    spec = ops.AttnSpec(q_heads=nq, window=0, scale=1 / math.sqrt(hd), m=m, causal=True, seq=None, args=rows)
    ya, yb = torch.empty_like(q), torch.empty_like(q)
    kv_store_rope(k_new, v_new, pools[0], 0, m, rows, rope)
    attn_rope(q, pools[0], 0, ya, spec, rope)
    kv_store_attn_rope(k_new, v_new, q, pools[1], 0, yb, spec, rope)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb), name
    ka, va = pools[0].read_layer(0)
    kb, vb = pools[1].read_layer(0)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb), name
    assert np.array_equal(kb, want_pool.k) and np.array_equal(vb, want_pool.v), name
    qr = _oracle_rope(q, positions, rot, cos, sin, qn)
    want = want_pool.attn(qr, oracle.row_meta(positions, seqs), m, nq, 1 / math.sqrt(hd))
    err = float(np.max(np.abs(yb.cpu().numpy() - want)))
    say("rope fused", name, "max abs err", err)
    assert err <= TOL


def test_rope_errors(torch_cuda):
    torch = torch_cuda
    from flint_amd import ThubanError
    from flint_amd.pool import RowMeta
    from flint_amd.rope import Rope, kv_store_rope, rope_rows

    pool = make_pool([40], kv_heads=2, head_dim=64, page_len=16)
    pool.alloc(0, 0, 40)
    rows = RowMeta(4)
    rows.write([20], [0], 1)
    k = torch.zeros(1, 2, 64, device="cuda")
    cos, sin = _tables(32, 64)
    bad_rot = Rope(cos[:, :12], sin[:, :12], 24)
    with pytest.raises(ThubanError) as e:
        kv_store_rope(k, k, pool, 0, 1, rows, bad_rot)
    assert e.value.kind == "Config" and "multiple of 16" in str(e.value)
    short = Rope(cos[:16], sin[:16], 64)
    with pytest.raises(ThubanError) as e:
        rope_rows(k, 2, short, rows, 1)  # position 20 >= 16 table rows
    assert e.value.kind == "Model" and "outside the rope tables" in str(e.value)
    with pytest.raises(ThubanError):
        kv_store_rope(k.to(torch.bfloat16), k.to(torch.bfloat16), pool, 0, 1, rows, Rope(cos, sin, 64))
    torch.cuda.synchronize()
