"""Writes the golden fixtures in this folder from the reference's own tests.

The reference (formetaohy/Flint, Rust) cannot be built here (no cargo), so
the fixtures are its test literals, transcribed with file:line citations, and
the inputs its tests generate with their deterministic LCG.  Floats are stored
as IEEE-754 bit patterns so that NaN, infinities and -0.0 survive JSON.

Run:  python tests/golden/make_golden.py   (rewrites the *.json files here)
"""

from __future__ import annotations

import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
U32_MAX = 0xFFFFFFFF


def fbits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ---------------------------------------------------------------- codecs
def codec_cases():
    """crates/thuban_num/src/lib.rs:78-139."""
    inf = float("inf")
    f16_to_f32 = [  # lib.rs:79-88
        (0x0000, 0.0), (0x8000, -0.0), (0x3C00, 1.0), (0xBC00, -1.0), (0x7BFF, 65504.0),
        (0x7C00, inf), (0xFC00, -inf), (0x0001, 2.0 ** -24),
    ]
    f32_to_f16 = [  # lib.rs:91-125
        (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-1.0, 0xBC00), (1.5, 0x3E00), (2.0, 0x4000),
        (-2.0, 0xC000), (0.5, 0x3800), (65504.0, 0x7BFF),
        (1.0 + 2.0 ** -11, 0x3C00), (1.0 + 2.0 ** -10, 0x3C01), (0.1, 0x2E66),
        (65520.0, 0x7C00), (1e30, 0x7C00), (-1e30, 0xFC00), (inf, 0x7C00),
        (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000), (-(2.0 ** -24), 0x8001), (1.5 * 2.0 ** -24, 0x0002),
    ]
    f32_to_f16_bits = [[fbits(v), h] for v, h in f32_to_f16]
    f32_to_f16_bits.append([0x7FC00000, 0x7E00])  # f32::NAN -> 0x7E00, lib.rs:116
    return {
        "cite": "crates/thuban_num/src/lib.rs:78-139",
        "f16_to_f32": [[h, fbits(v)] for h, v in f16_to_f32],
        "f32_to_f16": f32_to_f16_bits,
        "f16_round_trip": [fbits(v) for v in (0.0, 1.0, -1.0, 0.5, 65504.0, 1.5, 2.0, -2.0)],  # :128-132
        "bf16_round_trip": [fbits(v) for v in (0.0, 1.0, -1.0, 1.5, 123.0, -0.25, 65536.0)],  # :135-139
    }


# ------------------------------------------------------------------ arena
def arena_cases():
    """crates/thuban_model/tests/pool.rs:3-109 (page length 32)."""
    return [
        {"name": "alloc_grows_and_reuses_pages", "cite": "tests/pool.rs:3-26",
         "seq_lens": [64, 64], "pages": None, "steps": [
             {"expect": {"pages": 4, "used": 0}},
             {"op": "alloc", "args": [0, 0, 40]},
             {"expect": {"used": 2, "table_of": [0, [0, 1]]}},
             {"op": "alloc", "args": [0, 40, 24]},
             {"expect": {"used": 2, "table_len": [0, 2]}},
             {"op": "free_seq", "args": [0]},
             {"expect": {"used": 0}},
             {"op": "alloc", "args": [1, 0, 64]},
             {"expect": {"used": 2, "table_len": [1, 2]}}]},
        {"name": "truncate_keeps_prefix_and_frees_tail", "cite": "tests/pool.rs:28-45",
         "seq_lens": [128], "pages": None, "steps": [
             {"op": "alloc", "args": [0, 0, 128]},
             {"expect": {"table_len": [0, 4]}},
             {"op": "truncate", "args": [0, 70]},
             {"expect": {"table_len": [0, 3], "used": 3}},
             {"op": "alloc", "args": [0, 70, 30]},
             {"expect": {"table_len": [0, 4], "used": 4}}]},
        {"name": "free_seq_returns_every_page", "cite": "tests/pool.rs:47-62",
         "seq_lens": [96, 96], "pages": 3, "steps": [
             {"op": "alloc", "args": [0, 0, 96]},
             {"expect": {"used": 3}},
             {"op": "alloc", "args": [1, 0, 32], "error": ""},
             {"op": "free_seq", "args": [0]},
             {"op": "alloc", "args": [1, 0, 96]},
             {"expect": {"table_len": [1, 3], "used": 3}}]},
        {"name": "exhaustion_fails_fast", "cite": "tests/pool.rs:64-74",
         "seq_lens": [128], "pages": 2, "steps": [
             {"op": "alloc", "args": [0, 0, 128], "error": ""},
             {"op": "alloc", "args": [0, 0, 64]},
             {"expect": {"used": 2}}]},
        {"name": "context_limit_is_enforced", "cite": "tests/pool.rs:76-86",
         "seq_lens": [32], "pages": None, "steps": [
             {"op": "alloc", "args": [0, 0, 32]},
             {"op": "alloc", "args": [0, 32, 1], "error": "context limit 32"}]},
        {"name": "table_flattens_with_sentinels", "cite": "tests/pool.rs:88-109",
         "seq_lens": [32, 64], "pages": 4, "steps": [
             {"op": "alloc", "args": [1, 0, 40]},
             {"expect": {"table_size": 4, "table_eq": [[0, U32_MAX], [1, U32_MAX]],
                         "table_ne": [[2, U32_MAX], [3, U32_MAX]]}},
             {"op": "alloc", "args": [0, 0, 32]},
             {"expect": {"table_ne": [[0, U32_MAX]], "table_ne_idx": [[0, 2]]}}]},
    ]


# ---------------------------------------------------------------- kv_store
class Rng:
    """The reference tests' LCG: crates/thuban_backend/tests/kernels.rs:112-124."""

    def __init__(self, seed: int):
        self.state = seed

    def next(self) -> np.float32:
        self.state = (self.state * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        x = np.float32(self.state >> 33)
        return np.float32(np.float32(x / np.float32(2.0 ** 31)) * np.float32(2.0)) - np.float32(1.0)

    def fill(self, n: int):
        return [self.next() for _ in range(n)]


def cpu_ref_kv_store(src, cache, m, kv_heads, hd, max_seq, pos):
    """crates/thuban_backend/tests/support/cpu_ref.rs:154-170 (contiguous
    cache, value rounded to bf16 by truncation)."""
    for mi in range(m):
        for h in range(kv_heads):
            for d in range(hd):
                b = fbits(float(src[(mi * kv_heads + h) * hd + d])) >> 16
                cache[(h * max_seq + pos + mi) * hd + d] = b


def kv_store_cases():
    cases = []
    # anchor_layout_ops: kernels.rs:1396-1407
    cache = [0] * 8
    src = [1.0, 2.0, 3.0, 4.0]
    expect_vals = [0.0, 0.0, 1.0, 2.0, 3.0, 4.0, 0.0, 0.0]
    cases.append({"name": "anchor_layout_ops", "cite": "crates/thuban_backend/tests/kernels.rs:1404-1406",
                  "m": 2, "kv_heads": 1, "head_dim": 2, "max_seq": 4, "pos": 1,
                  "k_src": [fbits(x) for x in src], "v_src": [fbits(x) for x in src],
                  "expect_k": [fbits(x) >> 16 for x in expect_vals],
                  "expect_v": [fbits(x) >> 16 for x in expect_vals]})
    # kv_store_writes_both_caches: kernels.rs:1266-1308
    m, nkv, hd, max_seq, pos = 3, 2, 4, 8, 3
    rng = Rng(111)
    k_src = rng.fill(m * nkv * hd)
    v_src = rng.fill(m * nkv * hd)
    ck = [0] * (nkv * max_seq * hd)
    cv = [0] * (nkv * max_seq * hd)
    cpu_ref_kv_store(k_src, ck, m, nkv, hd, max_seq, pos)
    cpu_ref_kv_store(v_src, cv, m, nkv, hd, max_seq, pos)
    cases.append({"name": "kv_store_writes_both_caches", "cite": "crates/thuban_backend/tests/kernels.rs:1266-1308",
                  "m": m, "kv_heads": nkv, "head_dim": hd, "max_seq": max_seq, "pos": pos,
                  "k_src": [fbits(float(x)) for x in k_src], "v_src": [fbits(float(x)) for x in v_src],
                  "expect_k": ck, "expect_v": cv})
    return cases


# -------------------------------------------------------------------- attn
def attn_cases():
    """anchor_attn_causal_and_window: kernels.rs:1439-1481 (K = I2,
    V = [[1,2],[3,4]], q = [1,1], pos = 1, hd = 2, scale 1/sqrt(2))."""
    base = {"cite": "crates/thuban_backend/tests/kernels.rs:1439-1481", "m": 1, "q_heads": 1, "kv_heads": 1,
            "head_dim": 2, "max_seq": 2, "pos": 1, "causal": True,
            "q": [1.0, 1.0], "k": [1.0, 0.0, 0.0, 1.0], "v": [1.0, 2.0, 3.0, 4.0], "tol": 1e-6}
    return [dict(base, name="full_causal", window=0, expect=[2.0, 3.0]),
            dict(base, name="window_1", window=1, expect=[3.0, 4.0])]


# -------------------------------------------------------------------- rope
def rope_cases():
    """rope_case (kernels.rs:1200-1253) at the two shapes the reference runs
    (kernels.rs:1255-1263): x from Rng(seed), theta 1e7 tables built in
    double and rounded to f32 as the test does, rows at positions pos + r.
    The expectation is the rotation evaluated in double precision on those
    f32 inputs (cpu_ref.rs:132-152 is the same formula in f32); the
    reference accepts |gpu - cpu| <= 1e-5 |cpu| + 1e-6.  Plus anchor_rope
    (kernels.rs:1410-1436), whose expectation is spelled out in the test."""
    cases = []
    for m, heads, hd, rot, pos, seed in [(2, 2, 32, 16, 2, 51), (1, 1, 32, 32, 0, 53)]:
        half = rot // 2
        max_seq = pos + m + 2
        x = np.array(Rng(seed).fill(m * heads * hd), np.float32)
        cos = np.empty((max_seq, half), np.float32)
        sin = np.empty((max_seq, half), np.float32)
        for p in range(max_seq):
            for i in range(half):
                a = p * (1.0 / 1e7 ** ((2 * i) / rot))
                cos[p, i], sin[p, i] = np.float32(np.cos(a)), np.float32(np.sin(a))
        xv = x.astype(np.float64).reshape(m, heads, hd)
        want = xv.copy()
        for r in range(m):
            c, s_ = cos[pos + r].astype(np.float64), sin[pos + r].astype(np.float64)
            lo, hi = xv[r, :, :half], xv[r, :, half:rot]
            want[r, :, :half] = lo * c - hi * s_
            want[r, :, half:rot] = hi * c + lo * s_
        cases.append({"cite": "crates/thuban_backend/tests/kernels.rs:1200-1263", "m": m, "heads": heads,
                      "head_dim": hd, "rot": rot, "pos": [pos + r for r in range(m)], "seed": seed,
                      "x": x.tolist(), "cos": cos.reshape(-1).tolist(), "sin": sin.reshape(-1).tolist(),
                      "expect": want.reshape(-1).tolist(), "rel": 1e-5, "abs": 1e-6})
    inv1 = 1.0 / 10000.0 ** (2.0 / 4.0)
    c0, s0 = np.float32(np.cos(1.0)), np.float32(np.sin(1.0))
    c1, s1 = np.float32(np.cos(inv1)), np.float32(np.sin(inv1))
    f = np.float32
    want = [f(1) * c0 - f(3) * s0, f(2) * c1 - f(4) * s1, f(3) * c0 + f(1) * s0, f(4) * c1 + f(2) * s1]
    cases.append({"cite": "crates/thuban_backend/tests/kernels.rs:1410-1436", "m": 1, "heads": 1, "head_dim": 4,
                  "rot": 4, "pos": [1], "x": [1.0, 2.0, 3.0, 4.0], "cos": [0.0, 0.0, float(c0), float(c1)],
                  "sin": [0.0, 0.0, float(s0), float(s1)], "expect": [float(w) for w in want], "rel": 0.0,
                  "abs": 1e-6})
    return cases


def main():
    out = {
        "rope_cases.json": rope_cases(),
        "codec_cases.json": codec_cases(),
        "arena_cases.json": arena_cases(),
        "kv_store_cases.json": kv_store_cases(),
        "attn_cases.json": attn_cases(),
    }
    for name, data in out.items():
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(data, f, indent=1)
            f.write("\n")
        print("wrote", name)


if __name__ == "__main__":
    main()
