"""Host side of the rotary path: flint_amd.rope.rope_tables (the
reference's ops/rope.rs:52-87) against the reference tests' own constants
and closed forms.  CPU only."""

import json
import math
import os

import numpy as np

from flint_amd.rope import RopeScaling, rope_tables

HERE = os.path.dirname(os.path.abspath(__file__))


def test_anchor_constants():
    """anchor_rope (kernels.rs:1410-1415) uses row 1 of theta 10000, rot 4:
    cos/sin of 1 and of 1 / 10000^(2/4)."""
    cos, sin = rope_tables(2, 4, 4, 10000.0)
    assert cos.shape == (2, 2) and cos.dtype == np.float32
    assert np.array_equal(cos[0], [1.0, 1.0]) and np.array_equal(sin[0], [0.0, 0.0])
    inv1 = 1.0 / 10000.0 ** (2.0 / 4.0)
    assert np.array_equal(cos[1], np.array([math.cos(1.0), math.cos(inv1)], np.float32))
    assert np.array_equal(sin[1], np.array([math.sin(1.0), math.sin(inv1)], np.float32))


def test_matches_reference_test_tables():
    """rope_case (kernels.rs:1203-1215) builds theta 1e7 tables by hand; the
    committed fixture holds them."""
    with open(os.path.join(HERE, "golden", "rope_cases.json")) as f:
        cases = json.load(f)
    for case in cases[:2]:
        rot, half = case["rot"], case["rot"] // 2
        want_c = np.array(case["cos"], np.float32).reshape(-1, half)
        want_s = np.array(case["sin"], np.float32).reshape(-1, half)
        cos, sin = rope_tables(want_c.shape[0], rot, rot, 1e7)
        assert np.allclose(cos, want_c, rtol=0, atol=1e-7) and np.allclose(sin, want_s, rtol=0, atol=1e-7)


def test_partial_and_scaling():
    """ops/rope.rs:66-76: frequencies i >= partial do not rotate; a scaling
    divides frequency i by short[i] below original_max and long[i] from it."""
    cos, sin = rope_tables(8, 16, 16, 10000.0, partial=3)
    assert np.all(cos[:, 3:] == 1.0) and np.all(sin[:, 3:] == 0.0)
    assert np.all(sin[1:, :3] != 0.0)
    sc = RopeScaling(short=[2.0] * 8, long=[4.0, 4.0], original_max=4)
    cos, sin = rope_tables(8, 16, 16, 10000.0, scaling=sc)
    inv = 1.0 / 10000.0 ** (2.0 * np.arange(8) / 16)
    for p in range(8):
        for i in range(8):
            f = 2.0 if p < 4 else (4.0 if i < 2 else None)
            a = p * (inv[i] / f if f else inv[i])
            assert abs(float(cos[p, i]) - math.cos(a)) < 1e-7 and abs(float(sin[p, i]) - math.sin(a)) < 1e-7
