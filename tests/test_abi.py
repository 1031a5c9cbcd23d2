"""The C-ABI library loads and exports every symbol the header declares.
CPU only: no compute entry point is called."""

import ctypes
import os
import random
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    with open(os.path.join(ROOT, "include", "thuban_hip.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(thb_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_are_exported():
    from flint_amd import _lib

    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    bound = {n for n, _, _ in _lib.SIGNATURES}
    assert set(names) == bound, set(names) ^ bound


def test_abi_version_and_struct_layouts(tmp_path):
    """The ctypes mirrors of the header's structs match what a C compiler
    lays out (size and every field offset)."""
    import subprocess

    from flint_amd import _lib

    assert _lib.lib().thb_abi_version() == _lib.ABI_VERSION == 8
    structs = {"thb_pool_desc": _lib.PoolDesc, "thb_attn_spec": _lib.AttnSpecC,
               "thb_layer_info": _lib.LayerInfo, "thb_arena_info": _lib.ArenaInfo, "thb_rope": _lib.RopeC,
               "thb_attn_io": _lib.AttnIoC}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "thuban_hip.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                              check=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(cls, fname).offset, (cname, fname)


def test_check_head_dim():
    """ops::check_head_dim (ops/attn.rs:83-90) exactly: any value in
    [64, 512]; the backend's own limit (multiples of 8) is a separate check."""
    from flint_amd import ThubanError, _lib, check_head_dim

    for hd in (64, 80, 100, 127, 128, 256, 512):
        check_head_dim(hd)
    for hd, msg in ((32, "head_dim 32 outside [64, 512]"), (63, "outside"), (513, "outside")):
        with pytest.raises(ThubanError) as e:
            check_head_dim(hd)
        assert msg in str(e.value)
        assert e.value.kind == "Config"
    L = _lib.lib()
    for hd in (64, 80, 128, 512):
        assert L.thb_backend_head_dim(hd) == 0
    for hd, msg in ((100, "multiple of 8"), (127, "multiple of 8"), (32, "outside [64, 512]")):
        assert L.thb_backend_head_dim(hd) == _lib.THB_ERR_CONFIG
        assert msg in L.thb_last_error().decode()


def test_product_does_not_reference_the_oracle():
    """The product package never imports or loads the oracle."""
    for base, _, files in os.walk(os.path.join(ROOT, "flint_amd")):
        for fn in files:
            if fn.endswith((".py", ".hip", ".cpp", ".hpp", ".h")) or fn == "Makefile":
                with open(os.path.join(base, fn)) as f:
                    src = f.read()
                assert "oracle" not in src.lower(), os.path.join(base, fn)


def test_page_offsets_match_the_kernels_layout(tmp_path):
    """KvPool.page_offsets (the host-side conversion used by read_layer /
    write_layer) and flint_amd/csrc/layout.hpp (what every kernel uses) give
    the same offset for every (slot, dim) at several page lengths and head
    dims, and each is a permutation of the page."""
    import subprocess

    import numpy as np

    from flint_amd.pool import KvPool

    shapes = [(8, 64), (16, 128), (16, 80), (32, 200), (64, 512)]
    src = tmp_path / "offsets.cpp"
    src.write_text('#include <cstdio>\n#include "layout.hpp"\nint main() {\n' + "".join(
        f"for (unsigned j = 0; j < {P}; j++) for (unsigned d = 0; d < {hd}; d++) "
        f'std::printf("%llu %llu\\n", (unsigned long long)thb::k_off(j, d, {hd}, {P.bit_length() - 1}), '
        f"(unsigned long long)thb::v_off(j, d, {hd}));\n" for P, hd in shapes) + "return 0; }\n")
    exe = tmp_path / "offsets"
    subprocess.run(["g++", "-std=c++17", "-D__host__=", "-D__device__=", "-I",
                    os.path.join(ROOT, "flint_amd", "csrc"), str(src), "-o", str(exe)], check=True)
    got = np.array([list(map(int, line.split())) for line in
                    subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()])
    i = 0
    for P, hd in shapes:
        k, v = KvPool.page_offsets(P, hd)
        n = P * hd
        assert np.array_equal(got[i:i + n, 0], k.reshape(-1)), (P, hd)
        assert np.array_equal(got[i:i + n, 1], v.reshape(-1)), (P, hd)
        assert np.array_equal(np.sort(k.reshape(-1)), np.arange(n)) and np.array_equal(np.sort(v.reshape(-1)), np.arange(n))
        i += n


def test_partition_rule(tmp_path):
    """thb::part_split (flint_amd/csrc/partition.hpp, what both planners use):
    known answers at part_len 4096 (a span a few keys over 2 or 32 pieces
    keeps 2 or 32; one key more than PL / 64 per piece goes to the next power
    of two; a span just over one piece keeps two), and for every span of a
    sweep: pieces are aligned, cover the span with no empty trailing piece, are
    at most part_len + part_len / 64 (rounded up to the alignment) long, never
    outnumber ceil(span / part_len) rounded up to a power of two, and at the
    longest part_len the pool accepts (1008 pages) fit the kernels' 1024 staged
    page numbers.  thb::part_split32 (the device planner's 32-bit form, for
    spans below 2^31) gives the same result on every such case."""
    import subprocess

    known = {  # span -> (n_parts, plen) at part_len 4096, align 16
        1: (1, 16), 4096: (1, 4096), 4099: (2, 2064), 8192: (2, 4096), 8196: (2, 4112), 8320: (2, 4160),
        8321: (4, 2096), 12288: (4, 3072), 20000: (8, 2512), 131072: (32, 4096), 131073: (32, 4112),
        131072 + 2048: (32, 4160), 131072 + 2049: (64, 2096),
    }
    cases = [(s, 4096, 16) for s in known]
    for pl, align in ((64, 16), (512, 32), (4096, 16), (4096, 256), (1008 * 16, 16), (1008 * 8, 16), (1008 * 256, 256)):
        for s in list(range(1, 3 * pl, max(1, pl // 61))) + [k * pl + d for k in range(2, 40) for d in (0, 1, pl // 64 * k,
                                                                                                      pl // 64 * k + 1)]:
            cases.append((s, pl, align))
    rng = random.Random(7)
    for _ in range(4000):
        cases.append((rng.randrange(1, 1 << 31), rng.randrange(1, 1009) * 16, 1 << rng.randrange(4, 9)))
    cases += [((1 << 31) - 1, 4096, 16), ((1 << 31) - 1, 16128, 256), ((1 << 31) - 5000, 16, 16)]
    src = tmp_path / "parts.cpp"
    src.write_text('#include <cstdio>\n#include "partition.hpp"\nint main() {\n'
                   f"static const unsigned long long c[][3] = {{{','.join(f'{{{s},{p},{a}}}' for s, p, a in cases)}}};\n"
                   "for (const auto& x : c) { uint32_t n, plen, n32, plen32;"
                   " thb::part_split(x[0], (uint32_t)x[1], (uint32_t)x[2], n, plen);"
                   " thb::part_split32((uint32_t)x[0], (uint32_t)x[1], (uint32_t)x[2], n32, plen32);"
                   ' std::printf("%u %u %u %u\\n", n, plen, n32, plen32); }\nreturn 0; }\n')
    exe = tmp_path / "parts"
    subprocess.run(["g++", "-std=c++17", "-O1", "-D__host__=", "-D__device__=", "-I",
                    os.path.join(ROOT, "flint_amd", "csrc"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    got = [(int(out[4 * i]), int(out[4 * i + 1])) for i in range(len(cases))]
    got32 = [(int(out[4 * i + 2]), int(out[4 * i + 3])) for i in range(len(cases))]
    assert got32 == got
    for s, np_ in zip(known, got):
        assert np_ == known[s], (s, np_)
    for (s, pl, align), (n, plen) in zip(cases, got):
        assert plen % align == 0 and (n - 1) * plen < s <= n * plen, (s, pl, align, n, plen)
        assert plen <= -(-(pl + pl // 64) // align) * align, (s, pl, align, plen)
        n_ceil = -(-s // pl)
        assert n <= (1 << (n_ceil - 1).bit_length()), (s, pl, n)
        if s <= pl:
            assert n == 1
        if pl % 1008 == 0:
            page = pl // 1008
            assert plen // page <= 1024, (s, pl, plen)
