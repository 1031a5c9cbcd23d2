"""GPU checks of thb_hbm_stream (flint_amd/csrc/probe.hip), the streaming
probe bench.py's hbm_ceiling field times (no reference counterpart: a
measurement aid).

* Copy mode writes the source to the destination bit for bit, on sizes that
  do not divide evenly among the workgroups (ragged last slabs, empty
  workgroups) and on one 16-byte vector.
* Read mode writes one word per lane of each workgroup (its fold of the
  words it read) into the first 2 KiB per workgroup of dst and nothing past
  them.
* Arguments it cannot serve are refused before a launch."""

import ctypes

import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu


def _stream(src, dst, nbytes, mode, wg):
    from flint_amd import _lib
    from flint_amd.pool import _stream_ptr

    return _lib.lib().thb_hbm_stream(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), nbytes, mode,
                                     wg, _stream_ptr(None))


@pytest.mark.parametrize("vecs,wg", [(1, 1), (1, 3), (1000, 7), (4099, 256), (65536 + 5, 1024), (3 << 20, 4096)])
def test_copy_is_bit_exact(torch_cuda, vecs, wg):
    torch = torch_cuda
    say("hbm_stream copy", vecs, "vectors,", wg, "workgroups")
    src = torch.randint(0, 256, (16 * vecs,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros(16 * vecs + 64, dtype=torch.uint8, device="cuda")
    assert _stream(src, dst, 16 * vecs, 1, wg) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst[:16 * vecs], src)
    assert int(dst[16 * vecs:].count_nonzero()) == 0  # nothing past the copy


def test_read_writes_only_its_sink(torch_cuda):
    torch = torch_cuda
    wg, nbytes = 64, 1 << 22
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")
    assert _stream(src, dst, nbytes, 0, wg) == 0
    torch.cuda.synchronize()
    sink = 2048 * wg
    assert bool((dst[sink:] == 0xA5).all())
    # every word of the source was folded into some lane's word: the XOR of
    # all lanes' words equals the XOR of all source words
    want = np.bitwise_xor.reduce(src.cpu().numpy().view(np.uint32))
    got = np.bitwise_xor.reduce(dst[:sink].cpu().numpy().view(np.uint32))
    assert int(got) == int(want)


def test_refusals(torch_cuda):
    torch = torch_cuda
    from flint_amd import _lib

    src = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    dst = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    for nbytes, mode, wg in ((4096, 2, 1), (4096, 1, 0), (4096, 1, 65537), (4095, 1, 1), (4096, 0, 3)):
        assert _stream(src, dst, nbytes, mode, wg) == _lib.THB_ERR_INVALID, (nbytes, mode, wg)
    assert _stream(src[1:], dst, 4080, 1, 1) == _lib.THB_ERR_INVALID  # misaligned source
