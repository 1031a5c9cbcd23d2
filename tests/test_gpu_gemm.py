"""GPU parity of thb_gemm_acc (ops::gemm_acc, the o_proj product after
attention) against the oracle's restatement of cpu_ref::gemm / gemv
(crates/thuban_backend/tests/support/cpu_ref.rs:11-35).

* The reference's own bf16-weight cases, inputs drawn from its LCG:
  gemm_coop_bf16_acc and gemm_coop_bf16_multi_tile (kernels.rs:472-536),
  gemv_bf16 / gemv_bf16_wide_k (kernels.rs:630-680), and the shapes and
  seeds of gemm_acc_case (kernels.rs:542-598, which uses Q8_0 weights there;
  here the weights are bf16 draws of the same LCG), each within the
  reference's tolerance (rel 2e-2, abs 5e-2) of cpu_ref::gemm.
* A tight check against the oracle's double-precision sums: |gpu - exact|
  <= 2^-15 * sum |x w| + 1e-6 (the high/low split keeps ~16 bits of x against
  the exact weight), for every x type (f32, f16, bf16) x weight type (bf16,
  f16) over row counts that take both kernels and their edges.
* Identity weights give y = x exactly for an x of the weight's type;
  results are deterministic (two runs, same bits)."""

import zlib

import numpy as np
import pytest

import oracle
from gpu_util import say

pytestmark = pytest.mark.gpu


def _bf16_round(v):
    """bf16_round of kernels.rs:126-130: the upper 16 bits."""
    return (np.asarray(v, np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)


def _run(torch, x, w16, y0, acc, x_dtype=None, w_dtype=None):
    from flint_amd import ops

    m, k = x.shape
    tx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    if x_dtype is not None:
        tx = tx.to(x_dtype)
    tw = torch.from_numpy(np.ascontiguousarray(w16)).cuda().to(w_dtype or torch.bfloat16)
    ty = torch.from_numpy(np.ascontiguousarray(y0, np.float32)).cuda()
    ops.gemm_acc(tx, tw, ty, m, acc)
    torch.cuda.synchronize()
    return ty.cpu().numpy()


def _agree(got, want, rel, abs_):
    diff = np.abs(got - want)
    assert np.all(diff <= rel * np.abs(want) + abs_), float(np.max(diff - rel * np.abs(want)))


# (name, seed, m, n, k, acc): the reference's cases (kernels.rs lines above)
REF_CASES = [
    ("gemm_coop_bf16_acc", 13, 128, 128, 256, True),
    ("gemm_coop_bf16_multi_tile", 29, 128, 256, 1024, False),
    ("gemv_bf16", 31, 1, 32, 128, False),
    ("gemv_bf16_wide_k", 47, 1, 32, 1024, False),
    ("gemm_acc_coop_full", 31, 128, 128, 256, False),
    ("gemm_acc_coop_tail", 37, 144, 128, 256, False),
    ("gemm_acc_coop_tail_accumulates", 39, 144, 128, 256, True),
    ("gemm_acc_coop_long_k", 41, 128, 128, 8192, False),
    ("gemm_classic_segs_long_k", 43, 64, 64, 8192, False),
]


@pytest.mark.parametrize("case", REF_CASES, ids=[c[0] for c in REF_CASES])
def test_reference_cases(torch_cuda, case):
    torch = torch_cuda
    name, seed, m, n, k, acc = case
    say("gemm reference case", name)
    if name.startswith("gemm_coop_bf16") or name.startswith("gemv_bf16"):
        # one Rng: x, then w, then y0 (kernels.rs:479-482, 512-514, 633-634)
        draws = oracle.lcg_fill(seed, m * k + n * k + (m * n if acc else 0))
        x, w = draws[:m * k].reshape(m, k), draws[m * k:m * k + n * k].reshape(n, k)
        y0 = draws[m * k + n * k:].reshape(m, n) if acc else np.zeros((m, n), np.float32)
    else:
        # gemm_acc_case: Rng(seed) for x then y0; weights from seed ^ 0x1234
        draws = oracle.lcg_fill(seed, m * k + m * n)
        x, y0 = draws[:m * k].reshape(m, k), draws[m * k:].reshape(m, n)
        w = oracle.lcg_fill(seed ^ 0x1234, n * k).reshape(n, k)
        if not acc:
            y0 = np.zeros((m, n), np.float32)
    wb = _bf16_round(w)
    got = _run(torch, x, wb, y0, acc)
    want = oracle.gemm(x, wb, m, n, k, y0=y0 if acc else None)
    _agree(got, want, 2e-2, 5e-2)
    exact = oracle.gemm(x, wb, m, n, k, y0=y0 if acc else None, exact=True)
    scale = np.abs(x).astype(np.float64) @ np.abs(wb).astype(np.float64).T
    err = float(np.max(np.abs(got - exact) - 2.0 ** -15 * scale))
    say(name, "max |gpu - exact| over the bound", err)
    assert err <= 1e-6


@pytest.mark.parametrize("wt", ["bf16", "f16"])
@pytest.mark.parametrize("xt", ["f32", "f16", "bf16"])
def test_every_type_and_row_count(torch_cuda, xt, wt):
    torch = torch_cuda
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    rng = np.random.default_rng(zlib.crc32(f"{xt}-{wt}".encode()))  # the same inputs in every process
    n, k = 192, 512
    w = rng.standard_normal((n, k)).astype(np.float32)
    w = _bf16_round(w) if wt == "bf16" else w.astype(np.float16).astype(np.float32)
    for m in (1, 5, 16, 17, 32, 33, 48, 64, 65, 130):
        x = rng.standard_normal((m, k)).astype(np.float32)
        xq = torch.from_numpy(x).to(tdt[xt]).float().numpy()  # x as the kernel sees it
        y0 = rng.standard_normal((m, n)).astype(np.float32)
        got = _run(torch, x, w, y0, True, x_dtype=tdt[xt], w_dtype=tdt[wt])
        exact = oracle.gemm(xq, w, m, n, k, y0=y0, exact=True)
        scale = np.abs(xq).astype(np.float64) @ np.abs(w).astype(np.float64).T
        err = float(np.max(np.abs(got - exact) - 2.0 ** -15 * scale))
        assert err <= 1e-6, (xt, wt, m, err)
    say("gemm types", xt, wt, "ok")


def test_identity_weights_and_determinism(torch_cuda):
    torch = torch_cuda
    from flint_amd import ops

    k = 256
    eye = torch.eye(k, device="cuda", dtype=torch.bfloat16)
    for m in (3, 32, 100):
        x = torch.randn(m, k, device="cuda").to(torch.bfloat16)
        y = torch.zeros(m, k, device="cuda")
        ops.gemm_acc(x, eye, y, m, False)
        torch.cuda.synchronize()
        assert torch.equal(y, x.float()), m
    # Llama-3-8B o_proj at batch 32 (bf16 attention output into the residual)
    x = torch.randn(32, 4096, device="cuda").to(torch.bfloat16)
    w = (torch.randn(4096, 4096, device="cuda") * 0.02).to(torch.bfloat16)
    y0 = torch.randn(32, 4096, device="cuda")
    ya, yb = y0.clone(), y0.clone()
    ops.gemm_acc(x, w, ya, 32, True)
    ops.gemm_acc(x, w, yb, 32, True)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)
    exact = oracle.gemm(x.float().cpu().numpy(), w.float().cpu().numpy(), 32, 4096, 4096, y0=y0.cpu().numpy(),
                        exact=True)
    err = float(np.max(np.abs(ya.cpu().numpy() - exact)))
    say("o_proj 32 x 4096 x 4096 max abs err", err)
    assert err <= 1e-4


def test_gemm_errors(torch_cuda):
    torch = torch_cuda
    from flint_amd import ThubanError, ops

    x = torch.zeros(2, 96, device="cuda")
    w = torch.zeros(32, 96, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(2, 32, device="cuda")
    with pytest.raises(ThubanError) as e:
        ops.gemm_acc(x, w, y, 2, False)
    assert str(e.value) == "dimension pair (N=32, K=96) does not satisfy N%16 and K%64"
    assert e.value.kind == "Config"
    with pytest.raises(ThubanError):
        ops.check_gemm_dims([(4096, 4096), (40, 64)])
    ops.check_gemm_dims([(4096, 4096), (32, 128)])
