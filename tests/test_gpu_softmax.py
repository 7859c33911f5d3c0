"""Row softmax (cdna3_softmax_rows_f32) on gfx950 against the oracle (bench_softmax.hip:59-105).

Bound, element-wise: |gpu - ref| <= ref * (1e-6 + 1.2e-7 * |x - max|) + 1e-37. The kernel
computes exp(x - m) as 2^((x - m) * log2 e): rounding the product to fp32 moves the result by a
relative 2^-24 * |x - m| * log2(e) * ln(2) = 6e-8 * |x - m| (the slope, doubled), the exponential
itself by about one fp32 ulp, the row sum and the final product by a few more. The oracle takes
exp and the sum in double. The same outputs are also held to the north star's fp32 tolerance
(1e-4, absolute below 1) for the run's parity table."""
import ctypes

import numpy as np
import pytest
import torch

import cdna4
import oracle
from gpu_util import DEV, check_parity

pytestmark = pytest.mark.gpu


def _lcg(M, H):
    # bench_softmax.hip:117: ((i * 1103515245 + 12345) & 0xff) / 32 - 4
    i = np.arange(M * H, dtype=np.uint64)
    return ((((i * 1103515245 + 12345) & 0xFF).astype(np.float32)) / 32.0 - 4.0).reshape(M, H)


def _check(got, X, what):
    ref = oracle.softmax_rows(X).astype(np.float64)
    spread = X.max(axis=1, keepdims=True).astype(np.float64) - X
    spread = np.where(np.isfinite(spread), spread, 0.0)
    bound = ref * (1e-6 + 1.2e-7 * spread) + 1e-37
    d = np.abs(got.astype(np.float64) - ref)
    worst = float(np.max(d / bound))
    print(f"  softmax {what}: max |gpu-ref| / bound = {worst:.3f}", flush=True)
    assert np.all(d <= bound), f"{what}: {worst:.3f} x the bound"
    check_parity(got, ref, torch.float32, what=what)


@pytest.mark.parametrize("M,H", [(65536, 512), (65536, 64)])
def test_softmax_reference_benchmark_shapes(M, H):
    X = _lcg(M, H)
    got = cdna4.softmax_rows_f32(torch.from_numpy(X).to(DEV)).cpu().numpy()
    sums = got.sum(axis=1, dtype=np.float64)
    assert np.max(np.abs(sums - 1.0)) < 1e-5                  # bench_softmax.hip:123-133 checks row 0 to 1e-2
    _check(got, X, f"reference input {M}x{H}")


@pytest.mark.parametrize("M,H", [(1, 1), (9, 1), (17, 2), (4, 3), (33, 60), (300, 64), (5, 100), (3, 777),
                                 (64, 256), (40, 516), (7, 1024), (6, 2048), (7, 4096), (2, 5000), (3, 12345)])
def test_softmax_shapes_and_spreads(M, H):
    X = oracle.normal(M * 31 + H, M * H, 0.0, 8.0).reshape(M, H)
    got = cdna4.softmax_rows_f32(torch.from_numpy(X).to(DEV)).cpu().numpy()
    _check(got, X, f"N(0,8) {M}x{H}")


@pytest.mark.parametrize("H", [64, 512, 100])
def test_softmax_in_place_masked_and_misaligned(H):
    M = 129
    X = oracle.normal(H, M * H, 0.0, 3.0).reshape(M, H)
    X[::3, 1::5] = -np.inf                                     # masked entries carry no weight
    X[7, :] = 2.5                                              # a constant row is uniform
    t = torch.from_numpy(X).to(DEV)
    out = cdna4.softmax_rows_f32(t, out=t)                     # in place
    got = out.cpu().numpy()
    assert out.data_ptr() == t.data_ptr()
    assert np.all(got[::3, 1::5] == 0.0)
    np.testing.assert_allclose(got[7], 1.0 / H, rtol=2e-7)
    _check(got, X, f"in place {M}x{H}")
    # Rows starting 4 bytes past a 16-byte boundary take the element-wise kernel.
    buf = torch.zeros(M * H + 1, device=DEV)
    xin = buf[1:].view(M, H)
    xin.copy_(torch.from_numpy(X))
    out2 = torch.empty(M * H + 1, device=DEV)[1:].view(M, H)
    got2 = cdna4.softmax_rows_f32(xin, out=out2).cpu().numpy()
    _check(got2, X, f"misaligned {M}x{H}")


def test_softmax_through_the_c_abi_on_a_stream():
    M, H = 1000, 512
    X = _lcg(M, H)
    x = torch.from_numpy(X).to(DEV)
    y = torch.full_like(x, float("nan"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    rc = cdna4.lib().cdna3_softmax_rows_f32(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), M, H,
                                            ctypes.c_void_p(s.cuda_stream))
    assert rc == 0
    s.synchronize()
    _check(y.cpu().numpy(), X, "C ABI on a side stream")
