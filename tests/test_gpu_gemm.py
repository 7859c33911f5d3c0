"""The runtime's prompt GEMM (cdna4_gemm_f16_nt) on gfx950 against a PyTorch fp32 product of the
same fp16 operands: the session's four prompt shapes at cfg5 (Q|K|V, O, gate|up, down), ragged M
and N, each tile size the dispatcher picks, fp16 output, accumulation into Y, and the shapes the
kernel refuses (the session then uses rocBLAS)."""
import pytest
import torch

import cdna4
from gpu_util import DEV

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    X = torch.randn(M, K, device=DEV, generator=g).half()
    W = (torch.randn(N, K, device=DEV, generator=g) * 0.02).half()
    return X, W


@pytest.mark.parametrize("M,N,K,out_dtype,accum", [
    (512, 2304, 768, torch.float16, False),   # Q|K|V, cfg5
    (512, 768, 768, torch.float32, True),     # O projection into the residual
    (512, 6144, 768, torch.float32, False),   # gate|up
    (512, 768, 3072, torch.float32, True),    # down projection into the residual
    (4096, 4096, 256, torch.float32, False),  # 128 x 128 tiles, 128-wide K stages
    (2048, 2048, 192, torch.float32, True),   # 128 x 128 tiles, 64-wide K stages
    (512, 6144, 320, torch.float16, False),   # 64 x 128 tiles, 64-wide K stages
    (37, 100, 64, torch.float32, False),      # ragged M and N, one K step
    (1, 4, 128, torch.float16, True),
    (129, 260, 192, torch.float32, True),
    (300, 1000, 640, torch.float16, False),
])
def test_gemm_against_torch_fp32(M, N, K, out_dtype, accum):
    X, W = _operands(M, N, K, M * 31 + N * 7 + K)
    ref = X.float() @ W.float().t()
    Y0 = torch.randn(M, N, device=DEV).to(out_dtype) if accum else None
    out = Y0.clone() if accum else None
    got = cdna4.gemm_f16_nt(X, W, out=out, accum=accum, out_dtype=out_dtype)
    torch.cuda.synchronize()
    if accum:
        ref = ref + Y0.float()
    scale = max(1.0, ref.abs().max().item())
    # fp32 accumulation in another order: 1e-5 of the largest |Y|; fp16 output: half an fp16 ulp
    # of the largest |Y| on top of that
    tol = 1e-5 * scale if out_dtype == torch.float32 else 1e-5 * scale + 2.0 ** -11 * scale
    err = (got.float() - ref).abs().max().item()
    assert err <= tol, (M, N, K, err, tol)


def test_gemm_strided_output_rows():
    # Y with a leading dimension wider than N (a column slice of a wider buffer): only [:, :N] written
    M, N, K, ldy = 70, 96, 128, 160
    X, W = _operands(M, N, K, 5)
    buf = torch.full((M, ldy), 7.0, device=DEV)
    out = buf[:, :N]
    cdna4.gemm_f16_nt(X, W, out=out)
    torch.cuda.synchronize()
    ref = X.float() @ W.float().t()
    assert (out - ref).abs().max().item() <= 1e-5 * max(1.0, ref.abs().max().item())
    assert torch.equal(buf[:, N:], torch.full((M, ldy - N), 7.0, device=DEV))


@pytest.mark.parametrize("M,N,K", [(8, 64, 100), (8, 66, 128)])
def test_gemm_refuses_shapes_it_does_not_take(M, N, K):
    X, W = _operands(M, N, K, 9)
    with pytest.raises(RuntimeError):
        cdna4.gemm_f16_nt(X, W)
