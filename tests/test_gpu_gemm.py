"""The runtime's prompt GEMM (cdna4_gemm_f16_nt) on gfx950 against a PyTorch fp32 product of the
same fp16 operands: the session's four prompt shapes at cfg5 (Q|K|V, O, gate|up, down), ragged M
and N, every tile of the dispatcher's menu (checked with cdna4_gemm_f16_nt_tile), rings shorter
and longer than the K loop, fp16 output, accumulation into Y, and the shapes the kernel refuses
(the session then uses rocBLAS)."""
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


@pytest.mark.parametrize("M,N,K,out_dtype,accum,tile", [
    (512, 2304, 768, torch.float16, False, (64, 96)),    # Q|K|V, cfg5
    (512, 768, 768, torch.float32, True, (32, 32)),      # O projection into the residual
    (512, 6144, 768, torch.float32, False, (128, 96)),   # gate|up
    (512, 768, 3072, torch.float32, True, (32, 32)),     # down projection into the residual
    (37, 100, 64, torch.float32, False, (32, 32)),       # ragged M and N, one K stage
    (1, 4, 128, torch.float16, True, (32, 32)),
    (129, 260, 192, torch.float32, True, (32, 32)),
    (300, 1000, 640, torch.float16, False, (32, 32)),
    (100, 6144, 64, torch.float32, True, (64, 64)),
    (300, 6144, 64, torch.float16, False, (64, 128)),
    (4128, 448, 64, torch.float16, True, (128, 64)),
    (640, 6144, 64, torch.float32, False, (128, 128)),
    (4096, 4096, 256, torch.float32, False, (128, 128)),  # several rounds of workgroups
    (200, 6144, 960, torch.float16, False, (64, 96)),     # 15 stages through a 6-deep ring
])
def test_gemm_against_torch_fp32(M, N, K, out_dtype, accum, tile):
    # the tile the dispatcher takes on a 256-CU part (a part with another CU count may pick another)
    if torch.cuda.get_device_properties(DEV).multi_processor_count == 256:
        assert cdna4.gemm_f16_nt_tile(M, N, K) == tile
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


@pytest.mark.parametrize("M,F,K,tile", [
    (512, 3072, 768, (128, 128)),   # cfg5 gate|up with the SiLU product
    (37, 100, 64, (64, 64)),        # ragged M and F, one K stage
    (300, 3072, 64, (64, 128)),
    (4128, 224, 64, (128, 64)),
    (129, 260, 640, (64, 64)),
])
def test_gemm_silu_against_torch_fp32(M, F, K, tile):
    # Y = fp16(silu(X Wg^T) * (X Wu^T)) with W = [Wg; Wu]; the reference forms both products in fp32
    # and rounds the SiLU product once, as the separate silu_mul kernel does
    if torch.cuda.get_device_properties(DEV).multi_processor_count == 256:
        assert cdna4.gemm_f16_nt_silu_tile(M, F, K) == tile
    X, W = _operands(M, 2 * F, K, M * 13 + F * 5 + K)
    g = X.float() @ W[:F].float().t()
    u = X.float() @ W[F:].float().t()
    ref = g / (1 + torch.exp(-g)) * u
    got = cdna4.gemm_f16_nt_silu(X, W)
    torch.cuda.synchronize()
    assert got.dtype == torch.float16 and tuple(got.shape) == (M, F)
    # fp32 sums in another order (1e-5 of the largest |g| |u|), then one fp16 rounding of the product
    s = max(1.0, g.abs().max().item() * max(1.0, u.abs().max().item()))
    err = ((got.float() - ref).abs() - 2.0 ** -11 * ref.abs()).max().item()
    assert err <= 1e-5 * s, (M, F, K, err)


def test_gemm_silu_refuses_shapes_it_does_not_take():
    X, W = _operands(8, 2 * 6, 64, 3)   # F = 6, not a multiple of 4
    with pytest.raises(RuntimeError):
        cdna4.gemm_f16_nt_silu(X, W)
