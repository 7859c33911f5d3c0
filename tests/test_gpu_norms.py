"""RMSNorm, two-pass LayerNorm, RoPE and the RoPE table on gfx950 against the oracle."""
import numpy as np
import pytest
import torch

import cdna4
import oracle
from gpu_util import DEV

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,H", [(1, 768), (512, 768), (65536 // 64, 64), (37, 64), (17, 64), (16, 60), (5, 32), (1, 4), (300, 512), (7, 4096), (5, 1000), (3, 5000), (2, 3)])
def test_rmsnorm(M, H):
    X = oracle.normal(M * 7 + H, M * H, 0.0, 2.0).reshape(M, H)
    wv, wb = oracle.round16(oracle.normal(H, H, 1.0, 0.1), oracle.F16)
    Xt = torch.from_numpy(X).to(DEV)
    Wt = torch.from_numpy(wb.view(np.int16)).view(torch.float16).to(DEV)
    got = cdna4.rmsnorm_f32(Xt, Wt, 1e-6).cpu().numpy()
    np.testing.assert_allclose(got, oracle.rmsnorm(X, wb, 1e-6), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,H", [(65536 // 32, 64), (37, 64), (33, 64), (17, 16), (21, 48), (3, 8), (2048, 512), (512, 768), (4, 4096), (3, 6000), (5, 100), (9, 1)])
def test_layernorm(M, H):
    # The reference's input generator for its LayerNorm benchmark (bench_layernorm.hip:131).
    i = np.arange(M * H, dtype=np.uint64)
    X = ((((i * 1103515245 + 12345) & 0xFF).astype(np.float32)) / 32.0 - 4.0).reshape(M, H)
    g, b = oracle.uniform(1, H, 0.5, 1.5), oracle.uniform(2, H)
    got = cdna4.layernorm_f32(torch.from_numpy(X).to(DEV), torch.from_numpy(g).to(DEV), torch.from_numpy(b).to(DEV),
                              1e-5).cpu().numpy()
    np.testing.assert_allclose(got, oracle.layernorm(X, g, b, 1e-5), rtol=1e-4, atol=2e-5)
    if H >= 64:
        ones, zeros = torch.ones(H, device=DEV), torch.zeros(H, device=DEV)
        y = cdna4.layernorm_f32(torch.from_numpy(X).to(DEV), ones, zeros, 1e-5).double().cpu().numpy()
        np.testing.assert_allclose(y.mean(1), 0.0, atol=1e-4)      # bench_layernorm.hip:137-150
        np.testing.assert_allclose(y.var(1), 1.0, atol=1e-2)


@pytest.mark.parametrize("M,H", [(65536, 512), (262144, 64)])
def test_norms_streaming_policy_sizes(M, H):
    # Tensors of 64 MiB or more take the kernels with non-temporal loads and stores (the row-cached
    # form at 512 columns, the four-rows-per-wave form at 64); checked on a sample of rows.
    g = torch.Generator(device=DEV).manual_seed(M + H)
    Xt = torch.randn(M, H, device=DEV, generator=g) * 2.0
    rows = np.unique(np.concatenate([np.arange(8), np.arange(M - 8, M), oracle.integers(M + H, 200, 0, M - 1)]))
    X = Xt[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    wv, wb = oracle.round16(oracle.normal(H, H, 1.0, 0.1), oracle.F16)
    Wt = torch.from_numpy(wb.view(np.int16)).view(torch.float16).to(DEV)
    got = cdna4.rmsnorm_f32(Xt, Wt, 1e-6)[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    np.testing.assert_allclose(got, oracle.rmsnorm(X, wb, 1e-6), rtol=1e-5, atol=1e-5)
    gm, bt = oracle.uniform(1, H, 0.5, 1.5), oracle.uniform(2, H)
    got = cdna4.layernorm_f32(Xt, torch.from_numpy(gm).to(DEV), torch.from_numpy(bt).to(DEV),
                              1e-5)[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    np.testing.assert_allclose(got, oracle.layernorm(X, gm, bt, 1e-5), rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("seq,heads,D,pos0", [(512, 12, 64, 0), (1, 12, 64, 511), (33, 8, 128, 1000), (4, 2, 10, 3)])
def test_rope_table_and_rope(seq, heads, D, pos0):
    cos, sin = cdna4.rope_table_f32(pos0, seq, D, 10000.0)
    c_ref, s_ref = oracle.rope_table(pos0, seq, D, 10000.0)
    c_got, s_got = cos.cpu().numpy(), sin.cpu().numpy()
    # Device cosf/sinf/powf differ from glibc by a few ulp of the angle (pos up to ~1500 rad).
    np.testing.assert_allclose(c_got, c_ref, atol=2e-4)
    np.testing.assert_allclose(s_got, s_ref, atol=2e-4)
    vals, bits = oracle.round16(oracle.normal(seq + D, seq * heads * D), oracle.F16)
    T = torch.from_numpy(bits.view(np.int16)).view(torch.float16).to(DEV)
    ct, st = torch.from_numpy(c_ref).to(DEV), torch.from_numpy(s_ref).to(DEV)
    cdna4.rope_f16(T, ct, st, seq, heads, D)
    got = oracle.widen(T.view(torch.int16).cpu().numpy().view(np.uint16), oracle.F16)
    want = oracle.widen(oracle.rope(bits, c_ref, s_ref, seq, heads, D), oracle.F16)
    # Same fp32 formula and RNE; only FMA contraction may move a result by one fp16 ulp.
    np.testing.assert_allclose(got, want, rtol=2.0 ** -10, atol=2.0 ** -24)


# ---- the reference's __global__ kernels from <cdna3/runtime/forward.hpp>, launched as its layer
# loop launches them (hipLaunchKernelGGL, session.hpp:168-177, :193-207, :246-249) -------------

def _rt(which, a, b, c=None, d=None, ints=(0, 0, 0, 0, 0), f=0.0):
    from gpu_util import hooks, ptr, stream
    import ctypes
    p = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    rc = hooks().hook_runtime_kernels(which, p(a), p(b), p(c), p(d), *ints, f, stream())
    torch.cuda.synchronize()
    assert rc == 0


@pytest.mark.parametrize("M,H,block", [(1, 768, 256), (512, 768, 256), (37, 64, 256), (5, 1000, 256), (3, 5000, 256),
                                       (2, 3, 256), (64, 768, 64), (16, 4096, 1024)])
def test_rmsnorm_f32_kernel_as_launched_by_the_reference(M, H, block):
    X = oracle.normal(M * 3 + H, M * H, 0.0, 2.0).reshape(M, H)
    _, wb = oracle.round16(oracle.normal(H + 1, H, 1.0, 0.1), oracle.F16)
    Xt = torch.from_numpy(X).to(DEV)
    Wt = torch.from_numpy(wb.view(np.int16)).view(torch.float16).to(DEV)
    Y = torch.full_like(Xt, float("nan"))
    _rt(0, Xt, Y, Wt, None, (M, H, block, 0, 0), 1e-6)
    np.testing.assert_allclose(Y.cpu().numpy(), oracle.rmsnorm(X, wb, 1e-6), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("seq,heads,D", [(512, 12, 64), (1, 12, 64), (33, 8, 128), (5, 2, 10)])
def test_rope_kernel_as_launched_by_the_reference(seq, heads, D):
    c_ref, s_ref = oracle.rope_table(7, seq, D, 10000.0)
    _, bits = oracle.round16(oracle.normal(seq * D + heads, seq * heads * D), oracle.F16)
    T = torch.from_numpy(bits.view(np.int16)).view(torch.float16).to(DEV)
    _rt(1, None, T, torch.from_numpy(c_ref).to(DEV), torch.from_numpy(s_ref).to(DEV), (seq, heads, D, 0, 0))
    got = oracle.widen(T.view(torch.int16).cpu().numpy().view(np.uint16), oracle.F16)
    want = oracle.widen(oracle.rope(bits, c_ref, s_ref, seq, heads, D), oracle.F16)
    np.testing.assert_allclose(got, want, rtol=2.0 ** -10, atol=2.0 ** -24)


@pytest.mark.parametrize("seq,heads,D", [(77, 12, 64), (5, 2, 128)])
def test_repack_and_pack_kv_kernels(seq, heads, D):
    bits = (oracle.integers(seq, seq * heads * D, 0, 65535).astype(np.uint16) & 0x7bff)
    src = torch.from_numpy(bits.view(np.int16)).to(DEV)
    for direction in (0, 1):
        dst = torch.zeros_like(src)
        _rt(2, src, dst, ints=(seq, heads, D, direction, 0))
        assert np.array_equal(dst.cpu().numpy().view(np.uint16), oracle.repack(bits, seq, heads, D, direction))
    # pack_kv_kernel: the first N rows of each head of a [heads][max_seq][D] cache, packed.
    max_seq, N = seq + 9, seq - 3
    cache = oracle.integers(seq + 1, heads * max_seq * D, 0, 30000).astype(np.uint16)
    tc = torch.from_numpy(cache.view(np.int16)).to(DEV)
    packed = torch.zeros(heads * N * D, dtype=torch.int16, device=DEV)
    _rt(4, tc, packed, ints=(heads, N, D, max_seq, 0))
    want = cache.reshape(heads, max_seq, D)[:, :N].reshape(-1)
    assert np.array_equal(packed.cpu().numpy().view(np.uint16), want)


@pytest.mark.parametrize("T,pos0,max_seq", [(16, 0, 64), (1, 63, 64), (10, 60, 64)])
def test_scatter_kv_kernel(T, pos0, max_seq):
    heads, D = 4, 64
    src = oracle.integers(T + pos0, T * heads * D, 0, 30000).astype(np.uint16)
    cache = oracle.integers(7, heads * max_seq * D, 0, 30000).astype(np.uint16)
    ts = torch.from_numpy(src.view(np.int16)).to(DEV)
    tc = torch.from_numpy(cache.view(np.int16)).to(DEV)
    _rt(3, ts, tc, ints=(T, heads, D, pos0, max_seq))
    # Rows at or past max_seq are skipped (the reference wrote past the slot): compare with the
    # oracle's scatter of the rows that fit.
    fit = max(0, min(T, max_seq - pos0))
    want = oracle.scatter_kv(src.reshape(T, heads, D)[:fit].reshape(-1), cache, fit, heads, D, pos0, max_seq)
    assert np.array_equal(tc.cpu().numpy().view(np.uint16), want)
