"""The rest of the reference runtime's __global__ kernels (<cdna3/runtime/forward.hpp>, here
include/cdna3/runtime/forward_kernels.hpp), launched through a test hook with the reference's
launch geometry: the naive GEMMs (forward.hpp:70-131; 16 x 16 blocks, the lm_head call with
M = 1), SiLU product and residual add (:154-170), embedding gather (:174-184) and the greedy
argmax (:244-262).

Checks: the GEMMs against a float64 product of the same (rounded) inputs, within fp32
accumulation error (1e-5 of sum |x w|) plus, for fp16 outputs, the output's own rounding (2^-11
relative); SiLU within 1e-6 relative of a float64 evaluation; the add and the gather bit-exact;
the argmax index-exact against oracle.reference_argmax, which replays the reference kernel's
thread loop and tree step by step, on planted ties, all-(-inf) rows and NaNs.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import parity_log
from gpu_util import DEV, hooks, stream

pytestmark = pytest.mark.gpu


def _rt(which, a, b, c=None, d=None, ints=(0, 0, 0, 0, 0), f=0.0):
    p = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    rc = hooks().hook_runtime_kernels(which, p(a), p(b), p(c), p(d), *ints, f, stream())
    torch.cuda.synchronize()
    assert rc == 0


def _f16(x):
    vals, bits = oracle.round16(np.asarray(x, np.float32).reshape(-1), oracle.F16)
    return vals.astype(np.float64), torch.from_numpy(bits.view(np.int16)).view(torch.float16).to(DEV)


GEMMS = {5: ("f32", "f16", False), 6: ("f32", "f16", True), 7: ("f32", "f32", False), 8: ("f16", "f32", False),
         9: ("f16", "f16", False)}


@pytest.mark.parametrize("which", sorted(GEMMS))
@pytest.mark.parametrize("M,N,K,bx,by", [(1, 32000, 768, 16, 16), (37, 300, 768, 16, 16), (5, 100, 64, 16, 16),
                                         (3, 50, 30, 16, 16), (64, 64, 256, 8, 8), (7, 9, 100, 4, 4),
                                         (20, 48, 3072, 32, 8), (2, 17, 520, 10, 10)])
def test_reference_gemm_kernels(which, M, N, K, bx, by):
    xin, yout, bias = GEMMS[which]
    seed = which * 1000 + M + N + K
    xr = oracle.normal(seed, M * K, 0.0, 1.0)
    if xin == "f16":
        x, Xt = _f16(xr)
    else:
        x, Xt = xr.astype(np.float64), torch.from_numpy(xr.astype(np.float32)).to(DEV)
    w, Wt = _f16(oracle.normal(seed + 1, N * K, 0.0, 0.05))
    b, Bt = _f16(oracle.normal(seed + 2, N, 0.0, 0.5)) if bias else (np.zeros(N), None)
    Y = torch.full((M, N), float("nan"), device=DEV, dtype=torch.float16 if yout == "f16" else torch.float32)
    _rt(which, Xt, Y, Wt, Bt, (M, N, K, bx, by))
    X, W = x.reshape(M, K), w.reshape(N, K)
    ref = X @ W.T + b[None, :]
    mag = np.abs(X) @ np.abs(W).T + np.abs(b)[None, :]
    bound = 1e-5 * mag + (np.abs(ref) * 2.0 ** -11 + 2.0 ** -24 if yout == "f16" else 1e-30)
    got = Y.float().cpu().numpy().astype(np.float64)
    ratio = float(np.max(np.abs(got - ref) / bound))
    parity_log.record(ratio, 1.0, "gemm")
    print(f"gemm {which} {xin}->{yout} bias {bias} M{M} N{N} K{K} block {bx}x{by}: err/bound {ratio:.3f}")
    assert ratio <= 1.0


@pytest.mark.parametrize("n,off,block", [(1 << 20, 0, 256), (1000003, 0, 256), (1000, 1, 256), (77, 0, 64),
                                         (4097, 3, 1024)])
def test_silu_mul_and_add_kernels(n, off, block):
    g = oracle.normal(n, n + off, 0.0, 3.0).astype(np.float32)
    u = oracle.normal(n + 1, n + off, 0.0, 1.0).astype(np.float32)
    G = torch.from_numpy(g).to(DEV)
    U = torch.from_numpy(u).to(DEV)
    gate, up = G[off:], U[off:]                     # off > 0: not 16-byte aligned, the scalar path
    _rt(10, up, gate, ints=(n, block, 0, 0, 0))
    gg, uu = g[off:].astype(np.float64), u[off:].astype(np.float64)
    want = gg / (1.0 + np.exp(-gg)) * uu
    got = gate.cpu().numpy().astype(np.float64)
    err = float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)))
    parity_log.record(err, 1e-6, "silu")
    assert err <= 1e-6, err
    assert np.array_equal(G[:off].cpu().numpy(), g[:off])    # nothing before the view touched
    # add_f32_kernel: x += y in fp32, bit-exact
    x = oracle.normal(n + 2, n + off, 0.0, 1.0).astype(np.float32)
    X = torch.from_numpy(x).to(DEV)
    _rt(11, U[off:], X[off:], ints=(n, block, 0, 0, 0))
    assert np.array_equal(X[off:].cpu().numpy(), x[off:] + u[off:])
    assert np.array_equal(X[:off].cpu().numpy(), x[:off])


@pytest.mark.parametrize("T,H,V", [(33, 768, 32000), (1, 768, 32000), (5, 100, 50), (3, 8, 7)])
def test_embed_gather_kernel(T, H, V):
    _, bits = oracle.round16(oracle.normal(V + H, V * H, 0.0, 0.02), oracle.F16)
    E = torch.from_numpy(bits.view(np.int16)).view(torch.float16).to(DEV)
    ids = np.random.default_rng(T).integers(0, V, T).astype(np.int32)
    out = torch.full((T, H), float("nan"), device=DEV)
    _rt(12, E, out, torch.from_numpy(ids).to(DEV), ints=(T, H, 0, 0, 0))
    want = oracle.widen(bits, oracle.F16).reshape(V, H)[ids]
    assert np.array_equal(out.cpu().numpy(), want)


def _argmax(x16_bits, threads):
    L = torch.from_numpy(x16_bits.view(np.int16)).view(torch.float16).to(DEV)
    out = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    _rt(13, L, out, ints=(x16_bits.size, threads, 0, 0, 0))
    return int(out.item())


@pytest.mark.parametrize("threads", [256, 64, 1024, 32])
def test_argmax_kernel_ties_and_specials(threads):
    rng = np.random.default_rng(threads)
    cases = []
    V = 32000
    x = rng.normal(0, 1, V).astype(np.float32)
    cases.append(("random", x))
    t = x.copy()
    t[[3, 130, 200]] = 9.0                     # three threads tied: the smallest bit reversal wins
    cases.append(("ties across threads", t))
    t = x.copy()
    last = (V - 6) // threads
    t[[5 + threads * last, 5 + threads * (last // 2), 5 + threads]] = 9.0   # one thread: the first index wins
    cases.append(("ties in one thread", t))
    t = x.copy()
    t[rng.integers(0, V, 40)] = 9.0            # many ties
    cases.append(("many ties", t))
    t = x.copy()
    t[[17, 1000]] = [-0.0, 0.0]
    t[:] = np.minimum(t, -1.0)
    t[[17, 1000]] = [-0.0, 0.0]                # -0 and +0 tie (strict > sees them equal)
    cases.append(("signed zeros", t))
    cases.append(("all -inf", np.full(300, -np.inf, np.float32)))
    t = np.full(V, -np.inf, np.float32)
    t[31999] = -60000.0
    cases.append(("last element only", t))
    cases.append(("V = 1", np.array([1.5], np.float32)))
    cases.append(("V < threads", rng.normal(0, 1, 37).astype(np.float32)))
    t = x.copy()
    t[[10, 20]] = np.nan                       # NaN never chosen
    cases.append(("NaNs", t))
    for name, v in cases:
        _, bits = oracle.round16(v, oracle.F16)
        ref_in = oracle.widen(bits, oracle.F16)
        ref_in = np.where(np.isnan(ref_in), -np.inf, ref_in)       # the reference never picks a NaN
        want = oracle.reference_argmax(ref_in, threads)
        got = _argmax(bits, threads)
        print(f"argmax {threads} threads, {name}: {got} (reference {want})")
        assert got == want, name
