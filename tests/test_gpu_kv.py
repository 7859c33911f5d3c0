"""KV-cache append, layout repacks and the fused RoPE + append on gfx950 against the oracle."""
import numpy as np
import pytest
import torch

import cdna4
import oracle
from gpu_util import DEV

pytestmark = pytest.mark.gpu


def dev16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.float16).to(DEV)


def host16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


@pytest.mark.parametrize("T,heads,D,pos0,max_seq,offset", [(1, 8, 128, 100, 512, 0), (37, 12, 64, 0, 64, 0),
                                                            (512, 2, 128, 7, 1024, 0), (5, 3, 10, 2, 9, 0),
                                                            (9, 4, 64, 3, 16, 1)])
def test_scatter_kv_bit_exact(T, heads, D, pos0, max_seq, offset):
    rng = np.random.default_rng(T + D)
    src = rng.integers(0, 1 << 16, T * heads * D, dtype=np.uint16)
    cache = rng.integers(0, 1 << 16, heads * max_seq * D, dtype=np.uint16)
    # offset > 0 shifts both tensors off 16-byte alignment (the element-wise path).
    S = dev16(np.concatenate([np.zeros(offset, np.uint16), src]))[offset:]
    C = dev16(np.concatenate([np.zeros(offset, np.uint16), cache]))
    cdna4.scatter_kv_f16(S, C[offset:], T, heads, D, pos0, max_seq)
    got = host16(C)[offset:]
    assert np.array_equal(got, oracle.scatter_kv(src, cache, T, heads, D, pos0, max_seq).reshape(-1))


@pytest.mark.parametrize("seq,heads,D", [(512, 12, 64), (33, 8, 128), (7, 3, 10), (1, 32, 128)])
@pytest.mark.parametrize("direction", [0, 1])
def test_repack_bit_exact(seq, heads, D, direction):
    rng = np.random.default_rng(seq * heads + D + direction)
    src = rng.integers(0, 1 << 16, seq * heads * D, dtype=np.uint16)
    dst = torch.empty(seq * heads * D, dtype=torch.float16, device=DEV)
    cdna4.repack_f16(dev16(src), dst, seq, heads, D, direction)
    assert np.array_equal(host16(dst), oracle.repack(src, seq, heads, D, direction))


@pytest.mark.parametrize("T,nQH,nKVH,D,pos0,max_seq", [(512, 12, 12, 64, 0, 640), (1, 32, 8, 128, 700, 1024),
                                                        (17, 8, 2, 128, 40, 64), (3, 4, 4, 6, 1, 4)])
def test_rope_append_kv(T, nQH, nKVH, D, pos0, max_seq):
    c, s = oracle.rope_table(pos0, T, D, 10000.0)
    _, q = oracle.round16(oracle.normal(T + 1, T * nQH * D), oracle.F16)
    _, k = oracle.round16(oracle.normal(T + 2, T * nKVH * D), oracle.F16)
    _, v = oracle.round16(oracle.normal(T + 3, T * nKVH * D), oracle.F16)
    rng = np.random.default_rng(D)
    Kc0 = rng.integers(0, 0x7800, nKVH * max_seq * D, dtype=np.uint16)   # finite fp16 patterns
    Vc0 = rng.integers(0, 0x7800, nKVH * max_seq * D, dtype=np.uint16)
    q_out = torch.empty(nQH * T * D, dtype=torch.float16, device=DEV)
    Kc, Vc = dev16(Kc0), dev16(Vc0)
    Qd, Kd, Vd = dev16(q), dev16(k), dev16(v)
    cdna4.rope_append_kv_f16(Qd, Kd, Vd, q_out, Kc, Vc, torch.from_numpy(c).to(DEV), torch.from_numpy(s).to(DEV), T,
                             nQH, nKVH, D, pos0, max_seq)
    wq, wk, wv = oracle.rope_append_kv(q, k, v, Kc0, Vc0, c, s, T, nQH, nKVH, D, pos0, max_seq)
    # V rows and everything outside the slot are copies: bit-exact. Rotated values: the same fp32
    # formula and RNE, so only FMA contraction may move a result by one fp16 ulp.
    assert np.array_equal(host16(Vc), wv)
    got_k = host16(Kc).reshape(nKVH, max_seq, D)
    want_k = wk.reshape(nKVH, max_seq, D)
    outside = np.ones(max_seq, bool); outside[pos0:pos0 + T] = False
    assert np.array_equal(got_k[:, outside], want_k[:, outside])
    for got, want in ((host16(q_out), wq), (got_k[:, pos0:pos0 + T].reshape(-1), want_k[:, pos0:pos0 + T].reshape(-1))):
        np.testing.assert_allclose(oracle.widen(got, oracle.F16), oracle.widen(want, oracle.F16), rtol=2.0 ** -10,
                                   atol=2.0 ** -24)
    # Inputs are not modified.
    assert np.array_equal(host16(Qd), q) and np.array_equal(host16(Kd), k)
