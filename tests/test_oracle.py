"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something it does not restate: the reference's own
CPU references compiled from /root/reference (oracle/_ref, bit-exact), the reference's known-
answer tests, numpy / math routines, closed forms and invariants. One test plants a mistake in
the oracle's inputs to show the checks are sensitive to it.
"""
import math

import numpy as np
import pytest

import oracle

# Availability is decided from the file alone: collecting this module (also in a GPU test run)
# loads no reference-built library; only the tests below that run load oracle/_ref.
REF = oracle.ref_available("ref_attention_api")
needs_ref = pytest.mark.skipif(not REF, reason="oracle/_ref not built (no /root/reference checkout here)")


# ---- generators --------------------------------------------------------------------------

def test_splitmix64_known_answers():
    # Published first outputs of splitmix64 seeded with 0 (Vigna's reference implementation).
    assert oracle.splitmix64_at(0, 0) == 0xE220A8397B1DCDAF
    assert oracle.splitmix64_at(0, 1) == 0x6E789E6AA1B965F4
    assert oracle.splitmix64_at(0, 2) == 0x06C45D188009454F


def test_generators_ranges_and_moments():
    u = oracle.uniform(42, 1 << 20)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(float(u.mean())) < 5e-3 and abs(float(u.var()) - 1 / 3) < 5e-3
    z = oracle.normal(7, 1 << 20)
    assert abs(float(z.mean())) < 5e-3 and abs(float(z.std()) - 1.0) < 5e-3
    assert np.array_equal(oracle.normal(7, 1000), z[:1000])          # counter-based: prefix-stable
    k = oracle.integers(3, 1 << 16, -1000, 1000)
    assert k.min() == -1000 and k.max() == 1000
    k64 = oracle.integers(3, 1 << 16, -1000, 1000, np.int64)
    assert np.array_equal(k64, k.astype(np.int64))


# ---- fp16 / bf16 rounding ----------------------------------------------------------------

def _specials():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
            2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1e30, -1e30, np.inf, -np.inf]
    return np.array(vals, np.float32)


def test_round_f16_matches_numpy():
    x = np.concatenate([_specials(), oracle.normal(1, 200000, 0, 3), oracle.uniform(2, 100000, -1e-4, 1e-4),
                        oracle.uniform(3, 100000, -70000, 70000)]).astype(np.float32)
    vals, bits = oracle.round16(x, oracle.F16)
    ref = x.astype(np.float16)
    assert np.array_equal(bits, ref.view(np.uint16))
    assert np.array_equal(vals, ref.astype(np.float32))
    assert np.array_equal(oracle.widen(bits, oracle.F16), ref.astype(np.float32))


def test_round_bf16_is_nearest_even():
    x = np.concatenate([_specials(), oracle.normal(4, 200000, 0, 10), oracle.uniform(5, 1000, -1e-38, 1e-38)])
    x = x.astype(np.float32)
    vals, bits = oracle.round16(x, oracle.BF16)
    # Independent formulation: the two bf16 neighbours by truncation, pick the nearer, ties to even.
    u = x.view(np.uint32)
    lo = (u & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((u & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    fin = np.isfinite(x) & np.isfinite(hi)
    dlo, dhi = np.abs(xd - lo), np.abs(hi - xd)
    lo_even = ((u >> 16) & 1) == 0
    pick_lo = (dlo < dhi) | ((dlo == dhi) & lo_even)
    want = np.where(pick_lo, lo, hi)
    assert np.array_equal(vals[fin].astype(np.float64), want[fin])
    assert np.array_equal(oracle.widen(bits, oracle.BF16), vals)


# ---- attention ---------------------------------------------------------------------------

def _inputs(seed, B, HQ, HK, SQ, SK, D, dist="normal"):
    gen = oracle.normal if dist == "normal" else oracle.uniform
    Q = gen(seed, B * HQ * SQ * D).reshape(B, HQ, SQ, D)
    K = gen(seed + 1, B * HK * SK * D).reshape(B, HK, SK, D)
    V = gen(seed + 2, B * HK * SK * D).reshape(B, HK, SK, D)
    return Q, K, V


def _np_attention(Q, K, V, causal):
    """float64 softmax attention (numpy), GQA by head index h // group."""
    B, HQ, SQ, D = Q.shape
    HK, SK = K.shape[1], K.shape[2]
    g = HQ // HK
    out = np.empty((B, HQ, SQ, D))
    for b in range(B):
        for h in range(HQ):
            s = Q[b, h].astype(np.float64) @ K[b, h // g].astype(np.float64).T / math.sqrt(D)
            if causal:
                s = np.where(np.arange(SK)[None, :] > np.arange(SQ)[:, None], -np.inf, s)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            out[b, h] = (p / p.sum(axis=1, keepdims=True)) @ V[b, h // g].astype(np.float64)
    return out


CONFIGS = [  # (D, seqQ, seqK, nQH, nKVH, batch, causal) — the reference's validation set, scaled
    (128, 256, 256, 2, 2, 1, 0), (128, 256, 256, 4, 2, 1, 0), (128, 256, 256, 2, 2, 1, 1),
    (128, 256, 256, 4, 2, 1, 1), (64, 256, 256, 2, 2, 1, 0), (64, 96, 160, 4, 1, 2, 0), (128, 128, 128, 8, 2, 2, 1),
]


@needs_ref
@pytest.mark.parametrize("cfg", CONFIGS)
def test_prefill_bit_exact_vs_reference_cpu_prefill(cfg):
    D, SQ, SK, HQ, HK, B, causal = cfg
    Q, K, V = _inputs(11, B, HQ, HK, SQ, SK, D)
    ours = oracle.prefill(Q, K, V, D, SQ, SK, HQ, HK, B, causal)
    ref = oracle.ref_prefill(Q, K, V, D, SQ, SK, HQ, HK, B, causal)
    assert np.array_equal(ours, ref)


@needs_ref
@pytest.mark.parametrize("cfg", [(128, 128, 8, 8), (64, 128, 8, 8), (128, 512, 32, 8), (128, 1000, 4, 1)])
def test_decode_bit_exact_vs_reference_cpu_decode(cfg):
    D, N, HQ, HK = cfg
    q = oracle.normal(5, HQ * D)
    K = oracle.normal(6, HK * N * D)
    V = oracle.normal(7, HK * N * D)
    assert np.array_equal(oracle.decode(q, K, V, D, N, HQ, HK)[0], oracle.ref_decode(q, K, V, D, N, HQ, HK))


@pytest.mark.skipif(not oracle.ref_available("ref_fa_steps"), reason="oracle/_ref not built")
def test_prefill_bit_exact_vs_reference_fa_steps_cpu_ref():
    # The FA2 reference configuration (B1 H8 S512 D64), one head at a time as fa_naive.hip does.
    Q, K, V = _inputs(42, 1, 8, 8, 512, 512, 64, dist="uniform")
    ours = oracle.prefill(Q, K, V, 64, 512, 512, 8, 8, 1, 0)
    for h in range(8):
        assert np.array_equal(ours[0, h], oracle.ref_attn_cpu_ref(Q[0, h], K[0, h], V[0, h], 512, 512, 64))


@pytest.mark.parametrize("cfg", CONFIGS)
def test_prefill_matches_float64_softmax_attention(cfg):
    D, SQ, SK, HQ, HK, B, causal = cfg
    Q, K, V = _inputs(21, B, HQ, HK, SQ, SK, D)
    ours = oracle.prefill(Q, K, V, D, SQ, SK, HQ, HK, B, causal)
    np.testing.assert_allclose(ours, _np_attention(Q, K, V, causal), atol=2e-5, rtol=0)


def test_prefill_closed_forms():
    D, S, H = 64, 48, 2
    Q, K, V = _inputs(31, 1, H, H, S, S, D)
    # Causal row 0 sees only key 0: O = V[0] exactly.
    O = oracle.prefill(Q, K, V, D, S, S, H, H, 1, 1)
    assert np.array_equal(O[0, :, 0], V[0, :, 0])
    # Identical keys: uniform weights, O = mean of V.
    Kc = np.broadcast_to(K[:, :, :1], K.shape).copy()
    O = oracle.prefill(Q, Kc, V, D, S, S, H, H, 1, 0)
    np.testing.assert_allclose(O[0], np.broadcast_to(V[0].mean(axis=1, keepdims=True), O[0].shape), atol=1e-6)
    # One-hot V (V[k][d] = [k == d]): O[q][d] is the softmax probability of key d.
    Vh = np.zeros((1, H, S, D), np.float32)
    for k in range(S):
        Vh[0, :, k, k] = 1.0
    O = oracle.prefill(Q, K, Vh, D, S, S, H, H, 1, 0)
    s = np.einsum("hqd,hkd->hqk", Q[0].astype(np.float64), K[0].astype(np.float64)) / math.sqrt(D)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(O[0, :, :, :S], p, atol=1e-6)
    np.testing.assert_allclose(O[0].sum(-1), 1.0, atol=1e-5)


def test_planted_mistake_is_caught():
    # Swapping K and V (a transposed-operand class of mistake) must fail the float64 check.
    D, S, H = 64, 64, 2
    Q, K, V = _inputs(41, 1, H, H, S, S, D)
    good = _np_attention(Q, K, V, 0)
    wrong = oracle.prefill(Q, V, K, D, S, S, H, H, 1, 0)
    assert np.max(np.abs(wrong - good)) > 1e-2


def test_prefill_rows_and_decode_agree_with_prefill():
    D, SQ, SK, HQ, HK, B = 64, 40, 40, 4, 2, 2
    Q, K, V = _inputs(51, B, HQ, HK, SQ, SK, D)
    full = oracle.prefill(Q, K, V, D, SQ, SK, HQ, HK, B, 1)
    rows = np.array([[b, h, q] for b in range(B) for h in range(HQ) for q in (0, 7, 39)], np.int32)
    got = oracle.prefill_rows(Q, K, V, D, SQ, SK, HQ, HK, B, 1, rows)
    assert np.array_equal(got, full[rows[:, 0], rows[:, 1], rows[:, 2]])
    # A decode step is the last causal prefill row: same arithmetic, bit-identical.
    last = np.ascontiguousarray(Q[:, :, -1])
    dec = oracle.decode(last, K, V, D, SK, HQ, HK, B)
    assert np.array_equal(dec, full[:, :, -1])


def test_decode_strided_cache_equals_packed():
    D, N, HQ, HK, B, stride = 64, 33, 4, 2, 3, 48
    q = oracle.normal(61, B * HQ * D).reshape(B, HQ, D)
    Ks = oracle.normal(62, B * HK * stride * D).reshape(B, HK, stride, D)
    Vs = oracle.normal(63, B * HK * stride * D).reshape(B, HK, stride, D)
    strided = oracle.decode(q, Ks, Vs, D, N, HQ, HK, B, stride)
    packed = oracle.decode(q, np.ascontiguousarray(Ks[:, :, :N]), np.ascontiguousarray(Vs[:, :, :N]), D, N, HQ, HK, B)
    assert np.array_equal(strided, packed)


# ---- reduce / scan ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [oracle.F32, oracle.F64, oracle.I32, oracle.I64])
def test_reduce_scan_reference_kats(dtype):
    npt = {oracle.F32: np.float32, oracle.F64: np.float64, oracle.I32: np.int32, oracle.I64: np.int64}[dtype]
    lanes = np.arange(64).astype(npt)              # test_correctness.hip / bench_reduce_dpp_types.hip
    assert oracle.reduce(oracle.SUM, dtype, lanes) == 2016
    assert oracle.reduce(oracle.MAX, dtype, lanes) == 63
    assert oracle.reduce(oracle.MIN, dtype, lanes) == 0
    one_based = np.arange(1, 65).astype(npt)       # compile_smoke.hip
    assert oracle.reduce(oracle.SUM, dtype, one_based) == 2080
    assert oracle.reduce(oracle.MAX, dtype, one_based) == 64
    assert oracle.reduce(oracle.MIN, dtype, one_based) == 1
    ones = np.ones(64, npt)                        # probe_scan_dpp.hip: inclusive sum of ones = i + 1
    assert np.array_equal(oracle.scan_inclusive(oracle.SUM, dtype, ones), np.arange(1, 65))
    assert np.array_equal(oracle.scan_inclusive(oracle.MAX, dtype, lanes), np.arange(64))
    assert np.array_equal(oracle.scan_inclusive(oracle.MIN, dtype, lanes), np.zeros(64))


def test_reduce_integer_wraparound():
    x = np.array([2 ** 31 - 1, 1], np.int32)
    assert oracle.reduce(oracle.SUM, oracle.I32, x) == -(2 ** 31)
    y = np.array([2 ** 63 - 1, 2], np.int64)
    assert oracle.reduce(oracle.SUM, oracle.I64, y) == -(2 ** 63) + 1
    k = oracle.integers(9, 100003, -1000, 1000)
    assert oracle.reduce(oracle.SUM, oracle.I32, k) == int(k.astype(np.int64).sum())
    assert np.array_equal(oracle.scan_inclusive(oracle.SUM, oracle.I32, k), np.cumsum(k.astype(np.int64)).astype(np.int32))


def test_reduce_scan_floats_against_math():
    x = oracle.uniform(10, 100001)
    assert abs(oracle.reduce(oracle.SUM, oracle.F32, x) - math.fsum(x.astype(np.float64))) < 1e-9
    assert oracle.reduce(oracle.MAX, oracle.F32, x) == float(x.max())
    assert oracle.reduce(oracle.MIN, oracle.F32, x) == float(x.min())
    np.testing.assert_allclose(oracle.scan_inclusive(oracle.SUM, oracle.F32, x), np.cumsum(x.astype(np.float64)),
                               atol=1e-9)
    h = x.astype(np.float16)
    assert abs(oracle.reduce(oracle.SUM, oracle.F16, h.view(np.uint16)) - math.fsum(h.astype(np.float64))) < 1e-9
    _, bb = oracle.round16(x, oracle.BF16)
    wb = oracle.widen(bb, oracle.BF16).astype(np.float64)
    assert abs(oracle.reduce(oracle.SUM, oracle.BF16, bb) - math.fsum(wb)) < 1e-9
    np.testing.assert_allclose(oracle.scan_inclusive(oracle.MAX, oracle.BF16, bb), np.maximum.accumulate(wb))


def test_reduce_empty_is_identity():
    e = np.zeros(0, np.float32)
    assert oracle.reduce(oracle.SUM, oracle.F32, e) == 0.0
    assert oracle.reduce(oracle.MAX, oracle.F32, e) == float(np.finfo(np.float32).min)
    assert oracle.reduce(oracle.MAX, oracle.I32, np.zeros(0, np.int32)) == -(2 ** 31)
    assert oracle.reduce(oracle.MIN, oracle.I64, np.zeros(0, np.int64)) == 2 ** 63 - 1


# ---- norms / RoPE ----------------------------------------------------------------------------

def _lcg_rows(M, H):
    # bench_layernorm.hip:131 input generator: ((i * 1103515245 + 12345) & 0xff) / 32 - 4
    i = np.arange(M * H, dtype=np.uint64)
    return ((((i * 1103515245 + 12345) & 0xFF).astype(np.float32)) / 32.0 - 4.0).reshape(M, H)


def test_layernorm_invariants():
    X = _lcg_rows(64, 768)
    ones, zeros = np.ones(768, np.float32), np.zeros(768, np.float32)
    Y = oracle.layernorm(X, ones, zeros, 1e-5)
    np.testing.assert_allclose(Y.mean(axis=1), 0.0, atol=1e-5)
    np.testing.assert_allclose(Y.var(axis=1), 1.0, atol=1e-3)
    # Invariant under x -> a x + b (a > 0), and affine in (gamma, beta).
    Y2 = oracle.layernorm(3.0 * X + 5.0, ones, zeros, 1e-5)
    np.testing.assert_allclose(Y2, Y, atol=1e-4)
    g, b = oracle.uniform(1, 768, 0.5, 2.0), oracle.uniform(2, 768)
    np.testing.assert_allclose(oracle.layernorm(X, g, b, 1e-5), Y * g + b, atol=1e-5)


def test_rmsnorm_invariants():
    X = oracle.normal(3, 16 * 768, 0.0, 2.0).reshape(16, 768)
    w1 = np.full(768, 0x3C00, np.uint16)                   # fp16 1.0
    Y = oracle.rmsnorm(X, w1, 1e-6)
    np.testing.assert_allclose(np.sqrt((Y.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-5)
    np.testing.assert_allclose(oracle.rmsnorm(7.0 * X, w1, 0.0), oracle.rmsnorm(X, w1, 0.0), atol=1e-5)
    w2 = np.full(768, 0x4000, np.uint16)                   # fp16 2.0 doubles the output
    np.testing.assert_allclose(oracle.rmsnorm(X, w2, 1e-6), 2.0 * Y, atol=1e-6)


def test_softmax_rows_against_scipy_and_invariants():
    from scipy.special import softmax
    X = _lcg_rows(64, 512)                                  # bench_softmax.hip:117 input generator
    Y = oracle.softmax_rows(X)
    np.testing.assert_allclose(Y.sum(axis=1, dtype=np.float64), 1.0, atol=1e-6)   # bench_softmax.hip:123-133
    want = softmax(X.astype(np.float64), axis=1)
    np.testing.assert_allclose(Y, want, rtol=2e-7, atol=0)
    # Shift invariance (exact: the oracle subtracts the row maximum first), a constant row is
    # uniform, one dominant entry takes all the weight, and a permutation of a row permutes it.
    np.testing.assert_array_equal(oracle.softmax_rows(X + 2.0), Y)
    assert np.all(oracle.softmax_rows(np.full((2, 77), 3.5, np.float32)) == np.float32(1.0 / 77))
    row = np.zeros((1, 9), np.float32)
    row[0, 4] = 200.0
    assert oracle.softmax_rows(row)[0, 4] == 1.0 and oracle.softmax_rows(row).sum() == 1.0
    perm = np.random.default_rng(0).permutation(512)
    np.testing.assert_array_equal(oracle.softmax_rows(X[:, perm]), Y[:, perm])
    Z = oracle.normal(6, 3 * 1000, 0.0, 8.0).reshape(3, 1000)   # wide spread: tiny weights stay relative
    np.testing.assert_allclose(oracle.softmax_rows(Z), softmax(Z.astype(np.float64), axis=1), rtol=2e-7,
                               atol=1e-44)


def test_rope_table_and_rotation():
    D, T, heads = 64, 20, 3
    c, s = oracle.rope_table(0, T, D, 10000.0)
    np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-6)
    assert np.array_equal(c[:, : D // 2], c[:, D // 2:]) and np.array_equal(s[:, : D // 2], s[:, D // 2:])
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    ang = np.arange(T)[:, None] * 10000.0 ** (-2.0 * np.arange(D // 2)[None, :] / D)
    np.testing.assert_allclose(c[:, : D // 2], np.cos(ang), atol=2e-5)
    vals, bits = oracle.round16(oracle.normal(4, T * heads * D), oracle.F16)
    out = oracle.widen(oracle.rope(bits, c, s, T, heads, D), oracle.F16).reshape(T, heads, D)
    x = vals.reshape(T, heads, D).astype(np.float64)
    # Independent formulation: rotate-half RoPE multiplies (x_d + i x_{d+D/2}) by e^{i angle}.
    z = (x[..., : D // 2] + 1j * x[..., D // 2:]) * np.exp(1j * ang.astype(np.float64))[:, None, :]
    want = np.concatenate([z.real, z.imag], axis=-1)
    np.testing.assert_allclose(out, want, atol=2e-3 * np.abs(want).max())
    assert np.array_equal(out[0], vals.reshape(T, heads, D)[0])  # position 0 is the identity


def test_scatter_and_repack_are_the_reference_index_maps():
    # forward.hpp:190-220 restated; checked against numpy's own indexing and transposes.
    rng = np.random.default_rng(7)
    T, heads, D, pos0, max_seq = 5, 3, 10, 2, 9
    src = rng.integers(0, 1 << 16, T * heads * D, dtype=np.uint16)
    cache = rng.integers(0, 1 << 16, heads * max_seq * D, dtype=np.uint16)
    got = oracle.scatter_kv(src, cache, T, heads, D, pos0, max_seq).reshape(heads, max_seq, D)
    want = cache.reshape(heads, max_seq, D).copy()
    want[:, pos0:pos0 + T, :] = src.reshape(T, heads, D).transpose(1, 0, 2)
    assert np.array_equal(got, want)
    hm = oracle.repack(src, T, heads, D, 0)
    assert np.array_equal(hm.reshape(heads, T, D), src.reshape(T, heads, D).transpose(1, 0, 2))
    assert np.array_equal(oracle.repack(hm, T, heads, D, 1), src)


def test_rope_append_is_rope_then_layout():
    # The fused layer-loop step equals rope on token-major copies followed by the layout maps.
    T, nQH, nKVH, D, pos0, max_seq = 6, 4, 2, 16, 3, 12
    c, s = oracle.rope_table(pos0, T, D, 10000.0)
    _, q = oracle.round16(oracle.normal(1, T * nQH * D), oracle.F16)
    _, k = oracle.round16(oracle.normal(2, T * nKVH * D), oracle.F16)
    _, v = oracle.round16(oracle.normal(3, T * nKVH * D), oracle.F16)
    Kc0 = np.full(nKVH * max_seq * D, 0x7e00, np.uint16)    # a NaN pattern outside the slot
    Vc0 = np.full(nKVH * max_seq * D, 0x7e00, np.uint16)
    q_out, Kc, Vc = oracle.rope_append_kv(q, k, v, Kc0, Vc0, c, s, T, nQH, nKVH, D, pos0, max_seq)
    qr = oracle.rope(q, c, s, T, nQH, D).reshape(T, nQH, D)
    kr = oracle.rope(k, c, s, T, nKVH, D).reshape(T, nKVH, D)
    assert np.array_equal(q_out.reshape(nQH, T, D), qr.transpose(1, 0, 2))
    Kw = Kc0.reshape(nKVH, max_seq, D).copy(); Kw[:, pos0:pos0 + T] = kr.transpose(1, 0, 2)
    Vw = Vc0.reshape(nKVH, max_seq, D).copy(); Vw[:, pos0:pos0 + T] = v.reshape(T, nKVH, D).transpose(1, 0, 2)
    assert np.array_equal(Kc.reshape(nKVH, max_seq, D), Kw) and np.array_equal(Vc.reshape(nKVH, max_seq, D), Vw)
