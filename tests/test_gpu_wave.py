"""Lane-by-lane checks of the header-only device primitives on gfx950 (through the test hooks
in tests/native/wave_hooks.hip): wave::dpp reductions / scans / broadcast, the reference-
compatible wave:: API, ballots, the MFMA accessors and the dme async copies.
Known answers follow the reference's own tests (test_correctness.hip:43-260,
probe_scan_dpp.hip:13-35, bench_reduce_dpp_types.hip:60-81, compile_smoke.hip:24-50,
probe_mfma_mapping.hip:44-75, probe_dme.hip)."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DEV, hooks, ptr, stream

pytestmark = pytest.mark.gpu

DPP_SUM, DPP_MAX, DPP_MIN, DPP_SUM_B, DPP_SCAN, DPP_SCAN_MAX, DPP_SCAN_MIN, DPP_SCAN_EX, BCAST63, \
    PORT_SUM, PORT_SCAN, PORT_SCAN_EX, PORT_AND, PORT_OR, DPP_SCAN_EX_MAX, SOFTMAX, PORT_MAX, PORT_MIN, \
    DPP_MOVE_SHR1, DPP_STEP1, DPP_STEP4, DPP_STEP1248 = range(22)
TYPES = {oracle.F32: (np.float32, torch.float32), oracle.F64: (np.float64, torch.float64),
         oracle.I32: (np.int32, torch.int32), oracle.I64: (np.int64, torch.int64)}


def run(kind, dtype, x: np.ndarray) -> np.ndarray:
    nt, tt = TYPES[dtype]
    xin = torch.from_numpy(np.ascontiguousarray(x, nt)).to(DEV)
    out = torch.empty_like(xin)
    assert hooks().hook_wave(kind, dtype, ptr(xin), ptr(out), x.size // 64, stream()) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


def per_wave(x, fn):
    return np.concatenate([np.broadcast_to(fn(w), (64,)) if np.ndim(fn(w)) == 0 else fn(w) for w in x.reshape(-1, 64)])


@pytest.mark.parametrize("dtype", list(TYPES))
def test_reduce_known_answers_lane_by_lane(dtype):
    lanes = np.tile(np.arange(64), 3)
    for kind in (DPP_SUM, DPP_SUM_B, PORT_SUM):
        assert np.all(run(kind, dtype, lanes) == 2016), kind        # result on every lane
    assert np.all(run(DPP_MAX, dtype, lanes) == 63) and np.all(run(PORT_MAX, dtype, lanes) == 63)
    assert np.all(run(DPP_MIN, dtype, lanes) == 0) and np.all(run(PORT_MIN, dtype, lanes) == 0)
    one_based = np.tile(np.arange(1, 65), 2)
    assert np.all(run(DPP_SUM, dtype, one_based) == 2080)
    assert np.all(run(DPP_MAX, dtype, one_based) == 64) and np.all(run(DPP_MIN, dtype, one_based) == 1)
    neg = -np.tile(np.arange(1, 65), 2)      # max over negatives needs the right identity
    assert np.all(run(DPP_MAX, dtype, neg) == -1)


@pytest.mark.parametrize("dtype", list(TYPES))
def test_scan_known_answers_lane_by_lane(dtype):
    ones = np.ones(128)
    assert np.array_equal(run(DPP_SCAN, dtype, ones), np.tile(np.arange(1, 65), 2))
    assert np.array_equal(run(PORT_SCAN, dtype, ones), np.tile(np.arange(1, 65), 2))
    assert np.array_equal(run(DPP_SCAN_EX, dtype, ones), np.tile(np.arange(64), 2))
    assert np.array_equal(run(PORT_SCAN_EX, dtype, ones), np.tile(np.arange(64), 2))
    lanes = np.tile(np.arange(64), 2)
    assert np.array_equal(run(DPP_SCAN_MAX, dtype, lanes), lanes)
    assert np.array_equal(run(DPP_SCAN_MIN, dtype, lanes), np.zeros(128))
    rev = np.tile(np.arange(63, -1, -1), 2)
    assert np.array_equal(run(DPP_SCAN_MIN, dtype, rev), rev)
    assert np.array_equal(run(DPP_SCAN_MAX, dtype, rev), np.full(128, 63))
    assert np.array_equal(run(BCAST63, dtype, lanes), np.full(128, 63))


@pytest.mark.parametrize("dtype", list(TYPES))
def test_dpp_building_blocks_lane_by_lane(dtype):
    # dpp_move (wave_reduce_dpp.hpp:61-64) and scan_dpp_step (wave_scan_dpp.hpp:43-49): row_shr
    # moves within 16-lane rows; lanes without a source in their row take old / identity.
    lanes = np.tile(np.arange(64), 2)
    r = lanes % 16
    assert np.array_equal(run(DPP_MOVE_SHR1, dtype, lanes), np.where(r >= 1, lanes - 1, -7))
    assert np.array_equal(run(DPP_STEP1, dtype, lanes), np.where(r >= 1, 2 * lanes - 1, lanes))
    rev = np.tile(np.arange(63, -1, -1), 2)
    rr = np.tile(np.arange(64), 2) % 16
    assert np.array_equal(run(DPP_STEP4, dtype, rev), np.where(rr >= 4, rev + 4, rev))
    ones = np.ones(128)
    assert np.array_equal(run(DPP_STEP1248, dtype, ones), r + 1)   # in-row inclusive prefix


def test_integer_scans_and_reductions_bit_exact_random():
    for dtype, lo, hi in ((oracle.I32, -1000, 1000), (oracle.I64, -(2 ** 40), 2 ** 40)):
        nt = TYPES[dtype][0]
        x = oracle.integers(17, 64 * 64, lo, hi, nt).astype(nt)
        w = x.reshape(-1, 64).astype(np.int64)
        assert np.array_equal(run(DPP_SUM, dtype, x), np.repeat(w.sum(1), 64).astype(nt))
        assert np.array_equal(run(DPP_MAX, dtype, x), np.repeat(w.max(1), 64).astype(nt))
        assert np.array_equal(run(DPP_MIN, dtype, x), np.repeat(w.min(1), 64).astype(nt))
        inc = np.cumsum(w, axis=1)
        assert np.array_equal(run(DPP_SCAN, dtype, x), inc.reshape(-1).astype(nt))
        assert np.array_equal(run(DPP_SCAN_EX, dtype, x), (inc - w).reshape(-1).astype(nt))
        assert np.array_equal(run(DPP_SCAN_MAX, dtype, x), np.maximum.accumulate(w, 1).reshape(-1).astype(nt))
        assert np.array_equal(run(DPP_SCAN_MIN, dtype, x), np.minimum.accumulate(w, 1).reshape(-1).astype(nt))
        exmax = np.concatenate([np.full((w.shape[0], 1), np.iinfo(nt).min), np.maximum.accumulate(w, 1)[:, :-1]], 1)
        assert np.array_equal(run(DPP_SCAN_EX_MAX, dtype, x), exmax.reshape(-1).astype(nt))
        assert np.array_equal(run(BCAST63, dtype, x), np.repeat(w[:, 63], 64).astype(nt))
    x = np.full(64, 2 ** 31 - 1, np.int64)       # wrap-around of an int32 sum is defined
    got = run(DPP_SUM, oracle.I32, x.astype(np.int32))
    wrapped = np.array([((2 ** 31 - 1) * 64) % 2 ** 32], np.uint64).astype(np.uint32).view(np.int32)[0]
    assert np.all(got == wrapped)
    m = oracle.integers(5, 64 * 8, 0, 2 ** 30, np.int64).astype(np.int32)
    w = m.reshape(-1, 64)
    assert np.array_equal(run(PORT_AND, oracle.I32, m), np.repeat(np.bitwise_and.reduce(w, 1), 64))
    assert np.array_equal(run(PORT_OR, oracle.I32, m), np.repeat(np.bitwise_or.reduce(w, 1), 64))


def test_float_reductions_uniform_across_lanes_and_accurate():
    for dtype in (oracle.F32, oracle.F64):
        nt = TYPES[dtype][0]
        x = oracle.uniform(3, 64 * 32).astype(nt)
        got = run(DPP_SUM, dtype, x).reshape(-1, 64)
        assert np.all(got == got[:, :1])                  # bit-identical on every lane
        np.testing.assert_allclose(got[:, 0], x.reshape(-1, 64).astype(np.float64).sum(1), rtol=0,
                                   atol=1e-5 if dtype == oracle.F32 else 1e-12)
        scan = run(DPP_SCAN, dtype, x).reshape(-1, 64)
        np.testing.assert_allclose(scan, np.cumsum(x.reshape(-1, 64).astype(np.float64), 1), rtol=0,
                                   atol=1e-5 if dtype == oracle.F32 else 1e-12)
        ex = run(DPP_SCAN_EX, dtype, x).reshape(-1, 64)
        assert np.all(ex[:, 0] == 0)
        assert np.array_equal(ex[:, 1:], scan[:, :-1])     # exclusive = shifted inclusive, exactly


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_half_inputs_accumulate_in_fp32(tdt):
    kind = oracle.F16 if tdt == torch.float16 else oracle.BF16
    x = oracle.uniform(8, 64 * 16)
    vals, bits = oracle.round16(x, kind)
    xin = torch.from_numpy(bits.view(np.int16)).view(tdt).to(DEV)
    out = torch.empty(x.size, dtype=torch.float32, device=DEV)

    def go(k):
        assert hooks().hook_wave(k, kind, ptr(xin), ptr(out), x.size // 64, stream()) == 0
        torch.cuda.synchronize()
        return out.cpu().numpy().reshape(-1, 64)

    w = vals.reshape(-1, 64).astype(np.float64)
    np.testing.assert_allclose(go(DPP_SUM)[:, 0], w.sum(1), rtol=1e-3, atol=1e-5)
    np.testing.assert_allclose(go(DPP_SCAN), np.cumsum(w, 1), rtol=1e-3, atol=1e-5)
    assert np.array_equal(go(DPP_MAX)[:, 0], w.max(1)) and np.array_equal(go(DPP_MIN)[:, 0], w.min(1))
    # Reference bench input: 64 lanes of 0.1 (bench_bf16acc.hip:66): fp32 accumulation keeps 64 * x exactly.
    v01, b01 = oracle.round16(np.full(64, 0.1, np.float32), kind)
    xin = torch.from_numpy(b01.view(np.int16)).view(tdt).to(DEV)
    out = torch.empty(64, dtype=torch.float32, device=DEV)
    assert hooks().hook_wave(DPP_SUM, kind, ptr(xin), ptr(out), 1, stream()) == 0
    torch.cuda.synchronize()
    assert np.all(out.cpu().numpy() == np.float32(64 * np.float64(v01[0])))


def test_ballot_family():
    pred = np.tile((np.arange(64) % 2 == 0).astype(np.int32), 2)      # even lanes (test_correctness.hip)
    xin = torch.from_numpy(pred).to(DEV)
    out = torch.empty(128 * 5, dtype=torch.int64, device=DEV)
    assert hooks().hook_ballot(ptr(xin), ptr(out), 2, stream()) == 0
    torch.cuda.synchronize()
    o = out.cpu().numpy().view(np.uint64).reshape(128, 5)
    assert np.all(o[:, 0] == 0x5555555555555555) and np.all(o[:, 1] == 32)
    assert np.all(o[:, 2] == 1) and np.all(o[:, 3] == 0)
    assert np.array_equal(o[:64, 4], np.array([(1 << i) - 1 for i in range(64)], np.uint64))


def test_row_softmax_lane():
    x = oracle.uniform(12, 64 * 4, -4, 4)
    got = run(SOFTMAX, oracle.F32, x).reshape(-1, 64)
    w = x.reshape(-1, 64).astype(np.float64)
    p = np.exp(w - w.max(1, keepdims=True))
    np.testing.assert_allclose(got, p / p.sum(1, keepdims=True), atol=1e-6)


def _mm(which, A, B):
    if which == 5:   # fp32 operands
        ta = torch.from_numpy(np.ascontiguousarray(A, np.float32)).to(DEV)
        tb = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(DEV)
    else:
        half = which in (0, 1, 3)
        dt = torch.float16 if half else torch.bfloat16
        kind = oracle.F16 if half else oracle.BF16
        _, ab = oracle.round16(A.astype(np.float32), kind)
        _, bb = oracle.round16(B.astype(np.float32), kind)
        ta = torch.from_numpy(ab.view(np.int16)).view(dt).to(DEV)
        tb = torch.from_numpy(bb.view(np.int16)).view(dt).to(DEV)
    c = torch.zeros(A.shape[0] * B.shape[1], dtype=torch.float32, device=DEV)
    assert hooks().hook_mfma(which, ptr(ta), ptr(tb), ptr(c), stream()) == 0
    torch.cuda.synchronize()
    return c.cpu().numpy().reshape(A.shape[0], B.shape[1])


@pytest.mark.parametrize("which,shape", [(0, (16, 16, 16)), (1, (16, 32, 16)), (2, (16, 32, 16)),
                                         (3, (32, 16, 32)), (4, (32, 16, 32)), (5, (16, 4, 16))])
def test_mfma_lane_mapping_exact_gemm(which, shape):
    M, K, N = shape
    # Small integers: every product and sum is exact in fp32 (probe_mfma_mapping.hip style).
    A = ((np.arange(M * K).reshape(M, K) * 7) % 13 - 6).astype(np.float64)
    B = ((np.arange(K * N).reshape(K, N) * 5) % 11 - 5).astype(np.float64)
    assert np.array_equal(_mm(which, A, B), A @ B)
    # compile_smoke.hip: C[0] of a 16x16x16 tile of fp16(0.01) = 16 * fp16(0.01)^2.
    if which == 0:
        h = np.float64(np.float16(0.01))
        got = _mm(0, np.full((16, 16), 0.01), np.full((16, 16), 0.01))
        np.testing.assert_allclose(got, 16 * h * h, rtol=1e-6)


def test_dme_async_copies_are_byte_exact():
    src = torch.from_numpy((np.arange(4096) * 37 % 251).astype(np.uint8)).to(DEV)
    dst = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    fsrc = torch.from_numpy(oracle.uniform(1, 256)).to(DEV)
    fdst = torch.zeros(256, dtype=torch.float32, device=DEV)
    hs = oracle.round16(oracle.normal(2, 16 * 96), oracle.F16)[1].reshape(16, 96)
    hsrc = torch.from_numpy(hs.view(np.int16)).to(DEV)
    hdst = torch.zeros(16 * 64, dtype=torch.int16, device=DEV)
    assert hooks().hook_dme(ptr(src), ptr(dst), ptr(fsrc), ptr(fdst), ptr(hsrc), ptr(hdst), stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(src, dst) and torch.equal(fsrc, fdst)
    assert np.array_equal(hdst.cpu().numpy().view(np.uint16).reshape(16, 64), hs[:, :64])


def test_dme_forms_the_reference_kernels_call():
    # copy_element / copy_element_stream (per-lane slot tile[L], research/flash-attention-mi300x/
    # fa_dme.hip:129-155), copy_tile_1d_stream (tensor_prefetch.hpp:151-196), prefetch_tile2d_fp16
    # over two waves (fa_decode_dme_kernel.hpp:129-130) and AsyncTile2D's prologue / prefetch_next /
    # wait_next / advance over five tiles (probe_dme.hip semantics: out[i] == src[i]).
    fsrc = torch.from_numpy(np.arange(384, dtype=np.float32) * 1.5 - 100).to(DEV)
    fout = torch.zeros(384, dtype=torch.float32, device=DEV)
    hs = oracle.round16(oracle.normal(4, 32 * 64), oracle.F16)[1]
    hsrc = torch.from_numpy(hs.view(np.int16)).to(DEV)
    hout = torch.zeros(32 * 64, dtype=torch.int16, device=DEV)
    n_tiles = 5
    a = oracle.round16(oracle.normal(5, n_tiles * 16 * 64), oracle.F16)[1]
    asrc = torch.from_numpy(a.view(np.int16)).to(DEV)
    aout = torch.zeros(n_tiles * 16 * 64, dtype=torch.int16, device=DEV)
    assert hooks().hook_dme_forms(ptr(fsrc), ptr(fout), ptr(hsrc), ptr(hout), ptr(asrc), ptr(aout), n_tiles,
                                  stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(fout, fsrc)
    assert np.array_equal(hout.cpu().numpy().view(np.uint16), hs)
    assert np.array_equal(aout.cpu().numpy().view(np.uint16), a)


@pytest.mark.parametrize("n_tiles", [1, 3, 8])
def test_online_softmax_step_over_tiles(n_tiles):
    # cdna3::ex::online_softmax_step (cdna3-prims/examples/fused_softmax.hpp:37-48) folded over
    # several 64-wide tiles equals one softmax over all of them (float64 reference); later tiles
    # carry larger scores so the running maximum and the rescale factor change.
    s = (oracle.uniform(30 + n_tiles, 64 * n_tiles, -3, 3) + np.repeat(np.arange(n_tiles), 64)).astype(np.float32)
    v = oracle.uniform(40 + n_tiles, 64 * n_tiles, -1, 1)
    out = torch.zeros(3, dtype=torch.float32, device=DEV)
    ts, tv = torch.from_numpy(s).to(DEV), torch.from_numpy(v).to(DEV)
    assert hooks().hook_online_softmax(ptr(ts), ptr(tv), n_tiles, ptr(out), stream()) == 0
    torch.cuda.synchronize()
    m, l, o = out.cpu().numpy().astype(np.float64)
    x = s.astype(np.float64)
    assert m == x.max()
    p = np.exp(x - x.max())
    assert abs(l - p.sum()) <= 1e-5 * p.sum()
    assert abs(o - (p / p.sum()) @ v.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("which", [0, 1, 2])
def test_mma_tile_accumulate_exact_gemm(which):
    # cdna3::ex::mma_tile_accumulate (async_tiled_gemm.hpp:52-60) and its 16x16x32 form, with
    # leading dimensions wider than the tile; small integers make every product exact.
    K = 16 if which == 0 else 32
    ldA, ldB, ldC = K + 8, 24, 20
    A = ((np.arange(16 * ldA).reshape(16, ldA) * 7) % 13 - 6).astype(np.float32)
    B = ((np.arange(K * ldB).reshape(K, ldB) * 5) % 11 - 5).astype(np.float32)
    kind, dt = (oracle.BF16, torch.bfloat16) if which == 2 else (oracle.F16, torch.float16)
    ta = torch.from_numpy(oracle.round16(A, kind)[1].view(np.int16)).view(dt).to(DEV)
    tb = torch.from_numpy(oracle.round16(B, kind)[1].view(np.int16)).view(dt).to(DEV)
    c = torch.full((16 * ldC,), -1.0, dtype=torch.float32, device=DEV)
    assert hooks().hook_mma_tile(which, ptr(ta), ptr(tb), ptr(c), ldA, ldB, ldC, stream()) == 0
    torch.cuda.synchronize()
    got = c.cpu().numpy().reshape(16, ldC)
    assert np.array_equal(got[:, :16], A[:, :K].astype(np.float64) @ B[:, :16].astype(np.float64))
    assert np.all(got[:, 16:] == -1.0)   # nothing written past the tile's 16 columns
