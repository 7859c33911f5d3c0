"""Device-wide reduce / inclusive scan (cdna3_reduce, cdna3_scan_inclusive) against the oracle:
bit-exact for integers (two's-complement wrap), rel 1e-3 (or tighter) for floats, over ragged
and edge sizes, misaligned inputs, every op and dtype, and the full 2^26-element sweep."""
import numpy as np
import pytest
import torch

import cdna4
import oracle
from gpu_util import DEV

pytestmark = pytest.mark.gpu

TORCH = {oracle.F32: torch.float32, oracle.F64: torch.float64, oracle.I32: torch.int32, oracle.I64: torch.int64,
         oracle.F16: torch.float16, oracle.BF16: torch.bfloat16}
SIZES = [0, 1, 2, 63, 64, 65, 255, 1023, 4095, 4096, 4097, 8193, 100003, (1 << 20) + 7]


def make(dtype, n, seed, offset=0):
    """Host values (what the oracle reads) and a device tensor view starting `offset` elements in."""
    if dtype == oracle.I32:
        h = oracle.integers(seed, n + offset, -1000, 1000)
    elif dtype == oracle.I64:
        h = oracle.integers(seed, n + offset, -1000, 1000, np.int64)
    elif dtype == oracle.F64:
        h = oracle.uniform_f64(seed, n + offset)
    elif dtype == oracle.F32:
        h = oracle.uniform(seed, n + offset)
    else:
        h = oracle.round16(oracle.uniform(seed, n + offset), dtype)[1]
    t = torch.from_numpy(h.view(np.int16) if dtype in (oracle.F16, oracle.BF16) else h).to(DEV)
    if dtype in (oracle.F16, oracle.BF16):
        t = t.view(TORCH[dtype])
    return h[offset:], t[offset:]


def check_scalar(dtype, op, got, want, n):
    if dtype in (oracle.I32, oracle.I64):
        assert int(got) == int(want)
    elif op != oracle.SUM:
        assert float(got) == float(want)
    else:
        # fp32 accumulation: rel 1e-3 (the sweep's bound); fp64: n * 1e-13 absolute for n values
        # in [-1, 1] (the a-priori bound n * eps * sum|x| is far larger).
        tol = 1e-13 * max(1, n) if dtype == oracle.F64 else max(1e-6, 1e-3 * abs(want))
        assert abs(float(got) - want) <= tol, (got, want)


@pytest.mark.parametrize("dtype", [oracle.I32, oracle.I64, oracle.F32, oracle.F64, oracle.F16, oracle.BF16])
@pytest.mark.parametrize("op", [oracle.SUM, oracle.MAX, oracle.MIN])
def test_reduce_sizes(dtype, op):
    for i, n in enumerate(SIZES):
        h, t = make(dtype, n, 100 + i, offset=i % 3)    # offsets 1, 2 exercise the unaligned path
        got = cdna4.reduce(t, op).cpu().numpy()[0]
        check_scalar(dtype, op, got, oracle.reduce(op, dtype, h), n)


@pytest.mark.parametrize("dtype", [oracle.I32, oracle.I64, oracle.F32, oracle.F64, oracle.F16, oracle.BF16])
@pytest.mark.parametrize("op", [oracle.SUM, oracle.MAX, oracle.MIN])
def test_scan_sizes(dtype, op):
    for i, n in enumerate(SIZES[1:]):
        h, t = make(dtype, n, 200 + i, offset=i % 2)
        got = cdna4.scan_inclusive(t, op).cpu().numpy()
        want = oracle.scan_inclusive(op, dtype, h)
        if dtype in (oracle.I32, oracle.I64) or op != oracle.SUM:
            assert np.array_equal(got.astype(np.float64) if got.dtype.kind == "f" else got, want)
        else:
            tol = 1e-13 * n if dtype == oracle.F64 else 2e-5 * max(1.0, np.sqrt(n))
            assert np.max(np.abs(got.astype(np.float64) - want)) <= tol


@pytest.mark.parametrize("dtype", [oracle.I32, oracle.I64, oracle.F32, oracle.F64, oracle.F16, oracle.BF16])
def test_scan_tile_boundaries(dtype):
    # Inputs around multiples of every tile size the kernels use (64 lanes x 12-32 vectors of 2, 4
    # or 8 elements): the last tile full, one vector short, one element over, and a remainder below
    # one vector that the one-wave epilogue scans after the tiles. Odd sizes also run misaligned
    # (one element in), which takes the element-wise kernel with half-size tiles.
    sizes = sorted({m * k + d for m in (2048, 3072, 4096, 6144, 8192, 12288, 16384) for k in (1, 2)
                    for d in (-8, -1, 0, 1, 3, 7)})
    for i, n in enumerate(sizes):
        h, t = make(dtype, n, 900 + i, offset=n % 2)
        got = cdna4.scan_inclusive(t, "sum").cpu().numpy()
        want = oracle.scan_inclusive(oracle.SUM, dtype, h)
        if dtype in (oracle.I32, oracle.I64):
            assert np.array_equal(got, want), n
        else:
            tol = 1e-13 * n if dtype == oracle.F64 else 2e-5 * max(1.0, np.sqrt(n))
            assert np.max(np.abs(got.astype(np.float64) - want)) <= tol, n
        if dtype in (oracle.I32, oracle.F32):
            got = cdna4.scan_inclusive(t, "max").cpu().numpy()
            assert np.array_equal(got, oracle.scan_inclusive(oracle.MAX, dtype, h)), n


def test_scan_repeated_calls_reuse_workspace():
    # The look-back flags carry a per-call epoch, so one workspace serves many calls with no
    # clearing: calls alternate between two inputs and two dtypes, so that a flag left by the
    # previous call, if it were accepted, would hand a group the other input's prefix.
    n = 300007
    ha, ta = make(oracle.I32, n, 5)
    hb, tb = make(oracle.I32, n, 6)
    hc, tc = make(oracle.I64, n, 7)
    ws = torch.empty(cdna4.scan_workspace_size(n, cdna4.I64), dtype=torch.uint8, device=DEV)
    want = {id(ta): oracle.scan_inclusive(oracle.SUM, oracle.I32, ha), id(tb): oracle.scan_inclusive(oracle.SUM, oracle.I32, hb),
            id(tc): oracle.scan_inclusive(oracle.SUM, oracle.I64, hc)}
    for t in (ta, tb, ta, tc, tb, tc, ta, tb):
        got = cdna4.scan_inclusive(t, "sum", workspace=ws, check=False)
        assert cdna4.scan_status(ws) == 0
        assert np.array_equal(got.cpu().numpy(), want[id(t)])


@pytest.mark.parametrize("fill", ["zeros", "ones", "random", "stale_tags"])
def test_scan_workspace_needs_no_clearing(fill):
    # A workspace of any prior content: zeroed, all 0xFF, random bytes, or slot words whose upper
    # halves hold every small tag value (epoch 1, both kinds), never the call's own tag.
    n = (1 << 22) + 3
    h, t = make(oracle.F32, n, 9)
    size = cdna4.scan_workspace_size(n, cdna4.F32)
    if fill == "zeros":
        ws = torch.zeros(size, dtype=torch.uint8, device=DEV)
    elif fill == "ones":
        ws = torch.full((size,), 0xFF, dtype=torch.uint8, device=DEV)
    elif fill == "random":
        ws = torch.randint(0, 256, (size,), dtype=torch.uint8, device=DEV,
                           generator=torch.Generator(device=DEV).manual_seed(3))
    else:
        words = torch.arange(size // 8, dtype=torch.int64, device=DEV)
        ws = ((((words % 2) + 5) << 32) | (words & 0xFFFF)).view(torch.uint8)   # tags 5, 6 = epoch 1
    want = oracle.scan_inclusive(oracle.SUM, oracle.F32, h)
    for _ in range(3):
        got = cdna4.scan_inclusive(t, "sum", workspace=ws, check=False)
        assert cdna4.scan_status(ws) == 0
        g = got.cpu().numpy().astype(np.float64)
        scale = np.maximum(1.0, np.sqrt(np.arange(1, n + 1, dtype=np.float64)))
        assert np.max(np.abs(g - want) / scale) <= 1e-3


@pytest.mark.parametrize("dtype", [oracle.I32, oracle.I64, oracle.F32, oracle.F64, oracle.F16, oracle.BF16])
def test_full_sweep_2_26(dtype):
    n = 1 << 26
    h, t = make(dtype, n, 7)
    for op in (oracle.SUM, oracle.MAX, oracle.MIN):
        got = cdna4.reduce(t, op).cpu().numpy()[0]
        want = oracle.reduce(op, dtype, h)
        if dtype in (oracle.I32, oracle.I64) or op != oracle.SUM:
            assert float(got) == float(want) if dtype not in (oracle.I32, oracle.I64) else int(got) == int(want)
        else:
            assert abs(float(got) - want) <= 1e-3 * max(1.0, abs(want))
    got = cdna4.scan_inclusive(t, "sum")
    want = oracle.scan_inclusive(oracle.SUM, dtype, h)
    if dtype in (oracle.I32, oracle.I64):
        assert np.array_equal(got.cpu().numpy(), want)
    else:
        g = got.cpu().numpy().astype(np.float64)
        # rel 1e-3 of the running magnitude (the prefix of U(-1,1) wanders ~sqrt(i))
        scale = np.maximum(1.0, np.sqrt(np.arange(1, n + 1, dtype=np.float64)))
        assert np.max(np.abs(g - want) / scale) <= 1e-3
    # Checksum of checksums: the last prefix equals the total.
    if dtype in (oracle.I32, oracle.I64):
        assert int(got[-1].item()) == int(cdna4.reduce(t, "sum").item())


def test_scan_timeout_is_reported_not_silent(monkeypatch):
    # Force the look-back's bounded wait to give up at once (CDNA4_SCAN_SPIN_LIMIT=0): tiles whose
    # predecessors have not published yet stop waiting, every kernel still finishes, and the
    # workspace status word reports the invalid result, so the Python scan raises instead of
    # returning it. With the normal bound the same call is valid.
    n = 1 << 24
    h, t = make(oracle.I32, n, 11)
    ws = torch.empty(cdna4.scan_workspace_size(n, cdna4.I32), dtype=torch.uint8, device=DEV)
    monkeypatch.setenv("CDNA4_SCAN_SPIN_LIMIT", "0")
    with pytest.raises(cdna4.CDNA4Error):
        for _ in range(8):   # some tile must find its predecessor unpublished
            cdna4.scan_inclusive(t, "sum", workspace=ws)
    assert cdna4.scan_status(ws) != 0
    monkeypatch.delenv("CDNA4_SCAN_SPIN_LIMIT")
    got = cdna4.scan_inclusive(t, "sum", workspace=ws)
    assert cdna4.scan_status(ws) == 0
    assert np.array_equal(got.cpu().numpy(), oracle.scan_inclusive(oracle.SUM, oracle.I32, h))
