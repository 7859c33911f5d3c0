"""The machine's measured ceilings (tests/native/ceilings.hip): a streaming read of 1 GiB with
non-temporal and with default loads, a non-temporal 1 GiB copy, and a bare stream of
v_mfma_f32_16x16x32_bf16 on every CU (with and without one exponential per two MFMAs), and one CU's
asynchronous global -> LDS copy rate. The
kernels' roofline fractions are quoted against the published peaks; these figures are what the
design notes compare them with as achievable on the box (decode, reduce, scan, prefill). The test
prints them and checks only that they are plausible for an MI355X."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "ceilings")


def test_measured_ceilings():
    assert os.path.exists(EXE), "tests/native not built"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    c = json.loads(r.stdout.strip().splitlines()[-1])
    print("ceilings:", json.dumps(c), flush=True)
    assert 2000 < c["read_nt_GBs"] < 8000 and 2000 < c["read_GBs"] < 8000
    assert 2000 < c["copy_nt_GBs"] < 8000
    assert 300 < c["mfma_bf16_TFLOPs"] < 2600 and 300 < c["mfma_bf16_exp_TFLOPs"] < 2600
    assert 10 < c["lds_dma_cu_GBs"] < 1000
    assert 2000 < c["lds_dma_nt_GBs"] < 8000
