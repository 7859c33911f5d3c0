"""cdna3_attn_decode_noalloc, the allocation-free decode, through the C ABI.

It runs the split-K plan of cdna3_attn_decode with a workspace, with the partials in the
library's static per-GPU scratch array instead, so its output must equal that entry point's bit
for bit. Two calls in a row, the second on a smaller input (the array keeps the first call's
partials; the second must not read them), a call whose partials exceed the array is rejected
before anything is launched, and a call captured in a HIP graph replays correctly on new inputs.
"""
import ctypes

import pytest
import torch

import cdna4
from gpu_util import DEV

pytestmark = pytest.mark.gpu


def _inputs(cfg, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    st = cfg.stride_kv or cfg.N
    q = torch.randn(cfg.batch, cfg.nQHeads, cfg.D, device=DEV, generator=g).to(dtype)
    K = torch.randn(cfg.batch, cfg.nKVHeads, st, cfg.D, device=DEV, generator=g).to(dtype)
    V = torch.randn(cfg.batch, cfg.nKVHeads, st, cfg.D, device=DEV, generator=g).to(dtype)
    return q, K, V


def _noalloc_abi(q, K, V, o, cfg, dtype):
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return cdna4.lib().cdna3_attn_decode_noalloc(p(q), p(K), p(V), p(o), ctypes.byref(cfg),
                                                cdna4.BF16 if dtype == torch.bfloat16 else cdna4.F16, stream)


def _check_equal_to_workspace_entry_point(cfg, dtype, seed):
    plan = cdna4.decode_plan(cfg, dtype, with_workspace=True)
    print(f"noalloc D{cfg.D} N{cfg.N} {cfg.nQHeads}/{cfg.nKVHeads} B{cfg.batch} stride{cfg.stride_kv} {dtype} -> "
          f"{plan.name} P{plan.partials} ws {plan.workspace} B", flush=True)
    assert plan.name == "decode_split"
    assert plan.workspace <= cdna4.decode_noalloc_max_bytes()
    q, K, V = _inputs(cfg, dtype, seed)
    o_ws = torch.empty_like(q)
    ws = torch.empty(cdna4.decode_workspace_size(cfg), dtype=torch.uint8, device=DEV)
    cdna4.decode(q, K, V, o_ws, cfg, workspace=ws)
    o = torch.full_like(q, float("nan"))
    assert _noalloc_abi(q, K, V, o, cfg, dtype) == 0
    torch.cuda.synchronize()
    assert torch.equal(o, o_ws)


def test_noalloc_equals_decode_with_workspace_twice_second_smaller():
    _check_equal_to_workspace_entry_point(cdna4.DecodeCfg(128, 8192, 32, 8, 8), torch.float16, 1)
    _check_equal_to_workspace_entry_point(cdna4.DecodeCfg(128, 3000, 32, 8, 1, 4096), torch.bfloat16, 2)


def test_noalloc_short_cache_one_launch():
    # A short cache takes the one-launch plan, which needs no scratch at all.
    cfg = cdna4.DecodeCfg(64, 300, 12, 4, 2)
    assert cdna4.decode_plan(cfg, torch.float16).name == "decode_wg"
    q, K, V = _inputs(cfg, torch.float16, 3)
    o_ref = torch.empty_like(q)
    cdna4.decode(q, K, V, o_ref, cfg)
    o = torch.full_like(q, float("nan"))
    assert _noalloc_abi(q, K, V, o, cfg, torch.float16) == 0
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)


def test_noalloc_rejects_calls_beyond_the_scratch():
    # 1001 sequences x 64 query heads: one partial per head is 1001 * 64 * 130 * 4 B = 33 MB
    # (4,004 (batch, kv head) rows, not whole rounds of the CUs: the split-K plan).
    cfg = cdna4.DecodeCfg(128, 4096, 64, 4, 1001)
    assert cdna4.decode_workspace_size(cfg) > cdna4.decode_noalloc_max_bytes()
    small = torch.empty(4096, dtype=torch.float16, device=DEV)   # never read: rejected before launch
    rc = _noalloc_abi(small, small, small, small, cfg, torch.float16)
    assert rc == 0x4344, rc                     # CDNA4_ERR_SCRATCH_TOO_SMALL, outside the hipError_t range
    assert "static array" in cdna4.error_string(rc)
    assert "static array" not in cdna4.error_string(2)    # hipErrorOutOfMemory keeps its own message


def test_noalloc_captured_in_a_graph_and_replayed_with_new_inputs():
    # The entry point's purpose: a call captured into a HIP graph (no allocation inside the
    # capture), replayed after new inputs are written into the same buffers. Each replay, with
    # eager work and synchronisations between replays, must equal the workspace entry point on
    # the same inputs bit for bit.
    cfg = cdna4.DecodeCfg(128, 8192, 32, 8, 8)
    dtype = torch.float16
    assert cdna4.decode_plan(cfg, dtype, with_workspace=True).name == "decode_split"
    q, K, V = _inputs(cfg, dtype, 20)
    o = torch.empty_like(q)
    ws = torch.empty(cdna4.decode_workspace_size(cfg), dtype=torch.uint8, device=DEV)
    assert _noalloc_abi(q, K, V, o, cfg, dtype) == 0   # first call on the device outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _noalloc_abi(q, K, V, o, cfg, dtype)
    assert rc == 0
    for seed in (21, 22, 23):
        q2, K2, V2 = _inputs(cfg, dtype, seed)
        q.copy_(q2)
        K.copy_(K2)
        V.copy_(V2)
        o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        o_ws = torch.empty_like(q)
        cdna4.decode(q, K, V, o_ws, cfg, workspace=ws)
        torch.cuda.synchronize()
        print(f"replay seed {seed}: equal {torch.equal(o, o_ws)}", flush=True)
        assert torch.equal(o, o_ws)
