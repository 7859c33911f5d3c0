"""Every kernel the prefill and decode dispatchers can pick, against the CPU oracle.

Each case first asks the library which kernel it will launch (cdna3_attn_prefill_plan /
cdna3_attn_decode_plan) and asserts the one the case is meant to cover, then compares the GPU
output with the oracle (the restated cpu_prefill / cpu_decode of
cdna3-prims/tests/validate_attention_api.hip:27-72) on the same rounded inputs. Large prefill
shapes are checked on a seeded subsample of query rows of every (or every listed) head, with the
output pre-filled with NaN so that an unwritten row anywhere in the tensor fails the finiteness
check. Bound (gpu_util.check_parity): |gpu - ref| <= 2e-3 max(1, |ref|), plus half a bf16 ulp of ref for
bf16 outputs (the stored output's own rounding).
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import cdna4
import oracle
from gpu_util import DEV, check_parity

pytestmark = pytest.mark.gpu

_POOL = ThreadPoolExecutor(max_workers=8)   # the oracle is C called through ctypes (GIL released)


def _randn(shape, dtype, g):
    return torch.randn(*shape, device=DEV, generator=g).to(dtype)


def _rows(SQ, seed, n_random=64):
    """Query rows checked per head: the first 128, the middle, the last 64 and seeded random rows."""
    rows = set(range(min(SQ, 128))) | {SQ // 2 - 1, SQ // 2} | set(range(max(0, SQ - 64), SQ))
    rows |= set(int(r) for r in oracle.integers(seed, n_random, 0, SQ - 1))
    return sorted(r for r in rows if 0 <= r < SQ)


def _oracle_heads(q, k, v, heads, rows, D, SQ, SK, HQ, HK, causal):
    """Oracle rows of the listed (batch, head) pairs, computed per head in parallel."""
    grp = HQ // HK
    req = np.array([[0, 0, r] for r in rows], np.int32)

    def one(bh):
        b, h = bh
        return oracle.prefill_rows(q[b, h], k[b, h // grp], v[b, h // grp], D, SQ, SK, 1, 1, 1, causal, req)

    return dict(zip(heads, _POOL.map(one, heads)))


def check_prefill(D, SQ, SK, HQ, HK, B, causal, dtype, kernel, seed=0, heads=None):
    cfg = cdna4.PrefillCfg(D, SQ, SK, HQ, HK, B, causal)
    plan = cdna4.prefill_plan(cfg, dtype)
    print(f"prefill D{D} SQ{SQ} SK{SK} HQ{HQ} HK{HK} B{B} causal{causal} {dtype} -> {plan.name} "
          f"(grid {plan.grid})", flush=True)
    assert plan.name == kernel
    g = torch.Generator(device=DEV).manual_seed(seed)
    Q = _randn((B, HQ, SQ, D), dtype, g)
    K = _randn((B, HK, SK, D), dtype, g)
    V = _randn((B, HK, SK, D), dtype, g)
    O = torch.full_like(Q, float("nan"))
    cdna4.prefill(Q, K, V, O, cfg)
    torch.cuda.synchronize()
    assert torch.isfinite(O.float()).all(), "unwritten or non-finite output rows"
    heads = heads or [(b, h) for b in range(B) for h in range(HQ)]
    rows = _rows(SQ, seed + 1)
    q, k, v = (t.float().cpu().numpy() for t in (Q, K, V))
    want = _oracle_heads(q, k, v, heads, rows, D, SQ, SK, HQ, HK, causal)
    o = O.float().cpu().numpy()
    print(f"  {len(heads)} heads x {len(rows)} rows", flush=True)
    check_parity([o[b, h, rows] for b, h in heads], [want[(b, h)] for b, h in heads], dtype)


# ---- fa_pipe<D, 8, 2> (plan name fa_mfma_8w): batch * heads * ceil(seqQ / 256) >= CUs (causal) --
# ---- or >= CUs / 4 (non-causal) ---------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_8w_d128_causal_mha(dtype):
    check_prefill(128, 4096, 4096, 32, 32, 2, 1, dtype, "fa_mfma_8w", seed=1,
                  heads=[(b, h) for b in (0, 1) for h in range(0, 32, 3)])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_8w_d128_noncausal(dtype):
    check_prefill(128, 4096, 4096, 32, 32, 1, 0, dtype, "fa_mfma_8w", seed=2, heads=[(0, h) for h in range(0, 32, 4)])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_8w_gqa_4to1_causal(dtype):
    check_prefill(128, 4096, 4096, 32, 8, 1, 1, dtype, "fa_mfma_8w", seed=3, heads=[(0, h) for h in range(32)])


@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_8w_d64(dtype, causal):
    check_prefill(64, 2048, 2048, 64, 64, 1, causal, dtype, "fa_mfma_8w", seed=4, heads=[(0, h) for h in range(0, 64, 5)])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_8w_ragged_causal(dtype):
    # seqQ = seqK = 4093: the last q block and the last K/V tile are partial inside fa_mfma.
    check_prefill(128, 4093, 4093, 32, 32, 2, 1, dtype, "fa_mfma_8w", seed=5,
                  heads=[(0, 0), (0, 17), (1, 8), (1, 31)])


def test_fa_mfma_8w_ragged_cross_attention():
    # seqQ != seqK, neither a multiple of a tile, GQA 4:1, non-causal (heads not a multiple of 8:
    # the item mapping without the XCD grouping).
    check_prefill(64, 4096 + 37, 3001, 36, 9, 1, 0, torch.float16, "fa_mfma_8w", seed=6,
                  heads=[(0, 0), (0, 4), (0, 20), (0, 35)])


def test_fa_pipe_partial_odd_round():
    # 4 x 32 heads x 7 q blocks = 896 items: with 256 CUs each XCD holds 112 = 3 x 32 + 16 of them,
    # so the persistent grid's last round is partial and odd (taken in reverse over 16 entries).
    check_prefill(128, 1700, 1700, 32, 32, 4, 1, torch.bfloat16, "fa_mfma_8w", seed=11,
                  heads=[(0, 0), (1, 9), (2, 18), (3, 31)])


@pytest.mark.parametrize("D,S,H,dtype", [(128, 3000, 32, torch.bfloat16), (128, 2053, 32, torch.float16),
                                         (64, 2085, 64, torch.float16)])
def test_fa_pipe_causal_ragged_lengths(D, S, H, dtype):
    # Causal (seqQ == seqK) at lengths that are not multiples of 32: the tail's fixed mask of the
    # chunk at a wave's first query and the general mask of the ragged last chunk apply to the
    # same chunk in some waves and to different chunks in others.
    check_prefill(D, S, S, H, H, 1, 1, dtype, "fa_mfma_8w", seed=30 + S,
                  heads=[(0, 0), (0, H // 2 - 1), (0, H - 1)])


@pytest.mark.parametrize("SK", [1, 50, 95, 96, 97])
def test_fa_pipe_short_keys(SK):
    # Fewer keys than the pipelined main loop needs (t_main = 0 below 96): every tile in the tail.
    check_prefill(128, 4096, SK, 32, 32, 1, 0, torch.float16, "fa_mfma_8w", seed=12 + SK,
                  heads=[(0, 0), (0, 13), (0, 31)])


# ---- fa_mfma<D, 4, 1>: mid-size problems --------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_4w_d128_causal(dtype):
    check_prefill(128, 4096, 4096, 8, 8, 1, 1, dtype, "fa_mfma_4w", seed=7)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_mfma_4w_d64_gqa_causal(dtype):
    check_prefill(64, 2048, 2048, 16, 4, 1, 1, dtype, "fa_mfma_4w", seed=8)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fa_pipe_mid_size_d64_gqa_noncausal(dtype):
    # 16 heads x 8 blocks of 256 queries = 128 < one round: the non-causal 8-wave plan with a grid of
    # 128 workgroups, one work item each.
    check_prefill(64, 2048, 2048, 16, 4, 1, 0, dtype, "fa_mfma_8w", seed=8)


def test_fa_mfma_4w_ragged_causal():
    check_prefill(128, 4093, 4093, 8, 2, 1, 1, torch.float16, "fa_mfma_4w", seed=9)


def test_fa_pipe_mid_size_cross_attention():
    # non-causal, seqK 1003 (ragged last tile), 8 x 16 = 128 blocks
    check_prefill(64, 4096, 1003, 8, 8, 1, 0, torch.bfloat16, "fa_mfma_8w", seed=10)


def test_fa_pipe_quarter_round_noncausal():
    # the smallest non-causal 8-wave plan: 64 blocks (one per XCD-aligned group), D 128
    check_prefill(128, 2048, 2048, 8, 8, 1, 0, torch.bfloat16, "fa_mfma_8w", seed=13)


# ---- fa_small: both workgroup forms -------------------------------------------------------------

@pytest.mark.parametrize("D,SQ,HQ,HK,B", [(128, 512, 8, 8, 1), (64, 700, 12, 4, 2)])
def test_fa_small_forms(D, SQ, HQ, HK, B):
    cfg = cdna4.PrefillCfg(D, SQ, SQ, HQ, HK, B, 1)
    waves = cdna4.prefill_plan(cfg, torch.float16).waves
    print(f"fa_small waves {waves}", flush=True)
    check_prefill(D, SQ, SQ, HQ, HK, B, 1, torch.float16, "fa_small", seed=11)


# ---- the strided entry point (the runtime's prompt path) against the oracle ----------------------

@pytest.mark.parametrize("D,S,HQ,HK,dtype,kernel", [(64, 2048, 16, 4, torch.float16, "fa_mfma_4w"),
                                                     (128, 4096, 32, 8, torch.bfloat16, "fa_mfma_8w"),
                                                     (64, 300, 12, 12, torch.float16, "fa_small")])
def test_prefill_strided_against_oracle(D, S, HQ, HK, dtype, kernel):
    max_seq = (S + 100 + 7) // 8 * 8
    cfg = cdna4.PrefillCfg(D, S, S, HQ, HK, 1, 1)
    plan = cdna4.prefill_plan(cfg, dtype)
    print(f"strided prefill D{D} S{S} {HQ}/{HK} -> {plan.name}", flush=True)
    assert plan.name == kernel
    g = torch.Generator(device=DEV).manual_seed(S + D)
    Q = _randn((HQ, S, D), dtype, g)
    Kc = _randn((HK, max_seq, D), dtype, g)
    Vc = _randn((HK, max_seq, D), dtype, g)
    O_tok = torch.full((S, HQ, D), float("nan"), device=DEV, dtype=dtype)
    st = cdna4.PrefillStrides(HQ * S * D, S * D, D, HK * max_seq * D, max_seq * D, D, S * HQ * D, D, HQ * D)
    cdna4.prefill_strided(Q, Kc, Vc, O_tok, cfg, st)
    torch.cuda.synchronize()
    assert torch.isfinite(O_tok.float()).all()
    rows = _rows(S, 3)
    q = Q.float().cpu().numpy()[None]
    k = Kc[:, :S].float().cpu().numpy()[None]
    v = Vc[:, :S].float().cpu().numpy()[None]
    heads = [(0, h) for h in range(HQ)]
    want = _oracle_heads(q, k, v, heads, rows, D, S, S, HQ, HK, 1)
    o = O_tok.float().cpu().numpy()
    check_parity([o[rows, h] for _, h in heads], [want[(0, h)] for _, h in heads], dtype)


def test_prefill_strided_rows_4gib_apart():
    # K/V rows 2^25 elements apart: a 64-key tile spans 4 GiB, beyond the pipelined kernel's 32-bit
    # per-lane copy offsets, so every tile takes the clamped copy with 64-bit addresses (the plan is
    # still the 8-wave kernel). K and V share one ~4.5 GB allocation, heads interleaved in a row;
    # only the rows used are written. seqK 70: one full and one partial tile.
    D, SQ, SK, HQ, HK = 128, 2048, 70, 8, 2
    rs = 1 << 25
    cfg = cdna4.PrefillCfg(D, SQ, SK, HQ, HK, 1, 0)
    assert cdna4.prefill_plan(cfg, torch.bfloat16).name == "fa_mfma_8w"
    g = torch.Generator(device=DEV).manual_seed(77)
    Q = _randn((HQ, SQ, D), torch.bfloat16, g)
    Kd = _randn((HK, SK, D), torch.bfloat16, g)
    Vd = _randn((HK, SK, D), torch.bfloat16, g)
    big = torch.empty((SK - 1) * rs + 2 * HK * D, device=DEV, dtype=torch.bfloat16)
    big.as_strided((HK, SK, D), (D, rs, 1), 0).copy_(Kd)
    big.as_strided((HK, SK, D), (D, rs, 1), HK * D).copy_(Vd)
    O = torch.full((HQ, SQ, D), float("nan"), device=DEV, dtype=torch.bfloat16)
    st = cdna4.PrefillStrides(HQ * SQ * D, SQ * D, D, 0, D, rs, HQ * SQ * D, SQ * D, D)
    cdna4.prefill_strided(Q, big, big[HK * D:], O, cfg, st)
    torch.cuda.synchronize()
    assert torch.isfinite(O.float()).all()
    rows = _rows(SQ, 5)
    q = Q.float().cpu().numpy()[None]
    k = Kd.float().cpu().numpy()[None]
    v = Vd.float().cpu().numpy()[None]
    heads = [(0, h) for h in range(HQ)]
    want = _oracle_heads(q, k, v, heads, rows, D, SQ, SK, HQ, HK, 0)
    o = O.float().cpu().numpy()
    del big
    torch.cuda.empty_cache()
    check_parity([o[h, rows] for _, h in heads], [want[(0, h)] for _, h in heads], torch.bfloat16)


# ---- BASELINE config 3 at full size: every head of batches 0 and 3 -------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_config3_subsample_every_head_of_batches_0_and_3(dtype):
    # B4 H32 S8192 D128 causal N(0,1), bf16 (the config) and fp16 (the bench's prefill_fp16 leg);
    # rows 0..127, 4095, 8191 and 256 seeded random rows.
    B, H, S, D = 4, 32, 8192, 128
    cfg = cdna4.PrefillCfg(D, S, S, H, H, B, 1)
    plan = cdna4.prefill_plan(cfg, dtype)
    print(f"config 3 ({dtype}) -> {plan.name} (grid {plan.grid})", flush=True)
    assert plan.name == "fa_mfma_8w"
    g = torch.Generator(device=DEV).manual_seed(2024)
    Q = _randn((B, H, S, D), dtype, g)
    K = _randn((B, H, S, D), dtype, g)
    V = _randn((B, H, S, D), dtype, g)
    O = torch.full_like(Q, float("nan"))
    cdna4.prefill(Q, K, V, O, cfg)
    torch.cuda.synchronize()
    assert torch.isfinite(O.float()).all()
    rows = sorted(set(range(128)) | {4095, 8191} | set(int(r) for r in oracle.integers(77, 256, 0, S - 1)))
    gots, wants = [], []
    for b in (0, 3):
        q, k, v = (T[b:b + 1].float().cpu().numpy() for T in (Q, K, V))
        want = _oracle_heads(q, k, v, [(0, h) for h in range(H)], rows, D, S, S, H, H, 1)
        o = O[b].float().cpu().numpy()
        gots += [o[h, rows] for h in range(H)]
        wants += [want[(0, h)] for h in range(H)]
        print(f"  batch {b} done", flush=True)
    name = "bf16" if dtype == torch.bfloat16 else "fp16"
    check_parity(gots, wants, dtype,
                 what=f"cfg3 (B4 H32 S8192 D128 causal {name}), every head of batches 0 and 3 x {len(rows)} rows")


# ---- decode: split-K grid (decode_mfma + decode_merge) and the one-launch plan --------------------

def check_decode(D, N, HQ, HK, B, dtype, kernel, stride=0, seed=7, workspace="auto"):
    st = stride or N
    cfg = cdna4.DecodeCfg(D, N, HQ, HK, B, stride)
    plan = cdna4.decode_plan(cfg, dtype, with_workspace=workspace is not None)
    print(f"decode D{D} N{N} stride{st} {HQ}/{HK} B{B} {dtype} ws={workspace is not None} -> {plan.name} "
          f"(P {plan.partials}, keys/split {plan.rows})", flush=True)
    assert plan.name == kernel
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = _randn((B, HQ, D), dtype, g)
    K = _randn((B, HK, st, D), dtype, g)
    V = _randn((B, HK, st, D), dtype, g)
    o = torch.full_like(q, float("nan"))
    cdna4.decode(q, K, V, o, cfg, workspace=workspace)
    torch.cuda.synchronize()
    want = oracle.decode(q.float().cpu().numpy(), K.float().cpu().numpy(), V.float().cpu().numpy(), D, N, HQ, HK,
                         B, stride)
    check_parity(o.float().cpu().numpy(), want, dtype)
    return plan


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_split_strided_cache(dtype):
    # decode_dme's cache layout [nKVH][stride_kv][D] with stride_kv > N (the runtime's long-context
    # decode), N not a multiple of the 32-key chunk.
    check_decode(128, 5000, 32, 8, 2, dtype, "decode_split", stride=8192)


@pytest.mark.parametrize("HQ,HK", [(8, 8), (64, 8), (32, 1), (40, 2)])
def test_decode_split_gqa_groups(HQ, HK):
    # G = 1, 8, 32 (two 16-head column blocks per kv head) and 20 (a partial second block).
    check_decode(128, 4096, HQ, HK, 2, torch.float16, "decode_split", seed=HQ)


def test_decode_split_d64_ragged():
    check_decode(64, 4097, 12, 4, 3, torch.float16, "decode_split")


def test_decode_split_n8191():
    check_decode(128, 8191, 32, 8, 1, torch.bfloat16, "decode_split")


def test_decode_split_few_partials():
    # 64 (batch, kv head) rows: 16 partials per head, the sixteen-row form of the one-round-trip merge
    plan = check_decode(128, 4096, 32, 8, 8, torch.float16, "decode_split", seed=5)
    assert plan.partials <= 16


def test_decode_split_more_than_64_partials():
    # batch 1 with one kv head: P > 64, so the merge runs several 64-partial passes.
    plan = check_decode(128, 65536, 4, 1, 1, torch.float16, "decode_split", seed=3)
    assert plan.partials > 64


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def test_decode_whole_rounds_one_launch_d64_streaming():
    # batch x kv heads = the CU count: with a workspace the long cache still takes the one-launch
    # plan (one workgroup per CU); 327 MB of K/V, beyond the Infinity Cache: non-temporal copies.
    HK = 4
    check_decode(64, 5000, 16, HK, _cus() // HK, torch.float16, "decode_wg", seed=11)


def test_decode_whole_rounds_one_launch_d128_strided_cached():
    # whole rounds, a cache longer than the short-cache bound (1,024 keys at D 128) but K/V below
    # the Infinity Cache size (default copy policy), rows 2,048 apart
    HK = 8
    check_decode(128, 1500, 32, HK, _cus() // HK, torch.bfloat16, "decode_wg", stride=2048, seed=12)


def test_decode_whole_rounds_split_k_when_forced(monkeypatch):
    # CDNA4_DECODE_SPLIT_K=1: the whole-rounds shape above (config 4's kind) on the split-K grid and
    # its DPP merge instead of the one-launch plan.
    HK = 8
    monkeypatch.setenv("CDNA4_DECODE_SPLIT_K", "1")
    check_decode(128, 1500, 32, HK, _cus() // HK, torch.float16, "decode_split", seed=13)
    monkeypatch.delenv("CDNA4_DECODE_SPLIT_K")
    cfg = cdna4.DecodeCfg(128, 1500, 32, HK, _cus() // HK, 0)
    assert cdna4.decode_plan(cfg, torch.float16, with_workspace=True).name == "decode_wg"


@pytest.mark.parametrize("N,HQ,HK,B", [(8192, 32, 8, 1), (3000, 40, 2, 2), (4097, 12, 12, 1)])
def test_decode_without_workspace_one_launch(N, HQ, HK, B):
    # The reference launchers' contract: no workspace, one launch, any cache length.
    D = 64 if HQ == 12 else 128
    check_decode(D, N, HQ, HK, B, torch.float16, "decode_wg", workspace=None)


def test_decode_without_workspace_strided():
    check_decode(128, 1500, 32, 8, 2, torch.bfloat16, "decode_wg", stride=2048, workspace=None)


def test_decode_two_streams_with_different_inputs():
    # Calls on two streams at once, each with its own inputs: split-K calls with workspaces from
    # torch's allocator on their streams, and workspace-less calls. Every output is checked.
    D, N, HQ, HK = 128, 6000, 32, 8
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cases = []
    for i, s in enumerate(streams):
        g = torch.Generator(device=DEV).manual_seed(100 + i)
        with torch.cuda.stream(s):
            q = _randn((1, HQ, D), torch.float16, g)
            K = _randn((1, HK, N, D), torch.float16, g)
            V = _randn((1, HK, N, D), torch.float16, g)
        cases.append((s, q, K, V))
    torch.cuda.synchronize()
    cfg = cdna4.DecodeCfg(D, N, HQ, HK, 1)
    outs = {}
    for rep in range(4):
        for i, (s, q, K, V) in enumerate(cases):
            with torch.cuda.stream(s):
                o_ws = torch.empty_like(q)
                o_nows = torch.empty_like(q)
                cdna4.decode(q, K, V, o_ws, cfg)
                cdna4.decode(q, K, V, o_nows, cfg, workspace=None)
                outs[(rep, i)] = (o_ws, o_nows)
    torch.cuda.synchronize()
    for i, (s, q, K, V) in enumerate(cases):
        want = oracle.decode(q.float().cpu().numpy(), K.float().cpu().numpy(), V.float().cpu().numpy(), D, N, HQ,
                             HK)
        for rep in range(4):
            for o in outs[(rep, i)]:
                check_parity(o.float().cpu().numpy(), want, torch.float16)


def test_decode_auto_workspace_on_a_side_stream():
    # decode(workspace="auto", stream=s) while s is still busy: the call's split-K workspace is
    # freed on return, and the current stream then allocates a block of the same size and fills
    # it with 0xFF before the decode on s has run. The workspace must belong to s's pool, so the
    # fill cannot land in it (allocated on the current stream, it would be handed straight back).
    D, N, HQ, HK = 128, 8192, 32, 8
    cfg = cdna4.DecodeCfg(D, N, HQ, HK, 1)
    assert cdna4.decode_plan(cfg, torch.float16, with_workspace=True).name == "decode_split"
    g = torch.Generator(device=DEV).manual_seed(321)
    q = _randn((1, HQ, D), torch.float16, g)
    K = _randn((1, HK, N, D), torch.float16, g)
    V = _randn((1, HK, N, D), torch.float16, g)
    o = torch.full_like(q, float("nan"))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        torch.cuda._sleep(20_000_000)          # a bounded spin that keeps s busy for milliseconds
    cdna4.decode(q, K, V, o, cfg, workspace="auto", stream=s)
    junk = torch.empty(cdna4.decode_workspace_size(cfg), dtype=torch.uint8, device=DEV)
    junk.fill_(0xFF)
    torch.cuda.synchronize()
    want = oracle.decode(q.float().cpu().numpy(), K.float().cpu().numpy(), V.float().cpu().numpy(), D, N, HQ, HK)
    check_parity(o.float().cpu().numpy(), want, torch.float16)
