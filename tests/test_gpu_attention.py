"""Prefill and decode on gfx950 against the CPU oracle (the restated fp32 references of
cdna3-prims/tests/validate_attention_api.hip:27-72), on the rounded inputs the GPU sees.
Bound per output dtype (gpu_util.check_parity): |gpu - ref| <= tol * max(1, |ref|), tol 1e-4 (fp32),
2e-3 (fp16, bf16), plus half a bf16 ulp of ref for bf16 outputs (the stored output's own rounding)."""
import os
import subprocess

import numpy as np
import pytest
import torch

import cdna4
import oracle
from gpu_util import DEV, ROOT, check_abs, check_parity, host, max_rel_err, rounded

pytestmark = pytest.mark.gpu


def prefill_case(D, SQ, SK, HQ, HK, B, causal, dtype, seed=42, dist="normal", std=0.5):
    gen = (lambda s, n: oracle.normal(s, n, 0.0, std)) if dist == "normal" else (lambda s, n: oracle.uniform(s, n))
    q, Q = rounded(gen(seed, B * HQ * SQ * D), dtype)
    k, K = rounded(gen(seed + 1, B * HK * SK * D), dtype)
    v, V = rounded(gen(seed + 2, B * HK * SK * D), dtype)
    O = torch.empty_like(Q)
    cdna4.prefill(Q, K, V, O, cdna4.PrefillCfg(D, SQ, SK, HQ, HK, B, causal))
    ref = oracle.prefill(q, k, v, D, SQ, SK, HQ, HK, B, causal)
    return host(O).reshape(ref.shape), ref, (q, k, v)


# The reference's prefill validation set (validate_attention_api.hip:154-161).
REF_PREFILL = [(128, 256, 256, 2, 2, 1, 0), (128, 256, 256, 4, 2, 1, 0), (128, 256, 256, 2, 2, 1, 1),
               (128, 256, 256, 4, 2, 1, 1), (64, 256, 256, 2, 2, 1, 0), (128, 1024, 1024, 8, 8, 1, 0),
               (128, 512, 512, 32, 8, 1, 1)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cfg", REF_PREFILL)
def test_prefill_reference_validation_set(cfg, dtype):
    got, ref, _ = prefill_case(*cfg, dtype)
    check_parity(got, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_prefill_fa2_reference_config(dtype):
    # B1 H8 S512 D64, non-causal, U(-1,1) fp32 from seed 42; fp16-rounded arm.
    got, ref, _ = prefill_case(64, 512, 512, 8, 8, 1, 0, dtype, seed=42, dist="uniform")
    if dtype == torch.float32:
        check_abs(got, ref, 1e-4, what="cfg1 (B1 H8 S512 D64) fp32 arm, abs")
    else:
        check_parity(got, ref, dtype, what="cfg1 (B1 H8 S512 D64) fp16 arm")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cfg", [(64, 100, 200, 4, 2, 2, 0), (128, 77, 77, 3, 1, 1, 1), (64, 1, 1, 1, 1, 1, 1),
                                 (128, 130, 63, 2, 2, 1, 0), (64, 257, 257, 2, 1, 3, 1), (128, 16, 1000, 8, 8, 1, 0)])
def test_prefill_ragged_shapes(cfg, dtype):
    got, ref, _ = prefill_case(*cfg, dtype, seed=7)
    check_parity(got, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_closed_forms(dtype):
    D, S, H = 128, 320, 4
    got, ref, (q, k, v) = prefill_case(D, S, S, H, H, 1, 1, dtype, seed=3)
    vv = v.reshape(1, H, S, D)
    assert np.array_equal(got[0, :, 0], vv[0, :, 0])          # causal row 0 returns V[0] exactly
    # Identical keys -> mean of V.
    kc = np.broadcast_to(k.reshape(1, H, S, D)[:, :, :1], (1, H, S, D)).copy()
    _, Kc = rounded(kc.reshape(-1), dtype)
    _, Q = rounded(q, dtype)
    _, V = rounded(v, dtype)
    O = torch.empty_like(Q)
    cdna4.prefill(Q, Kc, V, O, cdna4.PrefillCfg(D, S, S, H, H, 1, 0))
    mean = vv.astype(np.float64).mean(axis=2, keepdims=True)
    check_parity(host(O).reshape(1, H, S, D), np.broadcast_to(mean, (1, H, S, D)), dtype)


def test_prefill_full_size_config_subsample():
    # BASELINE config 3 shape (B4 H32 S8192 D128 causal bf16). Heads are independent, so the
    # oracle-generated heads below are checked inside otherwise random full-size tensors.
    B, H, S, D = 4, 32, 8192, 128
    torch.manual_seed(0)
    Q = torch.randn(B, H, S, D, device=DEV, dtype=torch.bfloat16)
    K = torch.randn(B, H, S, D, device=DEV, dtype=torch.bfloat16)
    V = torch.randn(B, H, S, D, device=DEV, dtype=torch.bfloat16)
    heads = [(0, 0), (0, 31), (3, 5), (3, 31)]
    host_heads = {}
    for i, (b, h) in enumerate(heads):
        qkv = []
        for j, T in enumerate((Q, K, V)):
            vals, t = rounded(oracle.normal(1000 + 3 * i + j, S * D), torch.bfloat16)
            T[b, h] = t.reshape(S, D)
            qkv.append(vals.reshape(1, 1, S, D))
        host_heads[(b, h)] = qkv
    O = torch.empty_like(Q)
    cdna4.prefill(Q, K, V, O, cdna4.PrefillCfg(D, S, S, H, H, B, 1))
    rows = [0, 1, 63, 64, 127, 128, 4095, 4096, 8190, 8191] + list(oracle.integers(5, 10, 0, S - 1))
    gots, wants = [], []
    for (b, h), (q, k, v) in host_heads.items():
        wants.append(oracle.prefill_rows(q, k, v, D, S, S, 1, 1, 1, 1, np.array([[0, 0, r] for r in rows], np.int32)))
        gots.append(host(O[b, h, rows]))
    check_parity(gots, wants, torch.bfloat16, what="cfg3 (B4 H32 S8192 D128 causal bf16), 4 oracle heads x 20 rows")
    assert torch.isfinite(O.float()).all()


def decode_case(D, N, HQ, HK, B, dtype, seed=7, stride=0, std=0.5, workspace=None):
    st = stride or N
    q, qt = rounded(oracle.normal(seed, B * HQ * D, 0.0, std), dtype)
    k, K = rounded(oracle.normal(seed + 1, B * HK * st * D, 0.0, std), dtype)
    v, V = rounded(oracle.normal(seed + 2, B * HK * st * D, 0.0, std), dtype)
    o = torch.empty_like(qt)
    cdna4.decode(qt, K, V, o, cdna4.DecodeCfg(D, N, HQ, HK, B, stride), workspace=workspace)
    ref = oracle.decode(q, k, v, D, N, HQ, HK, B, stride)
    return host(o).reshape(ref.shape), ref


# The reference's decode validation set (validate_attention_api.hip:166-172).
REF_DECODE = [(128, 128, 8, 8), (64, 128, 8, 8), (128, 512, 32, 8), (128, 1024, 32, 8), (128, 4096, 32, 8),
              (128, 8192, 32, 8)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cfg", REF_DECODE)
def test_decode_reference_validation_set(cfg, dtype):
    got, ref = decode_case(*cfg, 1, dtype)
    check_parity(got, ref, dtype)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 3, 4, 7, 8, 16])
@pytest.mark.parametrize("N", [1, 2, 17, 100, 1000])
def test_decode_gqa_groups_and_lengths(D, group, N):
    HK = 2
    got, ref = decode_case(D, N, HK * group, HK, 3, torch.float16, seed=N + group)
    check_parity(got, ref, torch.float16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_strided_cache(dtype):
    # decode_dme's layout: [nKVH][stride_kv][D] with stride_kv = max_seq > N.
    got, ref = decode_case(128, 300, 32, 8, 2, dtype, stride=512)
    check_parity(got, ref, dtype)
    got, ref = decode_case(64, 37, 8, 8, 1, dtype, stride=64)
    check_parity(got, ref, dtype)


def test_decode_full_size_config_and_split_invariance():
    # batch 32, 32 q heads / 8 kv heads, D128, N8192, fp16 N(0,1).
    B, HQ, HK, D, N = 32, 32, 8, 128, 8192
    torch.manual_seed(1)
    q = torch.randn(B, HQ, D, device=DEV, dtype=torch.float16)
    K = torch.randn(B, HK, N, D, device=DEV, dtype=torch.float16)
    V = torch.randn(B, HK, N, D, device=DEV, dtype=torch.float16)
    checked = [0, 13, 31]
    hostv = {}
    for i, b in enumerate(checked):
        vals = []
        for j, (T, shape) in enumerate(((q, (HQ, D)), (K, (HK, N, D)), (V, (HK, N, D)))):
            x, t = rounded(oracle.normal(500 + 3 * i + j, int(np.prod(shape))), torch.float16)
            T[b] = t.reshape(shape)
            vals.append(x)
        hostv[b] = vals
    plan = cdna4.decode_plan(cdna4.DecodeCfg(D, N, HQ, HK, B), torch.float16, with_workspace=True)
    print(f"config-4 plan: {plan.name}", flush=True)   # the one-launch plan on a 256-CU part
    ws = torch.empty(cdna4.decode_workspace_size(cdna4.DecodeCfg(D, N, HQ, HK, B)), dtype=torch.uint8, device=DEV)
    o = torch.empty_like(q)
    cdna4.decode(q, K, V, o, cdna4.DecodeCfg(D, N, HQ, HK, B), workspace=ws)
    gots, refs = [], []
    for b, (qq, kk, vv) in hostv.items():
        refs.append(oracle.decode(qq, kk, vv, D, N, HQ, HK, 1)[0])
        gots.append(host(o[b]))
    check_parity(gots, refs, torch.float16, what="cfg4 (B32 32q/8kv D128 N8192 fp16), batches 0, 13, 31")
    # A batch-1 call splits the keys of one sequence into many more partials; same result.
    for b in (0, 31):
        o1 = torch.empty_like(q[b:b + 1])
        cdna4.decode(q[b:b + 1].contiguous(), K[b:b + 1].contiguous(), V[b:b + 1].contiguous(), o1,
                     cdna4.DecodeCfg(D, N, HQ, HK, 1))
        assert max_rel_err(host(o1[0]), host(o[b]).astype(np.float64)) <= 2e-3
    assert torch.isfinite(o.float()).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_full_size_config_on_the_split_k_plan(monkeypatch, dtype):
    # BASELINE config 4 names split-K across workgroups with a DPP final reduce: the same shape on
    # that plan (forced; the one-launch plan is the default on a 256-CU part), against the oracle;
    # fp16 as the config, and bf16 at the same size.
    B, HQ, HK, D, N = 32, 32, 8, 128, 8192
    monkeypatch.setenv("CDNA4_DECODE_SPLIT_K", "1")
    torch.manual_seed(2)
    q = torch.randn(B, HQ, D, device=DEV, dtype=dtype)
    K = torch.randn(B, HK, N, D, device=DEV, dtype=dtype)
    V = torch.randn(B, HK, N, D, device=DEV, dtype=dtype)
    checked = [1, 30]
    hostv = {}
    for i, b in enumerate(checked):
        vals = []
        for j, (T, shape) in enumerate(((q, (HQ, D)), (K, (HK, N, D)), (V, (HK, N, D)))):
            x, t = rounded(oracle.normal(700 + 3 * i + j, int(np.prod(shape))), dtype)
            T[b] = t.reshape(shape)
            vals.append(x)
        hostv[b] = vals
    cfg = cdna4.DecodeCfg(D, N, HQ, HK, B)
    plan = cdna4.decode_plan(cfg, dtype, with_workspace=True)
    print(f"config-4 forced plan ({dtype}): {plan.name}", flush=True)
    assert plan.name == "decode_split"
    ws = torch.empty(cdna4.decode_workspace_size(cfg), dtype=torch.uint8, device=DEV)
    o = torch.empty_like(q)
    cdna4.decode(q, K, V, o, cfg, workspace=ws)
    gots = [host(o[b]) for b in checked]
    refs = [oracle.decode(*hostv[b], D, N, HQ, HK, 1)[0] for b in checked]
    name = "fp16" if dtype == torch.float16 else "bf16"
    check_parity(gots, refs, dtype, what=f"cfg4 shape on the split-K plan, {name}, batches 1, 30")


def test_torch_op_mirrors():
    D, S, HQ, HK = 128, 192, 8, 2
    q, Q = rounded(oracle.normal(1, HQ * S * D, 0, 0.5), torch.float16)
    k, K = rounded(oracle.normal(2, HK * S * D, 0, 0.5), torch.float16)
    v, V = rounded(oracle.normal(3, HK * S * D, 0, 0.5), torch.float16)
    o = cdna4.flash_attn(Q.reshape(HQ, S, D), K.reshape(HK, S, D), V.reshape(HK, S, D))
    ref = oracle.prefill(q, k, v, D, S, S, HQ, HK, 1, 1)[0]
    check_parity(host(o), ref, torch.float16)
    od = cdna4.flash_attn_decode(Q.reshape(HQ, S, D)[:, -1].contiguous(), K.reshape(HK, S, D), V.reshape(HK, S, D))
    check_parity(host(od), ref[:, -1], torch.float16)


@pytest.mark.parametrize("D,S,HQ,HK,dtype", [(128, 192, 8, 2, torch.float16), (64, 333, 6, 6, torch.bfloat16)])
def test_registered_torch_ops_against_sdpa(D, S, HQ, HK, dtype):
    # torch.ops.amdinstinct.* as the reference's models call them, against PyTorch's own SDPA
    # in fp32 on the same rounded inputs (the reference's compare_vs_production_fa.py check).
    from cdna4 import torch_ops
    torch_ops.register()
    g = torch.Generator(device=DEV).manual_seed(D + S)
    q = torch.randn(HQ, S, D, device=DEV, generator=g).to(dtype)
    k = torch.randn(HK, S, D, device=DEV, generator=g).to(dtype)
    v = torch.randn(HK, S, D, device=DEV, generator=g).to(dtype)
    o = torch.ops.amdinstinct.flash_attn(q, k, v)
    rep = HQ // HK
    kf = k.float().repeat_interleave(rep, 0).contiguous()
    vf = v.float().repeat_interleave(rep, 0).contiguous()
    ref = torch.nn.functional.scaled_dot_product_attention(q.float()[None], kf[None], vf[None], is_causal=True)[0]
    check_parity(host(o), host(ref).astype(np.float64), dtype)
    od = torch.ops.amdinstinct.flash_attn_decode(q[:, -1].contiguous(), k, v)
    check_parity(host(od), host(ref[:, -1]).astype(np.float64), dtype)
    for bad in ((q.float(), k, v), (q[:, :, :32].contiguous(), k, v), (q, k[:, :-1].contiguous(), v)):
        with pytest.raises(RuntimeError):
            torch.ops.amdinstinct.flash_attn(*bad)
    with pytest.raises(RuntimeError):
        torch.ops.amdinstinct.flash_attn_decode(q[:, -1].contiguous(), k.transpose(1, 2), v)


def test_cpp_dropin_validation_program():
    exe = os.path.join(ROOT, "tests", "native", "validate_attention_api")
    assert os.path.exists(exe), "tests/native not built"
    r = subprocess.run([exe, os.path.join(ROOT, "oracle", "liboracle.so")], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Result: 17/17 PASS" in r.stdout


@pytest.mark.parametrize("D,S,HQ,HK,dtype", [(64, 512, 12, 12, torch.float16), (128, 300, 8, 2, torch.bfloat16),
                                              (64, 2048, 16, 4, torch.float16)])
def test_prefill_strided_reads_cache_and_writes_token_major(D, S, HQ, HK, dtype):
    # The layer loop's layout: Q head-major, K/V in place in a [nKVH][max_seq][D] cache, O token-major.
    max_seq = S + 77 if S % 8 == 0 else S + 3
    max_seq = (max_seq + 7) // 8 * 8
    g = torch.Generator(device=DEV).manual_seed(S)
    Q = torch.randn(HQ, S, D, device=DEV, generator=g).to(dtype)
    Kc = torch.randn(HK, max_seq, D, device=DEV, generator=g).to(dtype)
    Vc = torch.randn(HK, max_seq, D, device=DEV, generator=g).to(dtype)
    O_tok = torch.full((S, HQ, D), float("nan"), device=DEV, dtype=dtype)
    cfg = cdna4.PrefillCfg(D, S, S, HQ, HK, 1, 1)
    st = cdna4.PrefillStrides(HQ * S * D, S * D, D, HK * max_seq * D, max_seq * D, D, S * HQ * D, D, HQ * D)
    cdna4.prefill_strided(Q, Kc, Vc, O_tok, cfg, st)
    # Same kernel on packed copies: identical bits.
    K = Kc[:, :S].contiguous()
    V = Vc[:, :S].contiguous()
    O = torch.empty(HQ, S, D, device=DEV, dtype=dtype)
    cdna4.prefill(Q, K, V, O, cfg)
    assert torch.equal(O_tok.transpose(0, 1), O)
