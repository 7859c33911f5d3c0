"""The small-LLM runtime session (csrc/session.hip through the C ABI) against the CPU oracle.

Logits of every step are compared with the oracle's forward over the same token sequence
(teacher forcing: the oracle runs the prompt followed by the tokens the GPU chose), so one
near-tie cannot derail the rest of the comparison. A chosen token must be the oracle's argmax,
or within LOGIT_TOL of its maximum (a near-tie the fp16 rounding points can flip).
"""
import os

import numpy as np
import pytest

import cdna4
import oracle
import parity_log
from cdna4 import model_format as mf

pytestmark = pytest.mark.gpu

# |GPU - oracle| on the logits (the fp16 values both store), relative to the step's largest logit
# (at least 1): the fp16/bf16 bound 2e-3. The oracle rounds to fp16 where the reference does; the GPU accumulates its
# projections in another order, which moves an fp16 rounding by one ulp now and then, and these
# flips propagate through the layers.
LOGIT_TOL = 2e-3


def _row_err(got, ref):
    """max over rows of max|got - ref| / max(1, max|ref|) (one row per step)."""
    got, ref = np.atleast_2d(got), np.atleast_2d(ref)
    scale = np.maximum(1.0, np.abs(ref).max(axis=1))
    return float((np.abs(got - ref).max(axis=1) / scale).max())


MODELS = {
    "gqa_bias_d64": dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab_size=1000,
                         qkv_bias=True),
    "mha_d128_layernorm": dict(n_layers=2, hidden=256, n_heads=2, n_kv_heads=2, head_dim=128, ffn_dim=384,
                               vocab_size=777, norm="layernorm", rope_theta=1e6),
    "gqa3_d64": dict(n_layers=3, hidden=192, n_heads=3, n_kv_heads=1, head_dim=64, ffn_dim=256, vocab_size=500),
}


@pytest.fixture(scope="module", params=sorted(MODELS))
def model(request, tmp_path_factory):
    d = str(tmp_path_factory.mktemp(request.param))
    mf.random_model(d, seed=11, norm_jitter=0.2, **MODELS[request.param])
    meta, t = mf.read_model(d)
    print(f"model {request.param}", flush=True)
    return d, meta, t


def _prompt(meta, n, seed):
    return np.random.default_rng(seed).integers(0, int(meta["vocab_size"]), n).astype(np.int32)


def _check_generation(meta, t, ids, out, max_seq, what=""):
    toks, logits = out["tokens"], out["logits"]
    ref = oracle.LLM(meta, t, max_seq).forward(np.concatenate([ids, toks[:-1]]).astype(np.int32),
                                               all_logits=True)[len(ids) - 1:]
    assert ref.shape == logits.shape
    err = _row_err(logits, ref)
    print(f"  steps {len(toks)}: max |logit - oracle| / scale = {err:.2e}, "
          f"abs {float(np.abs(logits - ref).max()):.2e}", flush=True)
    parity_log.record(err, LOGIT_TOL, "logit", None, what)
    assert err < LOGIT_TOL, err
    for i, tok in enumerate(toks):
        best = oracle.reference_argmax(ref[i])
        near = 2 * LOGIT_TOL * max(1.0, float(np.abs(ref[i]).max()))
        assert tok == best or ref[i][best] - ref[i][tok] <= near, (i, tok, best)
        # The device argmax picks from its own (fp16) logits with the reference's tie-break.
        assert tok == oracle.reference_argmax(logits[i])


def test_config_read_from_meta(model):
    d, meta, _ = model
    with cdna4.Session(d, max_seq=64) as s:
        c = s.cfg.as_dict()
    for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab_size"):
        assert c[k] == int(meta[k]), k
    assert c["layernorm"] == int(meta.get("norm") == "layernorm")
    assert c["qkv_bias"] == int(meta["qkv_bias"])
    assert abs(c["norm_eps"] - (1e-5 if c["layernorm"] else 1e-6)) < 1e-9


@pytest.mark.parametrize("gemm", ["library", "rocblas"])
@pytest.mark.parametrize("n", [1, 5, 64, 100])
def test_prefill_logits_match_oracle(model, monkeypatch, n, gemm):
    # the prompt GEMMs on the library's MFMA GEMM (the default) or all on rocBLAS
    d, meta, t = model
    if gemm == "rocblas":
        monkeypatch.setenv("CDNA4_SESSION_ROCBLAS", "1")
    ids = _prompt(meta, n, n)
    with cdna4.Session(d, max_seq=128) as s:
        got = s.prefill_logits(ids)
    ref = oracle.LLM(meta, t, 128).forward(ids)
    err = _row_err(got, ref)
    print(f"  prompt {n} ({gemm} GEMMs): max |logit - oracle| / scale = {err:.2e}", flush=True)
    parity_log.record(err, LOGIT_TOL, "logit")
    assert err < LOGIT_TOL, err


@pytest.mark.parametrize("n,new", [(21, 16), (1, 8), (64, 12)])
def test_generate_matches_oracle(model, n, new):
    d, meta, t = model
    ids = _prompt(meta, n, 100 + n)
    with cdna4.Session(d, max_seq=96) as s:
        out = s.generate_ex(ids, cdna4.GenerateCfg(new), with_logits=True)
    assert len(out["tokens"]) == new
    assert out["ttft_ms"] > 0 and out["decode_ms"] > 0
    _check_generation(meta, t, ids, out, 96)


@pytest.mark.parametrize("parts", ["0", "1", "2", "4"])
@pytest.mark.parametrize("n,new", [(21, 16), (200, 12)])
def test_decode_attention_partials_match_oracle(model, monkeypatch, n, new, parts):
    # Short-cache decode steps run the attention as P split-K partials per head that the O
    # projection's GEMV merges (CDNA4_SESSION_ATTN_PARTS, default 3; "0" is the one-launch
    # attention and a plain GEMV). Every P, including key ranges left empty (P x 32-key chunks per
    # wave beyond the cache), against the oracle.
    d, meta, t = model
    monkeypatch.setenv("CDNA4_SESSION_ATTN_PARTS", parts)
    ids = _prompt(meta, n, 500 + n)
    with cdna4.Session(d, max_seq=256) as s:
        out = s.generate_ex(ids, cdna4.GenerateCfg(new), with_logits=True)
    _check_generation(meta, t, ids, out, 256, what=f"decode attention in {parts} partials")


def test_prompt_qkv_epilogue_equals_separate_append(model, monkeypatch):
    # Models without a Q|K|V bias project the prompt with RoPE and the cache append in the GEMM's
    # epilogue; CDNA4_SESSION_QKV_FUSED=0 runs the same GEMM with its plain output and the separate
    # append kernel. Both round each value to fp16 and rotate it alike: identical tokens and logits.
    d, meta, t = model
    ids = _prompt(meta, 77, 9)
    outs = []
    for fused in ("1", "0"):
        monkeypatch.setenv("CDNA4_SESSION_QKV_FUSED", fused)
        with cdna4.Session(d, max_seq=128) as s:
            outs.append(s.generate_ex(ids, cdna4.GenerateCfg(6), with_logits=True))
    assert outs[0]["tokens"] == outs[1]["tokens"]
    assert np.array_equal(outs[0]["logits"], outs[1]["logits"])


def test_session_reuse_and_plain_generate(model):
    # a second, shorter prompt on the same session sees none of the first one's cache rows
    d, meta, t = model
    a, b = _prompt(meta, 40, 1), _prompt(meta, 9, 2)
    with cdna4.Session(d, max_seq=64) as s:
        s.generate_ex(a, cdna4.GenerateCfg(10))
        second = s.generate(b, cdna4.GenerateCfg(6))
    with cdna4.Session(d, max_seq=64) as s:
        fresh = s.generate_ex(b, cdna4.GenerateCfg(6), with_logits=True)
    assert second == list(b) + fresh["tokens"]
    _check_generation(meta, t, b, fresh, 64)


@pytest.mark.parametrize("n,new,max_seq", [(7, 12, 64), (1000, 40, 1100)])
def test_captured_step_equals_separate_launches(model, monkeypatch, n, new, max_seq):
    # The decode step replayed as one captured graph (positions in device memory) against the
    # same kernels launched one by one: identical tokens and bit-identical logits. 1000 + 40
    # crosses the short-cache limit of the decode attention (1024 keys at D = 128, 2048 at
    # D = 64), so the graph is captured again when the attention plan changes.
    d, meta, t = model
    ids = _prompt(meta, n, 300 + n)
    outs = []
    for graph in ("1", "0"):
        monkeypatch.setenv("CDNA4_SESSION_GRAPH", graph)
        with cdna4.Session(d, max_seq=max_seq) as s:
            outs.append(s.generate_ex(ids, cdna4.GenerateCfg(new), with_logits=True))
            again = s.generate_ex(ids, cdna4.GenerateCfg(new), with_logits=True)   # graph reused
            assert again["tokens"] == outs[-1]["tokens"]
            assert np.array_equal(again["logits"], outs[-1]["logits"])
    assert outs[0]["tokens"] == outs[1]["tokens"]
    assert np.array_equal(outs[0]["logits"], outs[1]["logits"])


def test_graph_recaptured_when_scratch_grows(model):
    # A longer second prompt on the same session reallocates the per-token scratch buffers; the
    # captured decode step held the old addresses, so the session must drop it and capture again.
    d, meta, t = model
    short, long_ = _prompt(meta, 5, 41), _prompt(meta, 50, 42)
    with cdna4.Session(d, max_seq=64) as s:
        s.generate_ex(short, cdna4.GenerateCfg(4))
        grown = s.generate_ex(long_, cdna4.GenerateCfg(6), with_logits=True)
    with cdna4.Session(d, max_seq=64) as s:
        fresh = s.generate_ex(long_, cdna4.GenerateCfg(6), with_logits=True)
    assert grown["tokens"] == fresh["tokens"]
    assert np.array_equal(grown["logits"], fresh["logits"])


def test_eos_and_full_cache_stop_generation(model):
    d, meta, _ = model
    ids = _prompt(meta, 12, 3)
    with cdna4.Session(d, max_seq=64) as s:
        base = s.generate_ex(ids, cdna4.GenerateCfg(10))["tokens"]
        eos = base[4]
        stop = base.index(eos) + 1
        assert s.generate_ex(ids, cdna4.GenerateCfg(10, eos_token_id=eos))["tokens"] == base[:stop]
    with cdna4.Session(d, max_seq=len(ids) + 3) as s:
        assert s.generate_ex(ids, cdna4.GenerateCfg(10))["tokens"] == base[:4]


def test_invalid_requests_raise(model):
    d, meta, _ = model
    V = int(meta["vocab_size"])
    with cdna4.Session(d, max_seq=16) as s:
        for bad in ([V], [-1], list(range(17)), []):
            with pytest.raises((cdna4.CDNA4Error, ValueError)):
                s.generate_ex(bad, cdna4.GenerateCfg(2))
        with pytest.raises(cdna4.CDNA4Error):
            s.prefill_logits([0, V + 5])


def test_cfg5_shape_matches_oracle(tmp_path):
    # the benchmark's model shape (12 layers, d 768, 12 heads of 64, MLP 3072, vocab 32000,
    # LayerNorm with gains 1 and betas 0, weights N(0, 0.02)), on a prompt the oracle runs quickly
    d = str(tmp_path / "cfg5")
    mf.random_model(d, n_layers=12, hidden=768, n_heads=12, ffn_dim=3072, vocab_size=32000, norm="layernorm", seed=5)
    meta, t = mf.read_model(d)
    ids = _prompt(meta, 48, 9)
    with cdna4.Session(d, max_seq=128) as s:
        out = s.generate_ex(ids, cdna4.GenerateCfg(6), with_logits=True)
    _check_generation(meta, t, ids, out, 128)


def test_cfg5_full_workload_matches_oracle(tmp_path):
    # BASELINE config 5 exactly as bench.py runs it (Session::generate, session.hpp:263-296): the
    # bench's model (seed 5), its 512-token prompt (default_rng(5)) and 128 greedy tokens. Every
    # step's logits against the oracle under teacher forcing (the oracle runs the prompt and the
    # 127 tokens the GPU fed back, ~20 s on one host thread), every token against the oracle's
    # argmax with the reference's tie-break.
    L, H, nH, F, V, prompt, new = 12, 768, 12, 3072, 32000, 512, 128
    d = str(tmp_path / "cfg5_full")
    mf.random_model(d, n_layers=L, hidden=H, n_heads=nH, ffn_dim=F, vocab_size=V, norm="layernorm", seed=5)
    meta, t = mf.read_model(d)
    ids = np.random.default_rng(5).integers(0, V, prompt).astype(np.int32)
    with cdna4.Session(d, max_seq=prompt + new) as s:
        out = s.generate_ex(ids, cdna4.GenerateCfg(new), with_logits=True)
    assert len(out["tokens"]) == new
    print(f"cfg5 full workload: {prompt} + {new} tokens generated", flush=True)
    _check_generation(meta, t, ids, out, prompt + new,
                      what=f"cfg5 ({prompt}-token prompt + {new} greedy tokens, 12 layers d768) logits")


def test_cpp_session_program(model):
    # The reference's C++ usage (Session(model_dir, max_seq).generate(ids, GenerateCfg)) through
    # include/cdna3/runtime/session.hpp, built host-only (tests/native/generate_demo.cpp): same
    # tokens and logits as the Python mirror of the same library.
    import subprocess
    d, meta, t = model
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "generate_demo")
    assert os.path.exists(exe), "tests/native not built"
    ids = _prompt(meta, 17, 4)
    r = subprocess.run([exe, d, "64", "9"] + [str(i) for i in ids], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = dict(l.split(":", 1) for l in r.stdout.strip().splitlines())
    got = [int(x) for x in lines["tokens"].split()]
    assert "rejected" in lines["invalid id"]
    with cdna4.Session(d, max_seq=64) as s:
        ref = s.generate(ids, cdna4.GenerateCfg(9))
        lg = s.prefill_logits(ids)
    assert got == ref
    # The C++ process may bind another rocBLAS build than torch's (its prompt GEMMs then sum in
    # another order), so the logits agree to the parity bound, not bit for bit.
    assert np.allclose([float(x) for x in lines["logits0"].split()], lg[:4], atol=LOGIT_TOL)


def test_cpp_model_loader_and_kvcache(model):
    # The reference's ModelLoader / ModelWeights / KVCache used from C++ (include/cdna3/runtime/
    # model_loader.hpp, kv_cache.hpp; tests/native/runtime_types.cpp, host-only clang++): every
    # tensor read back from its device buffer equals the file, biases only with qkv_bias, and the
    # cache has the reference's [layers][kv heads][max_seq][D] layout, zero-filled.
    import subprocess
    d, meta, t = model
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "runtime_types")
    assert os.path.exists(exe), "tests/native not built"
    r = subprocess.run([exe, d, "96"], capture_output=True, text=True, timeout=120)
    print(r.stdout[-400:])
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [l.split() for l in r.stdout.strip().splitlines()]
    assert lines[-1] == ["kvcache", "ok"]
    sums = {l[0]: int(l[1]) for l in lines if len(l) == 2 and l[0] != "kvcache"}

    def fnv(path):
        s = 1469598103934665603
        for byte in open(path, "rb").read():
            s = ((s ^ byte) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
        return s

    expect = ["embed_tokens", "lm_head", "final_norm"]
    for i in range(int(meta["n_layers"])):
        names = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "norm_attn", "norm_mlp"]
        if int(meta["qkv_bias"]):
            names += ["q_bias", "k_bias", "v_bias"]
        expect += [f"layer_{i}_{n}" for n in names]
    assert set(sums) == set(expect)
    for n in expect:
        assert sums[n] == fnv(os.path.join(d, n + ".bin")), n
    assert r.stdout.startswith("ModelLoader: loaded")   # the reference loader's report line
    cfg = next(l for l in lines if l[0] == "cfg")
    assert [int(x) for x in cfg[1:8]] == [int(meta[k]) for k in (
        "n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab_size")]


def test_greedy_ties_break_as_the_reference(tmp_path):
    # lm_head rows 3, 130 and 200 hold the same vector and every other row is zero, so at every
    # step the logits of 3, 130 and 200 are bit-identical (and 0 elsewhere). The reference's
    # argmax_kernel then picks 200 when their logit is positive (smallest bitrev8(i % 256)) and
    # token 0 otherwise; the device must choose exactly as oracle.reference_argmax.
    d = str(tmp_path / "ties")
    mf.random_model(d, n_layers=2, hidden=128, n_heads=2, ffn_dim=256, vocab_size=300, seed=9)
    meta, t = mf.read_model(d)
    H = int(meta["hidden"])
    v = (np.random.default_rng(1).standard_normal(H) * 0.2).astype(np.float16)
    lm = np.zeros((300, H), np.float16)
    lm[[3, 130, 200]] = v
    lm.tofile(os.path.join(d, "lm_head.bin"))
    meta, t = mf.read_model(d)
    ids = _prompt(meta, 9, 2)
    with cdna4.Session(d, max_seq=64) as s:
        out = s.generate_ex(ids, cdna4.GenerateCfg(24), with_logits=True)
    toks = out["tokens"]
    for i, tok in enumerate(toks):
        assert tok == oracle.reference_argmax(out["logits"][i])
    ref = oracle.LLM(meta, t, 64).greedy(ids, 24)
    print(f"tokens {toks}", flush=True)
    assert toks == ref
    assert 200 in toks and 0 in toks     # both tie cases occurred
