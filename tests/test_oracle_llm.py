"""Pins the CPU oracle of the small-LLM runtime (oracle/llm.c) and the on-disk model format.

The oracle restates the reference's Session::run_layers with its fp16 rounding points. It is
pinned against an independent implementation of the same architecture: HuggingFace
transformers' Qwen2 / Llama decoders (the models the reference's exporter reads, and what its
own model-level check compares against), run in fp32 on the CPU with the model's weights mapped
back through the reference exporter's name map (runtime/export_model.py:83-115). The fp16
rounding points the oracle models and HF does not bound the difference (measured ~1e-3 on logits
of std ~0.3); a wrong RoPE sign or pairing, a transposed projection, a lost bias, residual or
GQA mapping, or a non-causal mask moves logits by O(0.1). Closed forms pin the embedding/final
norm/lm_head path on its own, and row independence pins the cache handling.
"""
import os

import numpy as np
import pytest

import oracle
from cdna4 import model_format as mf

HF_TOL = 4e-3   # |oracle - HF fp32| on logits: the oracle's fp16 rounding points, nothing else


def _hf_model(meta, t, arch):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    L, H, nH, nKV, D, F, V = (int(meta[k]) for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim",
                                                      "ffn_dim", "vocab_size"))
    layer = meta.get("norm") == "layernorm"
    kw = dict(vocab_size=V, hidden_size=H, intermediate_size=F, num_hidden_layers=L, num_attention_heads=nH,
              num_key_value_heads=nKV, head_dim=D, rope_theta=float(meta["rope_theta"]), rms_norm_eps=1e-6,
              tie_word_embeddings=False, max_position_embeddings=4096)
    if arch == "qwen2":
        model = transformers.Qwen2ForCausalLM(transformers.Qwen2Config(**kw))
    else:
        model = transformers.LlamaForCausalLM(transformers.LlamaConfig(attention_bias=False, mlp_bias=False, **kw))
    model = model.float().eval()
    f = lambda a: torch.from_numpy(np.asarray(a, np.float32))
    if layer:   # the LayerNorm extension: torch's own LayerNorm in place of the RMSNorms
        for lyr in model.model.layers:
            lyr.input_layernorm = torch.nn.LayerNorm(H, eps=1e-5)
            lyr.post_attention_layernorm = torch.nn.LayerNorm(H, eps=1e-5)
        model.model.norm = torch.nn.LayerNorm(H, eps=1e-5)
    sd = {"model.embed_tokens.weight": f(t["embed_tokens"]), "lm_head.weight": f(t["lm_head"]),
          "model.norm.weight": f(t["final_norm"])}
    if layer:
        sd["model.norm.bias"] = f(t["final_norm_bias"])
    for i in range(L):
        p = f"model.layers.{i}."
        for hf, ours in (("self_attn.q_proj", "q_proj"), ("self_attn.k_proj", "k_proj"), ("self_attn.v_proj", "v_proj"),
                         ("self_attn.o_proj", "o_proj"), ("mlp.gate_proj", "gate_proj"), ("mlp.up_proj", "up_proj"),
                         ("mlp.down_proj", "down_proj")):
            sd[p + hf + ".weight"] = f(t[f"layer_{i}_{ours}"])
        if arch == "qwen2":
            for x in "qkv":
                name = f"layer_{i}_{x}_bias"
                sd[p + f"self_attn.{x}_proj.bias"] = f(t[name]) if name in t else torch.zeros(
                    model.state_dict()[p + f"self_attn.{x}_proj.bias"].shape)
        sd[p + "input_layernorm.weight"] = f(t[f"layer_{i}_norm_attn"])
        sd[p + "post_attention_layernorm.weight"] = f(t[f"layer_{i}_norm_mlp"])
        if layer:
            sd[p + "input_layernorm.bias"] = f(t[f"layer_{i}_norm_attn_bias"])
            sd[p + "post_attention_layernorm.bias"] = f(t[f"layer_{i}_norm_mlp_bias"])
    res = model.load_state_dict(sd, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    return model


def _hf_logits(model, ids):
    import torch
    with torch.no_grad():
        return model(torch.tensor(np.asarray(ids, np.int64)[None])).logits[0].numpy()


MODELS = {
    # GQA 2:1, D=64, Q/K/V biases, RMSNorm (the reference's Qwen2 path)
    "qwen2_gqa_bias": (dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512,
                            vocab_size=1000, qkv_bias=True, rope_theta=10000.0), "qwen2"),
    # MHA, D=128, no bias (the Llama path), a large RoPE theta
    "llama_d128": (dict(n_layers=2, hidden=256, n_heads=2, n_kv_heads=2, head_dim=128, ffn_dim=384,
                        vocab_size=777, rope_theta=1e6), "llama"),
    # two-pass LayerNorm with gains and betas
    "layernorm": (dict(n_layers=2, hidden=192, n_heads=3, n_kv_heads=1, head_dim=64, ffn_dim=256,
                       vocab_size=500, norm="layernorm"), "llama"),
}


@pytest.fixture(scope="module", params=sorted(MODELS))
def model(request, tmp_path_factory):
    kw, arch = MODELS[request.param]
    d = str(tmp_path_factory.mktemp(request.param))
    mf.random_model(d, seed=7, norm_jitter=0.2, **kw)
    meta, t = mf.read_model(d)
    return meta, t, arch


def test_oracle_matches_huggingface_decoder(model):
    meta, t, arch = model
    hf = _hf_model(meta, t, arch)
    ids = np.random.default_rng(3).integers(0, int(meta["vocab_size"]), 48)
    ref = _hf_logits(hf, ids)
    got = oracle.LLM(meta, t, 64).forward(ids, all_logits=True)
    err = np.abs(got - ref).max()
    assert err < HF_TOL, err
    assert ref.std() > 0.1   # logits are not degenerate
    assert (got.argmax(1) == ref.argmax(1)).mean() > 0.95


def test_oracle_cache_is_row_independent(model):
    meta, t, _ = model
    ids = np.random.default_rng(4).integers(0, int(meta["vocab_size"]), 20)
    m = oracle.LLM(meta, t, 32)
    full = m.forward(ids, all_logits=True)
    m.reset()
    parts = [m.forward(ids[:7], all_logits=True), m.forward(ids[7:8], all_logits=True),
             m.forward(ids[8:], all_logits=True)]
    assert np.array_equal(np.vstack(parts), full)
    # causality: a prefix sees the same logits whatever follows
    m.reset()
    assert np.array_equal(m.forward(ids[:11], all_logits=True), full[:11])


def test_oracle_closed_form_without_layer_contributions(tmp_path):
    # o_proj = down_proj = 0: every layer adds nothing to the residual, so the logits are
    # final_norm(embed[id]) . lm_head^T, written here with numpy's own RMSNorm and matmul.
    d = str(tmp_path)
    mf.random_model(d, n_layers=2, hidden=128, n_heads=2, ffn_dim=256, vocab_size=300, seed=5, norm_jitter=0.3)
    meta, t = mf.read_model(d)
    for i in range(2):
        t[f"layer_{i}_o_proj"] = np.zeros_like(t[f"layer_{i}_o_proj"])
        t[f"layer_{i}_down_proj"] = np.zeros_like(t[f"layer_{i}_down_proj"])
    ids = np.array([0, 299, 17, 17, 250])
    got = oracle.LLM(meta, t, 8).forward(ids, all_logits=True)
    x = t["embed_tokens"].astype(np.float64)[ids]
    y = x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-6) * t["final_norm"].astype(np.float64)
    ref = y @ t["lm_head"].astype(np.float64).T
    # the logits are stored as fp16 (gemm_f32in_f16out_kernel): representable in fp16, and within
    # half an fp16 ulp (plus fp32 accumulation error) of the exact value
    assert np.array_equal(got, got.astype(np.float16).astype(np.float32))
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -11 + 1e-5)


def _bitrev8(x):
    return int(f"{x:08b}"[::-1], 2)


def test_reference_argmax_tie_break():
    # argmax_kernel (forward.hpp:244-262), restated step by step in oracle.reference_argmax:
    # thread t keeps the first maximum of indices t, t + 256, ...; the tree then merges thread
    # t + s into t for s = 128, 64, ..., 1 and keeps t on ties. Thread t therefore beats every
    # tied thread whose index, bit-reversed over 8 bits, is larger: the winner among equal maxima
    # has the smallest bitrev8(i % 256), then the smallest i.
    x = np.zeros(1000, np.float32)
    x[[5, 256]] = 3.0
    assert oracle.reference_argmax(x) == 256          # thread 0 beats thread 5
    x[:] = 0
    x[[44, 300]] = 3.0
    assert oracle.reference_argmax(x) == 44           # same thread: its first maximum
    assert oracle.reference_argmax(np.zeros(1000, np.float32)) == 0
    assert oracle.reference_argmax(np.array([1.0, 7.0, 7.0], np.float32)) == 2   # thread 2 merges into 0 first
    x[:] = 0
    x[[1, 128]] = 1.0
    assert oracle.reference_argmax(x) == 128          # bitrev8(128) = 1 < bitrev8(1) = 128
    rng = np.random.default_rng(0)
    for n in (3, 255, 256, 257, 1000, 32000):
        for _ in range(20):
            v = rng.integers(0, 4, n).astype(np.float32)     # many ties
            best = np.flatnonzero(v == v.max())
            want = min(best, key=lambda i: (_bitrev8(i % 256), i))
            assert oracle.reference_argmax(v) == want


def test_model_format_round_trip_and_validation(tmp_path):
    d = str(tmp_path / "m")
    meta = mf.random_model(d, n_layers=1, hidden=64, n_heads=1, ffn_dim=64, vocab_size=10, qkv_bias=True, seed=1)
    assert meta["head_dim"] == 64 and meta["n_kv_heads"] == 1 and meta["qkv_bias"] == 1
    meta2, t = mf.read_model(d)
    assert meta2 == meta
    assert set(t) == set(mf.tensor_shapes(meta))
    assert t["layer_0_q_bias"].shape == (64,) and t["lm_head"].shape == (10, 64)
    assert np.all(t["final_norm"] == 1) and t["embed_tokens"].dtype == np.float16
    assert 0.015 < float(np.std(t["lm_head"].astype(np.float32))) < 0.025
    # same seed, same weights; a different seed differs
    d2 = str(tmp_path / "m2")
    mf.random_model(d2, n_layers=1, hidden=64, n_heads=1, ffn_dim=64, vocab_size=10, qkv_bias=True, seed=1)
    assert open(os.path.join(d, "layer_0_up_proj.bin"), "rb").read() == \
        open(os.path.join(d2, "layer_0_up_proj.bin"), "rb").read()
    with open(os.path.join(d, "lm_head.bin"), "ab") as f:
        f.write(b"\0\0")
    with pytest.raises(ValueError):
        mf.read_model(d)
    out = str(tmp_path / "w")
    mf.write_model(out, meta, t)
    with pytest.raises(ValueError):
        bad = dict(t)
        bad["lm_head"] = t["lm_head"][:5]
        mf.write_model(out, meta, bad)
