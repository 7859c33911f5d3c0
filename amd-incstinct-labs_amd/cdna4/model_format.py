"""The small-LLM runtime's on-disk model format, as the reference's exporter writes it
(cdna3-prims/runtime/export_model.py:70-115) and its loader reads it
(cdna3-prims/include/cdna3/runtime/model_loader.hpp:143-193):

    meta.json     one flat JSON object: n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn_dim,
                  vocab_size, rope_theta, qkv_bias (0/1), optional model_id
    <name>.bin    one raw little-endian fp16 array per tensor, row-major, no header:
                  embed_tokens [V][H], lm_head [V][H], final_norm [H],
                  layer_<i>_q_proj [nH*D][H], layer_<i>_{k,v}_proj [nKV*D][H], layer_<i>_o_proj [H][nH*D],
                  layer_<i>_{q,k,v}_bias (when qkv_bias), layer_<i>_{gate,up}_proj [F][H],
                  layer_<i>_down_proj [H][F], layer_<i>_norm_{attn,mlp} [H]

Extensions read by this runtime (absent, the reference's behaviour holds): "norm": "layernorm"
(two-pass LayerNorm instead of RMSNorm), "norm_eps", and LayerNorm betas final_norm_bias and
layer_<i>_norm_{attn,mlp}_bias.

The reference's exporter needs a HuggingFace checkpoint; `random_model` writes a seeded
random-init model of any shape instead (weights N(0, std) rounded to fp16, norm gains 1 and
biases 0 unless asked otherwise).
"""
from __future__ import annotations

import json
import os
from typing import Dict, Optional, Tuple

import numpy as np

__all__ = ["tensor_shapes", "write_model", "read_model", "random_model"]


def _dims(meta: dict) -> Tuple[int, ...]:
    H, nH = int(meta["hidden"]), int(meta["n_heads"])
    nKV = int(meta.get("n_kv_heads", nH))
    D = int(meta.get("head_dim", H // nH))
    return int(meta["n_layers"]), H, nH, nKV, D, int(meta["ffn_dim"]), int(meta["vocab_size"])


def tensor_shapes(meta: dict) -> Dict[str, Tuple[int, ...]]:
    """Every tensor a model with this meta holds, in the order the loader reads them."""
    L, H, nH, nKV, D, F, V = _dims(meta)
    layer = meta.get("norm", "rms") == "layernorm"
    shapes = {"embed_tokens": (V, H), "lm_head": (V, H), "final_norm": (H,)}
    if layer:
        shapes["final_norm_bias"] = (H,)
    for i in range(L):
        p = f"layer_{i}_"
        shapes[p + "q_proj"] = (nH * D, H)
        shapes[p + "k_proj"] = (nKV * D, H)
        shapes[p + "v_proj"] = (nKV * D, H)
        if int(meta.get("qkv_bias", 0)):
            shapes[p + "q_bias"] = (nH * D,)
            shapes[p + "k_bias"] = (nKV * D,)
            shapes[p + "v_bias"] = (nKV * D,)
        shapes[p + "o_proj"] = (H, nH * D)
        shapes[p + "gate_proj"] = (F, H)
        shapes[p + "up_proj"] = (F, H)
        shapes[p + "down_proj"] = (H, F)
        shapes[p + "norm_attn"] = (H,)
        shapes[p + "norm_mlp"] = (H,)
        if layer:
            shapes[p + "norm_attn_bias"] = (H,)
            shapes[p + "norm_mlp_bias"] = (H,)
    return shapes


def write_model(model_dir: str, meta: dict, tensors: Dict[str, np.ndarray]) -> None:
    """Writes meta.json and one fp16 .bin per tensor (shapes checked against the meta)."""
    os.makedirs(model_dir, exist_ok=True)
    shapes = tensor_shapes(meta)
    missing = set(shapes) - set(tensors)
    if missing:
        raise ValueError(f"missing tensors: {sorted(missing)[:5]}")
    for name, shape in shapes.items():
        a = np.ascontiguousarray(np.asarray(tensors[name]), dtype="<f2")
        if a.shape != shape:
            raise ValueError(f"{name}: shape {a.shape}, expected {shape}")
        a.tofile(os.path.join(model_dir, name + ".bin"))
    with open(os.path.join(model_dir, "meta.json"), "w") as f:
        json.dump(meta, f, indent=2)


def read_model(model_dir: str) -> Tuple[dict, Dict[str, np.ndarray]]:
    """(meta, {name: fp16 array}) of a model directory; each file must hold exactly its tensor."""
    with open(os.path.join(model_dir, "meta.json")) as f:
        meta = json.load(f)
    tensors = {}
    for name, shape in tensor_shapes(meta).items():
        path = os.path.join(model_dir, name + ".bin")
        if name.endswith("_bias") and name.startswith(("final_norm", "layer_")) and "norm" in name \
                and not os.path.exists(path):
            continue   # LayerNorm betas are optional (zero)
        a = np.fromfile(path, dtype="<f2")
        if a.size != int(np.prod(shape)):
            raise ValueError(f"{path}: {a.size} elements, expected {int(np.prod(shape))}")
        tensors[name] = a.reshape(shape)
    return meta, tensors


def random_model(model_dir: str, n_layers: int, hidden: int, n_heads: int, ffn_dim: int, vocab_size: int,
                 n_kv_heads: Optional[int] = None, head_dim: Optional[int] = None, rope_theta: float = 10000.0,
                 qkv_bias: bool = False, norm: str = "rms", std: float = 0.02, norm_jitter: float = 0.0,
                 seed: int = 0) -> dict:
    """Writes a seeded random-init model and returns its meta. Weights (and biases) ~ N(0, std);
    norm gains 1 + U(-norm_jitter, norm_jitter), LayerNorm betas U(-norm_jitter, norm_jitter)
    (exactly 1 and 0 with the default jitter 0). Tensors are drawn in tensor_shapes order from
    one numpy PCG64 stream, so (shape, seed) fixes every weight."""
    if norm not in ("rms", "layernorm"):
        raise ValueError("norm must be 'rms' or 'layernorm'")
    n_kv_heads = n_kv_heads or n_heads
    head_dim = head_dim or hidden // n_heads
    meta = dict(n_layers=n_layers, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                ffn_dim=ffn_dim, vocab_size=vocab_size, rope_theta=float(rope_theta), qkv_bias=int(bool(qkv_bias)),
                model_id=f"random-init seed {seed}")
    if norm == "layernorm":
        meta["norm"] = "layernorm"
    rng = np.random.default_rng(seed)
    os.makedirs(model_dir, exist_ok=True)
    for name, shape in tensor_shapes(meta).items():
        n = int(np.prod(shape))
        if "norm" in name:
            u = rng.uniform(-norm_jitter, norm_jitter, n) if norm_jitter else np.zeros(n)
            a = u if name.endswith("_bias") else 1.0 + u
        else:
            a = rng.standard_normal(n, dtype=np.float32) * np.float32(std)
        np.asarray(a, dtype="<f2").reshape(shape).tofile(os.path.join(model_dir, name + ".bin"))
    with open(os.path.join(model_dir, "meta.json"), "w") as f:
        json.dump(meta, f, indent=2)
    return meta
