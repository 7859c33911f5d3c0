"""The reference's PyTorch custom ops, registered over libcdna4_attn.so.

    torch.ops.amdinstinct.flash_attn(q, k, v) -> o
        research/flash-attention-mi300x/llm_integration/torch_op/fa_torch_op.hip:36-66:
        causal GQA prefill on head-major q [nQH][seq][D], k, v [nKVH][seq][D] -> o [nQH][seq][D]
    torch.ops.amdinstinct.flash_attn_decode(q, k_cache, v_cache) -> o
        fa_decode_op.hip:26-57: one query per head, q [nQH][D], caches [nKVH][N][D] -> o [nQH][D]

Same schemas, namespace and dispatch key (CUDA, which is the HIP device on ROCm) as the
reference's TORCH_LIBRARY registration, so code written against those ops runs unchanged after
`register()`. Contract checks raise RuntimeError, as TORCH_CHECK does. Differences: fp16 and
bf16 are accepted (the reference: fp16 only) and any seq >= 1 is computed (the reference
required seq % 16 == 0 and kv seq % 64 == 0). Meta implementations give shapes for tracing.
"""
from __future__ import annotations

import torch

from . import DecodeCfg, PrefillCfg, decode, prefill

_LIB = None
_DTYPES = (torch.float16, torch.bfloat16)


def _check(t: torch.Tensor, name: str, dims: int) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU (HIP) tensor")
    if t.dtype not in _DTYPES:
        raise RuntimeError(f"{name} must be fp16 or bf16")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.dim() != dims:
        raise RuntimeError(f"{name} must have {dims} dimensions")


def _flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n, 3)
    nqh, seq, D = q.shape
    nkvh = k.shape[0]
    if k.shape[1] != seq or v.shape[1] != seq or tuple(v.shape) != tuple(k.shape):
        raise RuntimeError("k/v seq must match q")
    if k.shape[2] != D:
        raise RuntimeError("k/v head_dim must match q")
    if nqh % nkvh:
        raise RuntimeError("nQH must be a multiple of nKVH (GQA)")
    if D not in (64, 128):
        raise RuntimeError("D must be 64 or 128")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise RuntimeError("q, k, v must share one dtype")
    o = torch.empty_like(q)
    prefill(q, k, v, o, PrefillCfg(D, seq, seq, nqh, nkvh, 1, 1))
    return o


def _flash_attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> torch.Tensor:
    _check(q, "q", 2)
    _check(k_cache, "k_cache", 3)
    _check(v_cache, "v_cache", 3)
    nqh, D = q.shape
    nkvh, N, _ = k_cache.shape
    if k_cache.shape[2] != D or v_cache.shape[2] != D:
        raise RuntimeError("cache head_dim mismatch")
    if v_cache.shape[0] != nkvh or v_cache.shape[1] != N:
        raise RuntimeError("k/v cache shape mismatch")
    if nqh % nkvh:
        raise RuntimeError("nQH must be a multiple of nKVH (GQA)")
    if D not in (64, 128):
        raise RuntimeError("D must be 64 or 128")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise RuntimeError("q and the caches must share one dtype")
    o = torch.empty((nqh, D), dtype=q.dtype, device=q.device)
    # The split-K workspace comes from torch's caching allocator on the current stream.
    decode(q, k_cache, v_cache, o, DecodeCfg(D, N, nqh, nkvh, 1, 0), workspace="auto")
    return o


def register() -> None:
    """Defines torch.ops.amdinstinct.{flash_attn, flash_attn_decode} once per process. If the
    namespace already holds these ops (another library registered them), nothing is changed."""
    global _LIB
    if _LIB is not None:
        return
    ns = torch.ops.amdinstinct
    if hasattr(ns, "flash_attn") or hasattr(ns, "flash_attn_decode"):
        _LIB = "external"
        return
    lib = torch.library.Library("amdinstinct", "FRAGMENT")
    lib.define("flash_attn(Tensor q, Tensor k, Tensor v) -> Tensor")
    lib.define("flash_attn_decode(Tensor q, Tensor k_cache, Tensor v_cache) -> Tensor")
    lib.impl("flash_attn", _flash_attn, "CUDA")
    lib.impl("flash_attn_decode", _flash_attn_decode, "CUDA")
    lib.impl("flash_attn", lambda q, k, v: torch.empty_like(q), "Meta")
    lib.impl("flash_attn_decode", lambda q, k, v: torch.empty_like(q), "Meta")
    _LIB = lib
