"""Python host interface of libcdna4_attn.so, the MI355X (gfx950) attention hot path.

Mirrors the reference's host API for the path (cdna3-prims/include/cdna3/attention.hpp,
cdna3-prims/include/cdna3/runtime/forward.hpp) over the library's C ABI (include/cdna4_attn.h):

    prefill(Q, K, V, O, PrefillCfg(...))          cdna3::attn::prefill   (attention.hpp:86)
    decode(q, K, V, o, DecodeCfg(...))            cdna3::attn::decode    (attention.hpp:117)
    decode_dme(q, K, V, o, DecodeDmeCfg(...))     cdna3::attn::decode_dme (attention.hpp:152)
    rmsnorm_f32, layernorm_f32, rope_f16, rope_table_f32    runtime entry points
    Session(model_dir, max_seq).generate(ids, GenerateCfg(...))
                                                  cdna3::runtime::Session (runtime/session.hpp:47)
    reduce, scan_inclusive                        device-wide wave::dpp reductions / scans
    flash_attn(q, k, v), flash_attn_decode(q, k_cache, v_cache)
                                                  the reference's torch ops (fa_torch_op.hip:36,
                                                  fa_decode_op.hip:26), as plain functions

Tensors are torch tensors on the current HIP device; PyTorch only provides device memory and
the stream. Every call enqueues on torch's current stream (or the `stream` argument) and does
not synchronise. A non-zero library return code raises RuntimeError, as the reference's
launchers return hipErrorInvalidValue and its torch ops raise through TORCH_CHECK. There is no
fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import re
from typing import Optional

import torch

__all__ = [
    "F32", "F16", "BF16", "F64", "I32", "I64", "SUM", "MAX", "MIN",
    "PrefillCfg", "DecodeCfg", "DecodeDmeCfg", "library_path", "lib", "abi_version", "error_string",
    "prefill", "decode", "decode_dme", "decode_workspace_size", "reduce", "reduce_workspace_size",
    "scan_inclusive", "scan_workspace_size", "rmsnorm_f32", "layernorm_f32", "rope_f16",
    "rope_table_f32", "flash_attn", "flash_attn_decode", "CDNA4Error", "PrefillStrides", "prefill_strided",
    "scatter_kv_f16", "repack_f16", "rope_append_kv_f16", "ModelCfg", "GenerateCfg", "Session",
    "PlanInfo", "prefill_plan", "decode_plan", "scan_status", "KERNEL_NAMES", "decode_noalloc",
    "decode_noalloc_max_bytes", "softmax_rows_f32",
]

# Element types and operators (include/cdna4_attn.h).
F32, F16, BF16, F64, I32, I64 = 0, 1, 2, 3, 4, 5
SUM, MAX, MIN = 0, 1, 2
_OPS = {"sum": SUM, "max": MAX, "min": MIN, SUM: SUM, MAX: MAX, MIN: MIN}
_TORCH_DTYPES = {
    torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
    torch.float64: F64, torch.int32: I32, torch.int64: I64,
}


class CDNA4Error(RuntimeError):
    """A non-zero return code of libcdna4_attn.so; `.code` is the hipError_t value."""

    def __init__(self, what: str, code: int):
        super().__init__(f"{what}: {error_string(code)} (code {code})")
        self.code = code


class PrefillCfg(ctypes.Structure):
    """cdna3_prefill_cfg: field for field the reference's PrefillCfg (attention.hpp:63-71)."""
    _fields_ = [("D", ctypes.c_int), ("seqQ", ctypes.c_int), ("seqK", ctypes.c_int),
                ("nQHeads", ctypes.c_int), ("nKVHeads", ctypes.c_int), ("batch", ctypes.c_int),
                ("causal", ctypes.c_int)]


class PrefillStrides(ctypes.Structure):
    """cdna3_prefill_strides: element strides (batch, head, row) of Q, of K and V, and of O."""
    _fields_ = [(n, ctypes.c_longlong) for n in ("q_batch", "q_head", "q_row", "kv_batch", "kv_head", "kv_row",
                                                 "o_batch", "o_head", "o_row")]


class DecodeCfg(ctypes.Structure):
    """cdna3_decode_cfg: the reference's DecodeCfg {D, N, nQHeads, nKVHeads} (attention.hpp:73-78)
    plus batch (default 1) and stride_kv (0 = packed)."""
    _fields_ = [("D", ctypes.c_int), ("N", ctypes.c_int), ("nQHeads", ctypes.c_int),
                ("nKVHeads", ctypes.c_int), ("batch", ctypes.c_int), ("stride_kv", ctypes.c_int)]

    def __init__(self, D=0, N=0, nQHeads=0, nKVHeads=0, batch=1, stride_kv=0):
        super().__init__(D, N, nQHeads, nKVHeads, batch, stride_kv)


class ModelCfg(ctypes.Structure):
    """cdna3_model_cfg: the reference's ModelConfig (runtime/model_loader.hpp:52-61) plus the
    qkv_bias flag and the norm kind and epsilon."""
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                            "vocab_size")] + \
               [("rope_theta", ctypes.c_float), ("qkv_bias", ctypes.c_int), ("layernorm", ctypes.c_int),
                ("norm_eps", ctypes.c_float)]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class PlanInfo(ctypes.Structure):
    """cdna3_plan_info: the kernel a call would launch (CDNA4_KERNEL_*), its waves per workgroup,
    rows (prefill: queries per work item; decode: keys per split), split-K partials, grid and
    workspace bytes."""
    _fields_ = [("kernel", ctypes.c_int), ("waves", ctypes.c_int), ("rows", ctypes.c_int),
                ("partials", ctypes.c_int), ("grid", ctypes.c_longlong), ("workspace", ctypes.c_size_t)]

    @property
    def name(self) -> str:
        return KERNEL_NAMES.get(self.kernel, "?")


# CDNA4_KERNEL_* (include/cdna4_attn.h)
KERNEL_NAMES = {1: "fa_mfma_8w", 2: "fa_mfma_4w", 3: "fa_small", 4: "fa_f32", 5: "decode_split", 6: "decode_wg"}


def DecodeDmeCfg(D: int, N: int, nQHeads: int, nKVHeads: int, stride_kv: int, batch: int = 1) -> DecodeCfg:
    """The reference's DecodeDmeCfg {D, N, nQHeads, nKVHeads, stride_kv}
    (detail/fa_decode_dme_kernel.hpp:45-48) as a DecodeCfg."""
    return DecodeCfg(D, N, nQHeads, nKVHeads, batch, stride_kv)


_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return os.path.join(_HERE, "libcdna4_attn.so")


def _declare(l: ctypes.CDLL) -> None:
    c_int, c_size, vp, c_float = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float
    sig = {
        "cdna3_abi_version": (c_int, []),
        "cdna3_error_string": (ctypes.c_char_p, [c_int]),
        "cdna3_softmax_rows_f32": (c_int, [vp, vp, c_int, c_int, vp]),
        "cdna3_attn_prefill": (c_int, [vp, vp, vp, vp, ctypes.POINTER(PrefillCfg), c_int, vp]),
        "cdna3_attn_prefill_strided": (c_int, [vp, vp, vp, vp, ctypes.POINTER(PrefillCfg),
                                               ctypes.POINTER(PrefillStrides), c_int, vp]),
        "cdna3_attn_decode_workspace_size": (c_size, [ctypes.POINTER(DecodeCfg)]),
        "cdna3_attn_decode": (c_int, [vp, vp, vp, vp, ctypes.POINTER(DecodeCfg), c_int, vp, c_size, vp]),
        "cdna3_attn_decode_noalloc": (c_int, [vp, vp, vp, vp, ctypes.POINTER(DecodeCfg), c_int, vp]),
        "cdna3_attn_decode_noalloc_max_bytes": (c_size, []),
        "cdna3_attn_prefill_plan": (c_int, [ctypes.POINTER(PrefillCfg), c_int, ctypes.POINTER(PlanInfo)]),
        "cdna3_attn_decode_plan": (c_int, [ctypes.POINTER(DecodeCfg), c_int, c_int, ctypes.POINTER(PlanInfo)]),
        "cdna3_scan_status": (c_int, [vp, ctypes.POINTER(c_int), vp]),
        "cdna3_model_load": (c_int, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "cdna3_model_free": (None, [vp]),
        "cdna3_model_config": (c_int, [vp, vp]),
        "cdna3_model_weights_get": (c_int, [vp, vp]),
        "cdna3_reduce_workspace_size": (c_size, [c_size, c_int]),
        "cdna3_reduce": (c_int, [c_int, c_int, vp, c_size, vp, vp, c_size, vp]),
        "cdna3_scan_workspace_size": (c_size, [c_size, c_int]),
        "cdna3_scan_inclusive": (c_int, [c_int, c_int, vp, c_size, vp, vp, c_size, vp]),
        "cdna3_rmsnorm_f32": (c_int, [vp, vp, vp, c_int, c_int, c_float, vp]),
        "cdna3_layernorm_f32": (c_int, [vp, vp, vp, vp, c_int, c_int, c_float, vp]),
        "cdna4_gemm_f16_nt": (c_int, [vp, vp, vp, c_int, c_int, c_int, c_int, c_int, c_int, vp]),
        "cdna4_gemm_f16_nt_tile": (c_int, [c_int, c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
        "cdna4_gemm_f16_nt_silu": (c_int, [vp, vp, vp, c_int, c_int, c_int, c_int, vp]),
        "cdna4_gemm_f16_nt_silu_tile": (c_int, [c_int, c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
        "cdna3_rope_f16": (c_int, [vp, vp, vp, c_int, c_int, c_int, vp]),
        "cdna3_rope_table_f32": (c_int, [vp, vp, c_int, c_int, c_int, c_float, vp]),
        "cdna3_scatter_kv_f16": (c_int, [vp, vp] + [c_int] * 5 + [vp]),
        "cdna3_repack_f16": (c_int, [vp, vp] + [c_int] * 4 + [vp]),
        "cdna3_rope_append_kv_f16": (c_int, [vp] * 8 + [c_int] * 6 + [vp]),
        "cdna3_session_create": (c_int, [ctypes.c_char_p, c_int, ctypes.POINTER(vp)]),
        "cdna3_session_destroy": (None, [vp]),
        "cdna3_session_config": (c_int, [vp, ctypes.POINTER(ModelCfg)]),
        "cdna3_session_generate": (c_int, [vp, vp, c_int, c_int, c_int, vp, ctypes.POINTER(c_int), vp,
                                           ctypes.POINTER(c_float), ctypes.POINTER(c_float)]),
        "cdna3_session_prefill_logits": (c_int, [vp, vp, c_int, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def lib() -> ctypes.CDLL:
    """The loaded library. Raises if it has not been built (no fallback path exists)."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(f"libcdna4_attn.so not built ({path}); run __graft_entry__.build()")
        l = ctypes.CDLL(path)
        _declare(l)
        _LIB = l
    return _LIB


def header_symbols() -> list:
    """Every function name declared in include/cdna4_attn.h."""
    hdr = os.path.join(_HERE, "..", "..", "include", "cdna4_attn.h")
    text = open(hdr).read()
    return sorted(set(re.findall(r"\b(cdna3_[a-z0-9_]+)\s*\(", text)))


def abi_version() -> int:
    return lib().cdna3_abi_version()


def error_string(code: int) -> str:
    return lib().cdna3_error_string(code).decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise CDNA4Error(what, rc)


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, torch.cuda.Stream):
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(int(stream))


def _on_stream(stream):
    """Context under which torch allocations belong to the stream the call launches on. A
    temporary (split-K workspace, contiguous copy, scan workspace) freed when the call returns
    then goes back to that stream's pool, so the caching allocator can hand it out again only to
    work ordered after the kernels that still use it; allocated on another stream, it could be
    reused and overwritten while they run."""
    if stream is None:
        return contextlib.nullcontext()
    if not isinstance(stream, torch.cuda.Stream):
        stream = torch.cuda.ExternalStream(int(stream))
    return torch.cuda.stream(stream)


def _ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _dev(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("tensors must be on the GPU")
        if not t.is_contiguous():
            raise ValueError("tensors must be contiguous")


def _dtype(t: torch.Tensor) -> int:
    try:
        return _TORCH_DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


# ---- attention ----------------------------------------------------------------------------

def prefill(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, O: torch.Tensor, cfg: PrefillCfg,
            stream=None) -> None:
    """cdna3::attn::prefill: Q, O [batch][nQH][seqQ][D]; K, V [batch][nKVH][seqK][D];
    fp16, bf16 or fp32 (all four alike)."""
    _dev(Q, K, V, O)
    dt = _dtype(Q)
    if not (K.dtype == V.dtype == O.dtype == Q.dtype):
        raise ValueError("Q, K, V, O must share one dtype")
    nq = cfg.batch * cfg.nQHeads * cfg.seqQ * cfg.D
    nk = cfg.batch * cfg.nKVHeads * cfg.seqK * cfg.D
    if Q.numel() < nq or O.numel() < nq or K.numel() < nk or V.numel() < nk:
        raise ValueError("tensor smaller than the configuration")
    _check(lib().cdna3_attn_prefill(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), ctypes.byref(cfg), dt,
                                    _stream(stream)), "cdna3_attn_prefill")


def prefill_strided(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, O: torch.Tensor, cfg: PrefillCfg,
                    strides: PrefillStrides, stream=None) -> None:
    """Prefill over strided Q/K/V/O (fp16 or bf16), e.g. K/V in place in a KV cache and O
    token-major. The caller guarantees the strides stay inside the tensors."""
    _dev(Q, K, V, O)
    dt = _dtype(Q)
    if not (K.dtype == V.dtype == O.dtype == Q.dtype):
        raise ValueError("Q, K, V, O must share one dtype")
    _check(lib().cdna3_attn_prefill_strided(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), ctypes.byref(cfg),
                                            ctypes.byref(strides), dt, _stream(stream)), "cdna3_attn_prefill_strided")


def decode_workspace_size(cfg: DecodeCfg) -> int:
    return int(lib().cdna3_attn_decode_workspace_size(ctypes.byref(cfg)))


def decode(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, o: torch.Tensor, cfg: DecodeCfg,
           workspace="auto", stream=None) -> None:
    """cdna3::attn::decode with batch: q, o [batch][nQH][D]; K, V [batch][nKVH][stride][D];
    fp16 or bf16. `workspace`: "auto" (default) allocates the split-K workspace from torch's
    caching allocator on the stream the call launches on; a uint8 tensor of >= decode_workspace_size(cfg)
    bytes is used as given; None runs the one-launch plan that needs no workspace (the
    reference launchers' contract)."""
    _dev(q, K, V, o)
    dt = _dtype(q)
    if not (K.dtype == V.dtype == o.dtype == q.dtype):
        raise ValueError("q, K, V, o must share one dtype")
    stride = cfg.stride_kv or cfg.N
    if q.numel() < cfg.batch * cfg.nQHeads * cfg.D or o.numel() < cfg.batch * cfg.nQHeads * cfg.D:
        raise ValueError("q/o smaller than the configuration")
    if min(K.numel(), V.numel()) < cfg.batch * cfg.nKVHeads * stride * cfg.D:
        raise ValueError("K/V smaller than the configuration")
    if isinstance(workspace, str) and workspace != "auto":
        raise ValueError("workspace must be 'auto', None or a uint8 tensor")
    with _on_stream(stream):
        if isinstance(workspace, str):
            need = decode_workspace_size(cfg)
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device) if need > 0 else None
        ws_bytes = 0
        if workspace is not None:
            _dev(workspace)
            ws_bytes = workspace.numel() * workspace.element_size()
        _check(lib().cdna3_attn_decode(_ptr(q), _ptr(K), _ptr(V), _ptr(o), ctypes.byref(cfg), dt, _ptr(workspace),
                                       ws_bytes, _stream(stream)), "cdna3_attn_decode")


def decode_noalloc(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, o: torch.Tensor, cfg: DecodeCfg,
                   stream=None) -> None:
    """cdna3_attn_decode_noalloc: the split-K decode with its partials in the library's static
    per-GPU scratch array; allocates nothing. Calls that overlap on one GPU race (serialise them)."""
    _dev(q, K, V, o)
    dt = _dtype(q)
    if not (K.dtype == V.dtype == o.dtype == q.dtype):
        raise ValueError("q, K, V, o must share one dtype")
    stride = cfg.stride_kv or cfg.N
    if q.numel() < cfg.batch * cfg.nQHeads * cfg.D or o.numel() < cfg.batch * cfg.nQHeads * cfg.D:
        raise ValueError("q/o smaller than the configuration")
    if min(K.numel(), V.numel()) < cfg.batch * cfg.nKVHeads * stride * cfg.D:
        raise ValueError("K/V smaller than the configuration")
    _check(lib().cdna3_attn_decode_noalloc(_ptr(q), _ptr(K), _ptr(V), _ptr(o), ctypes.byref(cfg), dt,
                                           _stream(stream)), "cdna3_attn_decode_noalloc")


def decode_noalloc_max_bytes() -> int:
    return int(lib().cdna3_attn_decode_noalloc_max_bytes())


def prefill_plan(cfg: PrefillCfg, dtype=BF16) -> PlanInfo:
    """The kernel cdna3_attn_prefill would launch for cfg on the current device."""
    if isinstance(dtype, torch.dtype):
        dtype = _TORCH_DTYPES[dtype]
    out = PlanInfo()
    _check(lib().cdna3_attn_prefill_plan(ctypes.byref(cfg), dtype, ctypes.byref(out)), "cdna3_attn_prefill_plan")
    return out


def decode_plan(cfg: DecodeCfg, dtype=F16, with_workspace: bool = True) -> PlanInfo:
    """The kernels cdna3_attn_decode would launch for cfg, with or without a workspace."""
    if isinstance(dtype, torch.dtype):
        dtype = _TORCH_DTYPES[dtype]
    out = PlanInfo()
    _check(lib().cdna3_attn_decode_plan(ctypes.byref(cfg), dtype, 1 if with_workspace else 0, ctypes.byref(out)),
           "cdna3_attn_decode_plan")
    return out


def decode_dme(q, K, V, o, cfg: DecodeCfg, workspace="auto", stream=None) -> None:
    """cdna3::attn::decode_dme: decode reading a strided [nKVH][stride_kv][D] cache in place."""
    decode(q, K, V, o, cfg, workspace, stream)


# ---- device-wide reduce / scan ----------------------------------------------------------

def reduce_workspace_size(n: int, dtype: int) -> int:
    return int(lib().cdna3_reduce_workspace_size(n, dtype))


def scan_workspace_size(n: int, dtype: int) -> int:
    return int(lib().cdna3_scan_workspace_size(n, dtype))


def _acc_dtype(t: torch.Tensor) -> torch.dtype:
    return torch.float32 if t.dtype in (torch.float16, torch.bfloat16) else t.dtype


def reduce(x: torch.Tensor, op="sum", out: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Reduce a whole contiguous array with wave::dpp semantics; fp16/bf16 accumulate in fp32."""
    _dev(x)
    dt, o = _dtype(x), _OPS[op]
    n = x.numel()
    with _on_stream(stream):
        if out is None:
            out = torch.empty(1, dtype=_acc_dtype(x), device=x.device)
        if workspace is None:
            workspace = torch.empty(reduce_workspace_size(n, dt), dtype=torch.uint8, device=x.device)
        _check(lib().cdna3_reduce(o, dt, _ptr(x), n, _ptr(out), _ptr(workspace), workspace.numel(),
                                  _stream(stream)), "cdna3_reduce")
    return out


def scan_inclusive(x: torch.Tensor, op="sum", out: Optional[torch.Tensor] = None,
                   workspace: Optional[torch.Tensor] = None, stream=None, check: bool = True) -> torch.Tensor:
    """Inclusive scan of a whole contiguous array; fp16/bf16 accumulate (and return) fp32.
    With check (the default) the call synchronises the stream and raises CDNA4Error if the scan's
    look-back reported a wait past its bound (cdna3_scan_status), so a wrong result can never be
    returned silently; check=False leaves the call asynchronous (test with scan_status later)."""
    _dev(x)
    dt, o = _dtype(x), _OPS[op]
    n = x.numel()
    with _on_stream(stream):
        if out is None:
            out = torch.empty(n, dtype=_acc_dtype(x), device=x.device)
        if workspace is None:   # zeroed: no word of it can carry a valid look-back tag
            workspace = torch.zeros(max(1, scan_workspace_size(n, dt)), dtype=torch.uint8, device=x.device)
        _check(lib().cdna3_scan_inclusive(o, dt, _ptr(x), n, _ptr(out), _ptr(workspace), workspace.numel(),
                                          _stream(stream)), "cdna3_scan_inclusive")
        if check and n > 0:
            st = scan_status(workspace, stream)
            if st != 0:
                raise CDNA4Error("cdna3_scan_inclusive: look-back wait exceeded its bound; result invalid", 1)
    return out


def scan_status(workspace: torch.Tensor, stream=None) -> int:
    """cdna3_scan_status: 0 when the last scan on this workspace is valid (synchronises)."""
    st = ctypes.c_int(-1)
    _check(lib().cdna3_scan_status(_ptr(workspace), ctypes.byref(st), _stream(stream)), "cdna3_scan_status")
    return st.value


# ---- runtime norms and RoPE --------------------------------------------------------------

def rmsnorm_f32(X: torch.Tensor, W: torch.Tensor, eps: float = 1e-6, out: Optional[torch.Tensor] = None,
                stream=None) -> torch.Tensor:
    """rmsnorm_f32_kernel: X fp32 [M][H], W fp16 [H] -> Y fp32 [M][H]."""
    _dev(X, W)
    if X.dtype != torch.float32 or W.dtype != torch.float16:
        raise ValueError("X must be fp32 and W fp16")
    M, H = X.shape
    with _on_stream(stream):
        out = torch.empty_like(X) if out is None else out
    _check(lib().cdna3_rmsnorm_f32(_ptr(X), _ptr(W), _ptr(out), M, H, eps, _stream(stream)), "cdna3_rmsnorm_f32")
    return out


def layernorm_f32(X: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-5,
                  out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Two-pass layernorm: X, Y fp32 [M][H]; gamma, beta fp32 [H]."""
    _dev(X, gamma, beta)
    M, H = X.shape
    with _on_stream(stream):
        out = torch.empty_like(X) if out is None else out
    _check(lib().cdna3_layernorm_f32(_ptr(X), _ptr(gamma), _ptr(beta), _ptr(out), M, H, eps, _stream(stream)),
           "cdna3_layernorm_f32")
    return out


def softmax_rows_f32(X: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Row softmax of X fp32 [M][H] (softmax_kernel, bench_softmax.hip:59-105) into out (may be X)."""
    _dev(X)
    if X.dtype != torch.float32 or X.dim() != 2:
        raise ValueError("X must be fp32 [M][H]")
    M, H = X.shape
    with _on_stream(stream):
        out = torch.empty_like(X) if out is None else out
    _check(lib().cdna3_softmax_rows_f32(_ptr(X), _ptr(out), M, H, _stream(stream)), "cdna3_softmax_rows_f32")
    return out


def gemm_f16_nt(X: torch.Tensor, W: torch.Tensor, out: Optional[torch.Tensor] = None, accum: bool = False,
                out_dtype=torch.float32, stream=None) -> torch.Tensor:
    """Y = X W^T (+ Y when accum): X fp16 [M][K], W fp16 [N][K], Y fp32 or fp16 [M][N] (the
    runtime's prompt GEMM; raises for the shapes it does not take)."""
    _dev(X, W)
    M, K = X.shape
    N = W.shape[0]
    if W.shape[1] != K or X.dtype != torch.float16 or W.dtype != torch.float16:
        raise ValueError("gemm_f16_nt: X [M][K] and W [N][K] fp16")
    if out is not None and (out.dtype not in (torch.float32, torch.float16) or out.shape[0] != M
                            or out.shape[1] != N or out.stride(1) != 1):
        raise ValueError("gemm_f16_nt: out fp32 or fp16 [M][N], rows contiguous")
    with _on_stream(stream):       # the contiguous copies below live until the kernel has read them
        if out is None:
            out = (torch.zeros if accum else torch.empty)(M, N, device=X.device, dtype=out_dtype)
        Xc, Wc = X.contiguous(), W.contiguous()
        _check(lib().cdna4_gemm_f16_nt(_ptr(Xc), _ptr(Wc), _ptr(out), int(out.dtype == torch.float32), int(accum), M,
                                       N, K, out.stride(0), _stream(stream)), "cdna4_gemm_f16_nt")
    return out


def gemm_f16_nt_silu(X: torch.Tensor, W: torch.Tensor, out: Optional[torch.Tensor] = None,
                     stream=None) -> torch.Tensor:
    """Y = fp16(silu(X Wg^T) * (X Wu^T)), W = [Wg; Wu] fp16 [2F][K], X fp16 [M][K], Y fp16 [M][F]
    (the SwiGLU gate|up product and the SiLU product in one launch; raises for the shapes it does
    not take)."""
    _dev(X, W)
    M, K = X.shape
    if W.shape[0] % 2 or W.shape[1] != K or X.dtype != torch.float16 or W.dtype != torch.float16:
        raise ValueError("gemm_f16_nt_silu: X [M][K] and W [2F][K] fp16")
    F = W.shape[0] // 2
    if out is not None and (out.dtype != torch.float16 or tuple(out.shape) != (M, F) or out.stride(1) != 1):
        raise ValueError("gemm_f16_nt_silu: out fp16 [M][F], rows contiguous")
    with _on_stream(stream):
        if out is None:
            out = torch.empty(M, F, device=X.device, dtype=torch.float16)
        Xc, Wc = X.contiguous(), W.contiguous()
        _check(lib().cdna4_gemm_f16_nt_silu(_ptr(Xc), _ptr(Wc), _ptr(out), M, F, K, out.stride(0), _stream(stream)),
               "cdna4_gemm_f16_nt_silu")
    return out


def gemm_f16_nt_silu_tile(M: int, F: int, K: int):
    """(BM, BN): the tile gemm_f16_nt_silu takes (BN counts the gate and up rows together)."""
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    _check(lib().cdna4_gemm_f16_nt_silu_tile(M, F, K, ctypes.byref(bm), ctypes.byref(bn)),
           "cdna4_gemm_f16_nt_silu_tile")
    return bm.value, bn.value


def gemm_f16_nt_tile(M: int, N: int, K: int):
    """(BM, BN): the tile (rows of X, rows of W per workgroup) gemm_f16_nt takes for a shape."""
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    _check(lib().cdna4_gemm_f16_nt_tile(M, N, K, ctypes.byref(bm), ctypes.byref(bn)), "cdna4_gemm_f16_nt_tile")
    return bm.value, bn.value


def rope_f16(T: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, seq: int, heads: int, D: int,
             stream=None) -> None:
    """rope_kernel, in place on T fp16 [seq][heads*D] with cos/sin fp32 [seq][D]."""
    _dev(T, cos, sin)
    _check(lib().cdna3_rope_f16(_ptr(T), _ptr(cos), _ptr(sin), seq, heads, D, _stream(stream)), "cdna3_rope_f16")


def rope_table_f32(pos0: int, T: int, D: int, theta: float = 10000.0, device=None, stream=None):
    """Session::fill_rope on the device: cos, sin fp32 [T][D] for positions pos0 .. pos0+T-1."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    with _on_stream(stream):
        cos = torch.empty((T, D), dtype=torch.float32, device=device)
        sin = torch.empty((T, D), dtype=torch.float32, device=device)
    _check(lib().cdna3_rope_table_f32(_ptr(cos), _ptr(sin), pos0, T, D, theta, _stream(stream)),
           "cdna3_rope_table_f32")
    return cos, sin


# ---- KV cache and layouts of the runtime layer loop -----------------------------------------

def scatter_kv_f16(src: torch.Tensor, cache: torch.Tensor, T: int, heads: int, D: int, pos0: int, max_seq: int,
                   stream=None) -> None:
    """scatter_kv_kernel: cache [heads][max_seq][D] rows pos0 .. pos0+T-1 <- src [T][heads][D]."""
    _dev(src, cache)
    _check(lib().cdna3_scatter_kv_f16(_ptr(src), _ptr(cache), T, heads, D, pos0, max_seq, _stream(stream)),
           "cdna3_scatter_kv_f16")


def repack_f16(src: torch.Tensor, dst: torch.Tensor, seq: int, heads: int, D: int, direction: int,
               stream=None) -> None:
    """repack_kernel: direction 0 token-major [seq][heads][D] -> head-major [heads][seq][D], 1 back."""
    _dev(src, dst)
    _check(lib().cdna3_repack_f16(_ptr(src), _ptr(dst), seq, heads, D, direction, _stream(stream)),
           "cdna3_repack_f16")


def rope_append_kv_f16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_out: torch.Tensor,
                       K_cache: torch.Tensor, V_cache: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, T: int,
                       nQH: int, nKVH: int, D: int, pos0: int, max_seq: int, stream=None) -> None:
    """RoPE(q) -> q_out [nQH][T][D]; RoPE(k), v -> K_cache / V_cache [nKVH][max_seq][D] at pos0."""
    _dev(q, k, v, q_out, K_cache, V_cache, cos, sin)
    _check(lib().cdna3_rope_append_kv_f16(_ptr(q), _ptr(k), _ptr(v), _ptr(q_out), _ptr(K_cache), _ptr(V_cache),
                                          _ptr(cos), _ptr(sin), T, nQH, nKVH, D, pos0, max_seq, _stream(stream)),
           "cdna3_rope_append_kv_f16")


# ---- the reference's torch-op contracts, as plain functions ------------------------------

def flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """amdinstinct.flash_attn (fa_torch_op.hip:36-59): causal GQA prefill on head-major
    q [nQH][seq][D], k, v [nKVH][seq][D] (fp16; bf16 also accepted) -> o [nQH][seq][D]."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be [heads, seq, D]")
    nqh, seq, D = q.shape
    nkvh = k.shape[0]
    if k.shape[1] != seq or v.shape[1] != seq or k.shape[2] != D or v.shape[2] != D:
        raise ValueError("k/v shape must match q")
    o = torch.empty_like(q)
    prefill(q, k, v, o, PrefillCfg(D, seq, seq, nqh, nkvh, 1, 1))
    return o


def flash_attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> torch.Tensor:
    """amdinstinct.flash_attn_decode (fa_decode_op.hip:26-50): q [nQH][D], caches [nKVH][N][D]."""
    if q.dim() != 2 or k_cache.dim() != 3 or v_cache.dim() != 3:
        raise ValueError("q must be [nQH, D] and caches [nKVH, N, D]")
    nqh, D = q.shape
    nkvh, N, _ = k_cache.shape
    if k_cache.shape[2] != D or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("cache shape mismatch")
    o = torch.empty((nqh, D), dtype=q.dtype, device=q.device)
    decode(q, k_cache, v_cache, o, DecodeCfg(D, N, nqh, nkvh, 1, 0))
    return o


# ---- small-LLM runtime session ----------------------------------------------------------------

class GenerateCfg:
    """The reference's GenerateCfg (runtime/session.hpp:42-45)."""

    def __init__(self, max_new_tokens: int = 64, eos_token_id: int = -1):
        self.max_new_tokens = max_new_tokens
        self.eos_token_id = eos_token_id


class Session:
    """cdna3::runtime::Session (runtime/session.hpp:47-331) over the C ABI: loads a model
    directory in the reference's export format onto the current device and runs greedy batch-1
    generation. The session owns its own HIP stream; calls return after the device is done."""

    def __init__(self, model_dir: str, max_seq: int = 4096):
        handle = ctypes.c_void_p()
        _check(lib().cdna3_session_create(os.fsencode(model_dir), max_seq, ctypes.byref(handle)),
               "cdna3_session_create")
        self._h = handle
        self.max_seq = max_seq
        cfg = ModelCfg()
        _check(lib().cdna3_session_config(self._h, ctypes.byref(cfg)), "cdna3_session_config")
        self.cfg = cfg

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().cdna3_session_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _ids(ids):
        import numpy as np
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32).reshape(-1))
        return a, ctypes.c_void_p(a.ctypes.data)

    def generate_ex(self, input_ids, cfg: Optional[GenerateCfg] = None, with_logits: bool = False) -> dict:
        """Greedy generation. Returns {"tokens": generated ids, "logits": [steps][vocab] fp32 or
        None, "ttft_ms": device time of the prompt, "decode_ms": device time of the other steps}."""
        import numpy as np
        cfg = cfg or GenerateCfg()
        ids, ids_p = self._ids(input_ids)
        n = max(1, cfg.max_new_tokens)
        out = np.zeros(n, dtype=np.int32)
        logits = np.zeros((n, self.cfg.vocab_size), dtype=np.float32) if with_logits else None
        n_out, ttft, dec = ctypes.c_int(0), ctypes.c_float(0), ctypes.c_float(0)
        _check(lib().cdna3_session_generate(self._h, ids_p, len(ids), cfg.max_new_tokens, cfg.eos_token_id,
                                            ctypes.c_void_p(out.ctypes.data), ctypes.byref(n_out),
                                            ctypes.c_void_p(0 if logits is None else logits.ctypes.data),
                                            ctypes.byref(ttft), ctypes.byref(dec)), "cdna3_session_generate")
        k = n_out.value
        return {"tokens": out[:k].tolist(), "logits": None if logits is None else logits[:k],
                "ttft_ms": ttft.value, "decode_ms": dec.value}

    def generate(self, input_ids, cfg: Optional[GenerateCfg] = None) -> list:
        """Session::generate: the prompt followed by the generated tokens."""
        return [int(t) for t in input_ids] + self.generate_ex(input_ids, cfg)["tokens"]

    def prefill_logits(self, input_ids):
        """Session::prefill_logits: fp32 logits [vocab] of the last prompt token (numpy)."""
        import numpy as np
        ids, ids_p = self._ids(input_ids)
        out = np.zeros(self.cfg.vocab_size, dtype=np.float32)
        _check(lib().cdna3_session_prefill_logits(self._h, ids_p, len(ids), ctypes.c_void_p(out.ctypes.data)),
               "cdna3_session_prefill_logits")
        return out
