"""Helpers shared by the GPU tests: move oracle-generated host arrays to the device and back."""
import ctypes
import os

import numpy as np
import torch

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEV = torch.device("cuda", 0)
KIND = {torch.float16: oracle.F16, torch.bfloat16: oracle.BF16}


def rounded(x: np.ndarray, dtype: torch.dtype):
    """(fp32 values as the GPU will see them, device tensor of `dtype`) for fp32 host data."""
    if dtype == torch.float32:
        return x.astype(np.float32), torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV)
    vals, bits = oracle.round16(x, KIND[dtype])
    t = torch.from_numpy(bits.view(np.int16)).view(dtype).to(DEV)
    return vals, t


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def max_rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max(1, |ref|) (absolute below 1, relative above)."""
    return float(np.max(np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))))


def tolerance(dtype: torch.dtype) -> float:
    """Parity bound per output dtype, in max_rel_err units (|d| / max(1, |ref|)).
    fp32: 1e-4. fp16: 2e-3. bf16: 2e-3 plus two bf16 roundings the format forces (2^-9 relative
    each): the stored output (its half-ulp alone reaches 2e-3 * |O| for |O| >= 1) and the softmax
    weights P, which enter the P.V matrix product in the input precision. With P of a query with
    two visible keys rounded by 2^-9, O moves by up to 2^-9 * p0 p1 / (p0 + p1)^2 * |v0 - v1|."""
    return {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 2e-3 + 2 * 2.0 ** -9}[dtype]


_HOOKS = None


def hooks() -> ctypes.CDLL:
    global _HOOKS
    if _HOOKS is None:
        path = os.path.join(ROOT, "tests", "native", "libwave_hooks.so")
        if not os.path.exists(path):
            raise RuntimeError("tests/native/libwave_hooks.so not built; run __graft_entry__.build()")
        l = ctypes.CDLL(path)
        vp = ctypes.c_void_p
        l.hook_wave.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, ctypes.c_int, vp]
        l.hook_ballot.argtypes = [vp, vp, ctypes.c_int, vp]
        l.hook_mfma.argtypes = [ctypes.c_int, vp, vp, vp, vp]
        l.hook_dme.argtypes = [vp] * 7
        l.hook_dme_forms.argtypes = [vp] * 6 + [ctypes.c_int, vp]
        l.hook_online_softmax.argtypes = [vp, vp, ctypes.c_int, vp, vp]
        l.hook_mma_tile.argtypes = [ctypes.c_int, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        l.hook_runtime_kernels.argtypes = [ctypes.c_int, vp, vp, vp, vp] + [ctypes.c_int] * 5 + [ctypes.c_float, vp]
        _HOOKS = l
    return _HOOKS


def ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
