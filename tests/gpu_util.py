"""Helpers shared by the GPU tests: move oracle-generated host arrays to the device and back."""
import ctypes
import os

import numpy as np
import torch

import oracle
import parity_log

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


def output_quantum(ref: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Half a unit in the last place of `ref` in the output format, for bf16 outputs; 0 otherwise.
    bf16 keeps 8 significant bits, so for |ref| in [2^e, 2^(e+1)) its spacing is 2^(e-7) and the
    rounding of the stored output alone can move it by 2^(e-8) (3.9e-3 at |ref| = 1): more than
    the 2e-3 compute tolerance, whatever the kernel computes. fp16 (11 bits, 2^-11 relative) and
    fp32 outputs need no such term."""
    if dtype != torch.bfloat16:
        return np.zeros_like(ref, dtype=np.float64)
    _, e = np.frexp(np.abs(ref.astype(np.float64)))        # |ref| = m 2^e, m in [0.5, 1)
    return np.where(ref != 0, np.ldexp(1.0, e - 9), 0.0)


def parity_err(got: np.ndarray, ref: np.ndarray, dtype: torch.dtype) -> float:
    """Worst compute error: max over elements of (|got - ref| - output_quantum(ref)) / max(1, |ref|).
    `parity_err <= tolerance(dtype)` is the element-wise bound
    |got - ref| <= tolerance * max(1, |ref|) + half an output ulp of ref (bf16 only)."""
    ref = np.asarray(ref, np.float64)
    d = np.abs(np.asarray(got, np.float64) - ref)
    return float(np.max((d - output_quantum(ref, dtype)) / np.maximum(1.0, np.abs(ref))))


def tolerance(dtype: torch.dtype) -> float:
    """Parity bound per output dtype for parity_err: 1e-4 (fp32), 2e-3 (fp16 and bf16), the
    tolerances the north star states; bf16 additionally allows the output's own rounding (above)."""
    return {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 2e-3}[dtype]


DTYPE_NAME = {torch.float32: "fp32", torch.float16: "fp16", torch.bfloat16: "bf16"}


def check_parity(got, ref, dtype: torch.dtype, what: str = "") -> float:
    """Assert the element-wise bound (parity_err <= tolerance), record the worst error of the
    running test for the end-of-run table, and return it. `got` and `ref` may be sequences of
    arrays checked together (e.g. the sampled heads of one output)."""
    if isinstance(got, (list, tuple)):
        got = np.concatenate([np.asarray(g, np.float64).ravel() for g in got])
        ref = np.concatenate([np.asarray(r, np.float64).ravel() for r in ref])
    got = np.asarray(got)
    ref = np.asarray(ref, np.float64).reshape(got.shape)
    err = parity_err(got, ref, dtype)
    uni = max_rel_err(got, ref)
    parity_log.record(err, tolerance(dtype), DTYPE_NAME[dtype], uni, what)
    print(f"  parity {DTYPE_NAME[dtype]}: err {err:.2e} (uniform {uni:.2e}) bound {tolerance(dtype):.0e}"
          + (f" [{what}]" if what else ""), flush=True)
    assert err <= tolerance(dtype), f"parity {err} > {tolerance(dtype)} (uniform {uni})"
    return err


def check_abs(got, ref, bound: float, what: str = "") -> float:
    """max |got - ref| <= bound (the fp32 arm of the reference's FA2 config is held to 1e-4
    absolute), recorded like check_parity."""
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))
    parity_log.record(err, bound, "fp32a", err, what)
    print(f"  parity fp32 abs: err {err:.2e} bound {bound:.0e}" + (f" [{what}]" if what else ""), flush=True)
    assert err <= bound, f"abs error {err} > {bound}"
    return err


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
