"""NumPy interface of the CPU oracle (oracle/liboracle.so) and of the reference's own CPU
attention references built into oracle/_ref/.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the cpu_baseline leg
of bench.py, always as the checker or the CPU baseline, never as the thing measured or shipped.
The product library (libcdna4_attn.so) does not depend on it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = {}

F32, F16, BF16, F64, I32, I64 = 0, 1, 2, 3, 4, 5
SUM, MAX, MIN = 0, 1, 2
_NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16, F64: np.float64, I32: np.int32, I64: np.int64}

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def lib() -> ctypes.CDLL:
    """liboracle.so, built with gcc on first use if it is missing (no GPU, no ROCm needed)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            subprocess.run(["make", "-C", HERE, "oracle"], check=True, capture_output=True)
        l = ctypes.CDLL(path)
        c_int, c_size, c_u64, c_float, vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p
        l.orc_splitmix64_at.restype = c_u64
        l.orc_splitmix64_at.argtypes = [c_u64, c_u64]
        l.orc_fill_uniform_f32.argtypes = [c_u64, c_size, c_float, c_float, _f32p]
        l.orc_fill_normal_f32.argtypes = [c_u64, c_size, c_float, c_float, _f32p]
        l.orc_fill_int_i32.argtypes = [c_u64, c_size, ctypes.c_int32, ctypes.c_int32, _i32p]
        l.orc_fill_int_i64.argtypes = [c_u64, c_size, ctypes.c_int64, ctypes.c_int64, vp]
        l.orc_fill_uniform_f64.argtypes = [c_u64, c_size, ctypes.c_double, ctypes.c_double, vp]
        l.orc_round.argtypes = [c_int, _f32p, c_size, vp, vp]
        l.orc_widen.argtypes = [c_int, _u16p, c_size, _f32p]
        l.orc_prefill_f32.restype = c_int
        l.orc_prefill_f32.argtypes = [_f32p, _f32p, _f32p, _f32p] + [c_int] * 7
        l.orc_prefill_rows.restype = c_int
        l.orc_prefill_rows.argtypes = [_f32p, _f32p, _f32p] + [c_int] * 7 + [_i32p, c_size, _f32p]
        l.orc_decode_f32.restype = c_int
        l.orc_decode_f32.argtypes = [_f32p, _f32p, _f32p, _f32p] + [c_int] * 6
        l.orc_reduce.restype = c_int
        l.orc_reduce.argtypes = [c_int, c_int, vp, c_size, vp]
        l.orc_scan_inclusive.restype = c_int
        l.orc_scan_inclusive.argtypes = [c_int, c_int, vp, c_size, vp]
        l.orc_rmsnorm_f32.argtypes = [_f32p, _u16p, _f32p, c_int, c_int, c_float]
        l.orc_layernorm_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, c_int, c_int, c_float]
        l.orc_softmax_rows_f32.argtypes = [_f32p, _f32p, c_int, c_int]
        l.orc_rope_table.argtypes = [_f32p, _f32p, c_int, c_int, c_int, c_float]
        l.orc_rope_f16.argtypes = [_u16p, _f32p, _f32p, c_int, c_int, c_int]
        l.orc_scatter_kv_f16.argtypes = [_u16p, _u16p] + [c_int] * 5
        l.orc_repack_f16.argtypes = [_u16p, _u16p] + [c_int] * 4
        l.orc_rope_append_kv_f16.argtypes = [_u16p] * 6 + [_f32p, _f32p] + [c_int] * 6
        _LIB = l
    return _LIB


# ---- generators ---------------------------------------------------------------------------

def splitmix64_at(seed: int, i: int) -> int:
    return int(lib().orc_splitmix64_at(seed, i))


def uniform(seed: int, n: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform_f32(seed, n, lo, hi, out)
    return out


def uniform_f64(seed: int, n: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float64)
    lib().orc_fill_uniform_f64(seed, n, lo, hi, out.ctypes.data)
    return out


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal_f32(seed, n, mean, std, out)
    return out


def integers(seed: int, n: int, lo: int, hi: int, dtype=np.int32) -> np.ndarray:
    out = np.empty(n, dtype)
    if dtype == np.int32:
        lib().orc_fill_int_i32(seed, n, lo, hi, out)
    else:
        lib().orc_fill_int_i64(seed, n, lo, hi, out.ctypes.data)
    return out


# ---- fp16 / bf16 -----------------------------------------------------------------------------

def round16(x: np.ndarray, kind: int):
    """Round fp32 values to f16 (kind F16) or bf16 (kind BF16), RNE: (values as fp32, bits)."""
    x = np.ascontiguousarray(x, np.float32)
    vals = np.empty(x.shape, np.float32)
    bits = np.empty(x.shape, np.uint16)
    lib().orc_round(kind, x.reshape(-1), x.size, vals.ctypes.data, bits.ctypes.data)
    return vals, bits


def widen(bits: np.ndarray, kind: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_widen(kind, bits.reshape(-1), bits.size, out.reshape(-1))
    return out


# ---- attention ---------------------------------------------------------------------------------

def prefill(Q, K, V, D, seqQ, seqK, nQH, nKVH, batch, causal) -> np.ndarray:
    Q, K, V = (np.ascontiguousarray(a, np.float32).reshape(-1) for a in (Q, K, V))
    O = np.empty(batch * nQH * seqQ * D, np.float32)
    rc = lib().orc_prefill_f32(Q, K, V, O, D, seqQ, seqK, nQH, nKVH, batch, int(causal))
    if rc:
        raise ValueError("orc_prefill_f32: bad arguments")
    return O.reshape(batch, nQH, seqQ, D)


def prefill_rows(Q, K, V, D, seqQ, seqK, nQH, nKVH, batch, causal, rows) -> np.ndarray:
    Q, K, V = (np.ascontiguousarray(a, np.float32).reshape(-1) for a in (Q, K, V))
    rows = np.ascontiguousarray(rows, np.int32).reshape(-1)
    n = rows.size // 3
    out = np.empty(n * D, np.float32)
    rc = lib().orc_prefill_rows(Q, K, V, D, seqQ, seqK, nQH, nKVH, batch, int(causal), rows, n, out)
    if rc:
        raise ValueError("orc_prefill_rows: bad arguments")
    return out.reshape(n, D)


def decode(q, K, V, D, N, nQH, nKVH, batch=1, stride=0) -> np.ndarray:
    q, K, V = (np.ascontiguousarray(a, np.float32).reshape(-1) for a in (q, K, V))
    o = np.empty(batch * nQH * D, np.float32)
    rc = lib().orc_decode_f32(q, K, V, o, D, N, nQH, nKVH, batch, stride)
    if rc:
        raise ValueError("orc_decode_f32: bad arguments")
    return o.reshape(batch, nQH, D)


# ---- reduce / scan -----------------------------------------------------------------------------

def reduce(op: int, dtype: int, x: np.ndarray):
    """Float inputs (f32 / f16 bits / bf16 bits / f64) -> float (fp64 combine); ints -> int (wrap)."""
    x = np.ascontiguousarray(x, _NP[dtype])
    if dtype in (I32, I64):
        out = np.zeros(1, _NP[dtype])
    else:
        out = np.zeros(1, np.float64)
    if lib().orc_reduce(op, dtype, x.ctypes.data, x.size, out.ctypes.data):
        raise ValueError("orc_reduce: bad arguments")
    return out[0].item()


def scan_inclusive(op: int, dtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, _NP[dtype])
    out = np.empty(x.size, _NP[dtype] if dtype in (I32, I64) else np.float64)
    if lib().orc_scan_inclusive(op, dtype, x.ctypes.data, x.size, out.ctypes.data):
        raise ValueError("orc_scan_inclusive: bad arguments")
    return out


# ---- norms / RoPE -----------------------------------------------------------------------------

def rmsnorm(X: np.ndarray, W_bits: np.ndarray, eps: float) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    M, H = X.shape
    Y = np.empty_like(X)
    lib().orc_rmsnorm_f32(X.reshape(-1), np.ascontiguousarray(W_bits, np.uint16), Y.reshape(-1), M, H, eps)
    return Y


def layernorm(X: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    M, H = X.shape
    Y = np.empty_like(X)
    lib().orc_layernorm_f32(X.reshape(-1), np.ascontiguousarray(gamma, np.float32),
                            np.ascontiguousarray(beta, np.float32), Y.reshape(-1), M, H, eps)
    return Y


def softmax_rows(X: np.ndarray) -> np.ndarray:
    """Row softmax of a [M][H] fp32 array (bench_softmax.hip:59-105), exponentials and sums in
    double, rounded to fp32."""
    X = np.ascontiguousarray(X, np.float32)
    M, H = X.shape
    Y = np.empty_like(X)
    lib().orc_softmax_rows_f32(X.reshape(-1), Y.reshape(-1), M, H)
    return Y


def rope_table(pos0: int, T: int, D: int, theta: float = 10000.0):
    c = np.empty(T * D, np.float32)
    s = np.empty(T * D, np.float32)
    lib().orc_rope_table(c, s, pos0, T, D, theta)
    return c.reshape(T, D), s.reshape(T, D)


def rope(T_bits: np.ndarray, cos: np.ndarray, sin: np.ndarray, seq: int, heads: int, D: int) -> np.ndarray:
    t = np.ascontiguousarray(T_bits, np.uint16).copy()
    lib().orc_rope_f16(t.reshape(-1), np.ascontiguousarray(cos, np.float32).reshape(-1),
                       np.ascontiguousarray(sin, np.float32).reshape(-1), seq, heads, D)
    return t


def scatter_kv(src_bits: np.ndarray, cache_bits: np.ndarray, T: int, heads: int, D: int, pos0: int,
               max_seq: int) -> np.ndarray:
    """scatter_kv_kernel on fp16 bits: a copy of cache [heads][max_seq][D] with src [T][heads][D]
    written at token offset pos0."""
    out = np.ascontiguousarray(cache_bits, np.uint16).copy()
    lib().orc_scatter_kv_f16(np.ascontiguousarray(src_bits, np.uint16).reshape(-1), out.reshape(-1), T, heads, D,
                             pos0, max_seq)
    return out


def repack(src_bits: np.ndarray, seq: int, heads: int, D: int, direction: int) -> np.ndarray:
    """repack_kernel on fp16 bits: 0 token-major -> head-major, 1 the reverse."""
    out = np.empty(seq * heads * D, np.uint16)
    lib().orc_repack_f16(np.ascontiguousarray(src_bits, np.uint16).reshape(-1), out, seq, heads, D, direction)
    return out


def rope_append_kv(q_bits, k_bits, v_bits, K_cache_bits, V_cache_bits, cos, sin, T: int, nQH: int, nKVH: int,
                   D: int, pos0: int, max_seq: int):
    """The layer loop's RoPE + Q repack + K/V append: (q_out [nQH][T][D], K cache, V cache) bits."""
    q_out = np.empty(nQH * T * D, np.uint16)
    Kc = np.ascontiguousarray(K_cache_bits, np.uint16).copy().reshape(-1)
    Vc = np.ascontiguousarray(V_cache_bits, np.uint16).copy().reshape(-1)
    lib().orc_rope_append_kv_f16(np.ascontiguousarray(q_bits, np.uint16).reshape(-1),
                                 np.ascontiguousarray(k_bits, np.uint16).reshape(-1),
                                 np.ascontiguousarray(v_bits, np.uint16).reshape(-1), q_out, Kc, Vc,
                                 np.ascontiguousarray(cos, np.float32).reshape(-1),
                                 np.ascontiguousarray(sin, np.float32).reshape(-1), T, nQH, nKVH, D, pos0, max_seq)
    return q_out, Kc, Vc


# ---- the reference's own CPU references (oracle/_ref) ------------------------------------------

def ref_available(name: str) -> bool:
    """True when oracle/_ref/lib<name>.so was built here; checks the file only, loads nothing."""
    return os.path.exists(os.path.join(HERE, "_ref", f"lib{name}.so"))


def ref_lib(name: str) -> Optional[ctypes.CDLL]:
    """oracle/_ref/lib<name>.so if it was built here from /root/reference, else None."""
    if name not in _REF:
        path = os.path.join(HERE, "_ref", f"lib{name}.so")
        if not os.path.exists(path):
            _REF[name] = None
        else:
            l = ctypes.CDLL(path)
            if name == "ref_attention_api":
                l.ref_cpu_prefill.argtypes = [_f32p] * 4 + [ctypes.c_int] * 7
                l.ref_cpu_decode.argtypes = [_f32p] * 4 + [ctypes.c_int] * 4
            elif name == "ref_fa_steps":
                l.ref_attn_cpu_ref.argtypes = [_f32p] * 4 + [ctypes.c_int] * 3
            _REF[name] = l
    return _REF[name]


def ref_prefill(Q, K, V, D, seqQ, seqK, nQH, nKVH, batch, causal) -> np.ndarray:
    l = ref_lib("ref_attention_api")
    Q, K, V = (np.ascontiguousarray(a, np.float32).reshape(-1) for a in (Q, K, V))
    O = np.empty(batch * nQH * seqQ * D, np.float32)
    l.ref_cpu_prefill(Q, K, V, O, D, seqQ, seqK, nQH, nKVH, batch, int(causal))
    return O.reshape(batch, nQH, seqQ, D)


def ref_decode(q, K, V, D, N, nQH, nKVH) -> np.ndarray:
    l = ref_lib("ref_attention_api")
    q, K, V = (np.ascontiguousarray(a, np.float32).reshape(-1) for a in (q, K, V))
    o = np.empty(nQH * D, np.float32)
    l.ref_cpu_decode(q, K, V, o, D, N, nQH, nKVH)
    return o.reshape(nQH, D)


def ref_attn_cpu_ref(Q, K, V, seq_q, seq_k, d) -> np.ndarray:
    l = ref_lib("ref_fa_steps")
    Q, K, V = (np.ascontiguousarray(a, np.float32).reshape(-1) for a in (Q, K, V))
    O = np.empty(seq_q * d, np.float32)
    l.ref_attn_cpu_ref(Q, K, V, O, seq_q, seq_k, d)
    return O.reshape(seq_q, d)


# ---- small-LLM runtime (llm.c) ----------------------------------------------------------------

_PP = ctypes.POINTER(ctypes.c_void_p)


class _OrcLLM(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                            "vocab", "layernorm")] + \
               [("rope_theta", ctypes.c_float), ("eps", ctypes.c_float)] + \
               [(n, ctypes.c_void_p) for n in ("embed", "lm_head", "fnorm", "fnorm_b")] + \
               [(n, _PP) for n in ("wq", "wk", "wv", "wo", "bq", "bk", "bv", "wg", "wu", "wd", "n1", "n1b", "n2",
                                  "n2b")]


def reference_argmax(logits, threads: int = 256) -> int:
    """argmax_kernel (cdna3-prims/include/cdna3/runtime/forward.hpp:244-262), one block of
    `threads` threads (the reference launches 256; a power of two), restated step by step:
    thread t keeps the first strictly larger value of logits[t], logits[t + threads], ...
    starting from -1e30 (index 0), then a tree over the threads in which the right partner
    replaces the left only when strictly larger (strides threads/2, ..., 1)."""
    x = np.ascontiguousarray(logits, np.float32).reshape(-1)
    bv = np.full(threads, np.float32(-1e30), np.float32)
    bi = np.zeros(threads, np.int64)
    for t in range(min(threads, x.size)):
        col = x[t::threads]
        run = np.maximum.accumulate(col)
        first = int(np.argmax(col == run[-1]))          # first index of the column maximum
        if run[-1] > bv[t]:
            bv[t], bi[t] = run[-1], t + threads * first
    s = threads // 2
    while s > 0:
        for t in range(s):
            if bv[t + s] > bv[t]:
                bv[t], bi[t] = bv[t + s], bi[t + s]
        s //= 2
    return int(bi[0])


class LLM:
    """CPU forward of the runtime's decoder (llm.c: Session::run_layers with the reference's
    rounding points). `meta` and `tensors` are a model directory's meta.json dict and its fp16
    arrays by file name. Holds the KV cache; `forward` appends to it like the runtime does."""

    _KIND = {"wq": "q_proj", "wk": "k_proj", "wv": "v_proj", "wo": "o_proj", "bq": "q_bias", "bk": "k_bias",
             "bv": "v_bias", "wg": "gate_proj", "wu": "up_proj", "wd": "down_proj", "n1": "norm_attn",
             "n1b": "norm_attn_bias", "n2": "norm_mlp", "n2b": "norm_mlp_bias"}

    def __init__(self, meta: dict, tensors: dict, max_seq: int):
        L, H, nH = int(meta["n_layers"]), int(meta["hidden"]), int(meta["n_heads"])
        nKV = int(meta.get("n_kv_heads", nH))
        D = int(meta.get("head_dim", H // nH))
        layer = meta.get("norm", "rms") == "layernorm"
        eps = float(meta.get("norm_eps", 1e-5 if layer else 1e-6))
        self.meta, self.max_seq, self.vocab = meta, max_seq, int(meta["vocab_size"])
        self._keep = []

        def f32(a):
            a = np.ascontiguousarray(np.asarray(a, np.float16).astype(np.float32))
            self._keep.append(a)
            return a.ctypes.data

        m = _OrcLLM(L, H, nH, nKV, D, int(meta["ffn_dim"]), self.vocab, int(layer),
                    float(meta.get("rope_theta", 10000.0)), eps)
        m.embed, m.lm_head, m.fnorm = f32(tensors["embed_tokens"]), f32(tensors["lm_head"]), f32(tensors["final_norm"])
        m.fnorm_b = f32(tensors["final_norm_bias"]) if "final_norm_bias" in tensors else None
        for field, suffix in self._KIND.items():
            names = [f"layer_{i}_{suffix}" for i in range(L)]
            if not all(n in tensors for n in names):
                setattr(m, field, None)
                continue
            arr = (ctypes.c_void_p * L)(*[f32(tensors[n]) for n in names])
            self._keep.append(arr)
            setattr(m, field, ctypes.cast(arr, _PP))
        self._m = m
        self.Kc = np.zeros(L * nKV * max_seq * D, np.uint16)
        self.Vc = np.zeros_like(self.Kc)
        self.pos = 0
        l = lib()
        l.orc_llm_forward.restype = ctypes.c_int
        l.orc_llm_forward.argtypes = [ctypes.POINTER(_OrcLLM), _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_int, _f32p, ctypes.c_int]

    def reset(self) -> None:
        self.Kc[:] = 0
        self.Vc[:] = 0
        self.pos = 0

    def forward(self, ids, all_logits: bool = False) -> np.ndarray:
        """Runs ids at the next cache positions; logits [T][vocab] (all_logits) or [vocab], fp32
        arrays holding the fp16 values the reference stores."""
        ids = np.ascontiguousarray(np.asarray(ids, np.int32).reshape(-1))
        T = ids.size
        out = np.empty((T if all_logits else 1) * self.vocab, np.float32)
        rc = lib().orc_llm_forward(ctypes.byref(self._m), ids, T, self.pos, self.Kc.ctypes.data, self.Vc.ctypes.data,
                                   self.max_seq, out, int(all_logits))
        if rc:
            raise ValueError("orc_llm_forward: bad arguments")
        self.pos += T
        return out.reshape(T, self.vocab) if all_logits else out

    def greedy(self, ids, max_new_tokens: int) -> list:
        """Session::generate's loop on the CPU (session.hpp:262-296), greedy_from_last's argmax as
        the reference breaks ties (reference_argmax)."""
        self.reset()
        toks = [reference_argmax(self.forward(ids))]
        while len(toks) < max_new_tokens and self.pos < self.max_seq:
            toks.append(reference_argmax(self.forward([toks[-1]])))
        return toks
