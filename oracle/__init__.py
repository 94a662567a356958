"""CPU oracle for the entropy-gated precision path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm on the CPU (C in ee_oracle.c,
loaded through ctypes; numpy for array plumbing).  It exists to check the HIP
kernels: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it.  The product package never imports it and
has no CPU fallback.

Reference citations use EE = "entropy-engine (1)/entropy-engine" and
NB = Triton_Entropy_Based_Precision.ipynb (raw JSON line numbers).

Pinning (each function's independent checks live in tests/test_oracle_*.py):
  f32_to_f16 ........ exhaustive vs numpy's float16 cast (all 2^32 is too many:
                      every fp16 rounding boundary +-1 ulp of binary32)
  e4m3_from_f32 ..... all 65,536 fp16 inputs vs torch's float8_e4m3fn cast
                      below 464, closed-form saturation above
  quant_act_* ....... per-element closed forms with exact rationals
  gemm_i8_acc ....... torch._int_mm and brute-force Python integers
  epilogue_i8 ....... element-wise numpy float32 restatement
  gemm_*_f64 ........ numpy float64 matmul of the decoded codes
  softmax_entropy ... closed forms (uniform: ln S; one-hot: 0; two-point:
                      ln 2), shift invariance, numpy float64 recompute
  route ............. the reference's own tier answers (EE/python/
                      benchmark.py:185-210) and sweep table (NB:555-561)
  silu_mul .......... numpy restatement of the f32 evaluation with numpy's
                      casts, torch's CPU and GPU fp16 F.silu, closed forms
                      (silu(0) = 0, silu(x) - silu(-x) = x, large |x|)
  mlp_forward ....... composition of the pinned functions above, checked
                      against an independent numpy float64 MLP
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libee_oracle.so")
_lib = None

_i64 = ctypes.c_int64
_p = ctypes.c_void_p


def build(force: bool = False) -> str:
    """Compile ee_oracle.c into oracle/_build/libee_oracle.so with make."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", _HERE],
                       check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sigs = {
            "eo_f16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
            "eo_f32_to_f16": ([ctypes.c_float], ctypes.c_uint16),
            "eo_e4m3_from_f32": ([ctypes.c_float], ctypes.c_uint8),
            "eo_e4m3_to_f32": ([ctypes.c_uint8], ctypes.c_float),
            "eo_i8_trunc": ([ctypes.c_float], ctypes.c_int8),
            "eo_quant_act_i8_dispatch": ([_p, _i64, _i64, _i64, _p, _i64, _p], None),
            "eo_quant_act_i8_engine": ([_p, _i64, _i64, _i64, _p, _i64, _p], None),
            "eo_quant_act_f8": ([_p, _i64, _i64, _i64, _p, _i64, _p], None),
            "eo_quant_tensor_f8": ([_p, _i64, _i64, _i64, _p, _i64, _p], None),
            "eo_quant_weight_i8": ([_p, _i64, _i64, _i64, _p, _i64, _p], None),
            "eo_gemm_i8_acc": ([_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64], None),
            "eo_epilogue_i8": ([_p, _i64, _p, _p, _p, _i64, _i64, _i64], None),
            "eo_gemm_f8_f64": ([_p, _i64, _p, _i64, _p, _p, _p, _i64, _i64, _i64], None),
            "eo_dequant_w8a16": ([_p, _i64, _p, _p, _i64, _i64, _i64], None),
            "eo_gemm_w8a16_f64": ([_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64], None),
            "eo_softmax_entropy": ([_p, _i64, _i64, _i64, ctypes.c_int, _p, _p, _p], None),
            "eo_route": ([_p, _i64, ctypes.c_double, ctypes.c_double, _p, _p, _p], None),
            "eo_f32_to_f16_n": ([_p, _p, _i64], None),
            "eo_f16_to_f32_n": ([_p, _p, _i64], None),
            "eo_e4m3_from_f32_n": ([_p, _p, _i64], None),
            "eo_e4m3_to_f32_n": ([_p, _p, _i64], None),
            "eo_i8_trunc_n": ([_p, _p, _i64], None),
            "eo_f64_to_f16": ([ctypes.c_double], ctypes.c_uint16),
            "eo_f64_to_f16_n": ([_p, _p, _i64], None),
            "eo_silu_mul": ([_p, _i64, _p, _i64, _i64, _i64, _p], None),
            "eo_num_threads": ([], ctypes.c_int),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def num_threads() -> int:
    """OpenMP threads the oracle's parallel loops use."""
    return int(lib().eo_num_threads())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# scalar formats (array forms)
# --------------------------------------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    """binary32 -> binary16 RNE (bit level)."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().eo_f32_to_f16_n(_ptr(x), _ptr(y), x.size)
    return y.view(np.float16)


def f16_to_f32(x) -> np.ndarray:
    x = _c(np.asarray(x, np.float16).view(np.uint16), np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().eo_f16_to_f32_n(_ptr(x), _ptr(y), x.size)
    return y


def e4m3_from_f32(x) -> np.ndarray:
    """binary32 -> e4m3fn code, RNE, saturating to +-448 (EE/python/kernels.py:160,166)."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().eo_e4m3_from_f32_n(_ptr(x), _ptr(y), x.size)
    return y


def e4m3_to_f32(c) -> np.ndarray:
    c = _c(c, np.uint8)
    y = np.empty(c.shape, np.float32)
    lib().eo_e4m3_to_f32_n(_ptr(c), _ptr(y), c.size)
    return y


def i8_trunc(q) -> np.ndarray:
    q = _c(q, np.float32)
    y = np.empty(q.shape, np.int8)
    lib().eo_i8_trunc_n(_ptr(q), _ptr(y), q.size)
    return y


def e4m3_of_int8() -> np.ndarray:
    """Weight codes e4m3(fp16(b)) for every int8 b, indexed by b & 0xff."""
    b = np.arange(256, dtype=np.uint8).view(np.int8).astype(np.float32)
    return e4m3_from_f32(b)


# --------------------------------------------------------------------------
# quantisers
# --------------------------------------------------------------------------

def _f16_2d(a):
    a = np.asarray(a)
    assert a.dtype == np.float16 and a.ndim == 2, (a.dtype, a.shape)
    return np.ascontiguousarray(a).view(np.uint16)


def quant_act_i8(a, mode: str = "dispatcher"):
    """INT8 activation codes + per-row f32 scale.

    mode="dispatcher": EE/python/kernels.py:336-338 (fp16 scale, truncation).
    mode="engine":     EE/test_cubin.py:93-103 (f32 scale, round + clamp).
    """
    a16 = _f16_2d(a)
    M, K = a16.shape
    codes = np.empty((M, K), np.int8)
    scale = np.empty(M, np.float32)
    fn = {"dispatcher": lib().eo_quant_act_i8_dispatch, "engine": lib().eo_quant_act_i8_engine}[mode]
    fn(_ptr(a16), M, K, K, _ptr(codes), K, _ptr(scale))
    return codes, scale


def quant_act_f8(a):
    """FP8 tier activation codes (e4m3 as uint8) + per-row f32 scale,
    EE/python/kernels.py:361,144,159-160."""
    a16 = _f16_2d(a)
    M, K = a16.shape
    codes = np.empty((M, K), np.uint8)
    scale = np.empty(M, np.float32)
    lib().eo_quant_act_f8(_ptr(a16), M, K, K, _ptr(codes), K, _ptr(scale))
    return codes, scale


def quant_tensor_f8(a):
    """Per-tensor FP8 e4m3 codes (uint8) + f32 scale per row (all equal): the
    build's definition of benchmark config 1's scheme (no reference counterpart)."""
    a16 = _f16_2d(a)
    M, K = a16.shape
    codes = np.empty((M, K), np.uint8)
    scale = np.empty(M, np.float32)
    lib().eo_quant_tensor_f8(_ptr(a16), M, K, K, _ptr(codes), K, _ptr(scale))
    return codes, scale


def quantize_weights_int8(W):
    """EE/python/dispatch.py:43-48: W fp16 [N,K] -> (B int8 [K,N], scale f32 [N])."""
    w16 = _f16_2d(W)
    N, K = w16.shape
    B = np.empty((K, N), np.int8)
    scale = np.empty(N, np.float32)
    lib().eo_quant_weight_i8(_ptr(w16), N, K, K, _ptr(B), N, _ptr(scale))
    return B, scale


# --------------------------------------------------------------------------
# GEMMs
# --------------------------------------------------------------------------

def gemm_i8_acc(A, B) -> np.ndarray:
    """Exact int32 accumulators of int8 A [M,K] x int8 B [K,N]."""
    A = _c(A, np.int8)
    B = _c(B, np.int8)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    acc = np.empty((M, N), np.int32)
    lib().eo_gemm_i8_acc(_ptr(A), K, _ptr(B), N, _ptr(acc), N, M, N, K)
    return acc


def epilogue_i8(acc, a_scale, b_scale) -> np.ndarray:
    """EE/python/kernels.py:104-110: fp16((f32(acc) * a_s) * b_s)."""
    acc = _c(acc, np.int32)
    a_s = _c(a_scale, np.float32)
    b_s = _c(b_scale, np.float32)
    M, N = acc.shape
    C = np.empty((M, N), np.uint16)
    lib().eo_epilogue_i8(_ptr(acc), N, _ptr(a_s), _ptr(b_s), _ptr(C), N, M, N)
    return C.view(np.float16)


def gemm_i8(A, B, a_scale, b_scale) -> np.ndarray:
    return epilogue_i8(gemm_i8_acc(A, B), a_scale, b_scale)


def gemm_f8_f64(A8, B, a_scale, b_scale) -> np.ndarray:
    """FP8 tier in float64 from activation codes A8 [M,K] and int8 weights B [K,N]."""
    A8 = _c(A8, np.uint8)
    B = _c(B, np.int8)
    M, K = A8.shape
    _, N = B.shape
    C = np.empty((M, N), np.float64)
    lib().eo_gemm_f8_f64(_ptr(A8), K, _ptr(B), N, _ptr(_c(a_scale, np.float32)),
                         _ptr(_c(b_scale, np.float32)), _ptr(C), M, N, K)
    return C


def dequant_w8a16(B, b_scale) -> np.ndarray:
    """EE/python/kernels.py:215,233: fp16(fp16(b) * fp16(b_scale)) -> fp16 [K,N]."""
    B = _c(B, np.int8)
    K, N = B.shape
    W = np.empty((K, N), np.uint16)
    lib().eo_dequant_w8a16(_ptr(B), N, _ptr(_c(b_scale, np.float32)), _ptr(W), N, K, N)
    return W.view(np.float16)


def gemm_w8a16_f64(A, B, b_scale) -> np.ndarray:
    a16 = _f16_2d(A)
    B = _c(B, np.int8)
    M, K = a16.shape
    _, N = B.shape
    C = np.empty((M, N), np.float64)
    lib().eo_gemm_w8a16_f64(_ptr(a16), K, _ptr(B), N, _ptr(_c(b_scale, np.float32)), _ptr(C), M, N, K)
    return C


# --------------------------------------------------------------------------
# softmax + entropy, routing
# --------------------------------------------------------------------------

def softmax_entropy(X, causal: bool = False, probs: bool = True):
    """Per-row (H float64 [R], P16 fp16 [R,S] or None); EE/python/kernels.py:264-312."""
    x16 = _f16_2d(X)
    R, S = x16.shape
    H = np.empty(R, np.float64)
    P16 = np.empty((R, S), np.uint16) if probs else None
    lib().eo_softmax_entropy(_ptr(x16), R, S, S, int(bool(causal)), _ptr(H), None,
                             _ptr(P16) if probs else None)
    return H, (P16.view(np.float16) if probs else None)


def softmax_entropy_probs_f64(X, causal: bool = False) -> np.ndarray:
    x16 = _f16_2d(X)
    R, S = x16.shape
    H = np.empty(R, np.float64)
    P = np.empty((R, S), np.float64)
    lib().eo_softmax_entropy(_ptr(x16), R, S, S, int(bool(causal)), _ptr(H), _ptr(P), None)
    return P


def fused_softmax_entropy(logits, causal: bool = True):
    """EE/python/kernels.py:416-453: logits fp16 [B,H,S,S] -> (probs fp16, mean H per batch)."""
    logits = np.asarray(logits)
    B, Hh, S, S2 = logits.shape
    assert S == S2
    Hrow, P = softmax_entropy(logits.reshape(B * Hh * S, S), causal=causal)
    return P.reshape(B, Hh, S, S), Hrow.reshape(B, Hh, S).mean(axis=(1, 2))


def route(H, tau_low: float, tau_high: float):
    """(tier int32 [R], idx int32 [R] stable partition, counts int32 [3])."""
    H = _c(H, np.float32)
    R = H.size
    tier = np.empty(R, np.int32)
    idx = np.empty(R, np.int32)
    counts = np.empty(3, np.int32)
    lib().eo_route(_ptr(H), R, float(tau_low), float(tau_high), _ptr(tier), _ptr(idx), _ptr(counts))
    return tier, idx, counts


# --------------------------------------------------------------------------
# the reference launchers end to end
# --------------------------------------------------------------------------

def triton_int8_gemm(a, b_int8, b_scale) -> np.ndarray:
    """EE/python/kernels.py:330-351 end to end; fp16 [M,N], bit-exact."""
    codes, a_scale = quant_act_i8(a, "dispatcher")
    return gemm_i8(codes, b_int8, a_scale, b_scale)


def triton_fp8_gemm_f64(a, b_int8, b_scale) -> np.ndarray:
    """EE/python/kernels.py:354-373 end to end, float64 before the fp16 store."""
    codes, a_scale = quant_act_f8(a)
    return gemm_f8_f64(codes, b_int8, a_scale, b_scale)


def triton_fp16_gemm_f64(a, b_int8, b_scale) -> np.ndarray:
    """EE/python/kernels.py:380-409 end to end, float64 before the fp16 store."""
    return gemm_w8a16_f64(a, b_int8, b_scale)


# --------------------------------------------------------------------------
# the Llama MLP (EntropyMLPEngine, EE/test_engine.py:17-39)
# --------------------------------------------------------------------------

def f64_to_f16(x) -> np.ndarray:
    """binary64 -> binary16, correctly rounded."""
    x = _c(x, np.float64)
    y = np.empty(x.shape, np.uint16)
    lib().eo_f64_to_f16_n(_ptr(x), _ptr(y), x.size)
    return y.view(np.float16)


def silu_mul(gu, F: int | None = None, with_silu: bool = False):
    """act fp16 [M, F] = fp16(fp16(silu(gate)) * up) from gu fp16 [M, 2F] (gate | up), silu
    evaluated in f32 as torch does; with_silu also returns that f32 silu [M, F]."""
    gu16 = _f16_2d(gu)
    M, F2 = gu16.shape
    F = F2 // 2 if F is None else F
    act = np.empty((M, F), np.uint16)
    s = np.empty((M, F), np.float32) if with_silu else None
    lib().eo_silu_mul(_ptr(gu16), F2, _ptr(act), F, M, F, _ptr(s) if with_silu else None)
    return (act.view(np.float16), s) if with_silu else act.view(np.float16)


def mlp_weights(gate_w, up_w, down_w):
    """Per-channel int8 quantisation of the three projections (EE/python/dispatch.py:43-48):
    ((B_gu int8 [H, 2F], s_gu [2F]), (B_dn int8 [F, H], s_dn [H])); gate columns, then up."""
    Bg, sg = quantize_weights_int8(gate_w)
    Bu, su = quantize_weights_int8(up_w)
    Bd, sd = quantize_weights_int8(down_w)
    return (np.concatenate([Bg, Bu], axis=1), np.concatenate([sg, su])), (Bd, sd)


def mlp_linear(x, B, s, tier: int):
    """One dispatched linear of the tier: INT8 fp16 bit-exact; FP8 / FP16 float64 before the store."""
    if tier == 0:
        return triton_int8_gemm(x, B, s)
    if tier == 1:
        return triton_fp8_gemm_f64(x, B, s)
    return triton_fp16_gemm_f64(x, B, s)


def mlp_forward(x, gate_w, up_w, down_w, tier: int, act=None):
    """The MLP under one tier: (gu, act, out).  gu and out are fp16 for INT8, float64 (pre-store)
    otherwise; FP8 / FP16 intermediates are rounded to fp16 before the next op, as the GPU stores
    them.  `act` (fp16 [M, F]) replaces the computed activation for the down projection, to check
    the down GEMM on exactly the operand the device used."""
    (Bgu, sgu), (Bdn, sdn) = mlp_weights(gate_w, up_w, down_w)
    gu = mlp_linear(x, Bgu, sgu, tier)
    gu16 = f64_to_f16(gu) if tier != 0 else gu
    a = silu_mul(gu16) if act is None else np.asarray(act, np.float16)
    return gu, a, mlp_linear(a, Bdn, sdn, tier)
