"""Host-side launchers of the entropy-gated path on the gfx950 kernels.

Drop-in counterparts of EE/python/kernels.py (EE = "entropy-engine (1)/
entropy-engine" in the reference): the same function names, argument order,
dtypes and return values, running hand-written HIP kernels through the C ABI
(no Triton).  Every call launches on torch's current stream of the tensors'
device.

  triton_int8_gemm(a, b_int8, b_scale)   EE/python/kernels.py:330-351
  triton_fp8_gemm(a, b_int8, b_scale)    EE/python/kernels.py:354-373
  triton_fp16_gemm(a, b_int8, b_scale)   EE/python/kernels.py:380-409
  fused_softmax_entropy(logits, causal)  EE/python/kernels.py:416-453

b_int8 is the reference's weight buffer, int8 [K, N] (N contiguous).  The
MFMA kernels read weights K-contiguous, as [N, K]; the first call with a
given weight tensor derives the per-tier operands on the GPU (transpose, e4m3
codes, W8A16 fp16 weights -- all bit-exact functions of the int8 codes) and
caches them until that tensor is freed or modified in place.
"""
from __future__ import annotations

import weakref

import torch

from . import _lib
from ._lib import check, engine, ptr, stream_handle

__all__ = [
    "triton_int8_gemm", "triton_fp8_gemm", "triton_fp16_gemm", "fused_softmax_entropy",
    "softmax_entropy", "quantize_activations", "gemm", "route", "row_copy", "routed_linear",
    "prepare_weight", "PackedWeight", "quantize_weight_codes", "silu_mul", "add_rmsnorm", "qkv_rope",
    "interleave_gate_up",
]


def _require_cuda(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("entropy_engine kernels take GPU tensors (got a tensor on %s)" % t.device)
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _rowmajor(t: torch.Tensor, name: str) -> int:
    """Row stride of a 2-D tensor with unit column stride."""
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 and t.size(1) > 1:
        raise ValueError(f"{name} must be contiguous along its last dimension")
    return t.stride(0) if t.size(0) > 1 else max(t.stride(0), t.size(1))


# ---------------------------------------------------------------- softmax + entropy

def softmax_entropy(x: torch.Tensor, causal: bool = False, probs: bool = True,
                    thresholds: tuple[float, float] | None = None, out_probs: torch.Tensor | None = None):
    """Row softmax + Shannon entropy of fp16 rows x [R, S].

    Returns (probs fp16 [R, S] or None, entropy f32 [R], tier int32 [R] or
    None).  With `thresholds=(tau_low, tau_high)` the per-row precision tier
    is produced in the same pass.  causal: column c of row r is kept iff
    c <= r % S (the reference's [B, H, S, S] rows)."""
    dev = _require_cuda(x, out_probs)
    if x.dtype != torch.float16:
        raise TypeError("logits must be float16")
    ldx = _rowmajor(x, "logits")
    R, S = x.shape
    p = None
    if probs:
        p = out_probs if out_probs is not None else torch.empty((R, S), dtype=torch.float16, device=dev)
        if p.shape != (R, S) or p.dtype != torch.float16:
            raise ValueError("out_probs must be float16 of the logits' shape")
    ldp = _rowmajor(p, "probs") if p is not None else S
    h = torch.empty(R, dtype=torch.float32, device=dev)
    tier = torch.empty(R, dtype=torch.int32, device=dev) if thresholds is not None else None
    tl, th = thresholds if thresholds is not None else (0.0, 0.0)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_softmax_entropy(engine(), ptr(x), ptr(p), ptr(h), R, S, ldx, ldp, int(bool(causal)),
                                            ptr(tier), float(tl), float(th), stream_handle()))
    return p, h, tier


def fused_softmax_entropy(logits: torch.Tensor, causal: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """EE/python/kernels.py:416-453: logits fp16 [B, H, S, S] -> (probs fp16
    [B, H, S, S], mean row entropy per batch f32 [B])."""
    B, H, S, S2 = logits.shape
    assert S == S2
    if not logits.is_contiguous():
        logits = logits.contiguous()
    probs = torch.empty_like(logits, dtype=torch.float16)
    _, row_entropies, _ = softmax_entropy(logits.view(B * H * S, S), causal=causal, probs=True,
                                          out_probs=probs.view(B * H * S, S))
    per_batch_entropy = row_entropies.reshape(B, H, S).mean(dim=(1, 2))
    return probs, per_batch_entropy


# ---------------------------------------------------------------- quantisers

_MODES = {"dispatcher": _lib.EE_QUANT_I8_DISPATCH, "engine": _lib.EE_QUANT_I8_ENGINE, "fp8": _lib.EE_QUANT_F8_ROW}


def quantize_activations(a: torch.Tensor, mode: str = "dispatcher", idx=None, counts=None, tier: int = 0,
                         out_codes=None, out_scale=None):
    """Per-row activation codes + f32 scales.

    mode "dispatcher": int8, EE/python/kernels.py:336-338 (fp16 scale, truncation)
    mode "engine":     int8, EE/test_cubin.py:93-103 (f32 scale, round, clamp)
    mode "fp8":        e4m3 bytes (uint8), EE/python/kernels.py:361,144,159-160
    Routed form (idx, counts, tier): rows idx[off + r] of `a` are quantised
    into slot off + r of the outputs (off = rows of the lower tiers)."""
    dev = _require_cuda(a, idx, counts, out_codes, out_scale)
    if a.dtype != torch.float16:
        raise TypeError("activations must be float16")
    lda = _rowmajor(a, "a")
    M, K = a.shape
    code_dtype = torch.uint8 if mode == "fp8" else torch.int8
    codes = out_codes if out_codes is not None else torch.empty((M, K), dtype=code_dtype, device=dev)
    scale = out_scale if out_scale is not None else torch.empty(M, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_quant_act(engine(), ptr(a), M, K, lda, _MODES[mode], ptr(codes), _rowmajor(codes, "codes"),
                                      ptr(scale), ptr(idx), ptr(counts), int(tier), stream_handle()))
    return codes, scale


def quantize_tensor_fp8(x: torch.Tensor):
    """FP8 e4m3 codes with ONE scale for the whole tensor -- benchmark config 1's
    "per-tensor amax" scheme, which the reference does not have (its FP8 tier
    scales per row, EE/python/kernels.py:361):
        s = amax|x| / 448 (1 if amax is 0 or not finite); code = e4m3(f32(x) * f32(1/s)).
    x fp16 [R, K] (activations, or an nn.Linear weight [N, K]) -> (codes uint8
    [R, K], scale f32 [R] holding s in every entry, as the FP8 GEMM expects)."""
    dev = _require_cuda(x)
    if x.dtype != torch.float16:
        raise TypeError("x must be float16")
    ldx = _rowmajor(x, "x")
    R, K = x.shape
    codes = torch.empty((R, K), dtype=torch.uint8, device=dev)
    scale = torch.empty(R, dtype=torch.float32, device=dev)
    ws = torch.empty(_lib.EE_TENSOR_WS_FLOATS, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_quant_tensor_f8(engine(), ptr(x), R, K, ldx, ptr(codes), K, ptr(scale), ptr(ws),
                                            stream_handle()))
    return codes, scale


def quantize_weight_codes(weight: torch.Tensor):
    """nn.Linear weight fp16 [N, K] -> (int8 codes [N, K], f32 scale [N]),
    the per-channel quantiser of EE/python/dispatch.py:43-48 in operand order."""
    dev = _require_cuda(weight)
    w = weight.detach()
    if w.dtype != torch.float16:
        w = w.to(torch.float16)
    w = w.contiguous()
    N, K = w.shape
    codes = torch.empty((N, K), dtype=torch.int8, device=dev)
    scale = torch.empty(N, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_quant_weight_i8(engine(), ptr(w), N, K, K, ptr(codes), K, ptr(scale), stream_handle()))
    return codes, scale


def transpose_i8(src: torch.Tensor) -> torch.Tensor:
    dev = _require_cuda(src)
    if src.dtype not in (torch.int8, torch.uint8):
        raise TypeError("transpose_i8 takes int8/uint8")
    R, C = src.shape
    dst = torch.empty((C, R), dtype=src.dtype, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_transpose_i8(engine(), ptr(src), R, C, _rowmajor(src, "src"), ptr(dst), R, stream_handle()))
    return dst


# ---------------------------------------------------------------- weights

class PackedWeight:
    """The three tier operands of one int8 weight, in MFMA operand order [N, K].

    i8:  int8 codes                              (INT8 tier)
    f8:  e4m3(fp16(code))                        (FP8 tier, EE/python/kernels.py:166)
    f16: fp16(fp16(code) * fp16(scale[n]))       (W8A16 tier, EE/python/kernels.py:215,233)
    """

    def __init__(self, codes_nk: torch.Tensor, scale: torch.Tensor):
        self.i8 = codes_nk.contiguous()
        self.scale = scale.contiguous()
        self._f8 = None
        self._f16 = None

    @property
    def N(self) -> int:
        return self.i8.shape[0]

    @property
    def K(self) -> int:
        return self.i8.shape[1]

    @property
    def f8(self) -> torch.Tensor:
        if self._f8 is None:
            N, K = self.i8.shape
            out = torch.empty((N, K), dtype=torch.uint8, device=self.i8.device)
            with torch.cuda.device(self.i8.device):
                check(_lib.lib().ee_pack_b_f8(engine(), ptr(self.i8), N, K, K, ptr(out), K, stream_handle()))
            self._f8 = out
        return self._f8

    @property
    def f16(self) -> torch.Tensor:
        if self._f16 is None:
            N, K = self.i8.shape
            out = torch.empty((N, K), dtype=torch.float16, device=self.i8.device)
            with torch.cuda.device(self.i8.device):
                check(_lib.lib().ee_pack_b_f16(engine(), ptr(self.i8), ptr(self.scale), N, K, K, ptr(out), K,
                                               stream_handle()))
            self._f16 = out
        return self._f16

    def materialize(self) -> "PackedWeight":
        _ = self.f8, self.f16
        return self


_weight_cache: dict = {}


def prepare_weight(b_int8: torch.Tensor, b_scale: torch.Tensor) -> PackedWeight:
    """Tier operands of the reference's weight buffer int8 [K, N] + scale [N],
    cached per (tensor, version) and dropped when either tensor is freed."""
    _require_cuda(b_int8, b_scale)
    if b_int8.dtype != torch.int8 or b_int8.dim() != 2:
        raise TypeError("b_int8 must be a 2-D int8 tensor [K, N]")
    if b_scale.dtype != torch.float32 or b_scale.numel() != b_int8.shape[1]:
        raise TypeError("b_scale must be float32 [N]")
    key = (b_int8.data_ptr(), tuple(b_int8.shape), tuple(b_int8.stride()), b_int8._version,
           b_scale.data_ptr(), b_scale._version, b_int8.device.index)
    pw = _weight_cache.get(key)
    if pw is None:
        pw = PackedWeight(transpose_i8(b_int8), b_scale.contiguous())
        _weight_cache[key] = pw
        weakref.finalize(b_int8, _weight_cache.pop, key, None)
        weakref.finalize(b_scale, _weight_cache.pop, key, None)
    return pw


# ---------------------------------------------------------------- GEMMs

_KINDS = {"int8": _lib.EE_GEMM_I8, "fp8": _lib.EE_GEMM_F8, "fp16": _lib.EE_GEMM_F16, "w8a16": _lib.EE_GEMM_W8A16}


def gemm(kind: str, a: torch.Tensor, b_nk: torch.Tensor, a_scale=None, b_scale=None, out=None, *,
         M: int | None = None, a_idx=None, c_idx=None, counts=None, tier: int = 0, acc_out=None,
         swiglu: bool = False) -> torch.Tensor:
    """C = A @ B^T on the tier's MFMA kernel; A [M, K], B [N, K] (operand order).
    swiglu: B is a gate|up operand interleaved in blocks of 32 rows (interleave_gate_up)
    and the result is act [M, N/2] = fp16(fp16(silu(gate)) * up)."""
    dev = _require_cuda(a, b_nk, a_scale, b_scale, out, a_idx, c_idx, counts, acc_out)
    lda = _rowmajor(a, "a")
    ldb = _rowmajor(b_nk, "b")
    N, K = b_nk.shape
    if M is None:
        M = a.shape[0] if a_idx is None else a_idx.numel()
    if a.shape[1] != K:
        raise ValueError(f"K mismatch: a is {tuple(a.shape)}, b is [{N}, {K}] in operand order")
    c = out if out is not None else torch.empty((M, N // 2 if swiglu else N), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        if swiglu:
            if acc_out is not None:
                raise ValueError("acc_out is not available with swiglu")
            check(_lib.lib().ee_gemm_swiglu(engine(), _KINDS[kind], ptr(a), lda, ptr(b_nk), ldb, ptr(c),
                                            _rowmajor(c, "act"), ptr(a_scale), ptr(b_scale), M, N, K, ptr(a_idx),
                                            ptr(c_idx), ptr(counts), int(tier), stream_handle()))
        else:
            check(_lib.lib().ee_gemm(engine(), _KINDS[kind], ptr(a), lda, ptr(b_nk), ldb, ptr(c), _rowmajor(c, "c"),
                                     ptr(a_scale), ptr(b_scale), M, N, K, ptr(a_idx), ptr(c_idx), ptr(counts),
                                     int(tier), ptr(acc_out), stream_handle()))
    return c


def _check_gemm_inputs(a, b_int8, b_scale):
    if a.dim() != 2 or b_int8.dim() != 2:
        raise ValueError("a must be [M, K] and b_int8 [K, N]")
    if a.dtype != torch.float16:
        raise TypeError("a must be float16")
    if a.shape[1] != b_int8.shape[0]:
        raise ValueError(f"K mismatch: a is {tuple(a.shape)}, b is {tuple(b_int8.shape)}")


def triton_int8_gemm(a: torch.Tensor, b_int8: torch.Tensor, b_scale: torch.Tensor) -> torch.Tensor:
    """EE/python/kernels.py:330-351: per-row int8 activation quantisation
    (fp16 scale, truncation) + INT8 MFMA GEMM + dequant epilogue."""
    _check_gemm_inputs(a, b_int8, b_scale)
    pw = prepare_weight(b_int8, b_scale)
    a_int8, a_scale = quantize_activations(a, "dispatcher")
    return gemm("int8", a_int8, pw.i8, a_scale, pw.scale)


def triton_fp8_gemm(a: torch.Tensor, b_int8: torch.Tensor, b_scale: torch.Tensor) -> torch.Tensor:
    """EE/python/kernels.py:354-373: per-row e4m3 activation codes + FP8 MFMA GEMM."""
    _check_gemm_inputs(a, b_int8, b_scale)
    pw = prepare_weight(b_int8, b_scale)
    a_f8, a_scale = quantize_activations(a, "fp8")
    return gemm("fp8", a_f8, pw.f8, a_scale, pw.scale)


def triton_fp16_gemm(a: torch.Tensor, b_int8: torch.Tensor, b_scale: torch.Tensor) -> torch.Tensor:
    """EE/python/kernels.py:380-409: W8A16 GEMM (fp16 activations, int8
    weights dequantised to fp16 exactly as the reference does in SRAM)."""
    _check_gemm_inputs(a, b_int8, b_scale)
    if not a.is_contiguous():
        a = a.contiguous()
    pw = prepare_weight(b_int8, b_scale)
    return gemm("fp16", a, pw.f16)


def fp8_tensor_gemm(a: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """a fp16 [M, K] @ weight fp16 [N, K]^T with per-tensor e4m3 scaling of both
    operands (quantize_tensor_fp8) on the FP8 MFMA GEMM: fp16((acc * s_a) * s_w)."""
    ca, sa = quantize_tensor_fp8(a)
    cw, sw = quantize_tensor_fp8(weight)
    return gemm("fp8", ca, cw, sa, sw)


# ---------------------------------------------------------------- routing

def route(h: torch.Tensor, tau_low: float, tau_high: float):
    """Per-row tiers + stable partition: (tier int32 [R], idx int32 [R], counts int32 [3])."""
    dev = _require_cuda(h)
    if h.dtype != torch.float32 or h.dim() != 1 or not h.is_contiguous():
        raise TypeError("entropy must be a contiguous 1-D float32 tensor")
    R = h.numel()
    tier = torch.empty(R, dtype=torch.int32, device=dev)
    idx = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(3, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_route(engine(), ptr(h), R, float(tau_low), float(tau_high), ptr(tier), ptr(idx),
                                  ptr(counts), stream_handle()))
    return tier, idx, counts


def route_heads(h: torch.Tensor, tau_low: float, tau_high: float):
    """route() on the per-token mean over heads of h [B, heads, S] (float32): token
    b * S + s is routed on (h[b, 0, s] + ... + h[b, heads-1, s]) / heads, summed in
    head order.  Returns (tier int32 [B*S], idx int32 [B*S], counts int32 [3])."""
    dev = _require_cuda(h)
    if h.dtype != torch.float32 or h.dim() != 3 or not h.is_contiguous():
        raise TypeError("entropy must be a contiguous [B, heads, S] float32 tensor")
    B, Hh, S = h.shape
    R = B * S
    tier = torch.empty(R, dtype=torch.int32, device=dev)
    idx = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(3, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_route_heads(engine(), ptr(h), B, Hh, S, float(tau_low), float(tau_high), ptr(tier),
                                        ptr(idx), ptr(counts), stream_handle()))
    return tier, idx, counts


def row_copy(src: torch.Tensor, idx: torch.Tensor, counts=None, tier: int = 0, scatter: bool = False,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """Gather (dst[r] = src[idx[off+r]]) or scatter (dst[idx[off+r]] = src[r]) whole rows."""
    dev = _require_cuda(src, idx, counts, out)
    if src.dim() != 2:
        raise ValueError("src must be 2-D")
    rows = idx.numel()
    if out is None:
        out = torch.empty((rows, src.shape[1]) if not scatter else src.shape, dtype=src.dtype, device=dev)
    es = src.element_size()
    with torch.cuda.device(dev):
        check(_lib.lib().ee_row_copy(engine(), ptr(src), _rowmajor(src, "src") * es, ptr(out),
                                     _rowmajor(out, "out") * es, rows, src.shape[1] * es, ptr(idx), ptr(counts),
                                     int(tier), int(bool(scatter)), stream_handle()))
    return out


def routed_linear(x: torch.Tensor, pw: PackedWeight, idx: torch.Tensor, counts: torch.Tensor,
                  out: torch.Tensor | None = None, workspace=None, swiglu: bool = False,
                  quantized=None) -> torch.Tensor:
    """One tier per row: INT8 / FP8 / W8A16 GEMMs over the rows `idx`/`counts`
    assign them (from `route`), scattered back in place; no host sync.
    swiglu: pw is an interleaved gate|up weight; the result is act [M, N/2].
    quantized: (codes, scale) of x's INT8 and FP8 slots, from add_rmsnorm_route
    (the GEMM launch alone; K % 128 == 0)."""
    dev = _require_cuda(x, idx, counts, out)
    if x.dtype != torch.float16:
        raise TypeError("x must be float16")
    M, K = x.shape
    if K != pw.K:
        raise ValueError(f"K mismatch: x is {tuple(x.shape)}, weight is [{pw.N}, {pw.K}]")
    N = pw.N
    c = out if out is not None else torch.empty((M, N // 2 if swiglu else N), dtype=torch.float16, device=dev)
    if quantized is not None:
        ws_codes, ws_scale = quantized
        if ws_codes.shape != (M, K) or ws_codes.dtype != torch.uint8 or not ws_codes.is_contiguous() \
                or ws_scale.dtype != torch.float32 or ws_scale.numel() != M:
            raise ValueError("quantized must be (uint8 [M, K] contiguous, float32 [M]) from add_rmsnorm_route")
        fn = _lib.lib().ee_routed_gemm_swiglu if swiglu else _lib.lib().ee_routed_gemm
    else:
        if workspace is None:
            workspace = (torch.empty((M, K), dtype=torch.uint8, device=dev),
                         torch.empty(M, dtype=torch.float32, device=dev))
        ws_codes, ws_scale = workspace
        fn = _lib.lib().ee_routed_linear_swiglu if swiglu else _lib.lib().ee_routed_linear
    with torch.cuda.device(dev):
        check(fn(engine(), ptr(x), _rowmajor(x, "x"), M, K, N, ptr(idx), ptr(counts), ptr(pw.i8), ptr(pw.f8),
                 ptr(pw.f16), ptr(pw.scale), ptr(c), _rowmajor(c, "out"), ptr(ws_codes), ptr(ws_scale),
                 stream_handle()))
    return c


def interleave_gate_up(t: torch.Tensor) -> torch.Tensor:
    """Rows 0..F-1 (gate) and F..2F-1 (up) of t [2F, ...] interleaved in blocks of 32
    rows (the SwiGLU operand layout): rows 64k..64k+31 = gate 32k.., 64k+32.. = up 32k..."""
    dev = _require_cuda(t)
    t = t.contiguous()
    if t.shape[0] % 64:
        raise ValueError("gate|up needs 2F rows with F % 32 == 0")
    rb = t[0].numel() * t.element_size() if t.dim() > 1 else t.element_size()
    out = torch.empty_like(t)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_interleave_gate_up(engine(), ptr(t), rb, ptr(out), rb, t.shape[0] // 2, rb,
                                               stream_handle()))
    return out


# ---------------------------------------------------------------- MLP activation

def silu_mul(gu: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """act [M, F] = fp16(fp16(silu(gate)) * up) for gu fp16 [M, 2F] = [gate | up]:
    torch's fp16 F.silu(gate) * up, the activation of the Llama MLP the reference
    gates (EE/python/dispatch.py:199-203, EE/test_engine.py:35)."""
    dev = _require_cuda(gu, out)
    if gu.dtype != torch.float16:
        raise TypeError("gu must be float16")
    M, F2 = gu.shape
    if F2 % 2:
        raise ValueError("gu must hold [gate | up]: an even number of columns")
    F = F2 // 2
    act = out if out is not None else torch.empty((M, F), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_silu_mul(engine(), ptr(gu), _rowmajor(gu, "gu"), ptr(act), _rowmajor(act, "out"), M, F,
                                     stream_handle()))
    return act


# ---------------------------------------------------------------- Llama block elementwise work

def _rmsnorm_operands(x, w, y):
    D = x.shape[-1]
    x2 = x.reshape(-1, D)
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) % 8):
        x2 = x2.contiguous()
    y2 = None
    if y is not None:
        y2 = y.reshape(-1, D)
        if y2.stride(-1) != 1 or y2.data_ptr() % 16 or (y2.shape[0] > 1 and y2.stride(0) % 8):
            y2 = y2.contiguous()
    T = x2.shape[0]
    n = torch.empty((T, D), dtype=torch.float16, device=x.device)
    s = torch.empty((T, D), dtype=torch.float16, device=x.device) if y is not None else x2
    return x2, y2, s, n, w.contiguous(), T, D


def add_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, y: torch.Tensor | None = None):
    """(s, n): s = x + y (x itself when y is None), n = LlamaRMSNorm(s) with weight w,
    each op in torch's precision; rows of the last dimension D (D % 8 == 0, D <= 4096)."""
    dev = _require_cuda(x, w, y)
    x2, y2, s, n, w, T, D = _rmsnorm_operands(x, w, y)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_add_rmsnorm(engine(), ptr(x2), _rowmajor(x2, "x"), ptr(y2),
                                        _rowmajor(y2, "y") if y2 is not None else D, ptr(w),
                                        ptr(s) if y is not None else None, D, ptr(n), D, T, D, float(eps),
                                        stream_handle()))
    return s.view(x.shape), n.view(x.shape)


def add_rmsnorm_route(x: torch.Tensor, w: torch.Tensor, eps: float, y: torch.Tensor | None,
                      idx: torch.Tensor, counts: torch.Tensor, n_out: torch.Tensor | None = None):
    """(s, n, codes, scale): add_rmsnorm's s, plus the routed linear's INT8
    and FP8 operands of the rows of the partition idx/counts (from route or
    route_heads): codes uint8 [T, D] and scale f32 [T] in slot order, the bits
    routed_linear's quantiser writes from add_rmsnorm's n.  The normalised rows
    are written for the FP16 slots only (the INT8 and FP8 slots' rows reach the
    GEMM as codes): n is n_out (fp16 [T, D] contiguous), holding add_rmsnorm's
    rows at the FP16 slots' source rows and nothing elsewhere, when the caller
    passes it, and None otherwise.  Pass (codes, scale) to
    routed_linear(..., quantized=...) to skip that quantiser, with n_out as its
    input (its FP16 rows are the only ones it reads)."""
    dev = _require_cuda(x, w, y, idx, counts, n_out)
    x2, y2, s, n, w, T, D = _rmsnorm_operands(x, w, y)
    if idx.dtype != torch.int32 or counts.dtype != torch.int32 or idx.numel() != T:
        raise ValueError("idx must be int32 [T] and counts int32 [3] (from route)")
    if n_out is not None:
        if n_out.dtype != torch.float16 or tuple(n_out.shape) != (T, D) or not n_out.is_contiguous():
            raise ValueError("n_out must be a contiguous float16 [T, D] tensor")
        n = n_out
    codes = torch.empty((T, D), dtype=torch.uint8, device=dev)
    scale = torch.empty(T, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_add_rmsnorm_route(engine(), ptr(x2), _rowmajor(x2, "x"), ptr(y2),
                                              _rowmajor(y2, "y") if y2 is not None else D, ptr(w),
                                              ptr(s) if y is not None else None, D, ptr(n), D, T, D, float(eps),
                                              ptr(idx), ptr(counts), ptr(codes), D, ptr(scale), stream_handle()))
    return s.view(x.shape), (n.view(x.shape) if n_out is not None else None), codes, scale


def qkv_rope(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, B: int, S: int, Hq: int, Hkv: int, d: int,
             q_scale: float = 1.0, v_transposed: bool = False):
    """q [B, Hq, S, d], k, v [B, Hkv, S, d] from a fused projection output [B*S, (Hq+2Hkv)*d],
    rotary-embedded (x*cos + rotate_half(x)*sin per fp16 op; cos/sin [S, d]); q scaled by q_scale.
    v_transposed: the third output is attention_causal's vt [B, Hkv, d, S] instead (within each
    16-token group the order 0-3, 8-11, 4-7, 12-15; see VT_ORDER)."""
    dev = _require_cuda(qkv, cos, sin)
    ld = _rowmajor(qkv, "qkv")
    cos = cos.reshape(S, d).contiguous()
    sin = sin.reshape(S, d).contiguous()
    q = torch.empty((B, Hq, S, d), dtype=torch.float16, device=dev)
    k = torch.empty((B, Hkv, S, d), dtype=torch.float16, device=dev)
    v = torch.empty((B, Hkv, d, S) if v_transposed else (B, Hkv, S, d), dtype=torch.float16, device=dev)
    fn = _lib.lib().ee_qkv_rope_vt if v_transposed else _lib.lib().ee_qkv_rope
    with torch.cuda.device(dev):
        check(fn(engine(), ptr(qkv), ld, ptr(cos), ptr(sin), ptr(q), ptr(k), ptr(v), B, S, Hq, Hkv, d, float(q_scale),
                 stream_handle()))
    return q, k, v


# Token order of each 16-token group in attention_causal's vt layout: stored position p holds token VT_ORDER[p].
VT_ORDER = (0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15)


def attention_causal(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, out: torch.Tensor | None = None):
    """Fused causal grouped-query attention with per-row entropy (head_dim 64):
    q [B, Hq, S, 64] (already scaled), k [B, Hkv, S, 64], vt from qkv_rope(v_transposed=True).
    Returns (out [B*S, Hq*64] fp16, token-major, H [B, Hq, S] f32): softmax(q k^T) v over keys <= query,
    and each probability row's Shannon entropy."""
    dev = _require_cuda(q, k, vt, out)
    B, Hq, S, d = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, S, d) or vt.shape != (B, Hkv, d, S):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, vt {tuple(vt.shape)}")
    for t_, n in ((q, "q"), (k, "k"), (vt, "vt")):
        if t_.dtype != torch.float16 or not t_.is_contiguous():
            raise ValueError(f"{n} must be contiguous fp16")
    if out is None:
        out = torch.empty((B * S, Hq * d), dtype=torch.float16, device=dev)
    ld_out = _rowmajor(out, "out")
    h = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().ee_attention_causal(engine(), ptr(q), ptr(k), ptr(vt), ptr(out), ld_out, ptr(h), B, S, Hq,
                                             Hkv, d, stream_handle()))
    return out, h
