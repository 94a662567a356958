"""PyTorch-CPU restatement of the entropy-gated path (test infrastructure).

The CPU baseline bench.py times beside the GPU: the reference's own
PyTorch expressions for the quantisers and epilogues, evaluated with PyTorch
CPU ops, with the GEMMs the CPU has:
  * INT8 tier: the dispatcher quantiser (EE/python/kernels.py:336-338),
    torch._int_mm (int8 x int8 -> int32) for the kernel's K loop
    (EE/python/kernels.py:86-98) and its epilogue (:104).
  * FP8 tier: the per-row e4m3 codes (EE/python/kernels.py:361, 144, 159-160),
    the weight codes e4m3(fp16(b)) (:165-166), decoded to f32 and multiplied in
    f32 (the CPU has no fp8 GEMM), then the epilogue (:176-180).
  * softmax + entropy in f32 (EE/python/kernels.py:264-312).
Only tests/ and bench.py's cpu_baseline leg use it; the product never does.
tests/test_oracle_torch_cpu.py pins it against the C oracle (INT8 outputs and
FP8 codes bit for bit, FP8 outputs and entropies within tolerance).

Like the C oracle, the quantisers divide by a Python float the way PyTorch on
the GPU does (multiplication by the f32 reciprocal), which is what the
reference's launchers ran.
"""
import numpy as np
import torch

_INV127 = np.float32(1.0) / np.float32(127.0)
_INV448 = np.float32(1.0) / np.float32(448.0)


def quant_act_i8(a: torch.Tensor):
    """EE/python/kernels.py:336-338 on fp16 [M, K]: (int8 codes, f32 scale [M])."""
    amax = a.abs().amax(dim=1, keepdim=True).float()
    s = (amax * float(_INV127)).half().float()              # fp16 tensor / 127.0, then .to(f32)
    codes = torch.trunc(a.float() / s).to(torch.int8)       # .to(int8) truncates toward zero
    return codes, s.squeeze(1)


def gemm_i8(codes: torch.Tensor, b_kn: torch.Tensor, a_scale: torch.Tensor, b_scale: torch.Tensor):
    """EE/python/kernels.py:86-104: int32 accumulators, fp16((f32(acc) * as) * bs)."""
    acc = torch._int_mm(codes, b_kn)
    return ((acc.float() * a_scale[:, None]) * b_scale[None, :]).half()


def triton_int8_gemm(a, b_kn, b_scale):
    codes, s = quant_act_i8(a)
    return gemm_i8(codes, b_kn, s, b_scale)


def _e4m3(x16: torch.Tensor) -> torch.Tensor:
    """fp16 -> e4m3 RNE with saturation at 448 (the reference's |x| <= ~448.5)."""
    return x16.float().clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def quant_act_f8(a: torch.Tensor):
    """EE/python/kernels.py:361, 144, 159-160: (e4m3 codes, f32 scale [M])."""
    amax = a.abs().amax(dim=1, keepdim=True).float()
    s = (amax * float(_INV448)).half().float()
    inv16 = (1.0 / s).half()                                # (1.0 / a_scale).to(f16)
    p = (a.float() * inv16.float()).half()                  # fp16 x fp16 product, rounded to fp16
    return _e4m3(p), s.squeeze(1)


def weight_f8(b_kn: torch.Tensor) -> torch.Tensor:
    """EE/python/kernels.py:165-166: the FP8 tier's weight codes e4m3(fp16(b))."""
    return _e4m3(b_kn.half())


def gemm_f8(a8: torch.Tensor, b8: torch.Tensor, a_scale, b_scale):
    """EE/python/kernels.py:171-180 with the dot in f32 on decoded codes."""
    acc = a8.float() @ b8.float()
    return ((acc * a_scale[:, None]) * b_scale[None, :]).half()


def triton_fp8_gemm(a, b_kn, b_scale, b8=None):
    a8, s = quant_act_f8(a)
    return gemm_f8(a8, weight_f8(b_kn) if b8 is None else b8, s, b_scale)


def softmax_entropy(x: torch.Tensor):
    """EE/python/kernels.py:264-312 (non-causal rows) in f32: (fp16 probs, f32 H)."""
    xf = x.float()
    s = xf - xf.amax(dim=1, keepdim=True)
    e = torch.exp(s)
    z = e.sum(dim=1, keepdim=True)
    p = e / z
    h = torch.log(z.squeeze(1)) - (e * s).sum(dim=1) / z.squeeze(1)
    return p.half(), h
