"""entropy_engine -- the entropy-gated precision path on MI355X (gfx950).

Row softmax + Shannon entropy, tau_low/tau_high routing, and INT8 / FP8-e4m3
/ W8A16 GEMMs as hand-written CDNA4 HIP kernels, loaded from gfx950 code
objects by a C-ABI launcher (include/entropy_engine.h) and driven from
PyTorch-ROCm.  The Python API mirrors the reference's kernels.py and
dispatch.py (IqtedarU/triton-kernels-optimization, entropy-engine/python).
"""
from .dispatch import (TINYLLAMA_1B, EntropyDispatchedLinear, EntropyDispatchedLlamaBlock, EntropyGatedLlama,
                       PipelinedEntropyDispatcher, PrecisionTier, RowEntropyRouter, build_dispatched_llama,
                       quantize_weights_int8, tier_of)
from .engine import CubinEngine, EntropyMLPEngine, HsacoEngine
from .kernels import (VT_ORDER, PackedWeight, add_rmsnorm, add_rmsnorm_route, attention_causal, fp8_tensor_gemm, interleave_gate_up,
                      fused_softmax_entropy, gemm, prepare_weight,
                      qkv_rope, quantize_activations, quantize_tensor_fp8, quantize_weight_codes, route, route_heads,
                      routed_linear,
                      row_copy,
                      silu_mul, softmax_entropy, transpose_i8, triton_fp8_gemm, triton_fp16_gemm, triton_int8_gemm)

__all__ = [
    "EntropyDispatchedLinear", "PipelinedEntropyDispatcher", "PrecisionTier", "RowEntropyRouter",
    "EntropyDispatchedLlamaBlock", "EntropyGatedLlama", "TINYLLAMA_1B", "build_dispatched_llama",
    "quantize_weights_int8", "tier_of", "CubinEngine", "EntropyMLPEngine", "HsacoEngine", "PackedWeight", "fused_softmax_entropy",
    "gemm", "prepare_weight", "quantize_activations", "quantize_weight_codes", "route", "route_heads", "routed_linear", "row_copy",
    "fp8_tensor_gemm", "quantize_tensor_fp8",
    "silu_mul", "add_rmsnorm", "add_rmsnorm_route", "qkv_rope", "attention_causal", "VT_ORDER", "interleave_gate_up", "softmax_entropy",
    "transpose_i8",
    "triton_fp8_gemm", "triton_fp16_gemm", "triton_int8_gemm",
]
