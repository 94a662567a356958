"""Entropy-gated precision dispatch: the reference's dispatcher API on gfx950.

Drop-in counterparts of EE/python/dispatch.py:32-143 (EE = "entropy-engine
(1)/entropy-engine" in the reference):

  PrecisionTier                dispatch.py:32-36
  quantize_weights_int8        dispatch.py:43-48   (on the GPU, bit-exact)
  PipelinedEntropyDispatcher   dispatch.py:55-96   (same API; the tier read is
                                                    ordered after its copy)
  EntropyDispatchedLinear      dispatch.py:103-143 (+ forward_routed: one tier
                                                    per row instead of per call)

Routing rule (dispatch.py:12-15,74-79): entropy < tau_low -> INT8,
tau_low <= entropy < tau_high -> FP8, otherwise FP16; ties go up a tier.
"""
from __future__ import annotations

from enum import IntEnum
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import kernels as K


class PrecisionTier(IntEnum):
    """Precision tiers ordered by compute throughput (highest first)."""
    INT8 = 0
    FP8 = 1
    FP16 = 2


def tier_of(entropy: float, tau_low: float, tau_high: float) -> PrecisionTier:
    """The dispatcher's strict comparisons (EE/python/dispatch.py:74-79)."""
    if entropy < tau_low:
        return PrecisionTier.INT8
    if entropy < tau_high:
        return PrecisionTier.FP8
    return PrecisionTier.FP16


# ============================================================================ weights

def quantize_weights_int8(weight: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """EE/python/dispatch.py:43-48: nn.Linear weight [N, K] -> (int8 [K, N], f32 scale [N]).

    scale[n] = max(amax_k |w| / 127, 1e-8); code = clamp(round(w / scale), -127, 127).
    Runs on the current GPU (a CPU weight is copied there first)."""
    w = weight.detach()
    if not w.is_cuda:
        w = w.to(torch.device("cuda", torch.cuda.current_device()))
    codes_nk, scale = K.quantize_weight_codes(w)
    return K.transpose_i8(codes_nk), scale


# ============================================================================ dispatcher

class PipelinedEntropyDispatcher:
    """Scalar per-call routing of EE/python/dispatch.py:55-96.

    submit_entropy: max over the batch -> pinned host buffer, non-blocking,
    with an event recorded after the copy.  get_tier: waits on that event
    before reading, so the tier always reflects the last submission (the
    reference read the pinned value without any ordering, dispatch.py:72).
    Without a GPU the buffer is ordinary host memory (CPU tensors only)."""

    def __init__(self, tau_low: float = 2.0, tau_high: float = 3.5):
        self.tau_low = tau_low
        self.tau_high = tau_high
        self._pinned = torch.empty(1, dtype=torch.float32, pin_memory=torch.cuda.is_available())
        self._event = None
        self._has_value = False
        self.tier_counts = {PrecisionTier.INT8: 0, PrecisionTier.FP8: 0, PrecisionTier.FP16: 0}

    def submit_entropy(self, entropy_batch: torch.Tensor):
        max_entropy = entropy_batch.max()
        if max_entropy.is_cuda:
            self._pinned.copy_(max_entropy.unsqueeze(0).to(torch.float32), non_blocking=True)
            self._event = torch.cuda.Event()
            self._event.record(torch.cuda.current_stream(max_entropy.device))
        else:
            self._pinned.copy_(max_entropy.unsqueeze(0).to(torch.float32))
            self._event = None
        self._has_value = True

    def get_tier(self) -> PrecisionTier:
        if not self._has_value:
            return PrecisionTier.FP16
        if self._event is not None:
            self._event.synchronize()
        val = self._pinned[0].item()
        tier = tier_of(val, self.tau_low, self.tau_high)
        self.tier_counts[tier] += 1
        return tier

    def reset_stats(self):
        self._has_value = False
        self.tier_counts = {t: 0 for t in PrecisionTier}

    def get_stats(self) -> dict:
        total = sum(self.tier_counts.values())
        return {
            tier.name: {
                'count': self.tier_counts[tier],
                'pct': self.tier_counts[tier] / max(total, 1) * 100,
            }
            for tier in PrecisionTier
        }


class RowEntropyRouter:
    """Per-row routing on the device: entropy f32 [R] -> (tier, idx, counts).

    No reference counterpart: the reference routes a whole call by one scalar.
    Counts accumulate on the device; get_stats() syncs once to report them in
    the dispatcher's {name: {count, pct}} schema (counted in rows)."""

    def __init__(self, tau_low: float, tau_high: float):
        self.tau_low = tau_low
        self.tau_high = tau_high
        self._totals = None

    def route(self, entropy: torch.Tensor):
        tier, idx, counts = K.route(entropy.contiguous().to(torch.float32), self.tau_low, self.tau_high)
        c64 = counts.to(torch.int64)
        self._totals = c64 if self._totals is None else self._totals + c64
        return tier, idx, counts

    def reset_stats(self):
        self._totals = None

    def get_stats(self) -> dict:
        tot = [0, 0, 0] if self._totals is None else [int(v) for v in self._totals.tolist()]
        n = max(sum(tot), 1)
        return {t.name: {'count': tot[t], 'pct': tot[t] / n * 100} for t in PrecisionTier}


# ============================================================================ linear

class EntropyDispatchedLinear(nn.Module):
    """EE/python/dispatch.py:103-143 on the gfx950 GEMMs.

    Buffers: weight_int8 [K, N] and weight_scale [N] exactly as the
    reference (state dicts carry them), plus the tier operands in MFMA
    order: weight_i8_nk / weight_f8_nk (e4m3 bytes) / weight_f16_nk."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer('weight_int8', None)
        self.register_buffer('weight_scale', None)
        self.register_buffer('weight_i8_nk', None)
        self.register_buffer('weight_f8_nk', None)
        self.register_buffer('weight_f16_nk', None)
        if bias:
            self.register_buffer('bias', None)
        else:
            self.bias = None
        self._ws = None

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> 'EntropyDispatchedLinear':
        has_bias = linear.bias is not None
        layer = cls(linear.in_features, linear.out_features, bias=has_bias)
        w = linear.weight.detach()
        if not w.is_cuda:
            w = w.to(torch.device("cuda", torch.cuda.current_device()))
        codes_nk, scale = K.quantize_weight_codes(w)
        pw = K.PackedWeight(codes_nk, scale).materialize()
        layer.weight_int8 = K.transpose_i8(codes_nk)
        layer.weight_scale = scale
        layer.weight_i8_nk = pw.i8
        layer.weight_f8_nk = pw.f8
        layer.weight_f16_nk = pw.f16
        if has_bias:
            layer.bias = linear.bias.detach().to(device=w.device, dtype=torch.float16)
        return layer

    def _packed(self) -> K.PackedWeight:
        pw = K.PackedWeight(self.weight_i8_nk, self.weight_scale)
        pw._f8, pw._f16 = self.weight_f8_nk, self.weight_f16_nk
        return pw

    def forward(self, x: torch.Tensor, tier: PrecisionTier = PrecisionTier.FP16) -> torch.Tensor:
        orig_shape = x.shape
        x_2d = x.reshape(-1, self.in_features).contiguous().to(torch.float16)
        pw = self._packed()
        if tier == PrecisionTier.INT8:
            a, s = K.quantize_activations(x_2d, "dispatcher")
            out = K.gemm("int8", a, pw.i8, s, pw.scale)
        elif tier == PrecisionTier.FP8:
            a, s = K.quantize_activations(x_2d, "fp8")
            out = K.gemm("fp8", a, pw.f8, s, pw.scale)
        else:
            out = K.gemm("fp16", x_2d, pw.f16)
        if self.bias is not None:
            out = out + self.bias.unsqueeze(0)
        return out.reshape(orig_shape[:-1] + (self.out_features,))

    def forward_routed(self, x: torch.Tensor, idx: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
        """One tier per row: idx/counts from RowEntropyRouter.route over the
        rows of x.reshape(-1, in_features)."""
        orig_shape = x.shape
        x_2d = x.reshape(-1, self.in_features).contiguous().to(torch.float16)
        M = x_2d.shape[0]
        if self._ws is None or self._ws[0].shape[0] < M or self._ws[0].device != x_2d.device:
            self._ws = (torch.empty((M, self.in_features), dtype=torch.uint8, device=x_2d.device),
                        torch.empty(M, dtype=torch.float32, device=x_2d.device))
        ws = (self._ws[0][:M], self._ws[1][:M])
        out = K.routed_linear(x_2d, self._packed(), idx, counts, workspace=ws)
        if self.bias is not None:
            out = out + self.bias.unsqueeze(0)
        return out.reshape(orig_shape[:-1] + (self.out_features,))

    def extra_repr(self):
        return f'in={self.in_features}, out={self.out_features}, bias={self.bias is not None}'
