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

    def _scale_f32(self) -> torch.Tensor:
        """The per-channel scale as f32 for the kernels.  Module.half() casts the
        buffer to fp16 (as it does the reference's, whose Triton kernels then
        read fp16 scales, kernels.py:103-104); the f32 copy of those values is
        exact, so both see the same numbers."""
        s = self.weight_scale
        if s.dtype == torch.float32:
            return s
        key = (s.data_ptr(), s._version, s.dtype)
        if getattr(self, "_scale_key", None) != key:
            self._scale_cache = s.float().contiguous()
            self._scale_key = key
        return self._scale_cache

    def _packed(self) -> K.PackedWeight:
        pw = K.PackedWeight(self.weight_i8_nk, self._scale_f32())
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


# ============================================================================ Llama

def _rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotary embedding in the Llama convention: x*cos + rotate_half(x)*sin,
    cos/sin [B or 1, S, head_dim] broadcast over heads."""
    h = x.shape[-1] // 2
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return x * cos.unsqueeze(1) + rot * sin.unsqueeze(1)


def _attention_entropy(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scaling: float,
                       attention_mask: Optional[torch.Tensor] = None, causal: bool = False):
    """softmax(q k^T * scaling [+ mask]) v, the probabilities and their per-row
    Shannon entropy from the fused softmax+entropy kernel (one pass over the
    scores).  q [B, Hq, S, d], k/v [B, Hkv, Sk, d] fp16.  Grouped-query heads
    (Hq = G * Hkv, query head h reading kv head h // G) need no copies of k and
    v: the G query heads of a kv head are consecutive, so q viewed as
    [B, Hkv, G * S, d] multiplies k and v of [B, Hkv, Sk, d] directly.
    Returns (out [B, Hq, S, d] fp16, H [B, Hq, S] f32).  scaling == 1 skips the
    multiply (for q already scaled).  causal: key c of query s is kept iff
    c <= s (needs Sk == S)."""
    B, Hq, S, d = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    qg = q.contiguous().view(B, Hkv, G * S, d)
    scores = torch.matmul(qg, k.transpose(-1, -2).contiguous())          # [B, Hkv, G*S, Sk]
    if scaling != 1.0:
        scores = scores * scaling
    if attention_mask is not None:
        scores = scores.view(B, Hq, S, Sk) + attention_mask[..., :Sk].to(scores.dtype)
    probs, H, _ = K.softmax_entropy(scores.reshape(-1, Sk), causal=causal and attention_mask is None)
    out = torch.matmul(probs.view(B, Hkv, G * S, Sk), v.contiguous())   # [B, Hkv, G*S, d]
    return out.view(B, Hq, S, d), H.view(B, Hq, S)


class EntropyDispatchedLlamaBlock(nn.Module):
    """EE/python/dispatch.py:150-247 on the gfx950 path.

    Wraps an HF Llama decoder layer: the MLP projections become
    EntropyDispatchedLinear (one tier per call, from the dispatcher), and the
    attention probabilities come from the fused softmax+entropy kernel, which
    yields each probability row's Shannon entropy in the same pass.
    layer_entropy is the mean row entropy per batch element [B] (f32): the
    quantity the reference computes as -sum p ln(p + 1e-10) over HF's attention
    weights (dispatch.py:243-245); the kernel's exact H = ln Z - sum p*s differs
    from it only by the 1e-10 regulariser and the fp16 rounding of p.
    attention_mask follows HF attention: an additive [B, 1, S, Sk] mask; None
    means unmasked attention under eager attention (the reference's own test,
    benchmark.py:220-277) and causal attention (key c of query s kept iff
    c <= Sk - S + s) under the fused implementations, for which HF's LlamaModel
    passes None instead of a causal mask.

    KV cache (EE/python/dispatch.py:166-209, 214-247): keys and values are
    appended to an HF Cache after RoPE (cache.update(k, v, layer_idx)) and the
    attention runs over every cached key.  Two calling conventions: the
    reference's -- past_key_value=..., use_cache=..., returning (hidden,) or,
    with use_cache, (hidden, present_kv), present_kv being the updated cache or,
    without one, the (k, v) of this call -- and HF's LlamaModel's (transformers
    >= 5: past_key_values=..., returning the hidden tensor), so the block can
    replace an HF decoder layer inside a stock forward or generate()."""

    def __init__(self, llama_block, layer_idx: int = 0):
        super().__init__()
        self.layer_idx = layer_idx
        self.self_attn = llama_block.self_attn
        self.input_layernorm = llama_block.input_layernorm
        self.post_attention_layernorm = llama_block.post_attention_layernorm
        self.gate_proj = EntropyDispatchedLinear.from_linear(llama_block.mlp.gate_proj)
        self.up_proj = EntropyDispatchedLinear.from_linear(llama_block.mlp.up_proj)
        self.down_proj = EntropyDispatchedLinear.from_linear(llama_block.mlp.down_proj)
        self.act_fn = nn.SiLU()
        self.layer_entropy: Optional[torch.Tensor] = None
        self._rotary = None

    def forward(self, hidden_states: torch.Tensor, dispatcher: Optional[PipelinedEntropyDispatcher] = None,
                attention_mask: Optional[torch.Tensor] = None, position_ids: Optional[torch.Tensor] = None,
                past_key_value=None, use_cache: bool = False, **kwargs) -> Tuple[torch.Tensor, ...]:
        hf_call = "past_key_values" in kwargs               # HF LlamaModel (transformers >= 5) convention
        cache = kwargs.pop("past_key_values", None) if hf_call else past_key_value
        residual = hidden_states
        hidden_states = self.input_layernorm(hidden_states)
        attn_output, entropy_batch, present_kv = self._attention_with_fused_entropy(
            hidden_states, attention_mask=attention_mask, position_ids=position_ids, cache=cache, **kwargs)
        self.layer_entropy = entropy_batch
        if dispatcher is not None:
            dispatcher.submit_entropy(entropy_batch)
        hidden_states = residual + attn_output
        residual = hidden_states
        hidden_states = self.post_attention_layernorm(hidden_states)
        tier = dispatcher.get_tier() if dispatcher is not None else PrecisionTier.FP16
        gate = self.gate_proj(hidden_states, tier=tier)
        up = self.up_proj(hidden_states, tier=tier)
        hidden_states = self.down_proj(self.act_fn(gate) * up, tier=tier)
        hidden_states = residual + hidden_states
        if hf_call:
            return hidden_states
        outputs = (hidden_states,)
        if use_cache:
            outputs += (present_kv,)
        return outputs

    def _attention_with_fused_entropy(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None,
                                      cache=None, **kwargs):
        attn = self.self_attn
        B, S, _ = hidden_states.shape
        hd = attn.head_dim
        q = attn.q_proj(hidden_states).view(B, S, -1, hd).transpose(1, 2)
        k = attn.k_proj(hidden_states).view(B, S, -1, hd).transpose(1, 2)
        v = attn.v_proj(hidden_states).view(B, S, -1, hd).transpose(1, 2)
        pe = kwargs.get("position_embeddings")
        if pe is None:                      # isolated block: build the rotary tables from its config
            if self._rotary is None:
                from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
                self._rotary = LlamaRotaryEmbedding(config=attn.config, device=hidden_states.device)
            if position_ids is None:                        # after the cached positions, if any
                past = cache.get_seq_length(self.layer_idx) if cache is not None else 0
                position_ids = torch.arange(past, past + S, device=hidden_states.device).unsqueeze(0).expand(B, -1)
            pe = self._rotary(hidden_states, position_ids)
        cos, sin = pe
        q, k = _rope(q, cos, sin), _rope(k, cos, sin)
        if cache is not None:                               # append, then attend over every cached key
            k, v = cache.update(k, v, self.layer_idx)
        present = cache if cache is not None else (k, v)
        Sk = k.shape[2]
        causal = False
        if attention_mask is None and S > 1 and getattr(attn.config, "_attn_implementation", "eager") != "eager":
            if Sk == S:
                causal = True
            else:                                           # queries are the last S of Sk positions
                attention_mask = torch.full((S, Sk), float("-inf"), dtype=q.dtype, device=q.device)
                attention_mask = attention_mask.triu(Sk - S + 1).view(1, 1, S, Sk)
        out, H = _attention_entropy(q, k, v, attn.scaling, attention_mask, causal=causal)
        out = attn.o_proj(out.transpose(1, 2).reshape(B, S, -1).contiguous())
        return out, H.mean(dim=(1, 2)), present


def build_dispatched_llama(model, tau_low: float, tau_high: float):
    """EE/python/dispatch.py:250-260: every decoder layer of an HF Llama model
    as an EntropyDispatchedLlamaBlock (fp16, eval), plus one dispatcher."""
    device = next(model.parameters()).device
    blocks = []
    for i, layer in enumerate(model.model.layers):
        block = EntropyDispatchedLlamaBlock(layer, layer_idx=i).to(device).half()
        block.eval()
        blocks.append(block)
    return blocks, PipelinedEntropyDispatcher(tau_low=tau_low, tau_high=tau_high)


TINYLLAMA_1B = dict(layers=22, hidden=2048, heads=32, kv_heads=4, head_dim=64, ffn=5632, vocab=32000,
                    rope_theta=10000.0, eps=1e-5)

class EntropyGatedLlama:
    """A Llama forward in which EVERY linear layer routes each token row to the
    INT8, FP8 or FP16 (W8A16) GEMM by entropy -- benchmark config 4.  This
    extends EE/python/dispatch.py:150-260, which gates only the MLP and picks
    one tier per layer.

    A token's routing entropy is the mean over heads of its attention-row
    entropy: the fused attention kernel (attention_causal: scores,
    probabilities and entropies never leave the chip) where its shapes allow
    (head_dim 64, S % 64 == 0, an even number of query heads per kv head; the
    attribute fused_attention = False turns it off), else the scores, the
    fused softmax+entropy kernel and a product with v.  q/k/v of layer l use layer
    l-1's (layer 0 runs them on the FP16 tier), o/gate/up/down use layer l's,
    and the LM head uses the last layer's.  Rows are grouped per tier into one
    launch per tier and scattered back (routed_linear); q/k/v, and gate/up, run
    as one GEMM each on their concatenated weights (same input, same routing).
    Nothing syncs with the host inside forward.  forward(..., gated=False) is the all-FP16 run: every
    linear as a plain fp16 GEMM on the original weights (hipBLASLt).

    Weights: fp16 tensors in `params` (embed [V, D]; per layer ln1, q [Hq*d, D],
    k/v [Hkv*d, D], o [D, Hq*d], ln2, gate/up [F, D], down [D, F]; norm;
    lm_head [V, D]).  RMSNorm and RoPE follow the Llama definitions, as fused
    kernels (add_rmsnorm: residual add + norm; qkv_rope: RoPE + head-major q/k/v,
    q pre-scaled by 1/sqrt(d)); SwiGLU is silu_mul; grouped-query attention
    reads the shared k/v heads without copies.  A norm whose output feeds a
    routed linear also writes that linear's INT8/FP8 operands
    (add_rmsnorm_route; attribute fused_norm_quant = False turns it off), so the
    linear runs without its quantiser pass."""

    def __init__(self, params: dict, cfg: dict, tau_low: float = 2.34, tau_high: float = 6.03):
        self.p = params
        self.cfg = dict(cfg)
        self.tau_low, self.tau_high = tau_low, tau_high
        # q/k/v and gate/up share their input and routing: each pair runs as one
        # GEMM on the concatenated weights (one quantiser pass, one launch)
        self.fused = {}
        self.packed = {}
        for l in range(cfg["layers"]):
            self.fused[(l, "qkv")] = torch.cat([params[f"{l}.q"], params[f"{l}.k"], params[f"{l}.v"]], dim=0)
            self.fused[(l, "gu")] = torch.cat([params[f"{l}.gate"], params[f"{l}.up"]], dim=0)
            self.fused[(l, "o")] = params[f"{l}.o"]
            self.fused[(l, "down")] = params[f"{l}.down"]
        self.fused["lm_head"] = params["lm_head"]
        for key, w in self.fused.items():
            self.packed[key] = self._pack(w, swiglu=isinstance(key, tuple) and key[1] == "gu")
        self.last_fractions = None
        self._rope_cache = {}
        self.fused_attention = True
        self.fused_norm_quant = True
        # Test hooks (None: off).  linear_impl(key, x2d, route, swiglu) -> y replaces
        # the tier kernels of the gated linears (an independent restatement of their
        # arithmetic); linear_probe(key, x2d, route, y) sees each gated linear's
        # input, routing and output; route_replay: a list of (idx, counts), one per
        # layer, used instead of routing (routes holds the last forward's).
        self.linear_impl = None
        self.linear_probe = None
        self.route_replay = None
        self.routes = []
        # rows per tier over every linear call: layer l's route feeds o/gate/up/down
        # (4) plus layer l+1's q/k/v (3), the last layer's the LM head (1); the
        # weights live on the device, so the per-forward tally is a few kernels, not 3 per layer
        L = cfg["layers"]
        self._route_weights = torch.tensor([4 + (3 if l + 1 < L else 1) for l in range(L)], dtype=torch.int64,
                                           device=params["embed"].device).view(L, 1)

    @staticmethod
    def _pack(w: torch.Tensor, swiglu: bool = False) -> K.PackedWeight:
        """Tier operands of w [N, K]; swiglu: w is gate rows then up rows, packed
        interleaved in blocks of 32 for the SwiGLU epilogue (act = silu(gate) * up)."""
        codes, scale = K.quantize_weight_codes(w)
        if swiglu:
            codes, scale = K.interleave_gate_up(codes), K.interleave_gate_up(scale)
        return K.PackedWeight(codes, scale).materialize()

    @classmethod
    def random_init(cls, cfg: dict = TINYLLAMA_1B, seed: int = 0, device=None, std: float = 0.02, **kw):
        """Random-init weights N(0, std) (RMSNorm weights 1), generated on the GPU."""
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        D, F, V = cfg["hidden"], cfg["ffn"], cfg["vocab"]
        qd, kvd = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]

        def w(*shape):
            return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std).half()

        p = {"embed": w(V, D), "norm": torch.ones(D, device=dev, dtype=torch.float16), "lm_head": w(V, D)}
        for l in range(cfg["layers"]):
            p[f"{l}.ln1"] = torch.ones(D, device=dev, dtype=torch.float16)
            p[f"{l}.ln2"] = torch.ones(D, device=dev, dtype=torch.float16)
            p[f"{l}.q"], p[f"{l}.k"], p[f"{l}.v"], p[f"{l}.o"] = w(qd, D), w(kvd, D), w(kvd, D), w(D, qd)
            p[f"{l}.gate"], p[f"{l}.up"], p[f"{l}.down"] = w(F, D), w(F, D), w(D, F)
        return cls(p, cfg, **kw)

    # ---------------------------------------------------------------- pieces
    def _rope_tables(self, S: int, dev):
        key = (S, dev)
        if key not in self._rope_cache:
            d = self.cfg["head_dim"]
            inv = 1.0 / (self.cfg["rope_theta"] ** (torch.arange(0, d, 2, device=dev, dtype=torch.float32) / d))
            f = torch.outer(torch.arange(S, device=dev, dtype=torch.float32), inv)
            emb = torch.cat((f, f), dim=-1)
            self._rope_cache[key] = (emb.cos().half().unsqueeze(0), emb.sin().half().unsqueeze(0))
        return self._rope_cache[key]

    def _linear(self, x2d: torch.Tensor, key, route, gated: bool, swiglu: bool = False,
                quantized=None) -> torch.Tensor:
        """x2d @ W^T; swiglu: W is gate|up and the result is silu(gate) * up (fused
        into the GEMM epilogue on the gated path; a separate pass on the fp16 run).
        quantized: x2d's INT8/FP8 operands under `route`, from add_rmsnorm_route."""
        if not gated:
            y = torch.matmul(x2d, self.fused[key].t())
            return K.silu_mul(y) if swiglu else y
        if self.linear_impl is not None:
            y = self.linear_impl(key, x2d, route, swiglu)
        else:
            pw = self.packed[key]
            if route is None:                # no entropy yet: FP16 tier (W8A16), as the reference's default
                y = K.gemm("fp16", x2d, pw.f16, swiglu=swiglu)
            else:
                idx, counts = route
                y = K.routed_linear(x2d, pw, idx, counts, swiglu=swiglu, quantized=quantized)
        if self.linear_probe is not None:
            self.linear_probe(key, x2d, route, y)
        return y

    def _norm(self, x, w, res, route, gated: bool):
        """(x, xn, quantized): the residual add + RMSNorm; when the next linear is
        routed (and K % 128 == 0), the same kernel writes its INT8/FP8 operands,
        and xn then holds only the FP16 rows (a linear probe gets every row: the
        separate norm and quantiser, which give the same bits)."""
        if (gated and route is not None and self.fused_norm_quant and self.linear_impl is None
                and self.linear_probe is None and x.shape[-1] % 128 == 0):
            idx, counts = route
            xn = torch.empty((x.numel() // x.shape[-1], x.shape[-1]), dtype=torch.float16, device=x.device)
            x, xn, codes, scale = K.add_rmsnorm_route(x, w, self.cfg["eps"], res, idx, counts, n_out=xn)
            return x, xn, (codes, scale)
        x, xn = K.add_rmsnorm(x, w, self.cfg["eps"], res)
        return x, xn, None

    def _route_heads(self, h: torch.Tensor, counts_log: list):
        """Route tokens on the mean over heads of their attention-row entropies
        h [B, Hq, S] (the mean taken inside the routing kernel)."""
        if self.route_replay is not None:
            idx, counts = self.route_replay[len(counts_log)]
        else:
            _, idx, counts = K.route_heads(h, self.tau_low, self.tau_high)
        counts_log.append(counts)
        self.routes.append((idx, counts))
        return idx, counts

    # ---------------------------------------------------------------- forward
    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, gated: bool = True) -> torch.Tensor:
        """input_ids int64 [B, S] -> logits fp16 [B, S, V].  With gated=True,
        last_fractions holds the device tensor (int64 [3]) of rows per tier
        summed over every linear call (read it after the forward)."""
        c = self.cfg
        B, S = input_ids.shape
        T = B * S
        Hq, Hkv, d = c["heads"], c["kv_heads"], c["head_dim"]
        x = self.p["embed"][input_ids].reshape(T, -1)                    # [T, D] fp16
        cos, sin = self._rope_tables(S, x.device)
        # the fused attention kernel's shapes (attention_causal); others take the unfused path
        fused_att = self.fused_attention and d == 64 and S % 64 == 0 and (Hq // Hkv) % 2 == 0
        counts_log = []
        self.routes = []
        route_prev = None
        res = None                                    # the pending residual branch, added by the next norm
        for l in range(c["layers"]):
            x, xn, xq = self._norm(x, self.p[f"{l}.ln1"], res, route_prev, gated)
            qkv = self._linear(xn, (l, "qkv"), route_prev, gated, quantized=xq)
            # RoPE and the head-major layouts in one pass; q carries the 1/sqrt(d) scaling
            if fused_att:
                # scores, probabilities and entropies stay on chip; att comes out token-major
                q, k, vt = K.qkv_rope(qkv, cos, sin, B, S, Hq, Hkv, d, d ** -0.5, v_transposed=True)
                att, H = K.attention_causal(q, k, vt)
            else:
                q, k, v = K.qkv_rope(qkv, cos, sin, B, S, Hq, Hkv, d, d ** -0.5)
                att, H = _attention_entropy(q, k, v, 1.0, causal=True)
                att = att.transpose(1, 2).reshape(T, Hq * d)
            route_cur = self._route_heads(H, counts_log) if gated else None
            o = self._linear(att, (l, "o"), route_cur, gated)
            x, xn, xq = self._norm(x, self.p[f"{l}.ln2"], o, route_cur, gated)
            act = self._linear(xn, (l, "gu"), route_cur, gated, swiglu=True, quantized=xq)
            res = self._linear(act, (l, "down"), route_cur, gated)
            route_prev = route_cur
        x, xn, xq = self._norm(x, self.p["norm"], res, route_prev, gated)
        logits = self._linear(xn, "lm_head", route_prev, gated, quantized=xq)
        if gated:
            # rows per tier over every linear layer (weights in _route_weights); layer
            # 0's q/k/v run on the FP16 tier.  Device ops only: the forward stays
            # capturable as a HIP graph.
            total = (torch.stack(counts_log).to(torch.int64) * self._route_weights).sum(0)
            total[2] += 3 * T
            self.last_fractions = total
        return logits.view(B, S, -1)
