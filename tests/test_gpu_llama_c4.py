"""Config 4 at full size (TinyLlama-1.1B architecture: 22 layers, hidden 2048,
32 Q / 4 KV heads, FFN 5632, vocab 32000; batch 8 x 512 tokens; every linear
routed per token at (2.34, 6.03)).

Every gated linear of the forward is checked against an independent
restatement of its tier's arithmetic -- the reference's quantiser and epilogue
expressions (EE/python/kernels.py:336-338, 361, 144, 159-166, 104, 176-180,
215, 233; EE/python/dispatch.py:43-48) as torch ops, with exact int32 (via
float64) and float32 dots -- on the very input the kernels saw (INT8 rows bit
for bit, the rest within fp16 rounding).  End to end, the restatement run on
the kernel forward's routing is as far from the all-FP16 run as the gated
forward is: its ~1.5 max-abs logit error is the tiers' rounding.  Also: the
FP16 tier alone against a torch fp16 forward on the W8A16 weights, and sampled
rows of every routed linear of two layers against the C oracle (INT8
bit-exact, FP8 / W8A16 within 1e-2 of float64) on the inputs the kernels saw."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from test_gpu_parity import check_close_f64

pytestmark = pytest.mark.gpu

_E4M3_MAX = 448.0


class TierRestatement:
    """linear_impl for EntropyGatedLlama: each routed linear's rows computed
    per tier with torch ops on the original fp16 weights."""

    def __init__(self, model):
        self.m = model
        self.w = {}

    def _weights(self, key):
        if key not in self.w:
            W = self.m.fused[key]                                    # fp16 [N, K]
            w = W.float().t()                                        # dispatch.py:43-48
            scale = (w.abs().amax(dim=0) / 127).clamp(min=1e-8)
            codes = (w / scale).round().clamp(-127, 127).to(torch.int8)          # [K, N]
            w8 = codes.half().float().clamp(-_E4M3_MAX, _E4M3_MAX).to(torch.float8_e4m3fn).float()
            w16 = (codes.half() * scale.half()).float()              # kernels.py:215, 233
            self.w[key] = (codes.double(), scale, w8, w16)
        return self.w[key]

    def _tier(self, t, x, key):
        codes, scale, w8, w16 = self._weights(key)
        if t == 0:                                                   # kernels.py:336-338, 86-104
            s = (x.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=1e-8).float()
            a = (x.float() / s).to(torch.int8)
            acc = (a.double() @ codes).float()                       # exact int32 sums
            return ((acc * s) * scale[None, :]).half()
        if t == 1:                                                   # kernels.py:361, 144, 159-180
            s = (x.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12).float()
            inv = (1.0 / s).half()
            a8 = (x * inv).float().clamp(-_E4M3_MAX, _E4M3_MAX).to(torch.float8_e4m3fn).float()
            return (((a8 @ w8) * s) * scale[None, :]).half()
        return (x.float() @ w16).half()                              # kernels.py:192-246

    def __call__(self, key, x, route, swiglu):
        T = x.shape[0]
        N = self.m.fused[key].shape[0]
        y = torch.empty((T, N), dtype=torch.float16, device=x.device)
        if route is None:
            y = self._tier(2, x, key)
        else:
            idx, counts = route
            c = counts.tolist()
            off = 0
            for t in range(3):
                rows = idx[off:off + c[t]].long()
                off += c[t]
                if rows.numel():
                    y[rows] = self._tier(t, x[rows], key)
        if swiglu:                                                   # torch's fp16 F.silu(gate) * up
            Fh = N // 2
            y = (F.silu(y[:, :Fh].float()).half().float() * y[:, Fh:].float()).half()
        return y


@pytest.fixture(scope="module")
def c4():
    import entropy_engine as ee
    model = ee.EntropyGatedLlama.random_init(ee.TINYLLAMA_1B, seed=0, tau_low=2.34, tau_high=6.03)
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    ids = torch.randint(0, ee.TINYLLAMA_1B["vocab"], (8, 512), generator=g, device="cuda")
    return model, ids


def test_config4_gated_forward_is_tier_rounding(c4, orc):
    model, ids = c4
    fp16 = model.forward(ids, gated=False).float()
    restate = TierRestatement(model)
    worst = {}                                                      # key kind -> worst relative gap
    samples = {}
    sample_layers = (1, 11)

    def probe(key, x, route, y):
        # every gated linear against the restatement on the very input the kernels saw
        r = restate(key, x, route, key[1] == "gu" if isinstance(key, tuple) else False)
        kind = key[1] if isinstance(key, tuple) else key
        if route is not None:                                       # INT8 rows: bit for bit
            idx, counts = route
            rows = idx[:int(counts[0])].long()
            assert torch.equal(y[rows].view(torch.int16), r[rows].view(torch.int16)) or kind == "gu", key
        gap = ((y.float() - r.float()).abs().max() / r.float().abs().max()).item()
        worst[kind] = max(worst.get(kind, 0.0), gap)
        if isinstance(key, tuple) and key[0] in sample_layers and kind in ("qkv", "o", "down"):
            samples[key] = (x, route, y)

    model.linear_probe = probe
    try:
        gated = model.forward(ids).float()
        routes = [(i.clone(), c.clone()) for i, c in model.routes]
    finally:
        model.linear_probe = None
    rows = model.last_fractions.tolist()
    assert rows[1] > 0.8 * sum(rows) and rows[0] > 0 and rows[2] > 0          # mostly FP8, every tier used
    print("config 4, worst |kernel - restatement| / max per linear kind:",
          {k: round(v, 5) for k, v in worst.items()})
    # fp16 rounding of the same f32 sums in another order (SwiGLU: of gate, up and the product)
    assert max(v for k, v in worst.items() if k != "gu") <= 2e-3
    assert worst["gu"] <= 4e-3
    # end to end on the kernel forward's routing: the restatement's distance from the FP16
    # run is the gated forward's -- the error is the tiers' rounding -- and the two FP8
    # forwards are closer to each other than either is to FP16 (22 layers of rounding
    # at code boundaries make them drift apart, as any two such computations would)
    model.linear_impl, model.route_replay = restate, routes
    try:
        emu = model.forward(ids).float()
    finally:
        model.linear_impl = model.route_replay = None
    absmax = fp16.abs().max().item()
    err_gated = (gated - fp16).abs().max().item()
    err_emu = (emu - fp16).abs().max().item()
    gap = (gated - emu).abs().max().item()
    print(f"config 4: |gated - fp16| {err_gated:.4f}, |restated - fp16| {err_emu:.4f}, "
          f"|gated - restated| {gap:.4f}, fp16 absmax {absmax:.4f}")
    assert torch.isfinite(gated).all() and torch.isfinite(emu).all()
    assert abs(err_gated - err_emu) <= 0.25 * err_emu
    assert gap < min(err_gated, err_emu)
    # the GEMM kernels on the inputs they saw, sampled rows of every tier, against the oracle
    for key, (x, route, y) in samples.items():
        pw = model.packed[key]
        B_kn = pw.i8.t().contiguous().cpu().numpy()
        bs = pw.scale.cpu().numpy()
        idx, counts = (t.cpu().numpy() for t in route)
        off = 0
        for t in range(3):
            n = int(counts[t])
            if n:
                r = idx[off + np.unique([0, n // 2, n - 1])]
                xr = x[torch.from_numpy(r).long().cuda()].cpu().numpy()
                yr = y[torch.from_numpy(r).long().cuda()].cpu().numpy()
                if t == 0:
                    assert np.array_equal(yr.view(np.uint16), orc.triton_int8_gemm(xr, B_kn, bs).view(np.uint16)), key
                elif t == 1:
                    check_close_f64(yr, orc.triton_fp8_gemm_f64(xr, B_kn, bs))
                else:
                    check_close_f64(yr, orc.triton_fp16_gemm_f64(xr, B_kn, bs))
            off += n


def test_config4_fp16_tier_forward(c4):
    """Every row on the FP16 tier (thresholds below every entropy): the gated
    forward against a torch fp16 forward on the W8A16 weights (the
    restatement's FP16 tier), bounded as the 2-layer test bounds it."""
    model, ids = c4
    tl, th = model.tau_low, model.tau_high
    model.tau_low = model.tau_high = -1.0
    try:
        got = model.forward(ids).float()
        assert model.last_fractions.tolist()[:2] == [0, 0]
        routes = [(i.clone(), c.clone()) for i, c in model.routes]
        model.linear_impl, model.route_replay = TierRestatement(model), routes
        ref = model.forward(ids).float()
    finally:
        model.linear_impl = model.route_replay = None
        model.tau_low, model.tau_high = tl, th
    assert (got - ref).abs().max() <= 1e-2 * ref.abs().max()
