"""Pins of the oracle's MLP functions (CPU only).

silu_mul must equal torch's fp16 F.silu(gate) * up (the MLP activation of the
reference's baseline, EE/test_engine.py:35, and of the HF Llama MLP the
reference gates, EE/python/dispatch.py:199-203): silu evaluated in f32 as
x / (1 + exp(-x)) and rounded to fp16, then the fp16 product rounded.
Independent checks: a numpy restatement with numpy's own casts, closed forms
of silu, plausible mistakes (no intermediate rounding, gate and up swapped,
silu rounded from float64) that must fail, torch's CPU kernel, and the MLP
composition against a float64 MLP on the dequantised weights.  torch's GPU
kernel is compared in the GPU tests.
"""
import numpy as np
import pytest
import torch


def bits(a):
    return np.asarray(a, np.float16).view(np.uint16)


def test_f64_to_f16_is_correctly_rounded(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000) * s for s in (1e-6, 1e-3, 1.0, 100.0, 3e4)])
    # exact fp16 midpoints and their neighbours: double rounding through f32 would break these
    h = np.arange(0, 0x7BFF, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    ulp = np.spacing(h.astype(np.float16)).astype(np.float64)
    mids = h + ulp / 2
    x = np.concatenate([x, mids, mids + 1e-12 * ulp, mids - 1e-12 * ulp, -mids, [0.0, -0.0, 65519.0, 65520.0]])
    with np.errstate(over="ignore"):
        assert np.array_equal(bits(orc.f64_to_f16(x)), bits(x.astype(np.float16)))


def silu_mul_numpy(gu):
    F = gu.shape[1] // 2
    g = gu[:, :F].astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
        s16 = (g / (np.float32(1.0) + e)).astype(np.float16)
        return (s16.astype(np.float32) * gu[:, F:].astype(np.float32)).astype(np.float16)


def test_silu_mul_matches_numpy_restatement(orc):
    rng = np.random.default_rng(1)
    gu = (rng.standard_normal((64, 2 * 512)) * rng.choice([0.01, 1.0, 8.0, 40.0], (64, 1))).astype(np.float16)
    gu[0, :8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 65504, -65504, 6e-8]
    got, ref = orc.silu_mul(gu), silu_mul_numpy(gu)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(bits(got)[ok], bits(ref)[ok])


def test_silu_closed_forms(orc):
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    g = g[np.isfinite(g)]
    F = g.size
    gu = np.concatenate([g, np.ones(F, np.float16)])[None, :]
    act, s = orc.silu_mul(gu, with_silu=True)
    s, gd = s[0].astype(np.float64), g.astype(np.float64)
    assert np.all(s[gd == 0] == 0)
    # silu(x) - silu(-x) = x  (sigmoid(x) + sigmoid(-x) = 1), to f32 rounding
    pos = gd > 0
    order = np.argsort(gd)
    neg_of = {float(v): i for i, v in enumerate(gd)}
    idx = np.array([neg_of[-float(v)] for v in gd[pos]])
    assert np.allclose(s[pos] - s[idx], gd[pos], rtol=4e-7, atol=0)
    # large positive: silu(x) rounds to x; large negative: to -0 (or the smallest subnormal)
    big = gd >= 16
    assert np.array_equal(bits(act[0][big]), bits(g[big]))
    assert np.all(np.abs(act[0][gd <= -30].astype(np.float64)) <= 6e-8)
    # silu is increasing above its minimum at x = -1.2785 and bounded below by -0.2785
    a = act[0].astype(np.float64)
    assert np.all(np.diff(a[order][gd[order] > -1.2]) >= 0)
    assert s.min() > -0.2785 and s.min() < -0.2784
    # f32 evaluation, not a float64 one: for tiny |x| the f32 denominator is
    # exactly 2, so silu(x) is x / 2 exactly and an odd subnormal rounds to even
    tiny = np.array([6e-8, -6e-8, 1.8e-7], np.float16)
    t_act = orc.silu_mul(np.concatenate([tiny, np.ones(3, np.float16)])[None, :])[0]
    assert np.array_equal(bits(t_act), bits((tiny.astype(np.float64) / 2).astype(np.float16)))


def test_silu_mul_keeps_the_intermediate_rounding_and_operand_order(orc):
    """Plausible mistakes give different bits: rounding only once, or swapping gate and up."""
    rng = np.random.default_rng(2)
    gu = (rng.standard_normal((32, 2 * 256)) * 3).astype(np.float16)
    act = bits(orc.silu_mul(gu))
    F = 256
    g = gu[:, :F].astype(np.float64)
    once = (g / (1 + np.exp(-g)) * gu[:, F:].astype(np.float64)).astype(np.float16)
    swapped = silu_mul_numpy(np.concatenate([gu[:, F:], gu[:, :F]], axis=1))
    assert (act != bits(once)).mean() > 0.01
    assert (act != bits(swapped)).mean() > 0.5
    # silu rounded from float64 instead of evaluated in f32: differs where the
    # f32 denominator 1 + exp(-x) rounds to exactly 2 (x = +-2^-24)
    sub = np.arange(1, 1024, dtype=np.uint16).view(np.float16)
    sub = np.concatenate([sub, -sub])
    gu2 = np.concatenate([sub, np.ones_like(sub)])[None, :]
    g64 = sub.astype(np.float64)
    f64_rounded = (g64 / (1 + np.exp(-g64))).astype(np.float16)
    differ = np.nonzero(bits(orc.silu_mul(gu2)[0]) != bits(f64_rounded))[0]
    assert set(np.abs(sub[differ].astype(np.float64))) == {2.0 ** -24}


def test_silu_mul_matches_torch_cpu_fp16(orc):
    """torch's CPU fp16 kernels (f32 math, vectorised exp): at most one ulp from
    the correctly rounded silu, and almost always equal."""
    rng = np.random.default_rng(3)
    gu = (rng.standard_normal((128, 2 * 1024)) * 4).astype(np.float16)
    t = torch.from_numpy(gu)
    ref = (torch.nn.functional.silu(t[:, :1024]) * t[:, 1024:]).numpy()
    got = orc.silu_mul(gu)
    a = bits(got).astype(np.int32)
    b = bits(ref).astype(np.int32)
    same_sign = (a & 0x8000) == (b & 0x8000)
    d = np.abs(a - b)[same_sign]
    assert same_sign.mean() > 0.999 and d.max() <= 1 and (d == 0).mean() > 0.999


@pytest.mark.parametrize("tier,rtol", [(0, 0.1), (1, 0.1), (2, 0.03)])
def test_mlp_forward_against_float64_mlp(orc, tier, rtol):
    """The composed oracle MLP against an unquantised float64 MLP: relative
    error of the tier's quantisation (INT8 / FP8 activations, int8 weights)."""
    rng = np.random.default_rng(4)
    M, H, F = 32, 256, 384
    x = rng.standard_normal((M, H)).astype(np.float16)
    g = (rng.standard_normal((F, H)) / 16).astype(np.float16)
    u = (rng.standard_normal((F, H)) / 16).astype(np.float16)
    d = (rng.standard_normal((H, F)) / 20).astype(np.float16)
    X = x.astype(np.float64)
    G, U = X @ g.astype(np.float64).T, X @ u.astype(np.float64).T
    ref = (G / (1 + np.exp(-G)) * U) @ d.astype(np.float64).T
    gu, act, out = orc.mlp_forward(x, g, u, d, tier)
    out = np.asarray(out, np.float64)
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    assert rel < rtol
    # the gate|up stage on its own: columns 0..F-1 are gate, F..2F-1 are up
    guf = np.asarray(gu, np.float64)
    assert np.linalg.norm(guf[:, :F] - G) / np.linalg.norm(G) < rtol
    assert np.linalg.norm(guf[:, F:] - U) / np.linalg.norm(U) < rtol
    assert act.shape == (M, F) and act.dtype == np.float16
