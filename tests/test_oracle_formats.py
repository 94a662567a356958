"""Pins the oracle's scalar formats against independent implementations.

fp16: numpy's float16 cast.  e4m3: torch's float8_e4m3fn cast (RNE,
non-saturating, so compared below 464) plus the satfinite closed form the
reference's Triton casts use.  fp16(1/s): exact rational arithmetic.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

ALL_F16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
FINITE_F16 = ALL_F16[np.isfinite(ALL_F16)]


def test_f16_to_f32_exact(orc):
    got = orc.f16_to_f32(ALL_F16)
    ref = ALL_F16.astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))


def test_f32_to_f16_rounding_boundaries(orc):
    # Every fp16 value, every midpoint between neighbours, and the binary32
    # values one ulp either side of each: all of fp16's rounding decisions.
    h = np.sort(FINITE_F16[FINITE_F16 >= 0].astype(np.float32))
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    xs = np.concatenate([h, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(np.inf)),
                         np.float32([65504, 65519.996, 65520, 1e30, np.inf, 1e-30, 2.0 ** -25, 2.0 ** -24 * 1.5])])
    xs = np.concatenate([xs, -xs])
    got = orc.f32_to_f16(xs).view(np.uint16)
    ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    rng = np.random.default_rng(0)
    r = rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200000).astype(np.float32)
    assert np.array_equal(orc.f32_to_f16(r).view(np.uint16), r.astype(np.float16).view(np.uint16))
    assert np.isnan(orc.f32_to_f16(np.float32([np.nan]))[0])


def test_e4m3_all_fp16_inputs_vs_torch(orc):
    x = ALL_F16.astype(np.float32)
    got = orc.e4m3_from_f32(x)
    below = np.abs(x) < 464
    ref = torch.from_numpy(x[below]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got[below], ref)
    # satfinite: everything at or above 448 in magnitude (incl. inf) -> +-448
    sat = (np.abs(x) >= 448) & ~np.isnan(x)
    assert np.all(got[sat] & 0x7F == 0x7E)
    assert np.array_equal(got[sat] >> 7, (np.signbit(x[sat])).astype(np.uint8))
    assert np.all(got[np.isnan(x)] & 0x7F == 0x7F)


def test_e4m3_decode_vs_torch(orc):
    codes = np.arange(256, dtype=np.uint8)
    got = orc.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin], ref[fin])
    assert np.array_equal(np.isnan(got), np.isnan(ref))


def test_int8_to_e4m3_table(orc):
    """The weight re-cast of the FP8 tier, EE/python/kernels.py:166."""
    tab = orc.e4m3_of_int8()
    vals = orc.e4m3_to_f32(tab)
    b = np.arange(256, dtype=np.uint8).view(np.int8)
    assert len(set(vals[b != -128].tolist())) == 81          # 255 codes -> 81 values
    lut = dict(zip(b.tolist(), vals.tolist()))
    assert lut[127] == 128 and lut[17] == 16 and lut[19] == 20 and lut[-127] == -128
    assert all(lut[v] == v for v in range(-16, 17))           # small integers exact


def test_fp16_reciprocal_unambiguous():
    """fp16(1/s) is the same for a correctly rounded and a 2-ulp binary32
    divide (EE/python/kernels.py:144 uses Triton's approximate divide) for
    every positive finite fp16 s: no 1/s lies within 2 f32 ulps of an fp16
    rounding midpoint."""
    pos = FINITE_F16[(FINITE_F16 > 0)]
    hs = np.sort(FINITE_F16[FINITE_F16 >= 0].astype(np.float64))
    mids = [Fraction(a) / 2 + Fraction(b) / 2 for a, b in zip(hs[:-1], hs[1:])]
    mids_f = np.array([float(m) for m in mids])
    bad = 0
    for s in pos.astype(np.float64):
        q = Fraction(1) / Fraction(s)
        qf = float(q)
        if qf >= 65520:
            continue
        j = np.searchsorted(mids_f, qf)
        ulp = Fraction(2) ** (int(np.floor(np.log2(qf))) - 23)
        for jj in (j - 1, j):
            if 0 <= jj < len(mids) and abs(q - mids[jj]) <= 2 * ulp:
                bad += 1
    assert bad == 0


def test_i8_trunc_semantics(orc):
    q = np.float32([0.0, 1.7, -1.7, 126.99, -127.5, 127.06, 200.0, np.nan, -0.4])
    assert orc.i8_trunc(q).tolist() == [0, 1, -1, 126, -127, 127, -56, 0, 0]
