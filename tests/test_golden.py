"""The committed fixtures in tests/golden/ against the C oracle (CPU).

reference_known_answers.json holds answers of the reference's own harness
(EE/python/benchmark.py:185-210; NB:555-561); vectors_small.npz holds seeded
small inputs of every stage with the oracle outputs written when the oracle
passed its pins.  Integer, code and fp16 results must match bit for bit;
float64 recomputations to 1e-12 relative (their summation order may follow
the thread count)."""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def z():
    return np.load(os.path.join(GOLDEN, "vectors_small.npz"))


@pytest.fixture(scope="module")
def known():
    with open(os.path.join(GOLDEN, "reference_known_answers.json")) as f:
        return json.load(f)


def test_fixture_sizes_stay_small():
    for n in os.listdir(GOLDEN):
        assert os.path.getsize(os.path.join(GOLDEN, n)) < 256 * 1024, n


def test_reference_tier_answers(orc, known):
    t = known["tier_answers"]
    tier, idx, counts = orc.route(np.float32(t["entropy"]), t["tau_low"], t["tau_high"])
    assert tier.tolist() == t["tier"]


def test_reference_sweep_table(orc, known):
    ent = np.float32(known["sweep"]["entropy"])
    for tl, th, p0, p1, p2 in known["sweep"]["rows"]:
        _, _, counts = orc.route(ent, tl, th)
        assert (counts * 100 // ent.size).tolist() == [p0, p1, p2], (tl, th)


def test_quantisers_reproduce_fixture(orc, z):
    a = z["a"]
    for mode, key in (("dispatcher", "i8_dispatcher"), ("engine", "i8_engine")):
        c, s = orc.quant_act_i8(a, mode)
        assert np.array_equal(c, z["codes_" + key]) and np.array_equal(s.view(np.uint32),
                                                                       z["scale_" + key].view(np.uint32))
    c, s = orc.quant_act_f8(a)
    assert np.array_equal(c, z["codes_f8"]) and np.array_equal(s.view(np.uint32), z["scale_f8"].view(np.uint32))
    B, bs = orc.quantize_weights_int8(z["w"])
    assert np.array_equal(B, z["b_kn"]) and np.array_equal(bs, z["b_scale"])


def test_fixture_hazard_rows(z):
    # zero row: INT8 codes 0 and output 0; FP8 output NaN (0 * inf inverse scale)
    assert not z["codes_i8_dispatcher"][0].any() and not z["out_i8_bits"][0].any()
    assert np.isnan(z["out_f8_f64"][0]).all()
    # tiny row: fp16(1/scale) overflows, so every nonzero code saturates to +-448 (0x7e / 0xfe)
    c1 = z["codes_f8"][1]
    nz = z["a"][1] != 0
    assert np.all((c1[nz] & 0x7F) == 0x7E)


def test_gemms_reproduce_fixture(orc, z):
    acc = orc.gemm_i8_acc(z["codes_i8_dispatcher"], z["b_kn"])
    assert np.array_equal(acc, z["acc_i32"])
    out = orc.epilogue_i8(acc, z["scale_i8_dispatcher"], z["b_scale"])
    assert np.array_equal(out.view(np.uint16), z["out_i8_bits"])
    with np.errstate(invalid="ignore"):
        f8 = orc.gemm_f8_f64(z["codes_f8"], z["b_kn"], z["scale_f8"], z["b_scale"])
    np.testing.assert_allclose(f8, z["out_f8_f64"], rtol=1e-12, atol=0, equal_nan=True)
    w = orc.gemm_w8a16_f64(z["a"], z["b_kn"], z["b_scale"])
    np.testing.assert_allclose(w, z["out_w8a16_f64"], rtol=1e-12, atol=0)


def test_entropy_reproduces_fixture_and_closed_forms(orc, z):
    H, P = orc.softmax_entropy(z["logits"])
    np.testing.assert_allclose(H, z["entropy_f64"], rtol=1e-12, atol=1e-15)
    assert np.array_equal(P.view(np.uint16), z["probs_f16"].view(np.uint16))
    assert abs(z["entropy_f64"][0] - math.log(300)) < 1e-12
    assert z["entropy_f64"][1] == 0.0
    assert abs(z["entropy_f64"][2] - math.log(2)) < 1e-12
    Hc, Pc = orc.softmax_entropy(z["logits_causal"].reshape(12, 6), causal=True)
    np.testing.assert_allclose(Hc, z["entropy_causal_f64"], rtol=1e-12, atol=1e-15)
    assert np.array_equal(Pc.view(np.uint16), z["probs_causal_f16"].view(np.uint16))
    assert z["entropy_causal_f64"][0] == 0.0 and z["entropy_causal_f64"][6] == 0.0   # causal row 0 of each head


def test_route_reproduces_fixture(orc, z):
    for i, (tl, th) in enumerate(z["route_thresholds"]):
        tier, idx, counts = orc.route(z["route_h"], float(tl), float(th))
        assert np.array_equal(tier, z["route_tier"][i]) and np.array_equal(idx, z["route_idx"][i])
        assert np.array_equal(counts, z["route_counts"][i])


def test_e4m3_of_int8_matches_torch_table(orc, z):
    """The oracle's int8 -> e4m3 map against torch's float8_e4m3fn cast (an
    independent implementation), in code order -128 .. 127."""
    by_byte = orc.e4m3_of_int8()                            # indexed by b & 0xff
    assert np.array_equal(by_byte[np.arange(-128, 128) & 0xFF], z["e4m3_of_int8_torch"])
    vals = orc.e4m3_to_f32(z["e4m3_of_int8_torch"])
    assert len(set(vals.tolist())) == 81                    # 81 distinct e4m3 values; -128 lands on -127's
