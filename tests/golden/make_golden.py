#!/usr/bin/env python3
"""Writes the fixtures in tests/golden/.

reference_known_answers.json
    Answers the reference's own harness holds, typed in as data:
    * tier decisions at (tau_low, tau_high) = (2.0, 3.5) for entropies 1.0 /
      2.5 / 4.0 (EE/python/benchmark.py:185-210);
    * the dispatch sweep table, tier percentages for the entropies
      0.5, 1.0, ..., 5.0 (EE/python/benchmark.py:386 inputs; NB:555-561 output).
vectors_small.npz
    Seeded small inputs for every stage of the path and the C oracle's outputs
    for them.  They are written only after the oracle passes its pins
    (tests/test_oracle_formats.py, tests/test_oracle_path.py), so they pin
    the GPU path and later oracle edits against regressions.  The int8 ->
    e4m3 table comes from torch's own float8_e4m3fn cast, an independent
    source.

Regenerate from the repository root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

KNOWN = {
    "tier_answers": {                       # EE/python/benchmark.py:185-210
        "tau_low": 2.0, "tau_high": 3.5,
        "entropy": [1.0, 2.5, 4.0],
        "tier": [0, 1, 2],
    },
    "sweep": {                              # EE/python/benchmark.py:386 inputs, NB:555-561 table
        "entropy": [0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.5, 4.0, 4.5, 5.0],
        "rows": [  # tau_low, tau_high, INT8 %, FP8 %, FP16 %
            [1.0, 2.0, 10, 20, 70], [1.5, 2.5, 20, 20, 60], [2.0, 3.0, 30, 20, 50],
            [2.0, 3.5, 30, 30, 40], [2.5, 3.5, 40, 20, 40], [3.0, 4.0, 50, 20, 30],
            [3.5, 4.5, 60, 20, 20],
        ],
    },
}

# Routing thresholds of benchmark configs 3 and 4.
THRESHOLDS = np.float64([[0.41, 1.68], [2.34, 6.03]])


def activations(rng):
    """fp16 [24, 256]: N(0,1) rows at mixed scales, plus the hazard rows the
    reference path defines (zero row; a row small enough that the FP8 tier's
    fp16 inverse scale overflows; a row at fp16 extremes)."""
    M, K = 24, 256
    s = rng.choice(np.float32([0.01, 0.3, 1.0, 7.0, 300.0]), M)
    a = (rng.standard_normal((M, K)).astype(np.float32) * s[:, None]).astype(np.float16)
    a[0] = 0                                                    # INT8 -> 0 row, FP8 -> NaN row
    a[1] = (rng.standard_normal(K) * 1e-3).astype(np.float16)   # amax < 0.0068: fp16(1/scale) = inf
    a[2, :8] = np.float16([65504, -65504, 0.5, -0.5, 1.5, -2.5, 6e-8, -6e-8])
    return a


def entropy_rows(rng):
    """fp16 [10, 300] with closed-form rows first: constant (ln 300), one
    finite element (0), two equal maxima (ln 2); then N(0, s) rows."""
    R, S = 10, 300
    x = (rng.standard_normal((R, S)) * rng.choice([0.25, 1.0, 4.0, 16.0], R)[:, None]).astype(np.float16)
    x[0] = np.float16(3.0)
    x[1] = -np.inf
    x[1, 17] = 2.0
    x[2] = -np.inf
    x[2, [5, 250]] = np.float16(-1.0)
    return x


def e4m3_of_int8_torch():
    """torch's cast of every int8 code through fp16 to float8_e4m3fn bytes
    (|x| <= 127 never saturates)."""
    import torch
    codes = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8)
    return codes.to(torch.float16).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def main():
    import oracle
    rng = np.random.default_rng(20261201)
    a = activations(rng)
    W = (rng.standard_normal((40, 256)) * 0.02).astype(np.float16)        # nn.Linear [N, K]
    B, bs = oracle.quantize_weights_int8(W)                                 # [K, N], [N]
    ci, si = oracle.quant_act_i8(a, "dispatcher")
    ce, se = oracle.quant_act_i8(a, "engine")
    cf, sf = oracle.quant_act_f8(a)
    acc = oracle.gemm_i8_acc(ci, B)
    out_i8 = oracle.epilogue_i8(acc, si, bs)
    with np.errstate(invalid="ignore"):
        out_f8 = oracle.gemm_f8_f64(cf, B, sf, bs)
    out_w8a16 = oracle.gemm_w8a16_f64(a, B, bs)
    x = entropy_rows(rng)
    H, P = oracle.softmax_entropy(x)
    xc = (rng.standard_normal((1, 2, 6, 6)) * 2).astype(np.float16)       # causal [B, H, S, S]
    Hc, Pc = oracle.softmax_entropy(xc.reshape(12, 6), causal=True)
    h_route = np.concatenate([H.astype(np.float32), np.float32([0.41, 1.68, 2.34, 6.03, 0.0, 8.0]),
                              (rng.random(48) * 7).astype(np.float32)])
    routes = [oracle.route(h_route, float(t[0]), float(t[1])) for t in THRESHOLDS]

    np.savez_compressed(
        os.path.join(HERE, "vectors_small.npz"),
        a=a, w=W, b_kn=B, b_scale=bs,
        codes_i8_dispatcher=ci, scale_i8_dispatcher=si,
        codes_i8_engine=ce, scale_i8_engine=se,
        codes_f8=cf, scale_f8=sf,
        acc_i32=acc, out_i8_bits=out_i8.view(np.uint16), out_f8_f64=out_f8, out_w8a16_f64=out_w8a16,
        logits=x, entropy_f64=H, probs_f16=P,
        logits_causal=xc, entropy_causal_f64=Hc, probs_causal_f16=Pc,
        route_h=h_route, route_thresholds=THRESHOLDS,
        route_tier=np.stack([r[0] for r in routes]), route_idx=np.stack([r[1] for r in routes]),
        route_counts=np.stack([r[2] for r in routes]),
        e4m3_of_int8_torch=e4m3_of_int8_torch(),
    )
    with open(os.path.join(HERE, "reference_known_answers.json"), "w") as f:
        json.dump(KNOWN, f, indent=1)
        f.write("\n")
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
