"""Pins the oracle's path functions against independent evaluations.

Quantisers: the reference's PyTorch expressions evaluated by torch on the
CPU, with one substitution -- the reference ran them on the GPU, where
`tensor / python_float` multiplies by the binary32 reciprocal (ATen's
div_true for a CPU-scalar divisor).  That substitution is itself checked on
the GPU (tests/test_gpu_parity.py,
test_torch_gpu_scalar_division_is_reciprocal_multiply).
GEMMs: torch._int_mm, brute-force Python integers, numpy float64.
Entropy: closed forms, invariants and the textbook -sum p ln p in float64.
Routing: the reference's own known answers.
"""
import math

import numpy as np
import pytest
import torch

INV127 = (torch.tensor(1.0) / torch.tensor(127.0)).item()
INV448 = (torch.tensor(1.0) / torch.tensor(448.0)).item()


def _acts(rng, M, K, scale=1.0, outliers=0.0):
    a = (rng.standard_normal((M, K)) * scale).astype(np.float16)
    if outliers:
        n = int(M * K * outliers)
        pos = rng.choice(M * K, n, replace=False)
        a.reshape(-1)[pos] = (np.sign(rng.standard_normal(n)) * 20).astype(np.float16)
    return a


def _gpu_div(t, inv):
    """`t / python_float` as PyTorch computes it on the GPU: t * f32(1/d)."""
    return (t.float() * torch.tensor(inv, dtype=torch.float32)).to(t.dtype)


# ---------------------------------------------------------------- quantisers

@pytest.mark.parametrize("seed", [0, 1])
def test_quant_act_i8_dispatcher(orc, seed):
    rng = np.random.default_rng(seed)
    a = _acts(rng, 48, 640, outliers=0.002)
    a[5] = 0                                           # zero row: scale 0 -> NaN -> code 0
    a[7] *= np.float16(0.01)
    codes, scale = orc.quant_act_i8(a, "dispatcher")
    ta = torch.from_numpy(a)
    s = _gpu_div(ta.abs().amax(dim=1), INV127).clamp(min=1e-8).to(torch.float32)   # kernels.py:336
    ref = (ta / s[:, None]).to(torch.int8)                                        # kernels.py:338
    assert np.array_equal(scale.view(np.uint32), s.numpy().view(np.uint32))
    assert np.array_equal(codes, ref.numpy())
    assert np.all(codes[5] == 0) and scale[5] == 0


def test_quant_act_i8_engine(orc):
    rng = np.random.default_rng(2)
    a = _acts(rng, 40, 512)
    codes, scale = orc.quant_act_i8(a, "engine")
    ta = torch.from_numpy(a)
    s = _gpu_div(ta.float().abs().amax(dim=1), INV127).clamp(min=1e-8)            # test_cubin.py:93-94
    ref = (ta.float() / s.unsqueeze(1)).round().clamp(-127, 127).to(torch.int8)  # test_cubin.py:103
    assert np.array_equal(scale.view(np.uint32), s.numpy().view(np.uint32))
    assert np.array_equal(codes, ref.numpy())


@pytest.mark.parametrize("scale_in", [1.0, 0.1])
def test_quant_act_f8(orc, scale_in):
    rng = np.random.default_rng(3)
    a = _acts(rng, 40, 768, scale=scale_in, outliers=0.001)
    a[3] = 0                                           # zero row -> inv = inf -> 0*inf = NaN codes
    codes, scale = orc.quant_act_f8(a)
    ta = torch.from_numpy(a)
    s = _gpu_div(ta.abs().amax(dim=1), INV448).clamp(min=1e-12).to(torch.float32)  # kernels.py:361
    inv16 = (1.0 / s).to(torch.float16)                                            # kernels.py:144
    scaled = ta * inv16[:, None]                                                   # kernels.py:159 (fp16)
    ref = scaled.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)       # :160, satfinite
    assert np.array_equal(scale.view(np.uint32), s.numpy().view(np.uint32))
    assert np.array_equal(codes, ref.numpy())
    assert np.all(codes[3] & 0x7F == 0x7F)


def _tensor_f8_torch(a):
    """The per-tensor FP8 definition evaluated by numpy (f32 divisions and
    product, RNE) and torch's float8_e4m3fn cast (clamped to +-448 first:
    torch's cast does not saturate)."""
    amax = np.float32(np.abs(a.astype(np.float32)).max())
    s = np.float32(amax / np.float32(448)) if 0 < amax < np.inf else np.float32(1)
    inv = np.float32(1) / s
    x = a.astype(np.float32) * inv
    codes = torch.from_numpy(x).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, s


def test_quant_tensor_f8(orc):
    """Per-tensor FP8 (benchmark config 1's scheme; the build's own definition)."""
    rng = np.random.default_rng(30)
    for a in (_acts(rng, 64, 512, outliers=0.001),                      # config 1 style: +-20 outliers
              (rng.standard_normal((33, 100)) * 0.02).astype(np.float16),   # weight-like
              (rng.standard_normal((5, 64)) * 3e-5).astype(np.float16)):    # subnormal-heavy
        codes, scale = orc.quant_tensor_f8(a)
        ref, s = _tensor_f8_torch(a)
        assert np.all(scale == s) and np.array_equal(codes, ref)
    # amax = 448 * 2^k: s is a power of two and the max element codes to +-448 exactly
    a = np.float16([[896.0, -896.0, 1.0, 0.0]])
    codes, scale = orc.quant_tensor_f8(a)
    assert scale[0] == 2.0 and codes[0].tolist() == [0x7E, 0xFE, 0x30, 0x00]
    # all-zero or non-finite amax: s = 1
    codes, scale = orc.quant_tensor_f8(np.zeros((2, 8), np.float16))
    assert np.all(scale == 1.0) and not codes.any()
    a = np.float16([[np.inf, 1.0, -2.0, np.nan]])
    codes, scale = orc.quant_tensor_f8(a)
    assert scale[0] == 1.0 and codes[0, 1] == 0x38 and codes[0, 2] == 0xC0 and codes[0, 0] == 0x7E
    assert codes[0, 3] & 0x7F == 0x7F


def test_quantize_weights_int8(orc):
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((96, 320)) * 0.02).astype(np.float16)
    W[7] = 0                                                   # zero channel -> scale 1e-8
    B, scale = orc.quantize_weights_int8(W)
    w = torch.from_numpy(W).float().t().contiguous()           # dispatch.py:44
    s = _gpu_div(w.abs().amax(dim=0), INV127).clamp(min=1e-8)   # dispatch.py:45-46
    ref = (w / s.unsqueeze(0)).round().clamp(-127, 127).to(torch.int8)   # dispatch.py:47
    assert np.array_equal(scale.view(np.uint32), s.numpy().view(np.uint32))
    assert np.array_equal(B, ref.numpy())
    assert np.all(np.abs(B.astype(int)).max(axis=0)[np.arange(96) != 7] == 127)


# ---------------------------------------------------------------- GEMMs

def test_gemm_i8_acc_vs_int_mm(orc):
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, (64, 512), dtype=np.int8)
    B = rng.integers(-128, 128, (512, 200), dtype=np.int8)
    acc = orc.gemm_i8_acc(A, B)
    ref = torch._int_mm(torch.from_numpy(A), torch.from_numpy(B)).numpy()
    assert np.array_equal(acc, ref)


def test_gemm_i8_acc_bruteforce_and_extremes(orc):
    rng = np.random.default_rng(6)
    A = rng.integers(-128, 128, (5, 7), dtype=np.int8)
    B = rng.integers(-128, 128, (7, 3), dtype=np.int8)
    acc = orc.gemm_i8_acc(A, B)
    for i in range(5):
        for j in range(3):
            assert acc[i, j] == sum(int(A[i, k]) * int(B[k, j]) for k in range(7))
    # largest K on the path with all-extreme codes stays within int32
    K = 14336
    A = np.full((1, K), -127, np.int8)
    B = np.full((K, 2), -127, np.int8)
    assert orc.gemm_i8_acc(A, B)[0, 0] == K * 127 * 127


def test_epilogue_i8_vs_numpy(orc):
    rng = np.random.default_rng(7)
    acc = rng.integers(-(2 ** 26), 2 ** 26, (33, 70), dtype=np.int32)
    a_s = (rng.random(33) * 0.05).astype(np.float32)
    b_s = (rng.random(70) * 0.001).astype(np.float32)
    got = orc.epilogue_i8(acc, a_s, b_s)
    ref = ((acc.astype(np.float32) * a_s[:, None]).astype(np.float32) * b_s[None, :]).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_triton_int8_gemm_matches_reference_test_tolerance(orc):
    """EE/python/benchmark.py:93-113 semantics at a reduced shape: the INT8
    tier stays within the reference's own max-error bound of 10 against the
    weight-quant-only fp32 reference (benchmark.py:51-70)."""
    rng = np.random.default_rng(42)
    M, K, N = 64, 1024, 256
    A = rng.standard_normal((M, K)).astype(np.float16)
    W = rng.standard_normal((N, K)).astype(np.float16)
    B, bs = orc.quantize_weights_int8(W)
    ref = (A.astype(np.float32) @ (B.astype(np.float32) * bs[None, :])).astype(np.float16)
    out = orc.triton_int8_gemm(A, B, bs)
    err = np.abs(out.astype(np.float32) - ref.astype(np.float32))
    assert err.max() < 10.0 and err.mean() < 2.0


def test_gemm_f8_f64_vs_numpy(orc):
    rng = np.random.default_rng(8)
    A = (rng.standard_normal((24, 256)) * 0.1).astype(np.float16)
    W = (rng.standard_normal((40, 256)) * 0.02).astype(np.float16)
    B, bs = orc.quantize_weights_int8(W)
    codes, a_s = orc.quant_act_f8(A)
    got = orc.gemm_f8_f64(codes, B, a_s, bs)
    lut = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    bq = torch.from_numpy(B.astype(np.float16)).clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    ref = (lut[codes] @ bq) * a_s[:, None].astype(np.float64) * bs[None, :].astype(np.float64)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_w8a16_dequant_and_gemm(orc):
    rng = np.random.default_rng(9)
    A = rng.standard_normal((16, 128)).astype(np.float16)
    W = (rng.standard_normal((24, 128)) * 0.02).astype(np.float16)
    B, bs = orc.quantize_weights_int8(W)
    w16 = orc.dequant_w8a16(B, bs)
    tb = torch.from_numpy(B)
    ref_w = tb.to(torch.float16) * torch.from_numpy(bs).to(torch.float16)[None, :]    # kernels.py:215,233
    assert np.array_equal(w16.view(np.uint16), ref_w.numpy().view(np.uint16))
    got = orc.gemm_w8a16_f64(A, B, bs)
    ref = A.astype(np.float64) @ ref_w.numpy().astype(np.float64)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- entropy

def test_entropy_closed_forms(orc):
    S = 4096
    X = np.zeros((6, S), np.float16)
    X[1] = 3.5                                              # constant row -> ln S
    X[2] = -np.inf; X[2, 17] = 1.0                          # one finite entry -> 0
    X[3] = -np.inf; X[3, 5] = 2.0; X[3, 900] = 2.0          # two equal maxima -> ln 2
    X[4] = -30000.0; X[4, 3] = 0.0                          # others underflow -> ~0
    X[5] = np.arange(S) % 2                                 # two-level row, closed form below
    H, P = orc.softmax_entropy(X)
    assert H[0] == pytest.approx(math.log(S), rel=1e-15)
    assert H[1] == pytest.approx(math.log(S), rel=1e-15)
    assert H[2] == 0.0 and P[2, 17] == 1.0 and np.count_nonzero(P[2]) == 1
    assert H[3] == pytest.approx(math.log(2), rel=1e-15)
    assert H[4] == 0.0
    e = math.e
    Z = S / 2 * (1 + e)
    p0, p1 = 1 / Z, e / Z
    assert H[5] == pytest.approx(-(S / 2) * (p0 * math.log(p0) + p1 * math.log(p1)), rel=1e-13)
    assert np.all(P[1] == np.float16(1 / S))


def test_entropy_rows_without_a_finite_max(orc):
    """All -inf, or a NaN anywhere: the reference's e^(x - m) / Z is NaN for every
    column (m = -inf gives -inf - -inf; a NaN poisons Z), so H and p are NaN."""
    X = np.zeros((3, 64), np.float16)
    X[0] = -np.inf
    X[1, 7] = np.nan
    H, P = orc.softmax_entropy(X)
    assert np.isnan(H[0]) and np.isnan(H[1]) and np.isnan(P[:2]).all()
    assert H[2] == pytest.approx(math.log(64), rel=1e-15) and not np.isnan(P[2]).any()
    H, P = orc.softmax_entropy(np.full((2, 8), -np.inf, np.float16), causal=True)
    assert np.isnan(H).all() and np.isnan(P).all()


def test_entropy_vs_textbook_and_invariants(orc):
    rng = np.random.default_rng(10)
    R, S = 64, 1000
    sc = rng.choice([0.25, 1.0, 4.0, 16.0], R)
    X = (rng.standard_normal((R, S)) * sc[:, None]).astype(np.float16)
    H, P16 = orc.softmax_entropy(X)
    x = X.astype(np.float64)
    p = np.exp(x - x.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        Ht = -np.nansum(np.where(p > 0, p * np.log(p), 0.0), axis=1)
    assert np.allclose(H, Ht, rtol=1e-9, atol=1e-300)
    assert np.all((H >= 0) & (H <= math.log(S) + 1e-12))
    assert np.array_equal(P16.view(np.uint16), p.astype(np.float32).astype(np.float16).view(np.uint16)) or \
        np.abs(P16.astype(np.float64) - p).max() <= 2.0 ** -11
    # shift invariance: integer-valued logits, shifting by 8 is exact in fp16
    Xi = rng.integers(-20, 20, (8, S)).astype(np.float16)
    H1, _ = orc.softmax_entropy(Xi)
    H2, _ = orc.softmax_entropy((Xi.astype(np.float32) + 8).astype(np.float16))
    assert np.array_equal(H1, H2)


def test_entropy_causal(orc):
    rng = np.random.default_rng(11)
    S = 64
    X = rng.standard_normal((2 * S, S)).astype(np.float16)       # two heads of [S,S]
    H, P = orc.softmax_entropy(X, causal=True)
    assert H[0] == 0.0 and H[S] == 0.0                            # query 0 sees one key
    for r in (1, 5, S - 1, S + 3):
        q = r % S
        Hr, _ = orc.softmax_entropy(np.ascontiguousarray(X[r:r + 1, :q + 1]))
        assert H[r] == Hr[0]
        assert np.all(P[r, q + 1:] == 0)


def test_fused_softmax_entropy_4d(orc):
    rng = np.random.default_rng(12)
    L = rng.standard_normal((2, 3, 32, 32)).astype(np.float16)
    probs, ent = orc.fused_softmax_entropy(L, causal=True)
    H, _ = orc.softmax_entropy(L.reshape(-1, 32), causal=True)
    assert probs.shape == L.shape and ent.shape == (2,)
    assert np.allclose(ent, H.reshape(2, 3, 32).mean(axis=(1, 2)), rtol=1e-15)


# ---------------------------------------------------------------- routing

def test_route_reference_tier_answers(orc):
    """EE/python/benchmark.py:185-210: (2.0, 3.5) sends 1.0/2.5/4.0 to INT8/FP8/FP16."""
    tier, idx, counts = orc.route(np.float32([1.0, 2.5, 4.0]), 2.0, 3.5)
    assert tier.tolist() == [0, 1, 2] and counts.tolist() == [1, 1, 1]


SWEEP = [  # NB:555-561 (tau_low, tau_high, INT8%, FP8%, FP16%)
    (1.0, 2.0, 10, 20, 70), (1.5, 2.5, 20, 20, 60), (2.0, 3.0, 30, 20, 50),
    (2.0, 3.5, 30, 30, 40), (2.5, 3.5, 40, 20, 40), (3.0, 4.0, 50, 20, 30),
    (3.5, 4.5, 60, 20, 20),
]


@pytest.mark.parametrize("tl,th,p0,p1,p2", SWEEP)
def test_route_reference_sweep(orc, tl, th, p0, p1, p2):
    ent = np.float32([0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.5, 4.0, 4.5, 5.0])   # benchmark.py:386
    tier, idx, counts = orc.route(ent, tl, th)
    assert (counts * 10).tolist() == [p0, p1, p2]


def test_route_partition_and_threshold_precision(orc):
    rng = np.random.default_rng(13)
    H = rng.random(1000).astype(np.float32) * 8
    H[:3] = np.float32(0.41)                 # f32(0.41) vs the double threshold 0.41
    tier, idx, counts = orc.route(H, 0.41, 1.68)
    assert counts.sum() == 1000 and sorted(idx.tolist()) == list(range(1000))
    off = np.concatenate([[0], np.cumsum(counts)])
    for t in range(3):
        seg = idx[off[t]:off[t + 1]]
        assert np.all(np.diff(seg) > 0) and np.all(tier[seg] == t)
    expect = 0 if float(np.float32(0.41)) < 0.41 else 1
    assert np.all(tier[:3] == expect)
    nan_tier, _, _ = orc.route(np.float32([np.nan]), 1.0, 2.0)
    assert nan_tier[0] == 2
