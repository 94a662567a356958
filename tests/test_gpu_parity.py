"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (north star): int8 codes, int32 accumulators, INT8 fp16 outputs, e4m3
codes, W8A16 weights and routing decisions bit-exact; entropy within 1e-5
relative (absolute floor 1e-12 for rows whose entropy underflows); FP8 and
W8A16 outputs within 1e-2 relative of a float64 recompute from the same codes
(absolute floor 1e-3 x the output's RMS, for outputs that cancel to ~0);
probabilities within one fp16 ulp of the correctly rounded value.
Inputs are generated on the CPU from seeded numpy generators and copied to
the device, so both sides see identical bits.
"""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ENT_RTOL = 1e-5
ENT_ATOL = 1e-12
F_RTOL = 1e-2
F_ATOL_RMS = 1e-3


@pytest.fixture(scope="module")
def ee():
    import entropy_engine
    return entropy_engine


def cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _lib_set(ee, key, value):
    """Engine option through the C ABI (row-split overrides for coverage)."""
    from entropy_engine import _lib
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), key.encode(), value))


def logits_rows(rng, R, S, scales=(0.25, 1.0, 4.0, 16.0)):
    s = rng.choice(np.asarray(scales), R)
    return (rng.standard_normal((R, S)) * s[:, None]).astype(np.float16)


def check_entropy(h_gpu, h_ref):
    h_gpu = np.asarray(h_gpu, np.float64)
    err = np.abs(h_gpu - h_ref)
    bad = err > ENT_RTOL * np.abs(h_ref) + ENT_ATOL
    assert not bad.any(), f"{bad.sum()} rows off; worst rel {np.max(err / np.maximum(np.abs(h_ref), 1e-30)):.3e}"


def check_probs(p_gpu, p_ref16):
    a = p_gpu.view(np.uint16).astype(np.int32)
    b = p_ref16.view(np.uint16).astype(np.int32)
    assert np.abs(a - b).max() <= 1, "probabilities differ by more than one fp16 ulp"


def check_close_f64(out16, ref64):
    out = out16.astype(np.float64)
    fin = np.isfinite(ref64)
    rms = math.sqrt(np.mean(ref64[fin] ** 2)) if fin.any() else 0.0
    err = np.abs(out[fin] - ref64[fin])
    tol = F_RTOL * np.abs(ref64[fin]) + F_ATOL_RMS * rms
    assert (err <= tol).all(), f"max err {err.max():.3e}; worst excess {(err - tol).max():.3e}"
    assert np.array_equal(np.isnan(out), np.isnan(ref64))


# ---------------------------------------------------------------------------- torch semantics

def test_torch_gpu_scalar_division_is_reciprocal_multiply():
    """The oracle assumes `tensor / python_float` on the GPU is t * f32(1/d)
    (what the reference's launchers ran, EE/python/kernels.py:336,361 and
    dispatch.py:46).  Checked here on every fp16 value and on f32 amaxes."""
    x16 = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)
    t = cuda(x16)
    for d in (127.0, 448.0):
        inv = np.float32(1.0) / np.float32(d)
        ref = (x16.astype(np.float32) * inv).astype(np.float16)
        assert np.array_equal(host(t / d).view(np.uint16), ref.view(np.uint16)), d
    x32 = x16.astype(np.float32)
    inv = np.float32(1.0) / np.float32(127.0)
    assert np.array_equal(host(cuda(x32) / 127.0).view(np.uint32), (x32 * inv).view(np.uint32))


# ---------------------------------------------------------------------------- softmax + entropy

@pytest.mark.parametrize("R,S", [(64, 4096), (48, 512), (33, 1000), (8, 14336), (5, 40000), (3, 8)])
def test_softmax_entropy_rows(ee, orc, R, S):
    rng = np.random.default_rng(R * 7919 + S)
    X = logits_rows(rng, R, S)
    H_ref, P_ref = orc.softmax_entropy(X)
    p, h, _ = ee.softmax_entropy(cuda(X))
    check_entropy(host(h), H_ref)
    check_probs(host(p), P_ref)


@pytest.mark.parametrize("wpr,S", [(w, 2048) for w in range(1, 9)] + [(7, 14336), (8, 14336), (8, 30000), (3, 1000)])
def test_softmax_entropy_every_row_split(ee, orc, wpr, S):
    from entropy_engine import _lib
    rng = np.random.default_rng(wpr * 31 + S)
    X = logits_rows(rng, 40, S)
    H_ref, P_ref = orc.softmax_entropy(X)
    L = _lib.lib()
    _lib.check(L.ee_engine_set_option(_lib.engine(), b"se_wpr", wpr))
    try:
        p, h, _ = ee.softmax_entropy(cuda(X))
        check_entropy(host(h), H_ref)
        check_probs(host(p), P_ref)
    finally:
        _lib.check(L.ee_engine_set_option(_lib.engine(), b"se_wpr", 0))


@pytest.mark.parametrize("rpw", [1, 2, 4])
@pytest.mark.parametrize("R,S,causal", [(1027, 512, True), (1029, 512, False), (515, 1000, False), (7, 300, True),
                                        (2050, 1024, True)])
def test_softmax_entropy_rows_per_wave(ee, orc, R, S, causal, rpw):
    """Short rows with several rows per wave (all their loads issued first):
    ragged row counts (the last wave's rows past the end), causal rows, and the
    two-vector rows (S <= 1024) that only have a 2-rows variant."""
    from entropy_engine import _lib
    rng = np.random.default_rng(R + S + rpw)
    X = logits_rows(rng, R, S)
    H_ref, P_ref = orc.softmax_entropy(X, causal=causal)
    L = _lib.lib()
    _lib.check(L.ee_engine_set_option(_lib.engine(), b"se_rpw", rpw))
    try:
        p, h, _ = ee.softmax_entropy(cuda(X), causal=causal)
        check_entropy(host(h), H_ref)
        check_probs(host(p), P_ref)
        _, h2, _ = ee.softmax_entropy(cuda(X), causal=causal, probs=False)
        assert np.array_equal(host(h2), host(h))
    finally:
        _lib.check(L.ee_engine_set_option(_lib.engine(), b"se_rpw", 0))


@pytest.mark.parametrize("R,S,causal", [(300, 4096, False), (130, 14336, True), (1029, 512, False)])
def test_softmax_entropy_nontemporal_loads(ee, orc, R, S, causal):
    """Option se_nt: the logits read with non-temporal loads (2) or plain ones
    (1) give the same bits, both equal to the oracle's to its tolerance; the
    option rejects other values."""
    from entropy_engine import _lib
    rng = np.random.default_rng(R + S)
    X = logits_rows(rng, R, S)
    H_ref, P_ref = orc.softmax_entropy(X, causal=causal)
    L, E = _lib.lib(), _lib.engine()
    out = {}
    try:
        for v in (1, 2):
            _lib.check(L.ee_engine_set_option(E, b"se_nt", v))
            p, h, _ = ee.softmax_entropy(cuda(X), causal=causal)
            out[v] = (host(p), host(h))
    finally:
        _lib.check(L.ee_engine_set_option(E, b"se_nt", 0))
    check_entropy(out[2][1], H_ref)
    check_probs(out[2][0], P_ref)
    assert np.array_equal(out[1][1].view(np.uint32), out[2][1].view(np.uint32))
    assert np.array_equal(out[1][0].view(np.uint16), out[2][0].view(np.uint16))
    assert L.ee_engine_set_option(E, b"se_nt", 3) == _lib.EE_ERR_INVALID_ARG


def test_softmax_entropy_max_in_several_waves(ee, orc):
    """Rows whose maximum (and its ties) sit in different waves of the row, near
    one-hot rows, and +-0 maxima: the waves holding the max take the counting
    loop, the others the test-free one; H within 1e-5 relative either way."""
    S = 14336
    rng = np.random.default_rng(77)
    X = (rng.standard_normal((10, S)) * 0.5).astype(np.float16)
    X[0, [0, 3000, 9000, S - 1]] = 9.0          # four tied maxima in four waves
    X[1, 5] = 30.0                              # near one-hot
    X[2, [7, 8]] = 25.0                         # two ties in one lane
    X[3] = -1.0; X[3, 100] = 0.0                # max +0 ...
    X[4] = -1.0; X[4, 100] = -0.0; X[4, 2000] = 0.0   # ... and -0 tied with +0
    X[5] = -np.inf; X[5, 4096] = -3.0; X[5, 12000] = -3.0
    X[6] = 3.0                                  # constant row: every wave holds the max
    H_ref, P_ref = orc.softmax_entropy(X)
    try:
        for w in (0, 7, 8):
            _lib_set(ee, "se_wpr", w)
            p, h, _ = ee.softmax_entropy(cuda(X))
            check_entropy(host(h), H_ref)
            check_probs(host(p), P_ref)
    finally:
        _lib_set(ee, "se_wpr", 0)


def test_softmax_entropy_closed_forms(ee, orc):
    S = 4096
    X = np.zeros((6, S), np.float16)
    X[1] = 3.5
    X[2] = -np.inf; X[2, 17] = 1.0
    X[3] = -np.inf; X[3, 5] = 2.0; X[3, 900] = 2.0
    X[4] = -30000.0; X[4, 3] = 0.0
    X[5] = np.arange(S) % 2
    p, h, _ = ee.softmax_entropy(cuda(X))
    h = host(h)
    p = host(p)
    assert h[0] == pytest.approx(math.log(S), rel=1e-6) and h[1] == pytest.approx(math.log(S), rel=1e-6)
    assert h[2] == 0.0 and p[2, 17] == 1.0 and np.count_nonzero(p[2]) == 1
    assert h[3] == pytest.approx(math.log(2), rel=1e-6)
    assert h[4] == 0.0
    H_ref, _ = orc.softmax_entropy(X)
    check_entropy(h, H_ref)


@pytest.mark.parametrize("S", [64, 4096, 5000])
def test_softmax_entropy_rows_without_a_finite_max(ee, orc, S):
    """All -inf rows and rows holding a NaN are NaN in H and in every probability,
    as in the reference; other rows are unaffected.  Every row split."""
    rng = np.random.default_rng(S)
    X = rng.standard_normal((8, S)).astype(np.float16)
    X[1] = -np.inf
    X[3, S // 3] = np.nan
    X[5, :] = -np.inf
    X[5, S - 1] = np.nan
    H_ref, P_ref = orc.softmax_entropy(X)
    try:
        for w in range(0, 9):
            _lib_set(ee, "se_wpr", w)
            p, h, _ = ee.softmax_entropy(cuda(X))
            h, p = host(h), host(p)
            assert np.array_equal(np.isnan(h), np.isnan(H_ref)) and np.isnan(h[[1, 3, 5]]).all()
            assert np.isnan(p[[1, 3, 5]]).all() and not np.isnan(p[[0, 2, 4, 6, 7]]).any()
            ok = ~np.isnan(H_ref)
            check_entropy(h[ok], H_ref[ok])
            check_probs(p[ok], P_ref[ok])
    finally:
        _lib_set(ee, "se_wpr", 0)


def test_softmax_entropy_causal_4d(ee, orc):
    rng = np.random.default_rng(5)
    L = rng.standard_normal((2, 4, 128, 128)).astype(np.float16)
    probs, ent = ee.fused_softmax_entropy(cuda(L), causal=True)
    P_ref, ent_ref = orc.fused_softmax_entropy(L, causal=True)
    H_ref, _ = orc.softmax_entropy(L.reshape(-1, 128), causal=True)
    _, h, _ = ee.softmax_entropy(cuda(L.reshape(-1, 128)), causal=True)
    check_entropy(host(h), H_ref)
    check_probs(host(probs).reshape(-1, 128), P_ref.reshape(-1, 128))
    assert np.allclose(host(ent), ent_ref, rtol=1e-5)
    # the reference test's own bound (EE/python/benchmark.py:174) against -sum p log(p + 1e-10)
    pf = torch.softmax(torch.from_numpy(L).float().masked_fill(
        ~torch.tril(torch.ones(128, 128)).bool(), float("-inf")), dim=-1)
    ref_e = -(pf * torch.log(pf + 1e-10)).sum(-1).mean(dim=(1, 2)).numpy()
    assert np.abs(host(ent) - ref_e).max() < 0.1


def test_softmax_entropy_tiers_in_pass(ee, orc):
    rng = np.random.default_rng(6)
    X = logits_rows(rng, 300, 1024)
    _, h, tier = ee.softmax_entropy(cuda(X), probs=False, thresholds=(0.41, 1.68))
    t_ref, _, _ = orc.route(host(h), 0.41, 1.68)
    assert np.array_equal(host(tier), t_ref)


def test_softmax_entropy_full_size_properties(ee):
    """benchmark config 2's entropy shape [4096, 14336], log-uniform row scales:
    H in [0, ln S] and probabilities summing to 1 within fp16 rounding."""
    rng = np.random.default_rng(7)
    R, S = 4096, 14336
    sc = np.exp(rng.uniform(np.log(0.1), np.log(30.0), R)).astype(np.float32)
    X = (torch.from_numpy(rng.standard_normal((R, S), dtype=np.float32)) * torch.from_numpy(sc)[:, None]).half()
    p, h, _ = ee.softmax_entropy(X.cuda())
    h = host(h)
    assert np.all(h >= 0) and np.all(h <= math.log(S) * (1 + 1e-6))
    sums = p.float().sum(dim=1)
    assert torch.all((sums - 1).abs() < 5e-3).item()


# ---------------------------------------------------------------------------- quantisers

@pytest.mark.parametrize("mode", ["dispatcher", "engine", "fp8"])
@pytest.mark.parametrize("M,K", [(64, 4096), (37, 1024), (9, 14336), (13, 1000), (6, 24)])
def test_quant_codes_bit_exact(ee, orc, mode, M, K):
    rng = np.random.default_rng(M * 31 + K)
    A = rng.standard_normal((M, K)).astype(np.float16)
    A[1] = 0
    if M > 3:
        A[3] *= np.float16(0.01)
    codes, scale = ee.quantize_activations(cuda(A), mode)
    if mode == "fp8":
        ref_c, ref_s = orc.quant_act_f8(A)
    else:
        ref_c, ref_s = orc.quant_act_i8(A, mode)
    assert np.array_equal(host(scale).view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(host(codes).view(np.uint8), ref_c.view(np.uint8))


def test_e4m3_codes_every_fp16_value(ee, orc):
    """A row whose amax is 448 has scale fp16(448/448) = 1 and inverse 1, so its
    codes are e4m3(x) of the inputs themselves: all fp16 values |x| <= 448."""
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)
    h = h[h <= 448]
    vals = np.concatenate([h, -h]).astype(np.float16)
    K = 4096
    n = (len(vals) + K - 2) // (K - 1)
    A = np.zeros((n, K), np.float16)
    A[:, 0] = 448
    flat = A[:, 1:].reshape(-1)
    flat[:len(vals)] = vals
    A[:, 1:] = flat.reshape(n, K - 1)
    codes, scale = ee.quantize_activations(cuda(A), "fp8")
    assert np.all(host(scale) == 1.0)
    ref = orc.e4m3_from_f32(A.astype(np.float32))
    got = host(codes)
    bad = np.argwhere(got != ref)
    detail = [(float(A[i, j]), hex(int(A[i:i + 1, j:j + 1].view(np.uint16)[0, 0])), int(got[i, j]), int(ref[i, j]))
              for i, j in bad[:12]]
    assert len(bad) == 0, f"{len(bad)} codes differ (x, bits, gpu, oracle): {detail}"


def test_quant_routed_slots(ee, orc):
    rng = np.random.default_rng(8)
    A = rng.standard_normal((50, 512)).astype(np.float16)
    H = (rng.random(50) * 4).astype(np.float32)
    tier, idx, counts = ee.route(cuda(H), 1.0, 2.0)
    codes = torch.zeros((50, 512), dtype=torch.int8, device="cuda")
    scale = torch.zeros(50, dtype=torch.float32, device="cuda")
    ee.quantize_activations(cuda(A), "dispatcher", idx=idx, counts=counts, tier=1, out_codes=codes, out_scale=scale)
    c = host(counts)
    ix = host(idx)
    off = int(c[0])
    ref_c, ref_s = orc.quant_act_i8(A[ix[off:off + c[1]]], "dispatcher")
    assert np.array_equal(host(codes)[off:off + c[1]], ref_c)
    assert np.array_equal(host(scale)[off:off + c[1]], ref_s)
    assert np.all(host(codes)[:off] == 0) and np.all(host(codes)[off + c[1]:] == 0)


def test_quantize_weights_int8(ee, orc):
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((384, 640)) * 0.02).astype(np.float16)
    W[5] = 0
    B, s = ee.quantize_weights_int8(cuda(W))
    rB, rs = orc.quantize_weights_int8(W)
    assert np.array_equal(host(B), rB)
    assert np.array_equal(host(s).view(np.uint32), rs.view(np.uint32))


# ---------------------------------------------------------------------------- GEMMs

def weights(orc, rng, N, K, scale=0.02):
    W = (rng.standard_normal((N, K)) * scale).astype(np.float16)
    return orc.quantize_weights_int8(W)


@pytest.fixture(params=[0, 1, 2], ids=["auto", "loader-waves", "8-waves"])
def gemm_variant(request):
    """Runs a test on each GEMM pipeline (engine option gemm_variant)."""
    from entropy_engine import _lib
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_variant", request.param))
    yield request.param
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_variant", 0))


@pytest.fixture(params=[0, 1, 8, 13], ids=["persist-auto", "persist-off", "persist-grid8", "persist-grid13"])
def gemm_persist(request):
    """Runs a test with the persistent GEMM grids off, automatic, or forced to a
    few workgroups (8: XCD-contiguous tile ranges; 13: round robin) so that
    small shapes put many tiles on each workgroup."""
    from entropy_engine import _lib
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_persist", request.param))
    yield request.param
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_persist", 0))


@pytest.mark.parametrize("M,K,N", [(300, 512, 520), (1024, 2048, 1536), (129, 128, 4), (4096, 2048, 11264)])
def test_persistent_gemm(ee, orc, M, K, N, gemm_persist):
    """The persistent INT8 / FP8 kernels (one workgroup walking many tiles, the
    stage ring running across tile boundaries) against the oracle and, bit for
    bit, against the one-tile-per-workgroup kernels."""
    from entropy_engine import _lib
    rng = np.random.default_rng(M * 3 + K + N)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    big = M * N > 4096 * 4096 // 2
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    out_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs), acc_out=None if big else acc))
    out_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
    if not big:
        acc_ref = orc.gemm_i8_acc(codes, B)
        assert np.array_equal(host(acc), acc_ref)
        assert np.array_equal(out_i8.view(np.uint16), orc.epilogue_i8(acc_ref, a_s, bs).view(np.uint16))
        check_close_f64(out_f8, orc.gemm_f8_f64(c8, B, s8, bs))
    else:                                              # sampled rows against the oracle
        rows = np.array([0, 1, 127, 128, M // 2, M - 1])
        ref = orc.epilogue_i8(orc.gemm_i8_acc(codes[rows], B), a_s[rows], bs)
        assert np.array_equal(out_i8[rows].view(np.uint16), ref.view(np.uint16))
        check_close_f64(out_f8[rows], orc.gemm_f8_f64(c8[rows], B, s8[rows], bs))
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_persist", 1))
    try:
        one_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        one_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
    finally:
        _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_persist", gemm_persist))
    assert np.array_equal(out_i8.view(np.uint16), one_i8.view(np.uint16))
    assert np.array_equal(out_f8.view(np.uint16), one_f8.view(np.uint16))


@pytest.mark.parametrize("M,K,N", [(256, 1024, 512), (200, 512, 260), (1, 4096, 128), (130, 4112, 4), (1024, 4096, 4096),
                                   (128, 640, 128), (256, 768, 384)])
def test_int8_gemm_bit_exact(ee, orc, M, K, N, gemm_variant):
    rng = np.random.default_rng(M + K + N)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    acc_ref = orc.gemm_i8_acc(codes, B)
    out_ref = orc.epilogue_i8(acc_ref, a_s, bs)
    pw = ee.prepare_weight(cuda(B), cuda(bs))
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    out = ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs), acc_out=acc)
    assert np.array_equal(host(acc), acc_ref)
    assert np.array_equal(host(out).view(np.uint16), out_ref.view(np.uint16))
    # the reference launcher end to end (quantiser + GEMM)
    full = ee.triton_int8_gemm(cuda(A), cuda(B), cuda(bs))
    assert np.array_equal(host(full).view(np.uint16), out_ref.view(np.uint16))


def test_int8_gemm_extreme_codes(ee, orc):
    M, K, N = 128, 14336, 128
    A = np.full((M, K), -127, np.int8)
    A[::2] = 127
    B = np.full((K, N), -127, np.int8)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    pw = ee.prepare_weight(cuda(B), cuda(np.ones(N, np.float32)))
    ee.gemm("int8", cuda(A), pw.i8, cuda(np.ones(M, np.float32)), cuda(np.ones(N, np.float32)), acc_out=acc)
    assert np.array_equal(host(acc), orc.gemm_i8_acc(A, B))


@pytest.mark.parametrize("M,K,N,sc", [(256, 1024, 512, 1.0), (96, 4096, 260, 0.1), (1024, 4096, 4096, 1.0)])
def test_fp8_gemm(ee, orc, M, K, N, sc):
    rng = np.random.default_rng(M * 3 + N)
    A = (rng.standard_normal((M, K)) * sc).astype(np.float16)
    A[2] = 0                                    # zero row -> NaN row, as the reference
    B, bs = weights(orc, rng, N, K)
    codes, a_s = orc.quant_act_f8(A)
    ref = orc.gemm_f8_f64(codes, B, a_s, bs)
    out = ee.triton_fp8_gemm(cuda(A), cuda(B), cuda(bs))
    o = host(out)
    assert np.all(np.isnan(o[2]))
    check_close_f64(o, ref)
    pw = ee.prepare_weight(cuda(B), cuda(bs))
    assert np.array_equal(host(pw.f8), orc.e4m3_from_f32(B.T.astype(np.float32)))


@pytest.mark.parametrize("M,K,N", [(256, 1024, 512), (77, 2048, 132), (1024, 4096, 4096), (130, 320, 64)])
def test_w8a16_gemm(ee, orc, M, K, N, gemm_variant):
    rng = np.random.default_rng(M * 5 + N)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs))
    assert np.array_equal(host(pw.f16).view(np.uint16), orc.dequant_w8a16(B, bs).T.copy().view(np.uint16))
    out = ee.triton_fp16_gemm(cuda(A), cuda(B), cuda(bs))
    check_close_f64(host(out), orc.gemm_w8a16_f64(A, B, bs))


@pytest.mark.parametrize("M,K,N", [(256, 1024, 512), (77, 2048, 132), (1024, 4096, 4096), (130, 320, 64), (1, 64, 4),
                                   (300, 5632, 2048)])
def test_w8a16_int8_weights(ee, orc, M, K, N):
    """The W8A16 tier from int8 codes + scales, dequantised in the kernel
    (fp16(fp16(b) * fp16(s)), EE/python/kernels.py:215,233): within 1e-2 of the
    float64 recompute, and within fp16 rounding of the pre-dequantised fp16 kernel
    (same weights, another f32 summation order)."""
    rng = np.random.default_rng(M + 3 * K + N)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    out = ee.gemm("w8a16", cuda(A), pw.i8, None, pw.scale)
    check_close_f64(host(out), orc.triton_fp16_gemm_f64(A, B, bs))
    ref16 = host(ee.gemm("fp16", cuda(A), pw.f16)).astype(np.float64)
    assert np.abs(host(out).astype(np.float64) - ref16).max() <= 4e-3 * np.abs(ref16).max() + 1e-6


def test_gemm_full_size_sampled_rows(ee, orc):
    """benchmark configs 1-2 at full size (M=4096, K=4096, N=14336): INT8 int32
    accumulators bit-exact on 48 sampled rows (rows are independent)."""
    rng = np.random.default_rng(11)
    M, K, N = 4096, 4096, 14336
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    a, s = ee.quantize_activations(cuda(A), "dispatcher")
    pw = ee.prepare_weight(cuda(B), cuda(bs))
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    ee.gemm("int8", a, pw.i8, s, pw.scale, acc_out=acc)
    rows = np.sort(rng.choice(M, 48, replace=False))
    codes, _ = orc.quant_act_i8(A[rows], "dispatcher")
    assert np.array_equal(host(acc[torch.from_numpy(rows).cuda()]), orc.gemm_i8_acc(codes, B))


# ---------------------------------------------------------------------------- routing

@pytest.mark.parametrize("R", [1, 10, 1000, 4096, 70000])
def test_route_matches_oracle(ee, orc, R):
    rng = np.random.default_rng(R)
    H = (rng.random(R) * 8).astype(np.float32)
    H[: min(R, 3)] = np.float32(0.41)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    t_ref, i_ref, c_ref = orc.route(H, 0.41, 1.68)
    assert np.array_equal(host(tier), t_ref)
    assert np.array_equal(host(idx), i_ref)
    assert np.array_equal(host(counts), c_ref)


@pytest.mark.parametrize("B,Hh,S", [(8, 32, 512), (2, 4, 64), (3, 1, 100), (1, 5, 7), (3, 40, 2001)])
def test_route_heads_matches_oracle(ee, orc, B, Hh, S):
    """Routing on the per-token mean over heads: the oracle's route() applied to
    the f32 mean summed in head order then divided (the kernel's arithmetic)."""
    rng = np.random.default_rng(B * Hh + S)
    H = (rng.random((B, Hh, S)) * 3).astype(np.float32)
    acc = H[:, 0, :].copy()
    for j in range(1, Hh):
        acc = (acc + H[:, j, :]).astype(np.float32)
    mean = (acc / np.float32(Hh)).astype(np.float32).reshape(-1)
    tier, idx, counts = ee.route_heads(cuda(H), 0.41, 1.68)
    t_ref, i_ref, c_ref = orc.route(mean, 0.41, 1.68)
    assert np.array_equal(host(tier), t_ref)
    assert np.array_equal(host(idx), i_ref)
    assert np.array_equal(host(counts), c_ref)


def test_route_reference_sweep(ee):
    ent = cuda(np.float32([0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.5, 4.0, 4.5, 5.0]))   # EE/python/benchmark.py:386
    for (tl, th), pct in {(1.0, 2.0): [10, 20, 70], (2.0, 3.5): [30, 30, 40], (3.5, 4.5): [60, 20, 20]}.items():
        _, _, counts = ee.route(ent, tl, th)                                       # NB:555-561
        assert (host(counts) * 10).tolist() == pct


def test_row_copy_gather_scatter(ee):
    rng = np.random.default_rng(12)
    X = rng.standard_normal((40, 72)).astype(np.float16)
    idx = np.array(rng.permutation(40), np.int32)
    g = ee.row_copy(cuda(X), cuda(idx))
    assert np.array_equal(host(g), X[idx])
    s = ee.row_copy(g, cuda(idx), scatter=True, out=torch.empty((40, 72), dtype=torch.float16, device="cuda"))
    assert np.array_equal(host(s), X)


@pytest.mark.parametrize("M,K,N", [(300, 1024, 256), (4096, 4096, 4096)])
def test_routed_linear_equals_per_tier(ee, orc, M, K, N, gemm_variant, gemm_persist):
    """scatter(gemm_t(gather(X)))[r] == gemm_t(X)[r] bit for bit, every tier."""
    rng = np.random.default_rng(M + 1)
    X = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    H = (rng.random(M) * 3).astype(np.float32)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    out = ee.routed_linear(x, pw, idx, counts)
    full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
            ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
    o = host(out).view(np.uint16)
    t = host(tier)
    assert sorted(set(t.tolist())) == [0, 1, 2]
    for k in range(3):
        ref = host(full[k]).view(np.uint16)
        assert np.array_equal(o[t == k], ref[t == k]), f"tier {k}"


@pytest.mark.parametrize("M,K,N,H_hi", [(700, 1024, 384, 3.0), (300, 1008, 136, 3.0), (257, 512, 256, 0.3),
                                         (129, 256, 128, 10.0)])
def test_routed_linear_fused_equals_unfused(ee, orc, M, K, N, H_hi, gemm_variant, gemm_persist):
    """The two-launch routed linear (K % 128 == 0: one quantiser, one grid for
    the three tier GEMMs) and the five-launch sequence give the same bits; K =
    1008 takes the five-launch path.  Entropy ranges make some tiers empty."""
    rng = np.random.default_rng(M + K)
    X = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    H = (rng.random(M) * H_hi).astype(np.float32)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    fused = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
    try:
        _lib_set(ee, "routed_unfused", 1)
        unfused = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
    finally:
        _lib_set(ee, "routed_unfused", 0)
    assert np.array_equal(fused, unfused)
    t = host(tier)
    full = [host(ee.triton_int8_gemm(x, cuda(B), cuda(bs))).view(np.uint16),
            host(ee.triton_fp8_gemm(x, cuda(B), cuda(bs))).view(np.uint16),
            host(ee.triton_fp16_gemm(x, cuda(B), cuda(bs))).view(np.uint16)]
    for k in range(3):
        assert np.array_equal(fused[t == k], full[k][t == k]), f"tier {k}"


# ---------------------------------------------------------------------------- dispatcher API

def test_dispatcher_reference_answers(ee):
    """EE/python/benchmark.py:180-218 on GPU tensors."""
    d = ee.PipelinedEntropyDispatcher(tau_low=2.0, tau_high=3.5)
    assert d.get_tier() == ee.PrecisionTier.FP16
    for v, t in ((1.0, ee.PrecisionTier.INT8), (2.5, ee.PrecisionTier.FP8), (4.0, ee.PrecisionTier.FP16)):
        d.submit_entropy(torch.tensor([v], device="cuda"))
        assert d.get_tier() == t
    st = d.get_stats()
    assert [st[k]["count"] for k in ("INT8", "FP8", "FP16")] == [1, 1, 1]


def test_dispatched_linear_tiers(ee, orc):
    rng = np.random.default_rng(13)
    lin = torch.nn.Linear(512, 384, bias=True).half()
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy((rng.standard_normal((384, 512)) * 0.02).astype(np.float16)))
    lin = lin.cuda()
    layer = ee.EntropyDispatchedLinear.from_linear(lin)
    W = lin.weight.detach().cpu().numpy()
    B, bs = orc.quantize_weights_int8(W)
    assert np.array_equal(host(layer.weight_int8), B) and np.array_equal(host(layer.weight_scale), bs)
    x = rng.standard_normal((2, 10, 512)).astype(np.float16)
    y = layer(cuda(x), tier=ee.PrecisionTier.INT8)
    assert y.shape == (2, 10, 384)
    ref = orc.triton_int8_gemm(x.reshape(-1, 512), B, bs)
    ref = (torch.from_numpy(ref) + lin.bias.detach().cpu().unsqueeze(0)).numpy()
    assert np.array_equal(host(y).reshape(-1, 384).view(np.uint16), ref.view(np.uint16))
    for tier, fn in ((ee.PrecisionTier.FP8, orc.triton_fp8_gemm_f64), (ee.PrecisionTier.FP16, orc.triton_fp16_gemm_f64)):
        y = layer(cuda(x), tier=tier)
        r = fn(x.reshape(-1, 512), B, bs) + lin.bias.detach().cpu().double().numpy()[None, :]
        check_close_f64(host(y).reshape(-1, 384), r)


def test_cubin_engine_counterpart(ee, orc):
    """EE/test_cubin.py flow: round-based activation codes, int8 B [K, N], f32 scales."""
    import os
    from entropy_engine import engine as eng_mod
    rng = np.random.default_rng(14)
    M, K, N = 256, 1024, 512
    A = rng.standard_normal((M, K)).astype(np.float16)
    codes, a_s = orc.quant_act_i8(A, "engine")
    g_codes, g_s = ee.quantize_activations(cuda(A), "engine")
    assert np.array_equal(host(g_codes), codes) and np.array_equal(host(g_s), a_s)
    B = rng.integers(-127, 127, (K, N), dtype=np.int8)
    bs = (np.abs(rng.standard_normal(N)) * 0.01 + 0.001).astype(np.float32)
    e = ee.CubinEngine.from_metadata(eng_mod.DEFAULT_CODE_OBJECT, eng_mod.DEFAULT_META, "gemm_int8_kernel")
    out = e.forward(cuda(codes), cuda(B), cuda(a_s), cuda(bs))
    assert out.dtype == torch.float16 and out.shape == (M, N)
    assert np.array_equal(host(out).view(np.uint16), orc.gemm_i8(codes, B, a_s, bs).view(np.uint16))
    with pytest.raises(RuntimeError, match="a must be int8"):
        e.forward(cuda(A), cuda(B), cuda(a_s), cuda(bs))
    with pytest.raises(RuntimeError, match="K mismatch"):
        e.forward(cuda(codes[:, :512]), cuda(B), cuda(a_s), cuda(bs))
    assert os.path.exists(eng_mod.DEFAULT_META)


# ---------------------------------------------------------------------------- committed fixtures

def test_golden_vectors_through_the_abi(ee):
    """tests/golden/vectors_small.npz: every stage of the path on the GPU
    against the committed oracle outputs (hazard rows included: zero row, a
    row whose FP8 inverse scale overflows, fp16 extremes)."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vectors_small.npz"))
    a = cuda(z["a"])
    for mode, key in (("dispatcher", "i8_dispatcher"), ("engine", "i8_engine"), ("fp8", "f8")):
        c, s = ee.quantize_activations(a, mode)
        assert np.array_equal(host(c), z["codes_" + key]), mode
        assert np.array_equal(host(s).view(np.uint32), z["scale_" + key].view(np.uint32)), mode
    w_codes, w_scale = ee.quantize_weight_codes(cuda(z["w"]))
    assert np.array_equal(host(w_codes), z["b_kn"].T) and np.array_equal(host(w_scale), z["b_scale"])
    b_kn, bs = cuda(z["b_kn"]), cuda(z["b_scale"])
    pw = ee.prepare_weight(b_kn, bs)
    ci, si = cuda(z["codes_i8_dispatcher"]), cuda(z["scale_i8_dispatcher"])
    acc = torch.empty((24, 40), dtype=torch.int32, device="cuda")
    out = ee.gemm("int8", ci, pw.i8, si, pw.scale, acc_out=acc)
    assert np.array_equal(host(acc), z["acc_i32"])
    assert np.array_equal(host(out).view(np.uint16), z["out_i8_bits"])
    assert np.array_equal(host(ee.triton_int8_gemm(a, b_kn, bs)).view(np.uint16), z["out_i8_bits"])
    out8 = ee.gemm("fp8", cuda(z["codes_f8"]), pw.f8, cuda(z["scale_f8"]), pw.scale)
    check_close_f64(host(out8), z["out_f8_f64"])
    check_close_f64(host(ee.triton_fp8_gemm(a, b_kn, bs)), z["out_f8_f64"])
    check_close_f64(host(ee.triton_fp16_gemm(a, b_kn, bs)), z["out_w8a16_f64"])
    p, h, _ = ee.softmax_entropy(cuda(z["logits"]))
    check_entropy(host(h), z["entropy_f64"])
    check_probs(host(p), z["probs_f16"])
    p, h, _ = ee.softmax_entropy(cuda(z["logits_causal"].reshape(12, 6)), causal=True)
    check_entropy(host(h), z["entropy_causal_f64"])
    check_probs(host(p), z["probs_causal_f16"])
    for i, (tl, th) in enumerate(z["route_thresholds"]):
        tier, idx, counts = ee.route(cuda(z["route_h"]), float(tl), float(th))
        assert np.array_equal(host(tier), z["route_tier"][i]) and np.array_equal(host(idx), z["route_idx"][i])
        assert np.array_equal(host(counts), z["route_counts"][i])


# ---------------------------------------------------------------------------- config 1

def _config1_inputs(rng, M, K, N):
    a = rng.standard_normal((M, K)).astype(np.float16)
    n = M * K // 1000                                                   # 0.1% outliers of magnitude 20
    pos = rng.choice(M * K, n, replace=False)
    a.reshape(-1)[pos] = (np.sign(rng.standard_normal(n)) * 20).astype(np.float16)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    return a, w


def test_config1_three_gemms(ee, orc):
    """benchmark config 1 (M = K = N = 4096; activations N(0,1) with 0.1% +-20
    outliers, weights N(0,0.02)): INT8 per-row/per-channel (fp16 output
    bit-exact), FP8 e4m3 with per-tensor amax scaling (codes and scales
    bit-exact; outputs within the 1e-2 bar of float64) and the FP16 tier
    (W8A16, the reference's "FP16" GEMM), checked on sampled rows."""
    M = K = N = 4096
    rng = np.random.default_rng(41)
    a, w = _config1_inputs(rng, M, K, N)
    rows = np.sort(rng.choice(M, 48, replace=False))
    ga, gw = cuda(a), cuda(w)
    # FP8 per tensor
    ca, sa = ee.quantize_tensor_fp8(ga)
    cw, sw = ee.quantize_tensor_fp8(gw)
    oa, osa = orc.quant_tensor_f8(a)
    ow, osw = orc.quant_tensor_f8(w)
    assert np.array_equal(host(ca), oa) and np.array_equal(host(sa), osa)
    assert np.array_equal(host(cw), ow) and np.array_equal(host(sw), osw)
    out8 = host(ee.fp8_tensor_gemm(ga, gw))
    dec_a = orc.e4m3_to_f32(oa[rows]).astype(np.float64)
    dec_w = orc.e4m3_to_f32(ow).astype(np.float64)
    ref8 = (dec_a @ dec_w.T) * np.float64(osa[0]) * np.float64(osw[0])
    check_close_f64(out8[rows], ref8)
    # INT8 per row / per channel
    B, bs = orc.quantize_weights_int8(w)
    gB, gbs = ee.quantize_weights_int8(gw)
    assert np.array_equal(host(gB), B) and np.array_equal(host(gbs), bs)
    out_i8 = host(ee.triton_int8_gemm(ga, gB, gbs))
    assert np.array_equal(out_i8[rows].view(np.uint16), orc.triton_int8_gemm(a[rows], B, bs).view(np.uint16))
    # FP16 tier (W8A16)
    out16 = host(ee.triton_fp16_gemm(ga, gB, gbs))
    check_close_f64(out16[rows], orc.triton_fp16_gemm_f64(a[rows], B, bs))


def test_fp8_per_tensor_edge_cases(ee, orc):
    """All-zero tensor (s = 1, codes 0); inf and NaN entries (s = 1, NaN codes
    0x7f|sign); ragged K and an unaligned row stride (generic quantiser)."""
    cases = [np.zeros((3, 64), np.float16),
             np.float16([[np.inf, 1.0, -2.0, np.nan] * 4]),
             np.random.default_rng(42).standard_normal((37, 1000)).astype(np.float16)]
    for a in cases:
        c, s = ee.quantize_tensor_fp8(cuda(a))
        oc, os_ = orc.quant_tensor_f8(a)
        assert np.array_equal(host(c), oc) and np.array_equal(host(s), os_)
    big = np.random.default_rng(43).standard_normal((20, 1001)).astype(np.float16)
    view = cuda(big)[:, :999]                                           # row stride 1001: not 16-byte aligned
    c, s = ee.quantize_tensor_fp8(view)
    oc, os_ = orc.quant_tensor_f8(big[:, :999])
    assert np.array_equal(host(c), oc) and np.array_equal(host(s), os_)


# ---------------------------------------------------------------------------- config 3

def test_config3_dispatcher(ee, orc):
    """benchmark config 3: M = K = N = 4096 with row logits a seeded mixture of
    ~20% low / 40% mid / 40% high-entropy rows (bench.mixture_logits).
    entropy -> route under (0.41, 1.68) and under (2.34, 6.03) -> per-tier
    GEMMs on the gathered rows -> scatter.  Entropy within 1e-5 relative of
    the oracle; routing identical except rows within 1e-5 of a threshold;
    fractions near 20/40/40 at (0.41, 1.68); sampled output rows of each tier
    equal that tier's GEMM of the row (INT8 bit-exact, FP8 / FP16 within the
    1e-2 bar of float64)."""
    import bench
    M = K = N = 4096
    rng = np.random.default_rng(51)
    L, _ = bench.mixture_logits(rng, M, K)
    X = rng.standard_normal((M, K)).astype(np.float16)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    B, bs = orc.quantize_weights_int8(W)
    H_ref, _ = orc.softmax_entropy(L, probs=False)
    _, h, _ = ee.softmax_entropy(cuda(L), probs=False)
    check_entropy(host(h), H_ref)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    refs = (lambda r: orc.triton_int8_gemm(X[r], B, bs), lambda r: orc.triton_fp8_gemm_f64(X[r], B, bs),
            lambda r: orc.triton_fp16_gemm_f64(X[r], B, bs))
    for (tl, th), want in (((0.41, 1.68), (0.2, 0.4, 0.4)), ((2.34, 6.03), None)):
        tier, idx, counts = ee.route(h, tl, th)
        t = host(tier)
        t_ref, _, _ = orc.route(H_ref.astype(np.float32), tl, th)
        near = (np.abs(H_ref - tl) <= 1e-5) | (np.abs(H_ref - th) <= 1e-5)
        assert np.array_equal(t[~near], t_ref[~near])
        assert host(counts).tolist() == [int((t == k).sum()) for k in range(3)]
        if want is not None:
            assert np.allclose(host(counts) / M, want, atol=0.03)
        out = host(ee.routed_linear(x, pw, idx, counts))
        for k in range(3):
            rows = np.flatnonzero(t == k)
            if rows.size == 0:
                continue
            rows = np.sort(rng.choice(rows, min(12, rows.size), replace=False))
            if k == 0:
                assert np.array_equal(out[rows].view(np.uint16), refs[0](rows).view(np.uint16))
            else:
                check_close_f64(out[rows], refs[k](rows))


# ---------------------------------------------------------------------------- Llama (config 4)

def test_dispatched_linear_after_half(ee, orc):
    """Module.half() casts weight_scale to fp16, as it does the reference's
    buffer (whose kernels then read fp16 scales): the tiers use exactly those
    fp16-rounded scales -- INT8 bit-exact, FP8 within the 1e-2 bar."""
    rng = np.random.default_rng(61)
    lin = torch.nn.Linear(512, 384, bias=False)
    lin.weight.data = torch.from_numpy(rng.standard_normal((384, 512)).astype(np.float32) * 0.02)
    layer = ee.EntropyDispatchedLinear.from_linear(lin.half().cuda()).half()
    assert layer.weight_scale.dtype == torch.float16
    x = rng.standard_normal((100, 512)).astype(np.float16)
    B, bs16 = host(layer.weight_int8), host(layer.weight_scale).astype(np.float32)
    y = host(layer(cuda(x), tier=ee.PrecisionTier.INT8))
    assert np.array_equal(y.view(np.uint16), orc.triton_int8_gemm(x, B, bs16).view(np.uint16))
    check_close_f64(host(layer(cuda(x), tier=ee.PrecisionTier.FP8)), orc.triton_fp8_gemm_f64(x, B, bs16))


def test_dispatched_llama_block_against_hf(ee):
    """EE/python/dispatch.py:150-247 with the reference harness's tiny config
    (benchmark.py:220-277: hidden 256, 4 Q / 2 KV heads, eager attention, no
    mask).  layer_entropy equals -sum p ln(p + 1e-10) over HF's own attention
    weights (dispatch.py:243-245) within the fp16 rounding of p; the block's
    output equals HF's attention + an MLP on the FP16 tier's (W8A16) weights;
    with a dispatcher the tier follows the submitted entropy."""
    pytest.importorskip("transformers")
    from transformers import LlamaConfig, LlamaForCausalLM
    import torch.nn.functional as F
    torch.manual_seed(0)
    config = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=2, max_position_embeddings=128, vocab_size=1000,
                         attn_implementation="eager")
    model = LlamaForCausalLM(config).cuda().half().eval()
    layer = model.model.layers[0]
    block = ee.EntropyDispatchedLlamaBlock(layer, layer_idx=0).cuda().half().eval()
    B, S = 2, 32
    hidden = torch.randn(B, S, config.hidden_size, device="cuda", dtype=torch.float16)
    pos = torch.arange(S, device="cuda").unsqueeze(0).expand(B, -1)
    pe = model.model.rotary_emb(hidden, pos)
    with torch.no_grad():
        attn_ref, w = layer.self_attn(layer.input_layernorm(hidden), position_embeddings=pe, attention_mask=None)
        h_ref = -(w.float() * torch.log(w.float() + 1e-10)).sum(dim=-1).mean(dim=(1, 2))
        out = block(hidden, position_ids=pos, position_embeddings=pe)[0]
        assert torch.allclose(block.layer_entropy, h_ref, rtol=5e-3)
        h1 = hidden + attn_ref
        x2 = layer.post_attention_layernorm(h1)
        wg, wu, wd = block.gate_proj.weight_f16_nk, block.up_proj.weight_f16_nk, block.down_proj.weight_f16_nk
        ref = h1 + F.linear(F.silu(F.linear(x2, wg)) * F.linear(x2, wu), wd)
        assert out.shape == (B, S, config.hidden_size)
        assert (out.float() - ref.float()).abs().max() <= 2e-2 * ref.float().abs().max()
        d = ee.PipelinedEntropyDispatcher(tau_low=2.0, tau_high=3.5)
        out2 = block(hidden, dispatcher=d, position_ids=pos, position_embeddings=pe)[0]
        e = float(block.layer_entropy.max())
        want = ee.tier_of(e, 2.0, 3.5).name
        stats = d.get_stats()
        assert stats[want]["count"] == 1 and torch.isfinite(out2).all()
        blocks, disp = ee.build_dispatched_llama(model, 2.0, 3.5)
        assert len(blocks) == 2 and isinstance(disp, ee.PipelinedEntropyDispatcher)


SMALL_LLAMA = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                   rope_theta=10000.0, eps=1e-5)


def test_entropy_gated_llama_small(ee):
    """Config 4's model at a small size.  With thresholds below every entropy
    all rows take the FP16 tier, and the logits equal an fp16 forward on the
    W8A16-dequantised weights (up to GEMM summation order).  At (2.34, 6.03)
    the gated logits stay close to the all-FP16 run, the per-tier row counts
    cover every linear call, and routing mixes tiers per row."""
    m = ee.EntropyGatedLlama.random_init(SMALL_LLAMA, seed=3)
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    ids = torch.randint(0, SMALL_LLAMA["vocab"], (2, 64), generator=g, device="cuda")
    B, S = ids.shape
    fp16 = m.forward(ids, gated=False).float()
    out = m.forward(ids).float()
    fr = m.last_fractions.tolist()
    L = SMALL_LLAMA["layers"]
    assert sum(fr) == B * S * (7 * L + 1)
    assert torch.isfinite(out).all()
    assert (out - fp16).abs().max() <= 0.1 * fp16.abs().max()
    low = ee.EntropyGatedLlama(m.p, SMALL_LLAMA, tau_low=-1.0, tau_high=-1.0)
    deq = dict(m.p)
    D, F, Hd, KVd = SMALL_LLAMA["hidden"], SMALL_LLAMA["ffn"], 4 * 64, 2 * 64
    for key, pw in m.packed.items():
        w = pw.f16
        if key == "lm_head":
            deq["lm_head"] = w
        elif key[1] == "qkv":
            deq[f"{key[0]}.q"], deq[f"{key[0]}.k"], deq[f"{key[0]}.v"] = w[:Hd], w[Hd:Hd + KVd], w[Hd + KVd:]
        elif key[1] == "gu":                             # gate|up rows interleaved in blocks of 32
            v = w.view(F // 32, 2, 32, -1)
            deq[f"{key[0]}.gate"], deq[f"{key[0]}.up"] = v[:, 0].reshape(F, -1), v[:, 1].reshape(F, -1)
        else:
            deq[f"{key[0]}.{key[1]}"] = w
    ref = ee.EntropyGatedLlama(deq, SMALL_LLAMA).forward(ids, gated=False).float()
    got = low.forward(ids).float()
    assert low.last_fractions.tolist() == [0, 0, B * S * (7 * L + 1)]
    assert (got - ref).abs().max() <= 1e-2 * ref.abs().max()
    # the fused attention kernel against the unfused path (scores, softmax_entropy, product with v)
    m.fused_attention = False
    unfused = m.forward(ids, gated=False).float()
    m.fused_attention = True
    assert (fp16 - unfused).abs().max() <= 1e-2 * unfused.abs().max()
    # norms that write the routed linears' codes (add_rmsnorm_route + one GEMM
    # launch) against norms followed by routed_linear's own quantiser
    m.fused_norm_quant = False
    plain = m.forward(ids).float()
    m.fused_norm_quant = True
    assert torch.equal(plain, out)
