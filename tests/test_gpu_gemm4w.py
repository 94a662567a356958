"""GPU parity of the four-wave 256-row-tile GEMMs (eek_gemm4w_*: 256 x 256
tiles, eek_gemm4wn128_*: 256 x 128; one wave per SIMD owning a 128 x 128 or
128 x 64 quarter of the tile, accumulators in AGPRs).

They run the 8-wave 256-tile kernels' tiles, deal and per-block K order, so
every case checks them bit for bit against those kernels (gemm_waves = 8) and
against the oracle: INT8 int32 accumulators and fp16 outputs bit-exact, FP8 /
FP16 within 1e-2 of a float64 recompute.  The shapes cover ragged M and N,
tiles of two to twelve K stages, several tiles per workgroup on forced grids
(the stage ring and the tile-parity scale areas across tile boundaries, the
re-issued stages past a workgroup's last tile), grids whose last round runs as
256 x 128 halves, and the SwiGLU epilogue.  Each case asserts, through
ee_last_kernel, that the four-wave kernel is the one that ran.

The W8A16 kind (int8 codes + f32 scales, dequantised in registers) on the
four-wave kernels gives the bits of the FP16 kind on eek_pack_b_f16's weights
(the same MFMAs on the same weight values in the same order), on the same
shapes, grids and epilogues.
"""
import numpy as np
import pytest
import torch

from test_gpu_parity import check_close_f64, cuda, host, weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ee():
    import entropy_engine
    return entropy_engine


def _opt(key, value):
    from entropy_engine import _lib
    _lib.check(_lib.lib().ee_engine_set_option(_lib.engine(), key.encode(), value))


class _Options:
    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        for k, v in self.kv.items():
            _opt(k, v)

    def __exit__(self, *exc):
        for k in self.kv:
            _opt(k, 0)


def _last_kernel():
    from entropy_engine import _lib
    return _lib.lib().ee_last_kernel().decode()


def _operands(ee, orc, M, K, N, seed):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    return A, B, bs, pw


def _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw, acc=None, **opts):
    """INT8, FP8 and FP16 outputs under opts (and the INT8 int32 accumulators
    into acc); returns them with the names of the kernels that ran."""
    names = []
    with _Options(**opts):
        if acc is not None:
            ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs), acc_out=acc)
            names.append(_last_kernel())
        o_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        names.append(_last_kernel())
        o_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
        names.append(_last_kernel())
        o_f16 = host(ee.gemm("fp16", cuda(A), pw.f16))
        names.append(_last_kernel())
    return o_i8, o_f8, o_f16, names


# (M, K, N, gemm_persist): 0 = automatic grid
SHAPES = [
    (512, 512, 512, 0),        # 4 tiles, 4 stages each
    (300, 640, 520, 0),        # partial tiles in M and N, 5 stages
    (520, 256, 1028, 0),       # two K stages per tile; N % 8 == 4 tail
    (1, 256, 4, 0),            # a single row and 4 columns
    (1024, 512, 1024, 8),      # 16 tiles on 8 workgroups: 2 tiles each, ring across tiles
    (1024, 384, 1024, 3),      # 16 tiles on 3 workgroups (not a multiple of 8): 5-6 tiles each
    (768, 256, 2048, 5),       # 24 tiles on 5 workgroups, 2 stages per tile
    (1300, 1536, 900, 2),      # 24 tiles on 2 workgroups, 12 stages per tile
    # last round at most half full: it runs as 256 x 128 halves (256-wide tiles only)
    (512, 512, 2432, 8),       # 20 tiles on 8: 2 full rounds, 8 halves (one past N: skipped)
    (300, 640, 1800, 13),      # 16 tiles on 13: 1 round, 6 halves; partial in M and N
]


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,N,grid", SHAPES)
def test_gemm4w_small(ee, orc, M, K, N, grid, tn):
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 7 + K + N)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    o_i8, o_f8, o_f16, names = _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw, acc,
                                          gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid, gemm_waves=4)
    assert all("gemm4w" in n for n in names), names
    acc_ref = orc.gemm_i8_acc(codes, B)
    assert np.array_equal(host(acc), acc_ref)
    assert np.array_equal(o_i8.view(np.uint16), orc.epilogue_i8(acc_ref, a_s, bs).view(np.uint16))
    check_close_f64(o_f8, orc.gemm_f8_f64(c8, B, s8, bs))
    check_close_f64(o_f16, orc.gemm_w8a16_f64(A, B, bs))
    r_i8, r_f8, r_f16, rn = _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw,
                                       gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid, gemm_waves=8)
    assert all("gemm256" in n for n in rn), rn
    assert np.array_equal(o_i8.view(np.uint16), r_i8.view(np.uint16))
    assert np.array_equal(o_f8.view(np.uint16), r_f8.view(np.uint16))
    assert np.array_equal(o_f16.view(np.uint16), r_f16.view(np.uint16))


def test_gemm4w_one_stage_falls_back(ee, orc):
    """Tiles of a single K stage (K * element size = 128) keep the 8-wave kernel."""
    A, B, bs, pw = _operands(ee, orc, 520, 128, 1028, 3)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    with _Options(gemm_tile=256, gemm_waves=4):
        out = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        assert "gemm256" in _last_kernel()
    acc_ref = orc.gemm_i8_acc(codes, B)
    assert np.array_equal(out.view(np.uint16), orc.epilogue_i8(acc_ref, a_s, bs).view(np.uint16))


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (4096, 4096, 14336)], ids=["config1", "config2"])
def test_gemm4w_full_size(ee, orc, M, K, N):
    """Configs 1 and 2 at full size through the production epilogue: INT8 fp16
    outputs bit-exact and FP8 / FP16 within 1e-2 of float64 on sampled rows
    against the oracle; every output bit-identical to the 8-wave kernels'."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, 21 + N)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    o_i8, o_f8, o_f16, names = _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw, gemm_waves=4)
    assert all("gemm4w" in n for n in names), names
    rows = np.array([0, 1, 255, 256, 257, 1000, 2047, 2048, 3333, 4095])
    ref = orc.epilogue_i8(orc.gemm_i8_acc(codes[rows], B), a_s[rows], bs)
    assert np.array_equal(o_i8[rows].view(np.uint16), ref.view(np.uint16))
    check_close_f64(o_f8[rows], orc.gemm_f8_f64(c8[rows], B, s8[rows], bs))
    check_close_f64(o_f16[rows], orc.gemm_w8a16_f64(A[rows], B, bs))
    r_i8, r_f8, r_f16, _ = _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw, gemm_waves=8)
    assert np.array_equal(o_i8.view(np.uint16), r_i8.view(np.uint16))
    assert np.array_equal(o_f8.view(np.uint16), r_f8.view(np.uint16))
    assert np.array_equal(o_f16.view(np.uint16), r_f16.view(np.uint16))


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,F,grid", [(4096, 2048, 5632, 0), (600, 256, 640, 0), (512, 256, 1216, 8)])
def test_gemm4w_swiglu(ee, orc, M, K, F, grid, tn):
    """The four-wave SwiGLU epilogue gives the bits of the 8-wave one (every
    tier).  The forced grid of 8 leaves the last round half full: 256 x 128
    halves."""
    rng = np.random.default_rng(M + F)
    W = (rng.standard_normal((2 * F, K)) / np.sqrt(K)).astype(np.float16)
    codes, scale = ee.quantize_weight_codes(cuda(W))
    pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    ci, si = ee.quantize_activations(x, "dispatcher")
    cf, sf = ee.quantize_activations(x, "fp8")
    for kind, a, b, sa, sb in (("int8", ci, pw.i8, si, pw.scale), ("fp8", cf, pw.f8, sf, pw.scale),
                               ("fp16", x, pw.f16, None, None)):
        with _Options(gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid, gemm_waves=4):
            fused = ee.gemm(kind, a, b, sa, sb, swiglu=True)
            assert "gemm4w" in _last_kernel()
        with _Options(gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid, gemm_waves=8):
            ref = ee.gemm(kind, a, b, sa, sb, swiglu=True)
        assert torch.equal(fused.view(torch.int16), ref.view(torch.int16)), kind


def _sweep_cases(n=24, seed=4044):
    """Seeded shapes and forced grids: ragged M and N, K of 2-12 stages, grids of
    1-37 workgroups (multiples of 8 and not)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 1300))
        N = int(rng.integers(1, 700)) * 4
        K = int(rng.integers(2, 13)) * 128
        grid = int(rng.choice([1, 2, 3, 5, 7, 8, 13, 16, 24, 37]))
        out.append((M, K, N, grid))
    return out


@pytest.mark.parametrize("M,K,N,grid", _sweep_cases())
def test_gemm4w_seeded_sweep(ee, orc, M, K, N, grid):
    """Four-wave kernels on seeded shapes and grids: INT8 int32 accumulators equal
    the oracle's; INT8, FP8 and FP16 outputs equal the 8-wave kernels' bit for bit."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 31 + K + N + grid)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    o_i8, o_f8, o_f16, names = _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw, acc,
                                          gemm_tile=256, gemm_persist=grid, gemm_waves=4)
    assert all("gemm4w" in n for n in names), names
    assert np.array_equal(host(acc), orc.gemm_i8_acc(codes, B))
    r_i8, r_f8, r_f16, _ = _run_tiers(ee, A, codes, a_s, c8, s8, bs, pw, gemm_tile=256, gemm_persist=grid,
                                      gemm_waves=8)
    assert np.array_equal(o_i8.view(np.uint16), r_i8.view(np.uint16))
    assert np.array_equal(o_f8.view(np.uint16), r_f8.view(np.uint16))
    assert np.array_equal(o_f16.view(np.uint16), r_f16.view(np.uint16))


# ---------------------------------------------------------------------------- W8A16 from int8 codes

def _w8a16_and_f16(ee, A, pw, swiglu=False, **opts):
    """The W8A16 kind on the int8 codes + scales and the FP16 kind on the
    pre-dequantised weights under opts, with the names of the kernels that ran."""
    with _Options(**opts):
        o_w8 = host(ee.gemm("w8a16", cuda(A), pw.i8, None, pw.scale, swiglu=swiglu))
        n_w8 = _last_kernel()
        o_f16 = host(ee.gemm("fp16", cuda(A), pw.f16, swiglu=swiglu))
        n_f16 = _last_kernel()
    return o_w8, o_f16, n_w8, n_f16


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,N,grid", SHAPES + [(520, 128, 1028, 3), (257, 192, 516, 0)])
def test_gemm4w_w8a16_small(ee, orc, M, K, N, grid, tn):
    """eek_gemm4w[n128]_w8a16 dequantises the int8 codes in registers to exactly
    eek_pack_b_f16's weights and runs the FP16 kernel's MFMAs on them: its outputs
    equal eek_gemm4w[n128]_f16's on the pre-dequantised weights bit for bit (K of
    two stages of 64 elements and up, ragged M and N, several tiles per workgroup,
    half last rounds) and lie within 1e-2 of float64."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 11 + K + N)
    o_w8, o_f16, n_w8, n_f16 = _w8a16_and_f16(ee, A, pw, gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid,
                                              gemm_waves=4)
    assert "gemm4w" in n_w8 and n_w8.endswith("w8a16"), n_w8
    assert n_f16 == n_w8.replace("w8a16", "f16"), n_f16
    assert np.array_equal(o_w8.view(np.uint16), o_f16.view(np.uint16))
    check_close_f64(o_w8, orc.gemm_w8a16_f64(A, B, bs))


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (4096, 4096, 14336), (1024, 4096, 4096)],
                         ids=["config1", "config2", "config0"])
def test_gemm4w_w8a16_full_size(ee, orc, M, K, N):
    """Configs 0-2 at full size on the automatic choice of kernel: where the FP16
    kind runs the four-wave kernel the W8A16 kind does too, with the same bits;
    sampled rows within 1e-2 of float64."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, 5 + N + M)
    o_w8, o_f16, n_w8, n_f16 = _w8a16_and_f16(ee, A, pw)
    if "gemm4w" in n_f16:
        assert n_w8 == n_f16.replace("f16", "w8a16"), (n_w8, n_f16)
        assert np.array_equal(o_w8.view(np.uint16), o_f16.view(np.uint16))
    rows = np.array([0, 1, 255, 256, 257, 700, M // 2 - 1, M // 2, M - 2, M - 1])
    check_close_f64(o_w8[rows], orc.gemm_w8a16_f64(A[rows], B, bs))


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,F,grid", [(4096, 2048, 5632, 0), (600, 256, 640, 0), (512, 256, 1216, 8),
                                        (300, 128, 320, 3)])
def test_gemm4w_w8a16_swiglu(ee, orc, M, K, F, grid, tn):
    """The SwiGLU epilogue on int8 gate|up codes: the bits of the FP16 kind's
    four-wave SwiGLU GEMM on the pre-dequantised interleaved weights."""
    rng = np.random.default_rng(M + 3 * F)
    W = (rng.standard_normal((2 * F, K)) / np.sqrt(K)).astype(np.float16)
    codes, scale = ee.quantize_weight_codes(cuda(W))
    pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    x = rng.standard_normal((M, K)).astype(np.float16)
    o_w8, o_f16, n_w8, n_f16 = _w8a16_and_f16(ee, x, pw, swiglu=True, gemm_tile=256, gemm_tile_n=tn,
                                              gemm_persist=grid, gemm_waves=4)
    assert "gemm4w" in n_w8 and n_w8.endswith("w8a16_swiglu"), n_w8
    assert n_f16 == n_w8.replace("w8a16", "f16"), n_f16
    assert np.array_equal(o_w8.view(np.uint16), o_f16.view(np.uint16))


def _w8_sweep_cases(n=16, seed=808):
    """Seeded shapes and forced grids for the W8A16 kind: K of 2-24 stages of 64."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 1300))
        N = int(rng.integers(1, 700)) * 4
        K = int(rng.integers(2, 25)) * 64
        grid = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 37]))
        out.append((M, K, N, grid))
    return out


@pytest.mark.parametrize("M,K,N,grid", _w8_sweep_cases())
def test_gemm4w_w8a16_seeded_sweep(ee, orc, M, K, N, grid):
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 13 + K + N + grid)
    o_w8, o_f16, n_w8, n_f16 = _w8a16_and_f16(ee, A, pw, gemm_tile=256, gemm_persist=grid, gemm_waves=4)
    assert "gemm4w" in n_w8 and n_f16 == n_w8.replace("w8a16", "f16"), (n_w8, n_f16)
    assert np.array_equal(o_w8.view(np.uint16), o_f16.view(np.uint16))


def test_gemm4w_option_rejects_bad_value(ee):
    from entropy_engine import _lib
    assert _lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_waves", 6) == _lib.EE_ERR_INVALID_ARG


# ---------------------------------------------------------------------------- routed

@pytest.mark.parametrize("M,K,N,H_hi,grid", [(300, 512, 520, 3.0, 0), (700, 1024, 384, 3.0, 8), (700, 256, 264, 3.0, 3),
                                             (129, 256, 128, 10.0, 0), (257, 512, 256, 0.3, 0), (1500, 384, 1100, 3.0, 13)])
def test_gemm4w_routed_equals_8wave_and_per_tier(ee, orc, M, K, N, H_hi, grid):
    """The four-wave routed grid (phases FP16, INT8, FP8 per workgroup): every
    row equals the 8-wave routed grid's and the un-routed GEMM of its tier bit
    for bit.  Entropy ranges make tiers empty (H_hi 0.3: INT8 only; 10: mostly
    FP16)."""
    rng = np.random.default_rng(M * 5 + K + N)
    X = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    H = (rng.random(M) * H_hi).astype(np.float32)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    with _Options(gemm_tile=256, gemm_persist=grid):
        out = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
        assert _last_kernel() == "eek_gemm4w_routed"
    with _Options(gemm_tile=256, gemm_persist=grid, gemm_waves=8):
        ref8 = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
        assert _last_kernel() == "eek_gemm256_routed"
    assert np.array_equal(out, ref8)
    t = host(tier)
    full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
            ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
    for k in range(3):
        if (t == k).any():
            assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


@pytest.mark.parametrize("N,sw", [(2048, False), (2560, False), (1024, True)])
def test_gemm4w_routed_sparse_fp16_halves(ee, orc, N, sw):
    """Config 4's mix (2.3 / 95.8 / 1.9 % of 4096 rows): one sparse FP16 M-tile per
    column, run as 256 x 128 halves; rows equal the 8-wave routed grid's and, per
    tier, the un-routed GEMMs'."""
    M, K = 4096, 512
    rng = np.random.default_rng(N + 3 * sw)
    u = rng.random(M)
    H = np.where(u < 0.023, 0.1, np.where(u < 0.981, 1.0, 9.0)).astype(np.float32)
    if sw:
        W = (rng.standard_normal((2 * N, K)) / np.sqrt(K)).astype(np.float16)
        codes, scale = ee.quantize_weight_codes(cuda(W))
        pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    else:
        B, bs = weights(orc, rng, N, K)
        pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    tier, idx, counts = ee.route(cuda(H), 0.5, 5.0)
    assert all(c > 0 for c in counts.tolist())
    with _Options(gemm_tile=256):
        out = host(ee.routed_linear(x, pw, idx, counts, swiglu=sw)).view(np.uint16)
        assert _last_kernel().startswith("eek_gemm4w_routed")
    with _Options(gemm_tile=256, gemm_waves=8):
        ref8 = host(ee.routed_linear(x, pw, idx, counts, swiglu=sw)).view(np.uint16)
    assert np.array_equal(out, ref8)
    if not sw:
        t = host(tier)
        full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
                ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
        for k in range(3):
            assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


@pytest.mark.parametrize("mix,N,sw", [("c4", 11264, True), ("c4", 11264, False), ("int8", 5120, False),
                                      ("c3", 11264, True), ("int8", 1536, True), ("c4", 2048, False),
                                      ("c4", 2560, True), ("c4", 520, False), ("i8f8", 2048, False),
                                      ("i8f8", 2560, False), ("i8f8", 2560, True)])
def test_gemm4w_routed_last_round_halves(ee, orc, mix, N, sw):
    """A last round of 1-byte tiles at most half full runs as 256 x 128 halves on
    twice the workgroups (config 4's gate|up: 748 1-byte tiles, a fourth round of
    68; INT8 only at N = 5120: 320 tiles, a second round of 64 INT8 halves; N =
    1536: one round of 96 tiles, all halves; config 4's one-round grids at N =
    2048 / 2560 / 520 with FP16 halves beside them); config 4's INT8 + FP8 mix
    at N = 2048 / 2560 (one round, an INT8 tier of one tile row: its tiles run
    as halves beside the FP8 tiles): rows equal the 8-wave routed grid's and,
    per tier, the un-routed GEMMs'."""
    M, K = 4096, 256
    rng = np.random.default_rng(N + 7 * sw + len(mix))
    u = rng.random(M)
    lo, hi = {"c4": (0.023, 0.981), "c3": (0.2, 0.6), "int8": (1.0, 1.0), "i8f8": (0.023, 1.0)}[mix]
    H = np.where(u < lo, 0.1, np.where(u < hi, 1.0, 9.0)).astype(np.float32)
    if sw:
        W = (rng.standard_normal((2 * (N // 2), K)) / np.sqrt(K)).astype(np.float16)
        codes, scale = ee.quantize_weight_codes(cuda(W))
        pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    else:
        B, bs = weights(orc, rng, N, K)
        pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    tier, idx, counts = ee.route(cuda(H), 0.5, 5.0)
    with _Options(gemm_tile=256):
        out = host(ee.routed_linear(x, pw, idx, counts, swiglu=sw)).view(np.uint16)
        assert _last_kernel().startswith("eek_gemm4w_routed")
    with _Options(gemm_tile=256, gemm_waves=8):
        ref8 = host(ee.routed_linear(x, pw, idx, counts, swiglu=sw)).view(np.uint16)
    assert np.array_equal(out, ref8)
    if not sw:
        t = host(tier)
        full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
                ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
        for k in range(3):
            if (t == k).any():
                assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


@pytest.mark.parametrize("lo,hi,N", [(0.0, 1.0, 2048), (0.1, 1.0, 2048), (0.0, 1.0, 2560), (0.1, 0.99, 2048)])
def test_gemm4w_routed_one_round_spread(ee, orc, lo, hi, N):
    """One round of 1-byte tiles (4352 rows: 17 tile rows, 136-170 tiles) spread
    over the XCDs: all FP8, INT8 over two tile rows beside FP8, and with a few
    FP16 rows (the W8A16 deal): rows equal the 8-wave routed grid's and, per
    tier, the un-routed GEMMs'."""
    M, K = 4352, 256
    rng = np.random.default_rng(N + int(100 * lo) + int(1000 * hi))
    u = rng.random(M)
    H = np.where(u < lo, 0.1, np.where(u < hi, 1.0, 9.0)).astype(np.float32)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    tier, idx, counts = ee.route(cuda(H), 0.5, 5.0)
    with _Options(gemm_tile=256):
        out = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
        assert _last_kernel() == "eek_gemm4w_routed"
    with _Options(gemm_tile=256, gemm_waves=8):
        ref8 = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
    assert np.array_equal(out, ref8)
    t = host(tier)
    full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
            ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
    for k in range(3):
        if (t == k).any():
            assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


@pytest.mark.parametrize("n_i8,grid", [(100, 24), (100, 32), (0, 24), (300, 32)])
def test_gemm4w_routed_one_round_forced_grid(ee, orc, n_i8, grid):
    """One-round routed grids on forced workgroup counts (gemm_persist): 2000 rows,
    N = 512 (2 tile columns), INT8 rows first.  100 INT8 rows on 24 or 32 workgroups
    take the INT8-halves deal on 20 or 28 FP8 workgroups (not a multiple of 8);
    all-FP8 and two INT8 tile rows take the spread deal.  Rows equal the 8-wave
    routed grid's and, per tier, the un-routed GEMMs'."""
    M, K, N = 2000, 256, 512
    rng = np.random.default_rng(n_i8 + grid)
    H = np.where(rng.permutation(M) < n_i8, 0.1, 1.0).astype(np.float32)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    tier, idx, counts = ee.route(cuda(H), 0.5, 5.0)
    with _Options(gemm_tile=256, gemm_persist=grid):
        out = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
        assert _last_kernel() == "eek_gemm4w_routed"
    with _Options(gemm_tile=256, gemm_waves=8):
        ref8 = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
    assert np.array_equal(out, ref8)
    t = host(tier)
    full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs))]
    for k in range(2):
        if (t == k).any():
            assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


@pytest.mark.parametrize("M,K,F", [(4096, 2048, 1408), (600, 256, 320)])
def test_gemm4w_routed_swiglu(ee, orc, M, K, F):
    """SwiGLU epilogue of the four-wave routed grid: the bits of the 8-wave one."""
    rng = np.random.default_rng(M + 11 * F)
    W = (rng.standard_normal((2 * F, K)) / np.sqrt(K)).astype(np.float16)
    codes, scale = ee.quantize_weight_codes(cuda(W))
    pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    h = cuda((rng.random(M) * 3).astype(np.float32))
    _, idx, counts = ee.route(h, 0.41, 1.68)
    with _Options(gemm_tile=256):
        fused = ee.routed_linear(x, pw, idx, counts, swiglu=True)
        assert _last_kernel() == "eek_gemm4w_routed_swiglu"
    with _Options(gemm_tile=256, gemm_waves=8):
        ref = ee.routed_linear(x, pw, idx, counts, swiglu=True)
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))
