"""GPU parity of the 256-row-tile persistent GEMMs (eek_gemm256_*: 256 x 256
tiles; eek_gemm256n128_*: 256 x 128).  Every case runs at both tile widths.

They replace the 128 x 128 kernels for GEMMs and routed linears with more
128-tiles than CUs (configs 1-4), so each case checks them
against the oracle -- INT8 fp16 outputs and int32 accumulators bit-exact,
FP8 / FP16 within 1e-2 of a float64 recompute -- and, bit for bit, against the
128-tile kernels on the same inputs (same K order: FP8 and FP16 sum slice after
slice in both).  Ragged shapes, one-stage K, partial tiles and several tiles
per workgroup (forced grids, including one that is not a multiple of the 8
XCDs) exercise the stage ring across tile boundaries; grids whose last round
is at most half full run that round as 256 x 128 halves.
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


def _operands(ee, orc, M, K, N, seed):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    return A, B, bs, pw


# (M, K, N, gemm_persist): 0 = automatic grid
SHAPES = [
    (512, 512, 512, 0),        # 4 tiles, 4 stages each
    (300, 640, 520, 0),        # partial tiles in M and N, 5 stages
    (520, 128, 1028, 0),       # one K stage per tile; N % 8 == 4 tail
    (1, 256, 4, 0),            # a single row and 4 columns
    (1024, 512, 1024, 8),      # 16 tiles on 8 workgroups: 2 tiles each, ring across tiles
    (1024, 384, 1024, 3),      # 16 tiles on 3 workgroups (not a multiple of 8): 5-6 tiles each
    (768, 256, 2048, 5),       # 24 tiles on 5 workgroups, 2 stages per tile
    # last round at most half full: it runs as 256 x 128 halves (256-wide tiles only)
    (512, 512, 2432, 8),       # 20 tiles on 8: 2 full rounds, 8 halves (one past N: skipped)
    (300, 640, 1800, 13),      # 16 tiles on 13: 1 round, 6 halves; partial in M and N
]


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,N,grid", SHAPES)
def test_gemm256_int8_fp8_small(ee, orc, M, K, N, grid, tn):
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 7 + K + N)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    with _Options(gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid):
        o_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs), acc_out=acc)
        o_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
    acc_ref = orc.gemm_i8_acc(codes, B)
    assert np.array_equal(host(acc), acc_ref)
    assert np.array_equal(o_i8.view(np.uint16), orc.epilogue_i8(acc_ref, a_s, bs).view(np.uint16))
    check_close_f64(o_f8, orc.gemm_f8_f64(c8, B, s8, bs))
    with _Options(gemm_tile=128):
        r_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
    assert np.array_equal(o_f8.view(np.uint16), r_f8.view(np.uint16))


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,N,grid", SHAPES[:3] + SHAPES[4:6] + SHAPES[7:])
def test_gemm256_fp16_small(ee, orc, M, K, N, grid, tn):
    """The FP16 (W8A16) tier on the 256-tile kernel: within 1e-2 of float64 and
    bit-identical to the 128-tile loader-wave pipeline (same K order)."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, M + 5 * K + N)
    with _Options(gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid):
        out = host(ee.gemm("fp16", cuda(A), pw.f16))
    check_close_f64(out, orc.gemm_w8a16_f64(A, B, bs))
    with _Options(gemm_tile=128, gemm_variant=1):
        ref = host(ee.gemm("fp16", cuda(A), pw.f16))
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (4096, 4096, 14336)], ids=["config1", "config2"])
def test_gemm256_full_size(ee, orc, M, K, N):
    """Configs 1 and 2 at full size through the production epilogue (no int32
    debug output): INT8 fp16 outputs bit-exact and FP8 within 1e-2 of float64 on
    sampled rows against the oracle; all outputs bit-identical to the 128-tile
    kernels.  The automatic choice picks the 256 x 256-tile kernel at these shapes."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, 21 + N)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    o_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
    o_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
    rows = np.array([0, 1, 255, 256, 257, 1000, 2047, 2048, 3333, 4095])
    ref = orc.epilogue_i8(orc.gemm_i8_acc(codes[rows], B), a_s[rows], bs)
    assert np.array_equal(o_i8[rows].view(np.uint16), ref.view(np.uint16))
    check_close_f64(o_f8[rows], orc.gemm_f8_f64(c8[rows], B, s8[rows], bs))
    with _Options(gemm_tile=128):
        r_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        r_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
    assert np.array_equal(o_i8.view(np.uint16), r_i8.view(np.uint16))
    assert np.array_equal(o_f8.view(np.uint16), r_f8.view(np.uint16))


def test_gemm256_fp8_config1_per_tensor(ee, orc):
    """Config 1's FP8 leg (per-tensor e4m3 scales of A with 0.1% outliers of 20,
    and of the weights): the 256-tile kernel within 1e-2 of float64 on sampled
    rows and bit-identical to the 128-tile kernel."""
    M = K = N = 4096
    rng = np.random.default_rng(5)
    A = rng.standard_normal((M, K)).astype(np.float16)
    pos = rng.choice(M * K, M * K // 1000, replace=False)
    A.reshape(-1)[pos] = (20.0 * rng.choice([-1.0, 1.0], pos.size)).astype(np.float16)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    ca, sa = orc.quant_tensor_f8(A)
    cw, sw = orc.quant_tensor_f8(W)
    out = host(ee.gemm("fp8", cuda(ca), cuda(cw), cuda(sa), cuda(sw)))
    rows = np.array([0, 17, 2048, 4095])
    ref = orc.e4m3_to_f32(ca[rows]).astype(np.float64) @ orc.e4m3_to_f32(cw).astype(np.float64).T
    ref = ref * sa[rows].astype(np.float64)[:, None] * sw.astype(np.float64)[None, :]
    check_close_f64(out[rows], ref)
    with _Options(gemm_tile=128):
        r = host(ee.gemm("fp8", cuda(ca), cuda(cw), cuda(sa), cuda(sw)))
    assert np.array_equal(out.view(np.uint16), r.view(np.uint16))


@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,F,grid", [(4096, 2048, 5632, 0), (600, 256, 640, 0), (512, 256, 1216, 8)])
def test_gemm256_swiglu(ee, orc, M, K, F, grid, tn):
    """The SwiGLU epilogue of the 256-tile kernels gives the bits of the 128-tile
    SwiGLU kernels (every tier; FP16 on the loader-wave order).  The forced grid
    of 8 leaves the last round half full: 256 x 128 halves."""
    rng = np.random.default_rng(M + F)
    W = (rng.standard_normal((2 * F, K)) / np.sqrt(K)).astype(np.float16)
    codes, scale = ee.quantize_weight_codes(cuda(W))
    pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    ci, si = ee.quantize_activations(x, "dispatcher")
    cf, sf = ee.quantize_activations(x, "fp8")
    for kind, a, b, sa, sb in (("int8", ci, pw.i8, si, pw.scale), ("fp8", cf, pw.f8, sf, pw.scale),
                               ("fp16", x, pw.f16, None, None)):
        with _Options(gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid):
            fused = ee.gemm(kind, a, b, sa, sb, swiglu=True)
        with _Options(gemm_tile=128, gemm_variant=1):
            ref = ee.gemm(kind, a, b, sa, sb, swiglu=True)
        assert torch.equal(fused.view(torch.int16), ref.view(torch.int16)), kind


def _sweep_cases(n=24, seed=2024):
    """Seeded shapes and forced grids: ragged M and N, K of 1-12 stages, grids of
    1-37 workgroups (multiples of 8 and not), so that rounds end full, half full
    (256 x 128 halves) or otherwise."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 1300))
        N = int(rng.integers(1, 700)) * 4
        K = int(rng.integers(1, 13)) * 128
        grid = int(rng.choice([1, 2, 3, 5, 7, 8, 13, 16, 24, 37]))
        out.append((M, K, N, grid))
    return out


@pytest.mark.parametrize("M,K,N,grid", _sweep_cases())
def test_gemm256_seeded_sweep(ee, orc, M, K, N, grid):
    """256 x 256-tile kernels on seeded shapes and grids: INT8 int32 accumulators
    equal the oracle's; INT8, FP8 and FP16 outputs equal the 128-tile kernels'
    bit for bit."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 31 + K + N + grid)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    c8, s8 = orc.quant_act_f8(A)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    with _Options(gemm_tile=256, gemm_persist=grid):
        ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs), acc_out=acc)
        o_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        o_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
        o_f16 = host(ee.gemm("fp16", cuda(A), pw.f16))
    assert np.array_equal(host(acc), orc.gemm_i8_acc(codes, B))
    with _Options(gemm_tile=128, gemm_variant=1):
        r_i8 = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        r_f8 = host(ee.gemm("fp8", cuda(c8), pw.f8, cuda(s8), cuda(bs)))
        r_f16 = host(ee.gemm("fp16", cuda(A), pw.f16))
    assert np.array_equal(o_i8.view(np.uint16), r_i8.view(np.uint16))
    assert np.array_equal(o_f8.view(np.uint16), r_f8.view(np.uint16))
    assert np.array_equal(o_f16.view(np.uint16), r_f16.view(np.uint16))


def test_gemm256_option_rejects_bad_value(ee):
    from entropy_engine import _lib
    assert _lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_tile", 192) == _lib.EE_ERR_INVALID_ARG
    assert _lib.lib().ee_engine_set_option(_lib.engine(), b"gemm_tile_n", 64) == _lib.EE_ERR_INVALID_ARG


# ---------------------------------------------------------------------------- routed

@pytest.mark.parametrize("tn", [256, 128])
@pytest.mark.parametrize("M,K,N,H_hi,grid", [(300, 512, 520, 3.0, 0), (700, 1024, 384, 3.0, 8), (700, 256, 264, 3.0, 3),
                                             (129, 256, 128, 10.0, 0), (257, 512, 256, 0.3, 0), (1, 128, 64, 1.0, 0)])
def test_gemm256_routed_equals_per_tier(ee, orc, M, K, N, H_hi, grid, tn):
    """The 256-tile routed grid (three phases per workgroup: FP16, INT8, FP8
    tiles): every row equals the un-routed GEMM of its tier bit for bit, and the
    128-tile routed grid gives the same output.  Entropy ranges make tiers
    empty (H_hi 0.3: INT8 only; 10: mostly FP16)."""
    rng = np.random.default_rng(M * 3 + K + N)
    X = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    H = (rng.random(M) * H_hi).astype(np.float32)
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    with _Options(gemm_tile=256, gemm_tile_n=tn, gemm_persist=grid):
        out = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
    with _Options(gemm_tile=128):
        ref128 = host(ee.routed_linear(x, pw, idx, counts)).view(np.uint16)
    assert np.array_equal(out, ref128)
    t = host(tier)
    full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
            ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
    for k in range(3):
        if (t == k).any():
            assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


@pytest.mark.parametrize("N,sw", [(2048, False), (2560, False), (1024, True)])
def test_gemm256_routed_sparse_fp16_halves(ee, orc, N, sw):
    """Config 4's mix (2.3 / 95.8 / 1.9 % of 4096 rows): one sparse FP16 M-tile per
    column, which the routed grid runs as 256 x 128 halves.  Every row equals the
    128-tile routed grid's and, per tier, the un-routed GEMM of its tier bit for
    bit."""
    M, K = 4096, 512
    rng = np.random.default_rng(N + sw)
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
    with _Options(gemm_tile=128):
        ref128 = host(ee.routed_linear(x, pw, idx, counts, swiglu=sw)).view(np.uint16)
    assert np.array_equal(out, ref128)
    if not sw:
        t = host(tier)
        full = [ee.triton_int8_gemm(x, cuda(B), cuda(bs)), ee.triton_fp8_gemm(x, cuda(B), cuda(bs)),
                ee.triton_fp16_gemm(x, cuda(B), cuda(bs))]
        for k in range(3):
            assert np.array_equal(out[t == k], host(full[k]).view(np.uint16)[t == k]), f"tier {k}"


def test_gemm256_routed_config3(ee, orc):
    """Config 3's routed linear (M = K = N = 4096, 20/40/40 % tiers) takes the
    256-tile routed grid automatically: rows equal the per-tier GEMMs bit for bit,
    INT8 rows equal the oracle on sampled rows, FP8 / FP16 rows within 1e-2."""
    M = K = N = 4096
    rng = np.random.default_rng(3)
    X = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    H = rng.choice(np.array([0.2, 1.0, 3.0], np.float32), M, p=[0.2, 0.4, 0.4])
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    out = host(ee.routed_linear(x, pw, idx, counts))
    t = host(tier)
    for k, fn in enumerate((ee.triton_int8_gemm, ee.triton_fp8_gemm, ee.triton_fp16_gemm)):
        ref = host(fn(x, cuda(B), cuda(bs)))
        assert np.array_equal(out[t == k].view(np.uint16), ref[t == k].view(np.uint16)), f"tier {k}"
    rows = [np.nonzero(t == k)[0][[0, -1]] for k in range(3)]
    assert np.array_equal(out[rows[0]].view(np.uint16), orc.triton_int8_gemm(X[rows[0]], B, bs).view(np.uint16))
    check_close_f64(out[rows[1]], orc.triton_fp8_gemm_f64(X[rows[1]], B, bs))
    check_close_f64(out[rows[2]], orc.triton_fp16_gemm_f64(X[rows[2]], B, bs))


@pytest.mark.parametrize("M,K,F", [(4096, 2048, 1408), (600, 256, 320)])
@pytest.mark.parametrize("tn", [256, 128])
def test_gemm256_routed_swiglu(ee, orc, M, K, F, tn):
    """SwiGLU epilogue of the 256-tile routed grid: the bits of the 128-tile
    routed SwiGLU grid."""
    rng = np.random.default_rng(M + 7 * F)
    W = (rng.standard_normal((2 * F, K)) / np.sqrt(K)).astype(np.float16)
    codes, scale = ee.quantize_weight_codes(cuda(W))
    pw = ee.PackedWeight(ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    h = cuda((rng.random(M) * 3).astype(np.float32))
    _, idx, counts = ee.route(h, 0.41, 1.68)
    with _Options(gemm_tile=256, gemm_tile_n=tn):
        fused = ee.routed_linear(x, pw, idx, counts, swiglu=True)
    with _Options(gemm_tile=128):
        ref = ee.routed_linear(x, pw, idx, counts, swiglu=True)
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))


# (M, K, N): 128-tile routed grids that fit one round of the CUs with every FP16 tile
# split into two 128 x 64 halves (N % 128 of 0, 64, 32, 96, 4: the last half past N
# or partial), and one whose whole-tile grid takes between one and two rounds
# (2048 rows: 4 + 7 + 7 M-tiles x 16)
@pytest.mark.parametrize("M,K,N", [(1024, 512, 2048), (700, 256, 1984), (300, 384, 1056), (129, 128, 96),
                                   (1000, 640, 1540), (2048, 256, 2048)])
def test_routed_fp16_half_tiles(ee, orc, M, K, N):
    """The routed grid's FP16 tiles as 128 x 64 halves: every row equals its
    tier's un-routed GEMM bit for bit (the FP16 one runs whole 128 x 128 tiles),
    and FP16 rows are within 1e-2 of the oracle's float64 recompute."""
    rng = np.random.default_rng(M + N)
    X = rng.standard_normal((M, K)).astype(np.float16)
    B, bs = weights(orc, rng, N, K)
    H = rng.choice(np.array([0.2, 1.0, 3.0], np.float32), M, p=[0.2, 0.4, 0.4])
    pw = ee.prepare_weight(cuda(B), cuda(bs)).materialize()
    x = cuda(X)
    tier, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    with _Options(gemm_tile=128):
        out = host(ee.routed_linear(x, pw, idx, counts))
    t = host(tier)
    assert (t == 2).any()
    for k, fn in enumerate((ee.triton_int8_gemm, ee.triton_fp8_gemm, ee.triton_fp16_gemm)):
        ref = host(fn(x, cuda(B), cuda(bs)))
        assert np.array_equal(out[t == k].view(np.uint16), ref[t == k].view(np.uint16)), f"tier {k}"
    rows = np.nonzero(t == 2)[0][[0, -1]]
    check_close_f64(out[rows], orc.triton_fp16_gemm_f64(X[rows], B, bs))


# (M, K, N, swiglu): the automatic routed grid is 128 x 128 tiles for the first three
# (1-2 rounds of 128-tiles against 1 round of 256-tiles on 256 CUs) and 256 x 256
# tiles for the last two (3+ rounds against 1)
@pytest.mark.parametrize("M,K,N,sw", [(128, 256, 11264, True), (1024, 512, 4096, False), (2048, 384, 2048, False),
                                      (4096, 256, 2048, False), (4096, 256, 2816, True)])
@pytest.mark.parametrize("mix", [(1.0, 0.0, 0.0), (0.2, 0.4, 0.4)])
def test_routed_automatic_tile_choice(ee, orc, M, K, N, sw, mix):
    """The routed linear's automatic tile size (from the rounds of the CUs each
    grid takes) gives the bits of both forced sizes, plain and SwiGLU, with all
    rows INT8 and with a 20/40/40 % tier mix."""
    rng = np.random.default_rng(M + K + N + int(sw))
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float16)
    codes, scale = ee.quantize_weight_codes(cuda(W))
    if sw:
        codes, scale = ee.interleave_gate_up(codes), ee.interleave_gate_up(scale)
    pw = ee.PackedWeight(codes, scale).materialize()
    x = cuda(rng.standard_normal((M, K)).astype(np.float16))
    H = rng.choice(np.array([0.2, 1.0, 3.0], np.float32), M, p=list(mix))
    _, idx, counts = ee.route(cuda(H), 0.41, 1.68)
    outs = []
    for tile in (0, 128, 256):
        with _Options(gemm_tile=tile):
            outs.append(host(ee.routed_linear(x, pw, idx, counts, swiglu=sw)).view(np.uint16))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], outs[2])


# ---------------------------------------------------------------------------- 128-tile pipelines

def _sweep128_cases(n=16, seed=77):
    """Seeded ragged shapes for the 128 x 128-tile pipelines: grids of at most
    one tile per CU (the 8-wave INT8 kernel's automatic range) and K of 1-12
    stages (the 8-wave kernel peels its first stage and its last five)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 700))
        N = int(rng.integers(1, 400)) * 4
        K = int(rng.integers(1, 13)) * 128
        out.append((M, K, N))
    return out


@pytest.mark.parametrize("M,K,N", _sweep128_cases())
def test_gemm128_seeded_sweep(ee, orc, M, K, N):
    """The 128-tile INT8 and FP16 pipelines on seeded shapes: the 8-wave INT8
    kernel (16x16x64 MFMAs) gives the oracle's int32 accumulators and the
    loader-wave kernel's (32x32x32) fp16 outputs bit for bit; FP16 on the
    loader-wave kernel (16x16x32) equals the 256-tile kernel bit for bit and,
    like the 8-wave FP16 kernel (its own split-K f32 order), is within 1e-2 of
    the float64 recompute."""
    A, B, bs, pw = _operands(ee, orc, M, K, N, M * 7 + K + N)
    codes, a_s = orc.quant_act_i8(A, "dispatcher")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    with _Options(gemm_tile=128, gemm_variant=2):
        ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs), acc_out=acc)
        o8w = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        f16w = host(ee.gemm("fp16", cuda(A), pw.f16))
    assert np.array_equal(host(acc), orc.gemm_i8_acc(codes, B))
    with _Options(gemm_tile=128, gemm_variant=1):
        o8l = host(ee.gemm("int8", cuda(codes), pw.i8, cuda(a_s), cuda(bs)))
        f16l = host(ee.gemm("fp16", cuda(A), pw.f16))
    assert np.array_equal(o8w.view(np.uint16), o8l.view(np.uint16))
    with _Options(gemm_tile=256):
        f16g = host(ee.gemm("fp16", cuda(A), pw.f16))
    assert np.array_equal(f16l.view(np.uint16), f16g.view(np.uint16))
    ref = orc.gemm_w8a16_f64(A, B, bs)
    check_close_f64(f16l, ref)
    check_close_f64(f16w, ref)
