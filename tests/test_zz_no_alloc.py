"""ee_routed_linear_noalloc: the routed linear on the library's device-resident
workspace, called through the C ABI, against ee_routed_linear with a caller
workspace on the same inputs -- bit for bit in every tier (the same kernels run).
Two calls in a row, the second with a smaller input (fewer rows, other K, other
tier mix), so the second reads nothing the first left behind; sizes past the
workspace are rejected before any launch."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc(ee, x, pw, idx, counts, out):
    from entropy_engine import _lib
    M, K = x.shape
    rc = _lib.lib().ee_routed_linear_noalloc(
        _lib.engine(), x.data_ptr(), x.stride(0), M, K, pw.N, idx.data_ptr(), counts.data_ptr(), pw.i8.data_ptr(),
        pw.f8.data_ptr(), pw.f16.data_ptr(), pw.scale.data_ptr(), out.data_ptr(), out.stride(0),
        _lib.stream_handle())
    return rc


def _case(ee, orc, rng, M, K, N, h_hi):
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    B, bs = orc.quantize_weights_int8(W)
    pw = ee.prepare_weight(torch.from_numpy(B).cuda(), torch.from_numpy(bs).cuda()).materialize()
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda()
    h = torch.from_numpy((rng.random(M) * h_hi).astype(np.float32)).cuda()
    tier, idx, counts = ee.route(h, 0.41, 1.68)
    return x, pw, tier, idx, counts


def test_routed_linear_noalloc_matches_routed_linear():
    import entropy_engine as ee
    import oracle
    from entropy_engine import _lib
    rng = np.random.default_rng(2024)
    for M, K, N, h_hi in ((4096, 4096, 4096, 3.0), (700, 1024, 384, 3.0), (129, 256, 128, 10.0)):
        x, pw, tier, idx, counts = _case(ee, oracle, rng, M, K, N, h_hi)
        ref = ee.routed_linear(x, pw, idx, counts)
        out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
        _lib.check(_noalloc(ee, x, pw, idx, counts, out))
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (M, K, N)
        t = tier.cpu().numpy()
        assert len(set(t.tolist())) >= 2


def test_routed_linear_noalloc_rejects_sizes_past_the_workspace():
    import entropy_engine as ee
    from entropy_engine import _lib
    L = _lib.lib()
    rng = np.random.default_rng(1)
    K, N = 128, 64
    W = torch.from_numpy((rng.standard_normal((N, K)) * 0.02).astype(np.float16)).cuda()
    codes, scale = ee.quantize_weight_codes(W)
    pw = ee.PackedWeight(codes, scale).materialize()
    x = torch.zeros((_lib.EE_NOALLOC_MAX_ROWS + 1, K), dtype=torch.float16, device="cuda")
    idx = torch.zeros(x.shape[0], dtype=torch.int32, device="cuda")
    counts = torch.zeros(3, dtype=torch.int32, device="cuda")
    out = torch.empty((x.shape[0], N), dtype=torch.float16, device="cuda")
    assert _noalloc(ee, x, pw, idx, counts, out) == _lib.EE_ERR_UNSUPPORTED
    assert "at most" in L.ee_last_error().decode()
    big_k = _lib.EE_NOALLOC_MAX_CODE_BYTES // 1024 + 128
    assert L.ee_routed_linear_noalloc(_lib.engine(), x.data_ptr(), big_k, 1024, big_k, N, idx.data_ptr(),
                                      counts.data_ptr(), pw.i8.data_ptr(), pw.f8.data_ptr(), pw.f16.data_ptr(),
                                      pw.scale.data_ptr(), out.data_ptr(), N, None) == _lib.EE_ERR_UNSUPPORTED
