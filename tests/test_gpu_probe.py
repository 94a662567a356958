"""The hardware probes (probe.hip, ee_probe) that bench.py reports beside the
kernels: each runs and reads a rate in a plausible range for gfx950 (the
ranges are wide: the probes measure the box, they are not pinned values), and
bad arguments are rejected before any launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ee():
    import entropy_engine
    return entropy_engine


@pytest.mark.parametrize("kind,lo,hi", [("stream", 8.0, 128.0), ("stream_own", 2.0, 128.0), ("lds", 32.0, 257.0),
                                        ("mfma_i8", 16.0, 128.0), ("mfma_f8", 32.0, 256.0)])
def test_probe_rates_in_range(ee, kind, lo, hi):
    r = ee.probe(kind, iters=256)
    assert lo < r["value"] < hi, r
    assert 300 < r["sclk_mhz"] < 3500, r


@pytest.mark.parametrize("kind", ["frag_i8_32x32", "frag_i8_16x16", "frag_f16_32x32", "frag_f16_16x16"])
def test_probe_fragment_loops(ee, kind):
    # 8 MFMAs of 32 clocks (or 16 of 16) per wave and iteration, two waves per
    # SIMD: at least 512 clocks per iteration, and not far above
    r = ee.probe(kind, iters=512)
    assert 500 < r["value"] < 4000, r
    assert 300 < r["sclk_mhz"] < 3500, r


def test_probe_on_few_workgroups(ee):
    r = ee.probe("stream", iters=64, grid=3, window=65536)
    assert r["grid"] == 3 and r["value"] > 0


def test_probe_rejects_bad_arguments(ee):
    from entropy_engine import _lib
    L, E = _lib.lib(), _lib.engine()
    times = torch.zeros(16, dtype=torch.int64, device="cuda")
    sink = torch.zeros(4 * 512, dtype=torch.int32, device="cuda")
    src = torch.zeros(8 * 32768, dtype=torch.uint8, device="cuda")
    P = lambda t: t.data_ptr()
    assert L.ee_probe(E, 9, None, 0, 1, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG       # kind
    assert L.ee_probe(E, 5, None, 1 << 20, 1, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG # no src
    assert L.ee_probe(E, 6, P(src), 65536, 1, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG # src < 1 MiB
    assert L.ee_probe(E, 4, None, 32768, 1, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG   # no src
    assert L.ee_probe(E, 0, None, 32768, 1, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG   # no src
    assert L.ee_probe(E, 0, P(src), 1000, 1, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG  # window
    assert L.ee_probe(E, 2, None, 0, 0, 1, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG       # iters
    assert L.ee_probe(E, 2, None, 0, 1, 0, P(times), P(sink), None) == _lib.EE_ERR_INVALID_ARG       # grid
    with pytest.raises(ValueError):
        ee.probe("tlb")
