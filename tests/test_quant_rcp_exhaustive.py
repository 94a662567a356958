"""The INT8 dispatcher quantiser divides by the row scale on the reference
(EE/python/kernels.py:338); the gfx950 kernel multiplies by a biased
reciprocal instead.  tests/rcp_trunc_check.c proves the two give the same code
for every reachable (amax, x) fp16 pair (about 1e9 pairs, ~1 s on 8 cores),
and a deliberately unbiased reciprocal is shown to fail, so the check is not
vacuous."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "rcp_trunc_check.c")


def _build(tmp_path, extra=()):
    exe = tmp_path / "rcp_check"
    src = SRC
    if extra:
        text = open(SRC).read()
        for a, b in extra:
            assert a in text
            text = text.replace(a, b)
        src = tmp_path / "variant.c"
        src.write_text(text)
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-msse2", "-mfpmath=sse",
                    str(src), "-o", str(exe), "-lm"], check=True)
    return exe


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_biased_reciprocal_truncation_is_exact(tmp_path):
    out = subprocess.run([str(_build(tmp_path))], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    assert "mismatches 0" in out.stdout and "pairs 1007713280" in out.stdout


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_unbiased_reciprocal_is_caught(tmp_path):
    exe = _build(tmp_path, [("const float r_up = (one / s) * bias;", "const float r_up = (one / s);")])
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode != 0 and "mismatch" in out.stdout
