"""Exactness of the tiled kernels' division-free coordinate arithmetic (CPU).

The tiled kernels compute the reference's ``2*(p+c)/(S-1)`` and
``offset/(dim-1)`` with ``msd::div_rn`` (megaslide_amd/csrc/div_rn.h): a
reciprocal multiply plus one fused residual correction.  Corner choice at
lattice points depends on every bit of these quotients (grid_sample's
trilinear gradient is discontinuous there), so the routine must equal IEEE
division exactly.  The same header is compiled here with g++ and swept
against the host's correctly rounded divide:

* every fp32 mantissa against divisors 1..256 plus 64 divisors up to 32766
  (the offset divisors T-1, H-1, W-1);
* every base-grid numerator against every divisor up to 32766.

A wider sweep (divisors 1..4096 plus 600 up to 32766, 3.9e10 cases) was
run the same way during development with zero mismatches.
"""

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("divrn") / "div_rn_check"
    subprocess.run(
        ["g++", "-O2", "-ffp-contract=off", "-std=c++17",
         "-I", str(ROOT / "megaslide_amd" / "csrc"),
         str(ROOT / "tests" / "div_rn_check.cpp"), "-o", str(exe)],
        check=True)
    return exe


def test_div_rn_matches_ieee_division(checker):
    r = subprocess.run([str(checker), "256", "64"], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout


def test_small_integer_division_by_reciprocal():
    """The kernels split a tap index kap = (ci*kh + cj)*kw + ck with
    int((kap + 0.5) * RN(1/d)); exact for every window the tiled path accepts."""
    import numpy as np
    for d in range(1, 161):
        r = np.float32(1.0) / np.float32(d)
        kap = np.arange(0, 1 << 16, dtype=np.int64)
        q = ((kap.astype(np.float32) + np.float32(0.5)) * r).astype(np.int64)
        assert np.array_equal(q, kap // d), d
