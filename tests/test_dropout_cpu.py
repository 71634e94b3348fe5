"""Attention-dropout generator (no GPU).

The kernels draw the keep mask from Philox4x32-10 (megaslide_amd/csrc/
dropout.h); the oracle restates it in numpy (oracle/philox.py).  Both are
pinned here by the generator's published known-answer vectors (Random123,
Salmon et al., SC'11), checked against each other on many counters, and the
keep fraction is checked against 1 - p.
"""

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle.philox import dropout_scale, dropout_threshold, keep_mask, philox4x32_10

ROOT = Path(__file__).resolve().parents[1]

# Random123 kat_vectors, philox4x32_10: counter, key -> 4 output words
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_numpy_philox_known_answers(ctr, key, want):
    got = tuple(int(x) for x in philox4x32_10(*ctr, *key))
    assert got == want


@pytest.fixture(scope="module")
def header_exe(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("dropout") / "dropout_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "megaslide_amd" / "csrc"),
                    str(ROOT / "tests" / "dropout_check.cpp"), "-o", str(exe)], check=True)
    return exe


def _run(exe, lines):
    out = subprocess.run([str(exe)], input="\n".join(lines) + "\n", capture_output=True, text=True,
                         check=True).stdout.split()
    return out


def test_header_philox_known_answers(header_exe):
    lines = [f"p {' '.join(str(c) for c in ctr)} {' '.join(str(k) for k in key)}"
             for ctr, key, _ in KAT]
    got = [int(x) for x in _run(header_exe, lines)]
    assert got == [w[0] for _, _, w in KAT]


def test_header_mask_matches_oracle(header_exe):
    """Factor of every (row, head, tap) from the C header equals the oracle's mask."""
    p, seed, offset = 0.3, 0x123456789ABCDEF, 7
    rows = np.array([0, 1, 977, 65535, 2**32 + 5], dtype=np.int64)
    heads, taps = 3, 147
    keep = keep_mask(p, seed, offset, rows, heads, taps)
    thr, scale = dropout_threshold(p), dropout_scale(p)
    lines = [f"f {thr} {float(scale)!r} {seed & 0xFFFFFFFF} {seed >> 32} {offset} {r} {m} {k}"
             for r in rows for m in range(heads) for k in range(taps)]
    got = np.array([float(x) for x in _run(header_exe, lines)], dtype=np.float32)
    want = np.where(keep.reshape(-1), scale, np.float32(0.0))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_keep_fraction(p):
    rows = np.arange(4096)
    keep = keep_mask(p, 2024, 0, rows, 4, 147)
    n = keep.size
    sigma = np.sqrt(p * (1 - p) / n)
    assert abs(keep.mean() - (1 - p)) < 5 * sigma


def test_masks_differ_by_seed_offset_head_and_row():
    rows = np.arange(256)
    a = keep_mask(0.5, 1, 0, rows, 2, 147)
    assert not np.array_equal(a, keep_mask(0.5, 2, 0, rows, 2, 147))
    assert not np.array_equal(a, keep_mask(0.5, 1, 1, rows, 2, 147))
    assert not np.array_equal(a[:, 0], a[:, 1])
    assert not np.array_equal(a[0], a[1])


def test_threshold_and_scale():
    assert dropout_threshold(0.0) == 0
    assert dropout_threshold(0.5) == 2**31
    assert dropout_scale(0.2) == np.float32(1.0) / np.float32(0.8)
    with pytest.raises(ValueError):
        dropout_threshold(1.0)
