"""Load golden fixtures and regenerate their seeded inputs."""

from __future__ import annotations

import json
import os

import numpy as np
import torch

from inputs import C1, CASES, case_params  # noqa: F401  (tests/golden on sys.path)

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name: str):
    z = np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    return meta, {k: z[k] for k in z.files if k != "meta"}


def regenerate(meta):
    """Inputs of a case from its seed, checked against the sums in the fixture."""
    case = next(c for c in list(CASES) + [C1] if c["name"] == meta["name"])
    p, x, gy, off, extra = case_params(case)
    assert abs(float(x.sum()) - meta["x_sum"]) < 1e-9
    assert abs(float(gy.sum()) - meta["gy_sum"]) < 1e-9
    for k, v in p.items():
        assert abs(float(v.sum()) - meta["param_sums"][k]) < 1e-9, k
    if off is not None:
        assert abs(float(off.sum()) - meta["off_sum"]) < 1e-6
    if extra is not None:
        assert abs(float(extra.sum()) - meta["extra_sum"]) < 1e-9
    return case, p, x, gy, off, extra


def rel_err(a, b, floor: float = 1e-12) -> float:
    """max|a - b| / max(max|b|, floor): the relative error used by every parity test.

    ``floor`` keeps quantities that are mathematically zero (e.g. dq on a 1x1x1
    grid, where every tap samples the same voxel) from dividing rounding noise
    by ~0.
    """
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    if a.numel() == 0:
        return 0.0
    den = float(b.abs().max())
    return float((a - b).abs().max()) / max(den, floor)
