"""A non-finite K row reaches only the queries that sample it.

grid_sample with border padding (infinity/video/attention.py:262-268) clamps a
coordinate to [0, S-1] and skips a corner outside the volume, so a tap
clamped onto the last column x = W-1 never reads its upper x corner.  The
tiled forward reads each corner row's two x corners as one paired read of
table entries base and base + 1; for such a clamped tap entry base + 1 is a
different voxel (the next row's first column of the chunk), whose value the
kernel must not use, not even times its zero weight: an inf score there would
otherwise turn the tap's score into NaN for a query that grid_sample keeps
finite.

Volume T=2, H=8, W=16, zero offsets, one K voxel (y=3, x=9) set to +inf in
every frame.  Taps sit on the stretched lattice (w + c) 16/15 - 1/2, so the
queries at w >= 13 never sample x = 9 while w = 12 does; queries at w = 13-15
clamp their right taps onto x = 15, and in the tile of columns 12-15 the
corner box starts at x = 9, so x = 9 of the next row sits right after x = 15
in the table.  The oracle (CPU) pins which queries
stay finite; the kernels (GPU) must match it there.
"""

import pytest
import torch

from goldens import rel_err
from oracle.dsa3d_ref import dsa3d_core_ref

B, T, H, W, NH, HD = 1, 2, 8, 16, 1, 64
N, D, C = T * H * W, NH * HD, NH * 147 * 3
INF_Y, INF_X = 3, 9


def _inputs(dt=torch.float32):
    g = torch.Generator().manual_seed(99)
    q, k, v = (torch.randn(B, N, D, generator=g) for _ in range(3))
    for t in range(T):
        k[0, (t * H + INF_Y) * W + INF_X] = float("inf")
    off = torch.zeros(B, N, C)
    return [x.to(dt) for x in (q, k, v, off)]


def _token(t, y, x):
    return (t * H + y) * W + x


def test_oracle_keeps_queries_that_do_not_sample_the_voxel_finite():
    q, k, v, off = _inputs()
    out = dsa3d_core_ref(q, k, v, off, (T, H, W), NH, (3, 7, 7), 1.0)
    fin = torch.isfinite(out[0]).all(dim=-1).view(T, H, W)
    # the queries at w >= 13 read columns >= 10 only: finite
    assert fin[:, :, 13:].all()
    # a query whose window covers the voxel reads it with nonzero weight: not finite
    assert not fin[0, INF_Y, INF_X]
    assert not fin[:, :, 12].all()


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("algo", ["tiled", "direct"])
def test_kernels_match_oracle_finiteness(algo, dt):
    from megaslide_amd import dsa3d_core

    print(f"[non-finite K row] {algo} {dt}", flush=True)
    q, k, v, off = _inputs(dt)
    ref = dsa3d_core_ref(*(x.float() for x in (q, k, v, off)), (T, H, W), NH, (3, 7, 7), 1.0)
    with torch.no_grad():
        out = dsa3d_core(*(x.cuda() for x in (q, k, v, off)), (T, H, W), NH, (3, 7, 7), 1.0,
                         algo=algo).float().cpu()
    fin_ref = torch.isfinite(ref[0]).all(dim=-1)
    fin = torch.isfinite(out[0]).all(dim=-1)
    assert torch.equal(fin, fin_ref), (fin != fin_ref).nonzero().flatten().tolist()
    tol = 1e-4 if dt == torch.float32 else 2e-2
    assert rel_err(out[0][fin_ref], ref[0][fin_ref]) < tol
