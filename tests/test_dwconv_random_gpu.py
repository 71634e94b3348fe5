"""Depthwise 3-D conv kernels on seeded random shapes vs PyTorch's conv3d
(float64 on the CPU), forward and the x, weight and bias gradients.

Each case draws the window (odd sizes 1-5 deep, 1-7 high and wide), GELU or
none, channel counts on and off multiples of 8 and 64, grids with W on both
sides of the 16-output run and of the matrix-core weight gradient's row
widths, and fp32 or bf16: the kernel choice (register-tiled row kernels,
simple kernels, dot2 or matrix-core weight gradients, GELU epilogues) follows
from the shape.  Tolerances: 1e-4 (fp32), 2e-2 (bf16, inputs rounded to bf16
before the reference).
"""

import random

import pytest
import torch

from goldens import rel_err
from test_dwconv_gpu import reference

pytestmark = pytest.mark.gpu


def draw(seed):
    r = random.Random(30000 + seed)
    dtype, tol = r.choice([(torch.float32, 1e-4), (torch.bfloat16, 2e-2), (torch.bfloat16, 2e-2)])
    ks = (r.choice([1, 3, 5]), r.choice([1, 3, 5, 7]), r.choice([1, 3, 5, 7]))
    act = r.choice([None, "gelu"])
    B = r.choice([1, 2])
    C = r.choice([8, 16, 24, 40, 64, 96, 128, 136, 200, 256])
    T = r.choice([1, 2, 3, 5, 8])
    H = r.choice([1, 2, 4, 7, 9, 16, 23])
    W = r.choice([1, 3, 7, 15, 16, 17, 32, 33, 48, 64, 80, 100])
    while B * T * H * W * C > 3_000_000:
        if W >= max(T, H):
            W = (W + 1) // 2
        elif H >= T:
            H = (H + 1) // 2
        else:
            T = (T + 1) // 2
    return B, T, H, W, C, ks, act, dtype, tol


@pytest.mark.parametrize("seed", range(48))
def test_dwconv_random_shape_matches_conv3d(seed):
    from megaslide_amd import dwconv3d
    B, T, H, W, C, ks, act, dtype, tol = draw(seed)
    print(f"[dwconv random {seed}] B={B} T={T} H={H} W={W} C={C} window={ks} act={act} {dtype}",
          flush=True)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T * H * W, C, generator=g).to(dtype)
    w = (torch.randn(C, 1, *ks, generator=g) * 0.2).to(dtype)
    b = (torch.randn(C, generator=g) * 0.1).to(dtype)
    dy = torch.randn(B, T * H * W, C, generator=g).to(dtype)
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    yr = reference(xr, wr, br, (T, H, W), act)
    yr.backward(dy.double())
    xd, wd, bd = (t.to("cuda").requires_grad_(True) for t in (x, w, b))
    y = dwconv3d(xd, wd, bd, (T, H, W), act)
    y.backward(dy.to("cuda"))
    torch.cuda.synchronize()
    for name, a, r in (("y", y.detach(), yr.detach()), ("dx", xd.grad, xr.grad),
                       ("dw", wd.grad, wr.grad), ("db", bd.grad, br.grad)):
        e = rel_err(a.double().cpu(), r)
        print(f"  {name}: {e:.2e}", flush=True)
        assert e < tol, name
