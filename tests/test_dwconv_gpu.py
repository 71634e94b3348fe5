"""Depthwise 3-D conv kernels vs PyTorch's conv3d (float64 on the CPU).

Covers the register-tiled row kernels (kw in {3, 5, 7}), the simple kernels
(other odd sizes), the GELU epilogue and its backward, W not a multiple of the
16-output run, channel counts not a multiple of 64, and the bf16 matrix-core
weight gradient (kw >= 5, channels a multiple of 8, bands of at least 4 rows;
one or several 32-wide row segments, ragged row bands).  Tolerances: 1e-4
(fp32), 2e-2 (bf16, inputs rounded to bf16 before the reference).
"""

import pytest
import torch
import torch.nn.functional as F

from goldens import rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"


def reference(x, w, b, vs, act):
    B, N, C = x.shape
    T, H, W = vs
    kt, kh, kw = w.shape[-3:]
    y = F.conv3d(x.transpose(1, 2).reshape(B, C, T, H, W), w, b,
                 padding=(kt // 2, kh // 2, kw // 2), groups=C)
    if act == "gelu":
        y = F.gelu(y)
    return y.reshape(B, C, N).transpose(1, 2)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("cfg", [
    # B, T, H, W, C, kernel, act
    (1, 4, 6, 37, 96, (3, 7, 7), None),
    (2, 3, 5, 20, 130, (3, 3, 3), "gelu"),
    (1, 2, 9, 16, 64, (1, 5, 5), None),
    (1, 5, 4, 7, 40, (5, 3, 1), "gelu"),    # kw = 1: simple kernels
    (1, 3, 3, 3, 8, (3, 7, 7), None),       # window larger than the grid
    (1, 3, 9, 80, 64, (3, 7, 7), None),     # W = 80: the dot2 weight gradient
    (2, 4, 7, 45, 48, (3, 3, 3), "gelu"),
    (1, 2, 6, 70, 16, (3, 5, 5), "gelu"),   # W = 70, kw = 5: dot2 (bands would be 2 rows)
    (1, 4, 6, 48, 16, (3, 5, 5), "gelu"),   # kw = 5 on the matrix cores: 2 segments, bands 4 + 2
    (1, 4, 9, 32, 64, (3, 7, 7), None),     # the long-clip row width on the matrix cores: bands 4+4+1
    (2, 1, 9, 50, 32, (1, 5, 5), None),     # kt = 1 on the matrix cores: 2 segments, bands 8 + 1
])
def test_dwconv_matches_conv3d(cfg, dtype, tol):
    from megaslide_amd import dwconv3d
    B, T, H, W, C, ks, act = cfg
    print(f"[dwconv] {cfg} {dtype}", flush=True)
    g = torch.Generator().manual_seed(C + W)
    x = torch.randn(B, T * H * W, C, generator=g).to(dtype)
    w = (torch.randn(C, 1, *ks, generator=g) * 0.2).to(dtype)
    b = (torch.randn(C, generator=g) * 0.1).to(dtype)
    dy = torch.randn(B, T * H * W, C, generator=g).to(dtype)
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    yr = reference(xr, wr, br, (T, H, W), act)
    yr.backward(dy.double())
    xd, wd, bd = (t.to(DEV).requires_grad_(True) for t in (x, w, b))
    y = dwconv3d(xd, wd, bd, (T, H, W), act)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    assert rel_err(y.detach().double().cpu(), yr.detach()) < tol
    assert rel_err(xd.grad.double().cpu(), xr.grad) < tol
    assert rel_err(wd.grad.double().cpu(), wr.grad) < tol
    assert rel_err(bd.grad.double().cpu(), br.grad) < tol
