"""Matrix-core depthwise convolution (bf16, kh = kw in {5, 7}, kt in {1, 3}, C a
multiple of 8, W a multiple of 4 up to 256) against PyTorch's conv3d in float64
on the CPU.

The forward and the input gradient (the same kernel with mirrored taps) run
on the matrix cores for these shapes; the weight and bias gradients are
checked too.  The cases cover the band geometries the host picks: 16-row bands
of two x tiles (W = 32), 8-row bands of four (W = 64), partial x tiles (W = 20,
28, 36, 80, 100), a frame shorter than a band (H = 1, 3, 7), one frame (T = 1),
the widest row (W = 256), batches of two, channel counts of 8 to 136 (one to
seventeen 8-channel blocks), and clips long enough (T = 9, 11, 20) to be split
into several runs of frames, each with its own ring of staged input frames;
W = 33 takes the dot2 kernel instead.  The products are exact and summed in fp32, so
the error is the final bf16 rounding: max|y - ref| / max|ref| below 5e-3
(inputs rounded to bf16 before the reference).
"""

import pytest
import torch

from goldens import rel_err
from test_dwconv_gpu import reference

pytestmark = pytest.mark.gpu

TOL = 5e-3

CASES = [
    # B, T, H, W, C, kernel
    (1, 4, 32, 32, 64, (3, 7, 7)),
    (2, 3, 7, 36, 24, (3, 7, 7)),
    (1, 2, 5, 33, 16, (3, 7, 7)),
    (1, 2, 9, 64, 16, (3, 7, 7)),
    (1, 1, 5, 80, 8, (3, 7, 7)),
    (1, 3, 3, 100, 8, (3, 5, 5)),
    (1, 3, 1, 20, 8, (3, 7, 7)),
    (1, 2, 16, 256, 8, (1, 7, 7)),
    (2, 2, 12, 48, 136, (1, 5, 5)),
    (1, 5, 20, 40, 32, (3, 5, 5)),
    (1, 2, 33, 28, 40, (1, 7, 7)),
    (1, 2, 5, 4, 8, (3, 7, 7)),
    (1, 20, 8, 16, 8, (3, 7, 7)),
    (2, 11, 4, 12, 16, (3, 5, 5)),
    (1, 9, 3, 8, 8, (1, 7, 7)),
]


@pytest.mark.parametrize("cfg", CASES)
def test_dwconv_matrix_core_matches_conv3d(cfg):
    from megaslide_amd import dwconv3d
    B, T, H, W, C, ks = cfg
    print(f"[dwconv mfma] B={B} T={T} H={H} W={W} C={C} window={ks}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + T * 100 + H * 10 + W + C)
    x = torch.randn(B, T * H * W, C, generator=g).to(torch.bfloat16)
    w = (torch.randn(C, 1, *ks, generator=g) * 0.2).to(torch.bfloat16)
    b = (torch.randn(C, generator=g) * 0.1).to(torch.bfloat16)
    dy = torch.randn(B, T * H * W, C, generator=g).to(torch.bfloat16)
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    yr = reference(xr, wr, br, (T, H, W), None)
    yr.backward(dy.double())
    xd, wd, bd = (t.to("cuda").requires_grad_(True) for t in (x, w, b))
    y = dwconv3d(xd, wd, bd, (T, H, W), None)
    y.backward(dy.to("cuda"))
    torch.cuda.synchronize()
    for name, a, r, tol in (("y", y.detach(), yr.detach(), TOL), ("dx", xd.grad, xr.grad, TOL),
                            ("dw", wd.grad, wr.grad, 2e-2), ("db", bd.grad, br.grad, 2e-2)):
        e = rel_err(a.double().cpu(), r)
        print(f"  {name}: {e:.2e}", flush=True)
        assert e < tol, name


def test_dwconv_matrix_core_no_bias_and_repeat():
    """No bias, and two calls in a row on different shapes (the band geometry
    and the per-launch row stride change between them)."""
    from megaslide_amd import dwconv3d
    for (B, T, H, W, C) in ((1, 3, 10, 32, 16), (1, 2, 6, 72, 8)):
        g = torch.Generator().manual_seed(W)
        x = torch.randn(B, T * H * W, C, generator=g).to(torch.bfloat16)
        w = (torch.randn(C, 1, 3, 7, 7, generator=g) * 0.2).to(torch.bfloat16)
        yr = reference(x.double(), w.double(), None, (T, H, W), None)
        y = dwconv3d(x.cuda(), w.cuda(), None, (T, H, W), None)
        torch.cuda.synchronize()
        e = rel_err(y.double().cpu(), yr)
        print(f"[dwconv mfma no bias] W={W}: {e:.2e}", flush=True)
        assert e < TOL
