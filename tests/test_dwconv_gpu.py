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
    (1, 2, 8, 64, 64, (3, 7, 7), None),     # the large-block row width: the dot2 weight gradient
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


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("cfg", [(2, 3, 5, 20, 130, (3, 3, 3)), (1, 4, 9, 32, 64, (3, 3, 3)),
                                 (1, 5, 4, 7, 40, (5, 3, 1))])
def test_gelu_preact_kept_or_recomputed(cfg, dtype, tol):
    """The GELU form through the C ABI: the forward's optional pre-activation
    output equals the convolution before GELU, and the backward gives the same
    gradients from it as from recomputing it (preact NULL)."""
    import ctypes
    from megaslide_amd import _lib
    B, T, H, W, C, ks = cfg
    N = T * H * W
    print(f"[dwconv gelu preact] {cfg} {dtype}", flush=True)
    g = torch.Generator().manual_seed(3 * C + W)
    x = torch.randn(B, N, C, generator=g).to(dtype)
    w = (torch.randn(C, 1, *ks, generator=g) * 0.2).to(dtype)
    b = (torch.randn(C, generator=g) * 0.1).to(dtype)
    dy = torch.randn(B, N, C, generator=g).to(dtype)
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    zr = reference(xr, wr, br, (T, H, W), None)
    F.gelu(zr).backward(dy.double())
    lib = _lib.load()
    desc = _lib.ConvDesc(B, T, H, W, C, *ks, _lib.dtype_code(dtype), 1)
    xd, wd, bd, dyd = (t.to(DEV).contiguous() for t in (x, w.reshape(C, -1), b, dy))
    y, z = torch.empty_like(xd), torch.empty_like(xd)
    sh = torch.cuda.current_stream().cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731
    assert lib.msd_dwconv3d_fwd(ctypes.byref(desc), P(xd), P(wd), P(bd), P(y), P(z), sh) == 0
    nbytes = lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(desc))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    grads = {}
    for name, pre in (("kept", P(z)), ("recomputed", None)):
        dx, dw, db = torch.empty_like(xd), torch.empty_like(wd), torch.empty_like(bd)
        assert lib.msd_dwconv3d_bwd(ctypes.byref(desc), P(xd), P(wd), P(bd), pre, P(dyd), P(dx),
                                    P(dw), P(db), P(ws), nbytes, sh) == 0
        grads[name] = (dx, dw, db)
    torch.cuda.synchronize()
    assert rel_err(z.double().cpu(), zr.detach()) < tol
    assert rel_err(y.double().cpu(), F.gelu(zr).detach()) < tol
    for name, (dx, dw, db) in grads.items():
        assert rel_err(dx.double().cpu(), xr.grad) < tol, name
        assert rel_err(dw.double().cpu().reshape(wr.shape), wr.grad) < tol, name
        assert rel_err(db.double().cpu(), br.grad) < tol, name


def _saved_preacts(t):
    """The GELU input each depthwise-conv node of t's graph saved (None where
    it saved none), for the nodes with act = "gelu"."""
    seen, stack, found = set(), [t.grad_fn], []
    while stack:
        fn = stack.pop()
        if fn is None or fn in seen:
            continue
        seen.add(fn)
        if type(fn).__name__ == "DwConv3dFunctionBackward" and getattr(fn, "act", None) == "gelu":
            found.append(fn.saved_tensors[3])
        stack.extend(f for f, _ in fn.next_functions)
    return found


def test_module_keeps_gelu_input_for_backward():
    """Inside the module (autograd runs a Function's forward with gradients
    disabled) the offset predictor's conv still keeps the GELU input when a
    gradient will be taken, and keeps nothing under no_grad."""
    from megaslide_amd import DeformableSlideAttention3D

    print("[module GELU input kept]", flush=True)
    m = DeformableSlideAttention3D(128, 2).to(DEV)
    x = torch.randn(1, 2 * 4 * 5, 128, device=DEV, requires_grad=True)
    y = m(x, (2, 4, 5))
    z = _saved_preacts(y)
    assert len(z) == 1 and z[0] is not None and z[0].shape == x.shape
    y.sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    with torch.no_grad():
        assert m(x, (2, 4, 5)).grad_fn is None
    # parameters needing a gradient suffice (input without one)
    x2 = torch.randn(1, 2 * 4 * 5, 128, device=DEV)
    z2 = _saved_preacts(m(x2, (2, 4, 5)))
    assert len(z2) == 1 and z2[0] is not None
