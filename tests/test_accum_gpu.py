"""dK / dV accumulation of the tiled backward for bf16 storage (GPU).

Workgroups add their dK / dV partials into fp16 rows scaled by a power of two
per call (bounded from max|q|, max|dO|, head-row norms of dO and V and
max|dlse|), with packed two-channel atomics; a sum that leaves the fp16 range
becomes infinite, the conversion to bf16 flags it, and dK / dV are redone with
fp32 atomics.  These tests drive both paths: gradients of widely different
magnitudes against the oracle (the scale adapts, the tolerance is relative), an
engineered pile-up whose fp16 sum overflows (the redo must give the exact
closed-form value), and a mixed pile-up against the direct kernels, which
accumulate in fp32.
"""

import pytest
import torch

from goldens import rel_err
from oracle.dsa3d_ref import dsa3d_core_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16_TOL = 2e-2


def core():
    from megaslide_amd import dsa3d_core
    return dsa3d_core


@pytest.mark.parametrize("dout_scale", [1e-6, 1.0, 3e3])
def test_gradient_magnitudes_match_oracle(dout_scale):
    """dK / dV (and the rest) at bf16 tolerance whatever the gradients'
    magnitude: the fp16 scale is a power of two chosen per call."""
    B, T, H, W, nh, hd = 1, 3, 8, 9, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    print(f"[fp16 accumulation] dout x {dout_scale}", flush=True)
    g = torch.Generator().manual_seed(17)
    q, k, v = (torch.randn(B, N, D, generator=g).to(torch.bfloat16) for _ in range(3))
    dout = (torch.randn(B, N, D, generator=g) * dout_scale).to(torch.bfloat16)
    off = (torch.randn(B, N, C, generator=g) * 1.5).to(torch.bfloat16)
    ref_in = [t.float().clone().requires_grad_(True) for t in (q, k, v, off)]
    ref = dsa3d_core_ref(*ref_in, (T, H, W), nh, (3, 7, 7), 1.0)
    ref.backward(dout.float())
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
    out = core()(*ts, (T, H, W), nh, (3, 7, 7), 1.0, algo="tiled")
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    for name, t, r in zip(("dq", "dk", "dv", "doff"), ts, ref_in):
        e = rel_err(t.grad.float().cpu(), r.grad, floor=1e-2)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < BF16_TOL, name


@pytest.mark.parametrize("hd", [64, 96, 128])
def test_overflowing_pile_up_is_redone_in_fp32(hd):
    """Every tap of 8,192 queries clamps onto the volume's far corner (offsets
    +1000 voxels on every axis): each query's softmax weights sum to 1 on that
    one voxel, so dV[corner] = sum_q dO_q = 8,192 with dO = 1, and dV is zero
    elsewhere.  At the accumulator's scale that sum is far beyond the fp16
    range: the result must come from the fp32 redo, exact and finite (head_dim
    96: one 96-channel window; 128: two 64-channel windows)."""
    B, T, H, W, nh = 1, 8, 32, 32, 2
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    print(f"[fp16 overflow -> fp32 redo] 8192 queries on one voxel, head_dim {hd}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(3)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV).to(torch.bfloat16).requires_grad_(True)
               for _ in range(3))
    off = torch.full((B, N, C), 1000.0, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    out = core()(q, k, v, off, (T, H, W), nh, (3, 7, 7), 1.0, algo="tiled")
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    dv = v.grad.float()
    assert torch.isfinite(dv).all() and torch.isfinite(k.grad.float()).all()
    assert torch.equal(dv[0, N - 1], torch.full((D,), float(N), device=DEV))
    assert dv[0, : N - 1].abs().max().item() == 0.0
    # every query reads the corner row of V
    assert rel_err(out.detach().float().cpu(), v.detach().float()[:, N - 1:].expand(B, N, D).cpu()) < 1e-2


def test_mixed_pile_up_matches_direct_kernels():
    """Three quarters of 16,384 queries pile onto the far corner with dO ~ 1 +-
    0.1 (about 12,288 on one voxel: an fp16 overflow at the accumulator's
    scale, so the fp32 redo runs), the rest sample normally: every gradient
    equals the direct kernels' (fp32 accumulation) at bf16 tolerance."""
    B, T, H, W, nh, hd = 1, 16, 32, 32, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    print("[fp16 overflow, mixed] tiled vs direct", flush=True)
    g = torch.Generator(device=DEV).manual_seed(8)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
    off = torch.randn(B, N, C, generator=g, device=DEV) * 0.7
    off[:, : 3 * N // 4] = 1000.0
    off = off.to(torch.bfloat16)
    dout = (1.0 + 0.1 * torch.randn(B, N, D, generator=g, device=DEV)).to(torch.bfloat16)
    grads = {}
    for algo in ("tiled", "direct"):
        ts = [t.clone().requires_grad_(True) for t in (q, k, v, off)]
        out = core()(*ts, (T, H, W), nh, (3, 7, 7), 1.0, algo=algo)
        out.backward(dout)
        grads[algo] = [t.grad.float().cpu() for t in ts]
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "doff"), grads["tiled"], grads["direct"]):
        assert torch.isfinite(a).all(), name
        e = rel_err(a, b, floor=1e-2)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < BF16_TOL, name
