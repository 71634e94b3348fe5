"""dK / dV accumulation of the tiled backward for bf16 storage (GPU).

Workgroups add their dK / dV partials across query tiles in one of two ways,
chosen by the descriptor's dkv_accum:

- "fp32" (the default, the reference's precision): fp32 atomics into fp32 rows,
  rounded to bf16 once at the end;
- "fp16": fp16 rows scaled by a power of two per call (bounded from max|q|,
  max|dO|, the head-row L2 norms of dO and V and max|dlse|), with packed
  two-channel atomics; a sum that leaves the fp16 range becomes infinite, the
  conversion to bf16 flags it, and dK / dV are redone with fp32 atomics.

These tests drive both: gradients of widely different magnitudes against the
oracle (the fp16 scale adapts, the tolerance is relative), an engineered
pile-up whose fp16 sum overflows (the redo, and the fp32 path, must give the
exact closed-form value), a pile-up that takes the fp16 sums near the top of
their range without overflowing, a mixed pile-up against the direct kernels
(which accumulate in fp32), and outlier rows judged against the oracle per
head row, where a max-normalised error cannot see precision lost on the small
entries.
"""

import pytest
import torch

from goldens import rel_err
from oracle.dsa3d_ref import dsa3d_core_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16_TOL = 2e-2
ACCUMS = ("fp32", "fp16")


def core():
    from megaslide_amd import dsa3d_core
    return dsa3d_core


def row_err(a, b):
    """Per row of the last dimension: ||a - b|| / (||b|| + 5e-2 median ||b||);
    returns (99th percentile, max)."""
    a = a.double().reshape(-1, a.shape[-1])
    b = b.double().reshape(-1, b.shape[-1])
    nb = b.norm(dim=1)
    e = (a - b).norm(dim=1) / (nb + 5e-2 * nb.median().clamp_min(1e-30))
    return float(torch.quantile(e, 0.99)), float(e.max())


@pytest.mark.parametrize("accum", ACCUMS)
@pytest.mark.parametrize("dout_scale", [1e-6, 1.0, 3e3])
def test_gradient_magnitudes_match_oracle(dout_scale, accum):
    """dK / dV (and the rest) at bf16 tolerance whatever the gradients'
    magnitude: the fp16 scale is a power of two chosen per call."""
    B, T, H, W, nh, hd = 1, 3, 8, 9, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    print(f"[{accum} accumulation] dout x {dout_scale}", flush=True)
    g = torch.Generator().manual_seed(17)
    q, k, v = (torch.randn(B, N, D, generator=g).to(torch.bfloat16) for _ in range(3))
    dout = (torch.randn(B, N, D, generator=g) * dout_scale).to(torch.bfloat16)
    off = (torch.randn(B, N, C, generator=g) * 1.5).to(torch.bfloat16)
    ref_in = [t.float().clone().requires_grad_(True) for t in (q, k, v, off)]
    ref = dsa3d_core_ref(*ref_in, (T, H, W), nh, (3, 7, 7), 1.0)
    ref.backward(dout.float())
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
    out = core()(*ts, (T, H, W), nh, (3, 7, 7), 1.0, algo="tiled", dkv_accum=accum)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    for name, t, r in zip(("dq", "dk", "dv", "doff"), ts, ref_in):
        e = rel_err(t.grad.float().cpu(), r.grad, floor=1e-2)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < BF16_TOL, name


@pytest.mark.parametrize("accum", ACCUMS)
@pytest.mark.parametrize("hd", [64, 96, 128])
def test_overflowing_pile_up_is_exact(hd, accum):
    """Every tap of 8,192 queries clamps onto the volume's far corner (offsets
    +1000 voxels on every axis): each query's softmax weights sum to 1 on that
    one voxel, so dV[corner] = sum_q dO_q = 8,192 with dO = 1, and dV is zero
    elsewhere.  fp32 accumulation adds it exactly; at the fp16 accumulator's
    scale the sum is far beyond the fp16 range, so there the result must come
    from the fp32 redo, exact and finite (head_dim 96: one 96-channel window;
    128: two 64-channel windows)."""
    B, T, H, W, nh = 1, 8, 32, 32, 2
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    print(f"[{accum}: 8192 queries on one voxel] head_dim {hd}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(3)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV).to(torch.bfloat16).requires_grad_(True)
               for _ in range(3))
    off = torch.full((B, N, C), 1000.0, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    out = core()(q, k, v, off, (T, H, W), nh, (3, 7, 7), 1.0, algo="tiled", dkv_accum=accum)
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    dv = v.grad.float()
    assert torch.isfinite(dv).all() and torch.isfinite(k.grad.float()).all()
    assert torch.equal(dv[0, N - 1], torch.full((D,), float(N), device=DEV))
    assert dv[0, : N - 1].abs().max().item() == 0.0
    # every query reads the corner row of V
    assert rel_err(out.detach().float().cpu(), v.detach().float()[:, N - 1:].expand(B, N, D).cpu()) < 1e-2


def test_fp16_sums_near_the_top_of_their_range():
    """3,000 of 4,096 queries clamp every tap onto the far corner with dO =
    1 +- 0.1 (same sign), the rest sample normally.  The fp16 scale puts the
    largest dO at 8-16 scaled units, so the corner's dV sum lands between
    ~24,000 and ~48,000 of fp16's 65,504 (ulp 16-32) without overflowing: no
    redo runs, and every gradient must still match the oracle at bf16
    tolerance."""
    B, T, H, W, nh, hd = 1, 4, 32, 32, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    npile = 3000
    print(f"[fp16 near the top] {npile} queries on one voxel", flush=True)
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(B, N, D, generator=g).to(torch.bfloat16) for _ in range(3))
    off = torch.randn(B, N, C, generator=g) * 0.7
    off[:, :npile] = 1000.0
    off = off.to(torch.bfloat16)
    dout = (1.0 + 0.1 * torch.randn(B, N, D, generator=g)).to(torch.bfloat16)
    ref_in = [t.float().clone().requires_grad_(True) for t in (q, k, v, off)]
    ref = dsa3d_core_ref(*ref_in, (T, H, W), nh, (3, 7, 7), 1.0, head_chunk=1)
    ref.backward(dout.float())
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
    out = core()(*ts, (T, H, W), nh, (3, 7, 7), 1.0, algo="tiled", dkv_accum="fp16")
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    corner = float(ref_in[2].grad[0, N - 1].abs().max())
    assert 2000.0 < corner < 4200.0, corner  # the pile-up is where the test says
    for name, t, r in zip(("dq", "dk", "dv", "doff"), ts, ref_in):
        a = t.grad.float().cpu()
        assert torch.isfinite(a).all(), name
        e = rel_err(a, r.grad, floor=1e-2)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < BF16_TOL, name
    # the corner row itself, elementwise
    e = rel_err(ts[2].grad.float().cpu()[0, N - 1], ref_in[2].grad[0, N - 1])
    print(f"  dv[corner] {e:.2e}", flush=True)
    assert e < BF16_TOL


@pytest.mark.parametrize("accum", ACCUMS)
def test_mixed_pile_up_matches_direct_kernels(accum):
    """Three quarters of 16,384 queries pile onto the far corner with dO ~ 1 +-
    0.1 (about 12,288 on one voxel: an fp16 overflow at the accumulator's
    scale, so the fp32 redo runs), the rest sample normally: every gradient
    equals the direct kernels' (fp32 accumulation) at bf16 tolerance."""
    B, T, H, W, nh, hd = 1, 16, 32, 32, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    print(f"[{accum}, mixed pile-up] tiled vs direct", flush=True)
    g = torch.Generator(device=DEV).manual_seed(8)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
    off = torch.randn(B, N, C, generator=g, device=DEV) * 0.7
    off[:, : 3 * N // 4] = 1000.0
    off = off.to(torch.bfloat16)
    dout = (1.0 + 0.1 * torch.randn(B, N, D, generator=g, device=DEV)).to(torch.bfloat16)
    grads = {}
    for algo in ("tiled", "direct"):
        ts = [t.clone().requires_grad_(True) for t in (q, k, v, off)]
        out = core()(*ts, (T, H, W), nh, (3, 7, 7), 1.0, algo=algo, dkv_accum=accum)
        out.backward(dout)
        grads[algo] = [t.grad.float().cpu() for t in ts]
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "doff"), grads["tiled"], grads["direct"]):
        assert torch.isfinite(a).all(), name
        e = rel_err(a, b, floor=1e-2)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < BF16_TOL, name


@pytest.mark.parametrize("which", ["q", "v", "dout"])
def test_outlier_rows_per_voxel_row(which):
    """Gaussian inputs with three token rows of q, V or dO scaled by 50: the
    fp16 scale follows the largest magnitudes, so ordinary voxels' partial
    sums move toward fp16's subnormal range, and a x50 q row makes its query's
    softmax nearly one-hot, so its ds are small differences that its large q
    then carries into dK.  dq, dK and dV of the tiled kernels (both
    accumulations) against the oracle in fp32 on the same bf16 inputs, judged
    per head row (error over the row's own norm, floored at 5% of the median
    row norm), at the 99th percentile and the worst row."""
    B, T, H, W, nh, hd = 1, 8, 24, 24, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator().manual_seed(33)
    q, k, v, dout = (torch.randn(B, N, D, generator=g) for _ in range(4))
    off = torch.randn(B, N, C, generator=g) * 0.5
    rows = torch.tensor([17, N // 2 + 5, N - 40])
    t = {"q": q, "v": v, "dout": dout}[which]
    t[:, rows] *= 50.0
    q, k, v, dout, off = (x.to(torch.bfloat16) for x in (q, k, v, dout, off))
    ref_in = [x.float().clone().requires_grad_(True) for x in (q, k, v, off)]
    ref = dsa3d_core_ref(*ref_in, (T, H, W), nh, (3, 7, 7), 1.0, head_chunk=1)
    ref.backward(dout.float())
    for accum in ACCUMS:
        print(f"[{accum}, x50 rows of {which}] tiled vs oracle per row", flush=True)
        ts = [x.to(DEV).requires_grad_(True) for x in (q, k, v, off)]
        out = core()(*ts, (T, H, W), nh, (3, 7, 7), 1.0, algo="tiled", dkv_accum=accum)
        out.backward(dout.to(DEV))
        torch.cuda.synchronize()
        for name, i in (("dq", 0), ("dk", 1), ("dv", 2)):
            a = ts[i].grad.float().cpu().view(B, N, nh, hd)
            p99, worst = row_err(a, ref_in[i].grad.view(B, N, nh, hd))
            print(f"  {name} per-row p99 {p99:.2e} worst {worst:.2e}", flush=True)
            assert p99 < 1e-2 and worst < 5e-2, (accum, name)
