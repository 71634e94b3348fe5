"""Attention dropout in the HIP kernels (GPU).

The kernels drop tap weights with the Philox4x32-10 keep mask that
oracle.philox restates (pinned by the generator's known-answer vectors in
test_dropout_cpu.py).  With the same (p, seed, offset) the oracle applies the
same mask, so forward and every gradient must match it at the usual tolerance
(fp32 1e-4, bf16 2e-2, relative to max|ref|) -- a mask that differed in a
single tap, or a backward that used another mask than its forward, would not.
"""

import pytest
import torch

from goldens import rel_err
from oracle.dsa3d_ref import dsa3d_core_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"


def core():
    from megaslide_amd import dsa3d_core
    return dsa3d_core


@pytest.mark.parametrize("case", [
    # dtype, algo, B, T, H, W, nh, hd, kernel, off_std, p
    (torch.float32, "direct", 1, 3, 5, 6, 2, 32, (3, 7, 7), 1.0, 0.3),
    (torch.float32, "direct", 2, 2, 4, 4, 1, 64, (3, 3, 3), 0.5, 0.6),
    (torch.float32, "tiled", 2, 2, 4, 4, 1, 64, (3, 3, 3), 0.5, 0.6),
    (torch.float32, "tiled", 1, 3, 6, 10, 1, 96, (3, 5, 5), 2.0, 0.3),
    (torch.bfloat16, "tiled", 1, 3, 7, 9, 2, 64, (3, 7, 7), 0.5, 0.2),
    (torch.bfloat16, "tiled", 1, 2, 8, 8, 1, 128, (3, 7, 7), 1.0, 0.5),
    (torch.bfloat16, "tiled", 1, 3, 6, 10, 1, 96, (3, 5, 5), 2.0, 0.1),
])
def test_dropout_matches_oracle(case):
    dt, algo, B, T, H, W, nh, hd, ks, off_std, p = case
    print(f"[dropout] {case}", flush=True)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    N, D = T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator().manual_seed(55 + N + hd)
    q, k, v, dout = (torch.randn(B, N, D, generator=g).to(dt) for _ in range(4))
    off = (torch.randn(B, N, C, generator=g) * off_std).to(dt)
    seed, offset = 0x5EED0000 + N, 3
    qq, kk, vv, oo = (t.float().clone().requires_grad_(True) for t in (q, k, v, off))
    ref = dsa3d_core_ref(qq, kk, vv, oo, (T, H, W), nh, ks, 1.0, dropout=(p, seed, offset))
    ref.backward(dout.float())
    ts = [t.detach().to(DEV).requires_grad_(True) for t in (q, k, v, off)]
    out = core()(*ts, (T, H, W), nh, ks, 1.0, algo=algo, dropout_p=p, dropout_seed=seed,
                 dropout_offset=offset)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    errs = {"out": rel_err(out.detach().float().cpu(), ref.detach())}
    for name, t, r in zip(("dq", "dk", "dv", "doff"), ts, (qq, kk, vv, oo)):
        errs[name] = rel_err(t.grad.float().cpu(), r.grad)
    print("  " + "  ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        assert e < tol, name


@pytest.mark.parametrize("case", [
    # dtype, T, H, W, nh, hd, kernel, q scale, offsets, p
    # one tap per query: a kept tap carries p f = 1/(1-p) = 2.5 on one voxel
    (torch.float32, 3, 8, 8, 2, 64, (1, 1, 1), 1.0, "zero", 0.6),
    (torch.bfloat16, 3, 8, 8, 2, 64, (1, 1, 1), 1.0, "zero", 0.6),
    # peaked softmax (q x 8): most of a query's mass on one tap, factor 4
    (torch.float32, 3, 7, 9, 2, 64, (3, 7, 7), 8.0, "normal", 0.75),
    (torch.bfloat16, 3, 7, 9, 2, 64, (3, 7, 7), 8.0, "normal", 0.75),
    (torch.bfloat16, 2, 6, 8, 1, 128, (3, 7, 7), 8.0, "normal", 0.75),
    # +-50-voxel offsets: the border clamp piles taps onto the volume's edge voxels
    (torch.float32, 2, 6, 7, 2, 64, (3, 7, 7), 1.0, "clamp50", 0.6),
    (torch.bfloat16, 2, 6, 7, 2, 96, (3, 7, 7), 1.0, "clamp50", 0.6),
])
def test_dropout_large_kept_weights_match_oracle(case):
    """Kept weights scaled by 1/(1-p) can put more than a query's whole
    softmax mass on one voxel; the fixed-point scatter tables must still hold
    them.  Tiled kernels against the oracle with the same keep mask."""
    dt, T, H, W, nh, hd, ks, qscale, off_mode, p = case
    print(f"[dropout large] {case}", flush=True)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    B, N, D = 1, T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator().manual_seed(71 + N + hd)
    q = (torch.randn(B, N, D, generator=g) * qscale).to(dt)
    k, v, dout = (torch.randn(B, N, D, generator=g).to(dt) for _ in range(3))
    if off_mode == "zero":
        off = torch.zeros(B, N, C)
    elif off_mode == "normal":
        off = torch.randn(B, N, C, generator=g) * 0.5
    else:
        off = torch.sign(torch.randn(B, N, C, generator=g)) * 50.0
    off = off.to(dt)
    seed, offset = 0x0D1E0000 + N, 5
    qq, kk, vv, oo = (t.float().clone().requires_grad_(True) for t in (q, k, v, off))
    ref = dsa3d_core_ref(qq, kk, vv, oo, (T, H, W), nh, ks, 1.0, dropout=(p, seed, offset))
    ref.backward(dout.float())
    ts = [t.detach().to(DEV).requires_grad_(True) for t in (q, k, v, off)]
    out = core()(*ts, (T, H, W), nh, ks, 1.0, algo="tiled", dropout_p=p, dropout_seed=seed,
                 dropout_offset=offset)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    errs = {"out": rel_err(out.detach().float().cpu(), ref.detach())}
    # With one tap per query ds = p (f dp - dO.O) is zero up to the rounding of
    # two products of size |f dp| (~20 here), so dq and dk are fp32 noise: they
    # are measured against the scale of the gradient that does not vanish (dv).
    single = ks == (1, 1, 1)
    dv_scale = float(vv.grad.abs().max())
    for name, t, r in zip(("dq", "dk", "dv", "doff"), ts, (qq, kk, vv, oo)):
        floor = dv_scale if single and name in ("dq", "dk") else 1e-2
        errs[name] = rel_err(t.grad.float().cpu(), r.grad, floor=floor)
    print("  " + "  ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        assert e < tol, name


@pytest.mark.parametrize("algo,dt", [("direct", torch.float32), ("tiled", torch.float32),
                                     ("tiled", torch.bfloat16)])
def test_dropout_zero_and_determinism(algo, dt):
    B, T, H, W, nh, hd, ks = 1, 3, 8, 8, 2, 64, (3, 7, 7)
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(B, N, D, generator=g).to(dt).to(DEV) for _ in range(3))
    off = (torch.randn(B, N, C, generator=g) * 0.7).to(dt).to(DEV)
    f = core()
    with torch.no_grad():
        base = f(q, k, v, off, (T, H, W), nh, ks, algo=algo)
        zero = f(q, k, v, off, (T, H, W), nh, ks, algo=algo, dropout_p=0.0, dropout_seed=99)
        a1 = f(q, k, v, off, (T, H, W), nh, ks, algo=algo, dropout_p=0.4, dropout_seed=99)
        a2 = f(q, k, v, off, (T, H, W), nh, ks, algo=algo, dropout_p=0.4, dropout_seed=99)
        b1 = f(q, k, v, off, (T, H, W), nh, ks, algo=algo, dropout_p=0.4, dropout_seed=100)
        c1 = f(q, k, v, off, (T, H, W), nh, ks, algo=algo, dropout_p=0.4, dropout_seed=99,
               dropout_offset=1)
    torch.cuda.synchronize()
    assert torch.equal(base, zero)
    assert torch.equal(a1, a2)
    assert not torch.equal(a1, b1)
    assert not torch.equal(a1, c1)


def test_module_dropout_train_and_eval():
    from megaslide_amd import DeformableSlideAttention3D
    torch.manual_seed(0)
    B, T, H, W, D, nh = 1, 3, 6, 7, 128, 2
    m = DeformableSlideAttention3D(D, nh, dropout=0.5).to(DEV)
    with torch.no_grad():  # non-zero offsets
        m.offset_net[2].weight.normal_(0, 0.02)
    x = torch.randn(B, T * H * W, D, device=DEV)
    m.eval()
    with torch.no_grad():
        y_eval = m(x, (T, H, W))
        m.dropout.p = 0.0
        y_nodrop = m(x, (T, H, W))
        m.dropout.p = 0.5
    assert torch.equal(y_eval, y_nodrop)
    m.train()
    torch.manual_seed(1)
    y1 = m(x, (T, H, W))
    torch.manual_seed(1)
    y2 = m(x, (T, H, W))
    y3 = m(x, (T, H, W))
    assert torch.equal(y1, y2)  # the mask follows torch's generator
    assert not torch.equal(y1, y3)
    assert not torch.equal(y1, y_eval)
    y1.square().mean().backward()
    for name, prm in m.named_parameters():
        assert prm.grad is not None and torch.isfinite(prm.grad).all(), name


def test_module_dropout_with_extra_kv():
    """extra_kv path: local taps dropped in the kernel, extra keys by torch's
    dropout; p = 0 in training mode equals eval mode, and p > 0 trains."""
    from megaslide_amd import DeformableSlideAttention3D
    torch.manual_seed(3)
    B, T, H, W, D, nh, G = 1, 3, 5, 6, 128, 2, 8
    m = DeformableSlideAttention3D(D, nh, dropout=0.0).to(DEV)
    with torch.no_grad():
        m.offset_net[2].weight.normal_(0, 0.02)
    x = torch.randn(B, T * H * W, D, device=DEV)
    ekv = torch.randn(B, G, D, device=DEV)
    m.eval()
    with torch.no_grad():
        y_eval = m(x, (T, H, W), extra_kv=ekv)
    m.train()
    with torch.no_grad():
        y_train0 = m(x, (T, H, W), extra_kv=ekv)
    assert torch.equal(y_eval, y_train0)
    m.dropout.p = 0.3
    xg = x.clone().requires_grad_(True)
    eg = ekv.clone().requires_grad_(True)
    y = m(xg, (T, H, W), extra_kv=eg)
    assert not torch.equal(y.detach(), y_eval)
    y.square().mean().backward()
    assert torch.isfinite(xg.grad).all() and torch.isfinite(eg.grad).all()
    for name, prm in m.named_parameters():
        assert prm.grad is not None and torch.isfinite(prm.grad).all(), name
