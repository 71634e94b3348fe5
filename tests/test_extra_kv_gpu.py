"""Extra keys in the HIP attention core (GPU): the reference's extra_kv
(infinity/video/attention.py:160-173) appends G projected keys and values to
every query's taps before the softmax; HybridAttention3D feeds it G = 128
gated registers (infinity/video/hybrid_attention.py:89-93).

Forward and every gradient -- dq, dk, dv, d offsets and the extra keys' and
values' own -- against the oracle's autograd on the same inputs, at the parity
tolerance (fp32 1e-4, bf16 2e-2, relative to max|ref|), through the tiled and
the direct kernels, with and without dropout (extra key g is tap K + g of the
keep mask).
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


def _run(dt, algo, B, T, H, W, nh, hd, G, ks, off_std, p=0.0, seed=0):
    N, D = T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator().manual_seed(1000 + N + G + hd)
    q, k, v, dout = (torch.randn(B, N, D, generator=g).to(dt) for _ in range(4))
    ek, ev = (torch.randn(B, G, D, generator=g).to(dt) for _ in range(2))
    off = (torch.randn(B, N, C, generator=g) * off_std).to(dt)
    drop = (p, 0xE0E0 + seed, 2) if p > 0 else None
    ref_in = [t.float().clone().requires_grad_(True) for t in (q, k, v, off, ek, ev)]
    ref = dsa3d_core_ref(*ref_in[:4], (T, H, W), nh, ks, 1.0, extra_k=ref_in[4],
                         extra_v=ref_in[5], dropout=drop)
    ref.backward(dout.float())
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off, ek, ev)]
    kw = dict(dropout_p=p, dropout_seed=drop[1], dropout_offset=drop[2]) if drop else {}
    out = core()(*ts[:4], (T, H, W), nh, ks, 1.0, algo=algo, extra_k=ts[4], extra_v=ts[5], **kw)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    errs = {"out": rel_err(out.detach().float().cpu(), ref.detach())}
    for name, t, r in zip(("dq", "dk", "dv", "doff", "dek", "dev"), ts, ref_in):
        errs[name] = rel_err(t.grad.float().cpu(), r.grad, floor=1e-2)
    return errs


@pytest.mark.parametrize("case", [
    # dtype, algo, B, T, H, W, nh, hd, G, kernel, off_std
    (torch.bfloat16, "tiled", 1, 3, 8, 8, 16, 64, 128, (3, 7, 7), 0.5),   # D = 1024, 16 x 64, G = 128
    (torch.float32, "tiled", 2, 3, 5, 6, 2, 64, 20, (3, 7, 7), 1.0),      # G not a multiple of 16
    (torch.float32, "direct", 2, 3, 5, 6, 2, 64, 20, (3, 7, 7), 1.0),
    (torch.bfloat16, "tiled", 1, 2, 6, 7, 2, 128, 40, (3, 7, 7), 1.5),
    (torch.float32, "tiled", 1, 3, 6, 5, 1, 96, 256, (3, 5, 5), 0.7),     # the tiled kernels' largest G
    (torch.bfloat16, "tiled", 1, 3, 5, 6, 2, 32, 7, (3, 7, 7), 0.5),
    (torch.bfloat16, "tiled", 2, 2, 4, 9, 3, 96, 33, (1, 3, 3), 2.0),
    (torch.float32, "auto", 1, 2, 4, 5, 1, 64, 300, (3, 3, 3), 0.5),      # G > 256: direct kernels
])
def test_extra_keys_match_oracle(case):
    dt, algo, B, T, H, W, nh, hd, G, ks, off_std = case
    print(f"[extra keys] {case}", flush=True)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    errs = _run(dt, algo, B, T, H, W, nh, hd, G, ks, off_std)
    print("  " + "  ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        assert e < tol, name


@pytest.mark.parametrize("case", [
    (torch.float32, "tiled", 1, 3, 5, 6, 2, 64, 24, 0.3),
    (torch.bfloat16, "tiled", 1, 3, 6, 6, 2, 64, 64, 0.5),
    (torch.float32, "direct", 1, 3, 5, 6, 2, 64, 24, 0.3),
])
def test_extra_keys_with_dropout_match_oracle(case):
    dt, algo, B, T, H, W, nh, hd, G, p = case
    print(f"[extra keys dropout] {case}", flush=True)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    errs = _run(dt, algo, B, T, H, W, nh, hd, G, (3, 7, 7), 0.8, p=p, seed=G)
    print("  " + "  ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        assert e < tol, name


def test_extra_keys_tiled_equals_direct_fp32():
    """The two kernel families on the same fp32 inputs with extra keys."""
    B, T, H, W, nh, hd, G = 1, 3, 6, 6, 2, 64, 32
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator(device=DEV).manual_seed(77)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV) for _ in range(3))
    ek, ev = (torch.randn(B, G, D, generator=g, device=DEV) for _ in range(2))
    off = torch.randn(B, N, C, generator=g, device=DEV)
    with torch.no_grad():
        a, la = core()(q, k, v, off, (T, H, W), nh, return_lse=True, algo="tiled", extra_k=ek,
                       extra_v=ev)
        b, lb = core()(q, k, v, off, (T, H, W), nh, return_lse=True, algo="direct", extra_k=ek,
                       extra_v=ev)
    torch.cuda.synchronize()
    assert rel_err(a.cpu(), b.cpu()) < 1e-4
    assert rel_err(la.cpu(), lb.cpu()) < 1e-5


@pytest.mark.parametrize("algo", ["tiled", "direct"])
def test_extra_keys_peaked_softmax_delta(algo):
    """With extra keys and a peaked softmax (q x 8), ds = p (dP - Delta) is small
    next to p dP, so Delta must not carry the stored bf16 output's rounding:
    both kernel families sum it in fp32 over the taps and keys, and every
    gradient stays within 8e-3 of the oracle (Delta from dO . O gave dK 1.1e-2)."""
    B, T, H, W, nh, hd, ks, G = 1, 4, 8, 8, 2, 64, (3, 5, 5), 16
    K, N, D = 75, T * H * W, nh * hd
    print(f"[extra keys peaked] {algo}", flush=True)
    g = torch.Generator().manual_seed(7)
    q = (torch.randn(B, N, D, generator=g) * 8.0).to(torch.bfloat16)
    k, v = (torch.randn(B, N, D, generator=g).to(torch.bfloat16) for _ in range(2))
    off = (torch.randn(B, N, nh * K * 3, generator=g) * 0.5).to(torch.bfloat16)
    ek, ev = (torch.randn(B, G, D, generator=g).to(torch.bfloat16) for _ in range(2))
    dout = torch.randn(B, N, D, generator=g).to(torch.bfloat16)
    ins = [q, k, v, off, ek, ev]
    ri = [t.float().clone().requires_grad_(True) for t in ins]
    ref = dsa3d_core_ref(*ri[:4], (T, H, W), nh, ks, 1.0, extra_k=ri[4], extra_v=ri[5])
    ref.backward(dout.float())
    ts = [t.detach().to(DEV).requires_grad_(True) for t in ins]
    out = core()(*ts[:4], (T, H, W), nh, ks, 1.0, algo=algo, extra_k=ts[4], extra_v=ts[5])
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    for name, t, r in zip(("dq", "dk", "dv", "doff", "dek", "dev"), ts, ri):
        e = rel_err(t.grad.float().cpu(), r.grad)
        print(f"  {name}: {e:.2e}", flush=True)
        assert e < 8e-3, name
