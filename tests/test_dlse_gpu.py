"""Gradient through the returned log-sum-exp (GPU).

dsa3d_core(..., return_lse=True) returns each query's log-sum-exp over its
taps and extra keys; a caller that merges further keys outside (the reason
msd_dsa3d_bwd takes dlse) differentiates it.  The backward then uses
ds_k = p_k (dp_k - Delta) with Delta = dO . O - dlse (d lse / d s_k = p_k).

Both outputs are differentiated at once -- loss = sum(out * g_out) +
sum(lse * g_lse) -- and every gradient (dq, dk, dv, d offsets, and the extra
keys' and values') is compared with the oracle's autograd through its own
log-sum-exp of the scores (torch.logsumexp over the same tap and key list), at
the parity tolerance: fp32 1e-4, bf16 2e-2 relative to max|ref|.  Tiled and
direct kernels, fp32 and bf16 (both dK / dV accumulations), with and without
extra keys; one case with dO = 0 isolates the lse path.
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
    # dtype, algo, dkv_accum, G, hd, dout_zero
    (torch.float32, "tiled", "fp32", 0, 64, False),
    (torch.float32, "direct", "fp32", 0, 64, False),
    (torch.float32, "tiled", "fp32", 12, 64, False),
    (torch.float32, "direct", "fp32", 12, 64, False),
    (torch.float32, "tiled", "fp32", 0, 64, True),
    (torch.bfloat16, "tiled", "fp32", 0, 64, False),
    (torch.bfloat16, "tiled", "fp16", 0, 64, False),
    (torch.bfloat16, "direct", "fp32", 0, 64, False),
    (torch.bfloat16, "tiled", "fp32", 20, 64, False),
    (torch.bfloat16, "tiled", "fp16", 20, 96, False),
    (torch.bfloat16, "direct", "fp32", 20, 64, False),
    (torch.bfloat16, "tiled", "fp32", 0, 128, True),
])
def test_lse_gradient_matches_oracle(case):
    dt, algo, accum, G, hd, dout_zero = case
    print(f"[dlse] {case}", flush=True)
    B, T, H, W, nh = 1, 3, 7, 6, 2
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator().manual_seed(500 + G + hd)
    q, k, v = (torch.randn(B, N, D, generator=g).to(dt) for _ in range(3))
    off = (torch.randn(B, N, C, generator=g) * 1.2).to(dt)
    ek, ev = (torch.randn(B, G, D, generator=g).to(dt) for _ in range(2))
    gout = torch.randn(B, N, D, generator=g).to(dt)
    if dout_zero:
        gout.zero_()
    glse = torch.randn(B, N, nh, generator=g)  # d loss / d lse, fp32 like lse

    names = ["q", "k", "v", "off"] + (["ek", "ev"] if G else [])
    src = [q, k, v, off] + ([ek, ev] if G else [])
    ref_in = [t.float().clone().requires_grad_(True) for t in src]
    xk = dict(extra_k=ref_in[4], extra_v=ref_in[5]) if G else {}
    out_r, lse_r = dsa3d_core_ref(*ref_in[:4], (T, H, W), nh, (3, 7, 7), 1.0, return_lse=True, **xk)
    # the gradient of the out term alone, to show that the lse term matters
    dq_out_only = torch.autograd.grad((out_r * gout.float()).sum(), ref_in[0], retain_graph=True)[0]
    loss = (out_r * gout.float()).sum() + (lse_r.transpose(1, 2) * glse).sum()
    loss.backward()
    assert rel_err(dq_out_only, ref_in[0].grad) > 0.1

    ts = [t.to(DEV).requires_grad_(True) for t in src]
    xk = dict(extra_k=ts[4], extra_v=ts[5]) if G else {}
    out, lse = core()(*ts[:4], (T, H, W), nh, (3, 7, 7), 1.0, return_lse=True, algo=algo,
                      dkv_accum=accum, **xk)
    assert lse.shape == (B, N, nh) and lse.dtype == torch.float32
    loss = (out.float() * gout.to(DEV).float()).sum() + (lse * glse.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()

    tol = 1e-4 if dt == torch.float32 else 2e-2
    errs = {"out": rel_err(out.detach().float().cpu(), out_r.detach()),
            "lse": rel_err(lse.detach().cpu(), lse_r.detach().transpose(1, 2))}
    for name, t, r in zip(names, ts, ref_in):
        errs["d" + name] = rel_err(t.grad.float().cpu(), r.grad, floor=1e-2)
    print("  " + "  ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        assert e < tol, name
