"""The drop-in DeformableSlideAttention3D on seeded random configurations
against the oracle module (attention.py:82-192 restated), GPU.

Each case draws dim and heads (head sizes on and off the tiled kernels' set),
the window, offset_scale, the offset net's bias spread, the grid (unit axes
included), B, extra_kv keys and bf16 or fp32.  The oracle samples at the
offsets the module's own offset net produced (sampling is piecewise linear in
the offsets, so independently rounded offsets would move taps across lattice
lines) and chains the offset gradient through its own offset net.  Output,
dx, d extra_kv and every parameter gradient must agree: fp32 1e-4, bf16 2e-2
(relative to max|ref|).  Where every tap of a query samples one point (a
1 x 1 grid with a window one frame deep), ds and with it the q and k
projections' gradients vanish identically, and the k bias's always does (the
softmax's shift invariance); those are checked against an absolute bound
instead (1e-3, or 5e-2 in bf16, of max|d v_proj.weight|).
"""

import math
import random

import pytest
import torch
import torch.nn.functional as F

from goldens import rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"


def draw(seed):
    r = random.Random(40000 + seed)
    dtype, tol = r.choice([(torch.bfloat16, 2e-2), (torch.float32, 1e-4)])
    nh = r.choice([1, 2, 4])
    hd = r.choice([32, 64, 96, 48])
    ks = r.choice([(3, 7, 7), (3, 5, 5), (1, 3, 3), (3, 3, 3)])
    oscale = r.choice([0.5, 1.0, 2.0])
    B = r.choice([1, 2])
    T = r.choice([1, 2, 4, 6])
    H = r.choice([1, 3, 6, 9, 12])
    W = r.choice([1, 4, 7, 13, 16])
    G = r.choice([0, 0, 4, 16])
    bias_a = r.choice([0.0, 2.0, 4.0])
    return dtype, tol, nh, hd, ks, oscale, B, T, H, W, G, bias_a


@pytest.mark.parametrize("seed", range(24))
def test_module_random_config_vs_oracle(seed):
    from megaslide_amd import DeformableSlideAttention3D, dwconv3d
    from oracle.dsa3d_ref import dsa3d_module_ref, predict_offsets_ref
    dtype, tol, nh, hd, ks, oscale, B, T, H, W, G, bias_a = draw(seed)
    D, N = nh * hd, T * H * W
    print(f"[module random {seed}] {dtype} B={B} T={T} H={H} W={W} nh={nh} hd={hd} window={ks} "
          f"offset_scale={oscale} G={G} bias=U(-{bias_a}, {bias_a})", flush=True)
    g = torch.Generator().manual_seed(seed)
    m = DeformableSlideAttention3D(D, nh, kernel_size=ks, offset_scale=oscale)
    with torch.no_grad():
        for name, prm in m.named_parameters():
            if name == "offset_net.2.bias":
                prm.copy_(torch.rand(prm.shape, generator=g) * 2 * bias_a - bias_a)
            elif name.endswith("weight") and prm.dim() >= 2 and "offset_net" not in name \
                    and "dw_conv" not in name:
                prm.copy_(torch.randn(prm.shape, generator=g) * (1.0 / math.sqrt(D)))
            else:
                prm.copy_(torch.randn(prm.shape, generator=g) * 0.05)
    m = m.to(DEV, dtype)
    x = torch.randn(B, N, D, generator=g).to(dtype)
    gy = torch.randn(B, N, D, generator=g).to(dtype)
    ekv = torch.randn(B, G, D, generator=g).to(dtype) if G else None
    xd = x.to(DEV).requires_grad_(True)
    ed = ekv.to(DEV).requires_grad_(True) if G else None
    y = m(xd, (T, H, W), extra_kv=ed)
    y.backward(gy.to(DEV))
    # the offsets the module sampled at (same kernels and inputs: same bits)
    with torch.no_grad():
        on2 = m.offset_net[2]
        feat = dwconv3d(xd.detach(), m.offset_net[0].weight, m.offset_net[0].bias, (T, H, W),
                        act="gelu")
        off_mod = F.linear(feat, on2.weight.view(on2.weight.shape[0], -1), on2.bias)
    torch.cuda.synchronize()

    params = {n: prm.detach().float().cpu().requires_grad_(True) for n, prm in m.named_parameters()}
    xr = x.float().requires_grad_(True)
    er = ekv.float().requires_grad_(True) if G else None
    offr = off_mod.float().cpu().requires_grad_(True)
    yr = dsa3d_module_ref(xr, params, (T, H, W), nh, kernel_size=ks, offset_scale=oscale,
                          offsets=offr, extra_kv=er)
    yr.backward(gy.float())
    if offr.grad is not None:  # offsets reach the output (not a 1 x 1 x 1 grid)
        predict_offsets_ref(xr, params, (T, H, W)).backward(offr.grad)

    one_point = G == 0 and H == 1 and W == 1 and (ks[0] == 1 or T == 1)
    errs = {"y": rel_err(y.detach().float().cpu(), yr.detach()),
            "dx": rel_err(xd.grad.float().cpu(), xr.grad)}
    if G:
        errs["d extra_kv"] = rel_err(ed.grad.float().cpu(), er.grad)
    for n, prm in m.named_parameters():
        got = prm.grad.float().cpu() if prm.grad is not None else torch.zeros_like(params[n])
        ref = params[n].grad if params[n].grad is not None else torch.zeros_like(params[n])
        if n == "k_proj.bias" or (one_point and n.split(".")[0] in ("q_proj", "k_proj")):
            # zero: the softmax's shift invariance (k bias; the extra keys carry
            # it too), or ds = 0 (one point).  It is left as the cancellation of
            # separately rounded rows (dK, d extra keys), so bf16 leaves more.
            scale = max(1.0, float(params["v_proj.weight"].grad.abs().max()))
            bound = 1e-3 if dtype == torch.float32 else 5e-2
            assert float(got.abs().max()) < bound * scale, n
            continue
        errs[n] = rel_err(got, ref, floor=1e-2)
    print("  " + "  ".join(f"{k} {v:.1e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e < tol, k
