"""Tiled attention core on seeded random shapes against the fp32 oracle (GPU).

Each case draws a grid (partial tiles, T, H or W of 1 included), a window,
head size, batch and offsets (Gaussian per query, optionally a per-(head, tap)
shift as an offset net's bias gives) from its seed, then checks the output and
every gradient (dq, dK, dV, d offsets) against the oracle:
  - bf16, default accumulation (the column-streaming dq/dK/dV kernel, with its
    pair walks and the tile kernel for listed columns), 2e-2 of max|ref|;
  - bf16 with dK/dV summed in scaled fp16 (the tile kernel), 2e-2;
  - fp32 storage (fp32 matrix-core kernels), 1e-4;
  - bf16 with G shared extra keys (their gradients checked too), 2e-2;
  - bf16 with attention dropout (the oracle applies the same Philox keep mask), 2e-2;
  - head sizes and windows the tiled kernels do not take (head_dim 8 to 112 off the
    32/64/96/128 set, windows of more than 160 taps), which the default dispatch
    sends to the general (direct) kernels: bf16 2e-2, fp32 1e-4;
  - the returned log-sum-exp differentiated with the output (loss = sum(out g_out)
    + sum(lse g_lse), the dlse input of the backward), bf16 and fp32; lse itself
    within 1e-4 (bf16: 2e-3 of max|lse|).
"""

import random

import pytest
import torch

from goldens import rel_err
from oracle.dsa3d_ref import dsa3d_core_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16_TOL = 2e-2
FP32_TOL = 1e-4
MODES = {"bf16": (torch.bfloat16, "fp32", BF16_TOL), "bf16-f16acc": (torch.bfloat16, "fp16", BF16_TOL),
         "fp32": (torch.float32, "fp32", FP32_TOL), "bf16-extra": (torch.bfloat16, "fp32", BF16_TOL),
         "bf16-dropout": (torch.bfloat16, "fp32", BF16_TOL),
         "general-bf16": (torch.bfloat16, "fp32", BF16_TOL), "general-fp32": (torch.float32, "fp32", FP32_TOL),
         "bf16-lse": (torch.bfloat16, "fp32", BF16_TOL), "fp32-lse": (torch.float32, "fp32", FP32_TOL)}
WINDOWS = [(1, 1, 1), (1, 3, 3), (3, 3, 3), (3, 5, 5), (3, 7, 7), (1, 7, 7), (3, 1, 3),
           (5, 3, 3), (2, 3, 5), (3, 5, 7)]


def draw(seed):
    r = random.Random(seed)
    ks = r.choice(WINDOWS)
    hd = r.choice([32, 64, 96, 128])
    B = r.choice([1, 1, 2])
    nh = r.choice([1, 2])
    T = r.choice([1, 2, 3, 5, 8, 11])
    H = r.choice([1, 3, 4, 7, 9, 13])
    W = r.choice([1, 4, 6, 9, 14, 21])
    while B * T * H * W > 2400:  # keeps the CPU oracle to about a second
        if T >= max(H, W):
            T = (T + 1) // 2
        elif H >= W:
            H = (H + 1) // 2
        else:
            W = (W + 1) // 2
    off_std = r.choice([0.2, 0.6, 1.5, 3.0])
    shift = r.choice([0.0, 0.0, 2.0, 4.0])  # per-(head, tap) shift amplitude, voxels of offset
    scale = round(r.uniform(0.7, 1.3), 3)
    return B, T, H, W, nh, ks, hd, off_std, shift, scale


CASES = ([("bf16", s) for s in range(48)] + [("bf16-f16acc", s) for s in range(48, 64)] +
         [("fp32", s) for s in range(64, 80)] + [("bf16-extra", s) for s in range(80, 96)] +
         [("bf16-dropout", s) for s in range(96, 112)] + [("general-bf16", s) for s in range(112, 120)] +
         [("general-fp32", s) for s in range(120, 128)] + [("bf16-lse", s) for s in range(128, 144)] +
         [("fp32-lse", s) for s in range(144, 152)])


@pytest.mark.parametrize("mode,seed", CASES)
def test_tiled_random_shape_vs_oracle(mode, seed):
    dtype, accum, tol = MODES[mode]
    B, T, H, W, nh, ks, hd, off_std, shift, scale = draw(seed)
    general = mode.startswith("general")
    if general:
        # a head size off the tiled set, or (every third case) a 5x7x7 window of 245 taps
        hd = [8, 16, 40, 48, 80, 112][seed % 6]
        if seed % 3 == 0:
            hd, ks = 64, (5, 7, 7)
    K = ks[0] * ks[1] * ks[2]
    N, D = T * H * W, nh * hd
    print(f"[tiled random {mode} {seed}] B={B} T={T} H={H} W={W} nh={nh} hd={hd} window={ks} "
          f"off_std={off_std} shift={shift} scale={scale}", flush=True)
    g = torch.Generator().manual_seed(5000 + seed)
    q, k, v = (torch.randn(B, N, D, generator=g).to(dtype) for _ in range(3))
    off = torch.randn(B, N, nh * K * 3, generator=g) * off_std
    if shift > 0:
        off = off + (torch.rand(nh * K * 3, generator=g) * 2.0 - 1.0) * shift
    off = off.to(dtype)
    dout = torch.randn(B, N, D, generator=g).to(dtype)
    G = [1, 7, 32, 128][seed % 4] if mode == "bf16-extra" else 0
    inputs = [q, k, v, off]
    if G:
        inputs += [torch.randn(B, G, D, generator=g).to(dtype) for _ in range(2)]
    drop = (0.1 if seed % 2 else 0.3, 1000 + seed, seed % 3) if mode == "bf16-dropout" else None
    if G or drop:
        print(f"  extra keys G={G} dropout={drop}", flush=True)

    with_lse = mode.endswith("-lse")
    glse = torch.randn(B, N, nh, generator=g) if with_lse else None

    ref_in = [t.float().clone().requires_grad_(True) for t in inputs]
    ref = dsa3d_core_ref(*ref_in[:4], (T, H, W), nh, ks, scale,
                         extra_k=ref_in[4] if G else None, extra_v=ref_in[5] if G else None,
                         dropout=drop, return_lse=with_lse)
    if with_lse:
        ref, ref_lse = ref
        ((ref * dout.float()).sum() + (ref_lse.transpose(1, 2) * glse).sum()).backward()
    else:
        ref.backward(dout.float())

    from megaslide_amd import dsa3d_core
    ts = [t.detach().to(DEV).requires_grad_(True) for t in inputs]
    kw = dict(algo="auto" if general else "tiled", dkv_accum=accum)
    if G:
        kw.update(extra_k=ts[4], extra_v=ts[5])
    if drop:
        kw.update(dropout_p=drop[0], dropout_seed=drop[1], dropout_offset=drop[2])
    out = dsa3d_core(*ts[:4], (T, H, W), nh, ks, scale, return_lse=with_lse, **kw)
    if with_lse:
        out, lse = out
        ((out.float() * dout.to(DEV).float()).sum() + (lse * glse.to(DEV)).sum()).backward()
    else:
        out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    if with_lse:
        e_lse = rel_err(lse.detach().cpu(), ref_lse.detach().transpose(1, 2))
        print(f"  lse: {e_lse:.2e}", flush=True)
        assert e_lse < (1e-4 if dtype == torch.float32 else 2e-3)

    e_out = rel_err(out.detach().float().cpu(), ref.detach())
    print(f"  out: {e_out:.2e}", flush=True)
    assert e_out < tol
    names = ("dq", "dk", "dv", "doff", "dek", "dev")
    for name, r, t in zip(names, ref_in, ts):
        # an input that cannot reach the output (offsets on a 1x1x1 grid) gets no
        # reference gradient: it must be zero
        r = r.grad if r.grad is not None else torch.zeros_like(r)
        # every tap of a query samples one point (one tap, or a 1 x 1 grid with a
        # window one frame deep or one frame): ds = p (f dp - sum p f dp) sums
        # to 0 against one interpolated key, so dq and dK (both carried by ds)
        # are zero up to rounding (the oracle's are exactly 0); the inputs are O(1)
        one_point = K == 1 or (H == 1 and W == 1 and (ks[0] == 1 or T == 1))
        if name in ("dq", "dk") and one_point and G == 0 and not with_lse:
            m = t.grad.float().abs().max().item()
            print(f"  {name} (one point, zero): max |{name}| {m:.2e}", flush=True)
            assert m < 1e-4, name
            continue
        e = rel_err(t.grad.float().cpu(), r)
        print(f"  {name}: {e:.2e}", flush=True)
        assert e < tol, name
