"""Parity of the HIP attention core and module against the reference (GPU).

Tolerances (the parity contract), relative error = max|a-b| / max(max|b|, floor)
(tests/goldens.py:rel_err):
  * fp32 kernels vs the reference: 1e-4;
  * bf16 kernels vs an fp32 evaluation of the reference on the bf16-rounded
    inputs: 2e-2.

Random and full-size cases compare against the oracle evaluated in float32, the
reference's own precision: the sampling coordinate's rounding decides which
cell a tap lands in when it sits exactly on a voxel (frequent with
bf16-quantised offsets), and the coordinate gradient is discontinuous there.
The kernels compute that coordinate op for op as the fp32 reference does.
The float64 golden vectors (continuous random inputs) are compared directly.
``floor`` = 1e-2 covers gradients that vanish identically (e.g. dq with a single
tap); k_proj.bias, whose gradient is zero by the softmax's shift invariance, is
checked against the scale of the k_proj.weight gradient instead.
"""

import math
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from goldens import C1, CASES, load, regenerate, rel_err
from oracle.dsa3d_ref import PARAM_NAMES, dsa3d_core_ref, dsa3d_module_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
FP32_TOL = 1e-4
BF16_TOL = 2e-2


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def core():
    from megaslide_amd import dsa3d_core
    return dsa3d_core


def _grad_or_zero(t):
    return t.grad if t.grad is not None else torch.zeros_like(t)


@pytest.mark.parametrize("name", [c["name"] for c in CASES if "extra_g" not in c])
def test_core_fp32_matches_reference_goldens(name):
    meta, arrs = load(name)
    case, _, _, _, off_np, _ = regenerate(meta)
    print(f"[core golden] {name}", flush=True)
    off_src = off_np if off_np is not None else arrs["offsets"]
    q, k, v, off = (dev(a).requires_grad_(True) for a in (arrs["q"], arrs["k"], arrs["v"], off_src))
    out = core()(q, k, v, off, (case["T"], case["H"], case["W"]), case["nh"], case["kernel"],
                 case["scale"])
    out.backward(dev(arrs["dattn"]))
    torch.cuda.synchronize()
    assert rel_err(out.detach().cpu(), arrs["attn"]) < FP32_TOL
    # floor: dq/dk vanish identically with one tap or on a 1x1x1 grid
    assert rel_err(q.grad.cpu(), arrs["dq"], floor=1e-2) < FP32_TOL
    assert rel_err(k.grad.cpu(), arrs["dk"], floor=1e-2) < FP32_TOL
    assert rel_err(v.grad.cpu(), arrs["dv"]) < FP32_TOL
    assert rel_err(off.grad.cpu(), arrs["doffsets"], floor=1e-2) < FP32_TOL


def _module_from_case(case, p, dtype=torch.float32):
    from megaslide_amd import DeformableSlideAttention3D
    m = DeformableSlideAttention3D(case["D"], case["nh"], kernel_size=tuple(case["kernel"]),
                                   offset_scale=case["scale"])
    with torch.no_grad():
        for n, prm in m.named_parameters():
            prm.copy_(torch.from_numpy(p[n]))
    return m.to(DEV, dtype)


@pytest.mark.parametrize("name", [c["name"] for c in CASES if c["mode"] == "net"])
def test_module_fp32_matches_reference_goldens(name):
    meta, arrs = load(name)
    case, p, x_np, gy_np, _, extra_np = regenerate(meta)
    print(f"[module golden] {name}", flush=True)
    m = _module_from_case(case, p)
    x = dev(x_np).requires_grad_(True)
    extra = None if extra_np is None else dev(extra_np).requires_grad_(True)
    y = m(x, (case["T"], case["H"], case["W"]), extra_kv=extra)
    (y * dev(gy_np)).sum().backward()
    torch.cuda.synchronize()
    assert rel_err(y.detach().cpu(), arrs["y"]) < FP32_TOL
    assert rel_err(x.grad.cpu(), arrs["dx"]) < FP32_TOL
    if extra is not None:
        assert rel_err(extra.grad.cpu(), arrs["dextra_kv"]) < FP32_TOL
    grads = {n: _grad_or_zero(prm).cpu() for n, prm in m.named_parameters()}
    for n, gr in grads.items():
        if n == "k_proj.bias":  # zero by shift invariance of the softmax
            assert float(gr.abs().max()) <= FP32_TOL * float(grads["v_proj.weight"].abs().max())
            continue
        assert rel_err(gr, arrs["grad." + n], floor=1e-2) < FP32_TOL, n


def test_c1_forward_fp32_matches_reference_rows():
    meta, arrs = load("c1_fwd_fp32")
    case, p, x_np, _, _, _ = regenerate(meta)
    print("[c1 forward]", flush=True)
    m = _module_from_case(case, p)
    with torch.no_grad():
        y = m(dev(x_np), (case["T"], case["H"], case["W"]))
    torch.cuda.synchronize()
    rows = torch.from_numpy(arrs["rows"])
    assert rel_err(y[:, rows.to(DEV)].cpu(), arrs["y_rows"]) < FP32_TOL


def _oracle_core(q, k, v, off, vs, nh, ks, scale, dout, query_index=None, head_chunk=4,
                 dtype=torch.float32):
    """Oracle fwd + autograd bwd on CPU copies of the given tensors (fp32 = the
    reference's precision)."""
    qq, kk, vv, oo = (t.detach().cpu().to(dtype).requires_grad_(True) for t in (q, k, v, off))
    out = dsa3d_core_ref(qq, kk, vv, oo, vs, nh, ks, scale, head_chunk=head_chunk,
                         query_index=query_index)
    out.backward(dout.detach().cpu().to(dtype))
    return out.detach(), _grad_or_zero(qq), _grad_or_zero(kk), _grad_or_zero(vv), _grad_or_zero(oo)


@pytest.mark.parametrize("dtype,tol,algo", [(torch.float32, FP32_TOL, "auto"),
                                             (torch.float32, FP32_TOL, "direct"),
                                             (torch.bfloat16, BF16_TOL, "auto")])
@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, hd, kernel, off_std, scale
    (2, 4, 12, 12, 2, 64, (3, 7, 7), 1.5, 1.0),
    (1, 5, 9, 11, 3, 32, (3, 5, 5), 2.0, 0.7),
    (1, 3, 6, 10, 2, 96, (3, 7, 7), 0.5, 1.0),
    (1, 2, 5, 7, 1, 128, (3, 7, 7), 4.0, 1.0),
])
def test_core_vs_oracle_random(shape, dtype, tol, algo):
    B, T, H, W, nh, hd, ks, off_std, scale = shape
    print(f"[core oracle] {shape} {dtype} {algo}", flush=True)
    N, D = T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator().manual_seed(1234 + N + hd)
    q, k, v = (torch.randn(B, N, D, generator=g) for _ in range(3))
    off = torch.randn(B, N, C, generator=g) * off_std
    dout = torch.randn(B, N, D, generator=g)
    # the bf16 kernels see bf16-rounded inputs; the oracle sees the same values in fp32
    q, k, v, off, dout = (t.to(dtype) for t in (q, k, v, off, dout))
    ref = _oracle_core(q, k, v, off, (T, H, W), nh, ks, scale, dout)
    qd, kd, vd, od = (t.to(DEV).requires_grad_(True) for t in (q, k, v, off))
    out = core()(qd, kd, vd, od, (T, H, W), nh, ks, scale, algo=algo)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    assert out.dtype == dtype
    assert rel_err(out.detach().float().cpu(), ref[0]) < tol
    assert rel_err(qd.grad.float().cpu(), ref[1]) < tol
    assert rel_err(kd.grad.float().cpu(), ref[2]) < tol
    assert rel_err(vd.grad.float().cpu(), ref[3]) < tol
    assert rel_err(od.grad.float().cpu(), ref[4]) < tol


def _offsets(spec, B, T, H, W, D, C, dtype, g):
    """Raw offsets [B, N, C] on the device: ("normal", std), or ("net", conv std,
    1x1 weight std, bias) from an offset net (depthwise 3x3x3 conv + GELU + 1x1
    conv, as the module predicts them) on x ~ N(0, 1), with the bias ("normal",
    std) or ("uniform", a) ~ U(-a, a) voxels."""
    from megaslide_amd import dwconv3d
    N = T * H * W
    if spec[0] == "normal":
        return (torch.randn(B, N, C, generator=g, device=DEV) * spec[1]).to(dtype)
    _, conv_std, w_std, (kind, a) = spec
    x = torch.randn(B, N, D, generator=g, device=DEV).to(dtype)
    w0 = (torch.randn(D, 1, 3, 3, 3, generator=g, device=DEV) * conv_std).to(dtype)
    b0 = (torch.randn(D, generator=g, device=DEV) * conv_std).to(dtype)
    w2 = (torch.randn(C, D, generator=g, device=DEV) * w_std).to(dtype)
    if kind == "uniform":
        b2 = (torch.rand(C, generator=g, device=DEV) * 2 * a - a).to(dtype)
    else:
        b2 = (torch.randn(C, generator=g, device=DEV) * a).to(dtype)
    with torch.no_grad():
        return F.linear(dwconv3d(x, w0, b0, (T, H, W), act="gelu"), w2, b2).contiguous()


@pytest.mark.parametrize("cfg", [
    # name, dtype, B, T, H, W, nh, hd, offsets, algo
    ("fp32 B2 16x32x32 8x64", torch.float32, 2, 16, 32, 32, 8, 64, ("normal", 1.5), "auto"),
    ("fp32 B2 16x32x32 8x64 direct", torch.float32, 2, 16, 32, 32, 8, 64, ("normal", 1.5),
     "direct"),
    ("bf16 65536 tokens 16x64", torch.bfloat16, 1, 64, 32, 32, 16, 64, ("normal", 0.5), "auto"),
    # offsets from the offset net, conv weights ~ N(0, 0.05)
    ("bf16 131072 tokens 24x128", torch.bfloat16, 1, 32, 64, 64, 24, 128,
     ("net", 0.05, 0.05, ("normal", 0.05)), "auto"),
    # offsets from the offset net with its bias ~ U(-4, 4) voxels
    ("bf16 46800 tokens 16x96 (13x45x80)", torch.bfloat16, 1, 13, 45, 80, 16, 96,
     ("net", 0.02, 0.02, ("uniform", 4.0)), "auto"),
])
def test_core_full_size_sampled_queries_and_checksums(cfg):
    """Full-size shapes: exact per-query parity on sampled queries (fwd, dq,
    d offsets), element-wise dK and dV over the whole volume for those
    queries, and size-independent checksums of dK and dV.

    Sum over voxels of dV equals the sum over queries of dO (per channel),
    because every query's tap weights p_k * w_c sum to one; the sum of dK is
    zero because sum_k ds_k = 0.  A second backward whose upstream gradient is
    zero except at the sampled queries gives dK and dV that only those queries
    feed (a query with dO = 0 has p dO = 0 and ds = p (dp - dO.O) = 0), so the
    whole tensors are compared with the oracle's autograd over the same queries:
    a scatter to a wrong voxel or a dropped or doubled flush shows there.
    """
    name, dtype, B, T, H, W, nh, hd, off_spec, algo = cfg
    print(f"[full size] {name}", flush=True)
    ks = (3, 7, 7)
    N, D = T * H * W, nh * hd
    C = nh * 147 * 3
    g = torch.Generator(device=DEV).manual_seed(7)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV).to(dtype) for _ in range(3))
    off = _offsets(off_spec, B, T, H, W, D, C, dtype, g)
    dout = torch.randn(B, N, D, generator=g, device=DEV).to(dtype)
    qd, kd, vd, od = (t.clone().requires_grad_(True) for t in (q, k, v, off))
    out = core()(qd, kd, vd, od, (T, H, W), nh, ks, 1.0, algo=algo)
    out.backward(dout)
    torch.cuda.synchronize()
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    # checksums over every voxel
    sum_dv = vd.grad.double().sum(dim=1)
    sum_do = dout.double().sum(dim=1)
    assert rel_err(sum_dv.cpu(), sum_do.cpu()) < (1e-5 if dtype == torch.float32 else 1e-2)
    sum_dk = kd.grad.double().sum(dim=1).abs().max().item()
    scale_dk = kd.grad.double().abs().sum(dim=1).max().item()
    assert sum_dk < (1e-5 if dtype == torch.float32 else 1e-2) * scale_dk
    # parity for sampled queries (first, last, random) against the fp32 oracle
    idx = torch.cat([torch.tensor([0, N - 1]), torch.randperm(N, generator=torch.Generator().manual_seed(3))[:30]])
    ref_out, ref_dq, ref_dk, ref_dv, ref_doff = _oracle_core(
        q.float(), k.float(), v.float(), off.float(), (T, H, W), nh, ks, 1.0,
        dout.float()[:, idx], query_index=idx, head_chunk=2)
    assert rel_err(out.detach()[:, idx.to(DEV)].float().cpu(), ref_out) < tol
    qgrad = qd.grad[:, idx.to(DEV)].float().cpu()
    ref_dq_rows = ref_dq[:, idx]
    assert rel_err(qgrad, ref_dq_rows) < tol
    assert rel_err(od.grad[:, idx.to(DEV)].float().cpu(), ref_doff[:, idx]) < tol
    # the whole dK and dV of the sampled queries alone
    dsparse = torch.zeros_like(dout)
    dsparse[:, idx.to(DEV)] = dout[:, idx.to(DEV)]
    for t in (qd, kd, vd, od):
        t.grad = None
    out = core()(qd, kd, vd, od, (T, H, W), nh, ks, 1.0, algo=algo)
    out.backward(dsparse)
    torch.cuda.synchronize()
    e_dk = rel_err(kd.grad.float().cpu(), ref_dk)
    e_dv = rel_err(vd.grad.float().cpu(), ref_dv)
    print(f"  sampled-query dK {e_dk:.2e}  dV {e_dv:.2e}  (non-zero voxel rows: "
          f"{int((ref_dv.abs().sum(-1) > 0).sum())})", flush=True)
    assert e_dk < tol and e_dv < tol


def test_nograd_forward_matches_grad_forward_and_streams():
    B, T, H, W, nh, hd = 1, 3, 8, 8, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator(device=DEV).manual_seed(5)
    q, k, v = (torch.randn(B, N, D, generator=g, device=DEV) for _ in range(3))
    off = torch.randn(B, N, C, generator=g, device=DEV)
    with torch.no_grad():
        a = core()(q, k, v, off, (T, H, W), nh)
    b = core()(q.requires_grad_(True), k, v, off, (T, H, W), nh)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        c = core()(q.detach(), k, v, off, (T, H, W), nh)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(a, b.detach())
    assert torch.equal(a, c)


def test_strided_qkv_views():
    """q, k, v as column slices of one fused [B, N, 3D] projection output."""
    B, T, H, W, nh, hd = 1, 3, 6, 7, 2, 32
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator(device=DEV).manual_seed(9)
    qkv = torch.randn(B, N, 3 * D, generator=g, device=DEV, requires_grad=True)
    off = torch.randn(B, N, C, generator=g, device=DEV)
    q, k, v = qkv.split(D, dim=-1)
    out = core()(q, k, v, off, (T, H, W), nh)
    out.sum().backward()
    qkv2 = qkv.detach().clone().requires_grad_(True)
    q2, k2, v2 = (t.contiguous() for t in qkv2.split(D, dim=-1))
    out2 = core()(q2, k2, v2, off, (T, H, W), nh)
    out2.sum().backward()
    torch.cuda.synchronize()
    assert rel_err(out.detach().cpu(), out2.detach().cpu()) < 1e-6
    assert rel_err(qkv.grad.cpu(), qkv2.grad.cpu()) < 1e-5


def test_invariant_constant_values():
    """A constant V volume gives that constant for any q and offsets."""
    B, T, H, W, nh, hd = 1, 4, 9, 9, 2, 64
    N, D, C = T * H * W, nh * hd, nh * 147 * 3
    g = torch.Generator(device=DEV).manual_seed(11)
    q, k = (torch.randn(B, N, D, generator=g, device=DEV) for _ in range(2))
    const = torch.randn(D, generator=g, device=DEV)
    v = const.expand(B, N, D).contiguous()
    off = torch.randn(B, N, C, generator=g, device=DEV) * 3
    out = core()(q, k, v, off, (T, H, W), nh)
    torch.cuda.synchronize()
    assert rel_err(out.cpu(), const.expand(B, N, D).cpu()) < 1e-5


def test_cpu_tensor_raises():
    with pytest.raises(RuntimeError, match="ROCm"):
        core()(torch.zeros(1, 8, 16), torch.zeros(1, 8, 16), torch.zeros(1, 8, 16),
               torch.zeros(1, 8, 2 * 27 * 3), (2, 2, 2), 2, (3, 3, 3))


@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, kernel, off_std, scale  (head_dim 64, bf16: the matrix-core kernels)
    (1, 3, 7, 9, 2, (3, 7, 7), 0.5, 1.0),     # grid not a multiple of the 4x4 tile
    (2, 4, 8, 8, 1, (3, 5, 5), 1.5, 0.8),
    (1, 2, 5, 6, 2, (1, 3, 3), 0.7, 1.0),
    (1, 5, 12, 40, 1, (3, 7, 7), 8.0, 1.0),   # large offsets: corner boxes span several chunks
    (1, 1, 4, 4, 2, (3, 3, 3), 1.0, 1.0),     # T = 1
])
def test_tiled_forward_vs_oracle_and_direct(shape):
    B, T, H, W, nh, ks, off_std, scale = shape
    print(f"[tiled fwd] {shape}", flush=True)
    hd = 64
    N, D = T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator().manual_seed(99 + N)
    q, k, v = (torch.randn(B, N, D, generator=g).to(torch.bfloat16) for _ in range(3))
    off = (torch.randn(B, N, C, generator=g) * off_std).to(torch.bfloat16)
    ref, ref_lse = dsa3d_core_ref(q.float(), k.float(), v.float(), off.float(), (T, H, W), nh, ks,
                                  scale, return_lse=True)
    qd, kd, vd, od = (t.to(DEV) for t in (q, k, v, off))
    with torch.no_grad():
        out_t, lse_t = core()(qd, kd, vd, od, (T, H, W), nh, ks, scale, return_lse=True,
                              algo="tiled")
        out_d, lse_d = core()(qd, kd, vd, od, (T, H, W), nh, ks, scale, return_lse=True,
                              algo="direct")
    torch.cuda.synchronize()
    assert rel_err(out_t.float().cpu(), ref) < BF16_TOL
    assert rel_err(lse_t.cpu(), ref_lse.permute(0, 2, 1)) < 1e-5
    assert rel_err(out_t.float().cpu(), out_d.float().cpu()) < BF16_TOL
    assert rel_err(lse_t.cpu(), lse_d.cpu()) < 1e-5


def test_tiled_rejects_ineligible_calls():
    q = torch.zeros(1, 8, 16, device=DEV, dtype=torch.bfloat16)  # head_dim 16
    off = torch.zeros(1, 8, 27 * 3, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="tiled"):
        core()(q, q, q, off, (2, 2, 2), 1, (3, 3, 3), algo="tiled")


@pytest.mark.parametrize("D,nh", [(256, 4), (192, 2)])
def test_module_bf16_tiled_matches_oracle(D, nh):
    """Whole module in bf16 (matrix-core attention kernels, bf16 dwconvs, bf16
    GEMMs) on a non-tile-aligned grid, with offsets from an offset net whose
    bias ~ U(-4, 4) voxels as in the DiT-block configuration, against the fp32
    oracle module on the same bf16-rounded parameters and inputs.

    Sampling is piecewise linear in the offsets, so the oracle must sample at
    the offsets the bf16 module used: fp32 offsets differ from them by ~0.01
    voxels, which moves a few percent of the taps across a lattice line or the
    border clamp and changes their offset gradient by O(1).  The oracle
    therefore runs the attention with the module's bf16 offsets injected and
    chains the offset gradient it returns through its own fp32 offset net.
    """
    from megaslide_amd import DeformableSlideAttention3D, dwconv3d
    from oracle.dsa3d_ref import dsa3d_module_ref, predict_offsets_ref
    T, H, W, B = 5, 9, 14, 1
    N = T * H * W
    print(f"[module bf16] D={D} nh={nh}", flush=True)
    g = torch.Generator().manual_seed(404 + D)
    m = DeformableSlideAttention3D(D, nh)
    with torch.no_grad():
        for name, prm in m.named_parameters():
            if name == "offset_net.2.bias":
                prm.copy_(torch.rand(prm.shape, generator=g) * 8 - 4)
            elif name.endswith("weight") and prm.dim() >= 2 and "offset_net" not in name \
                    and "dw_conv" not in name:
                prm.copy_(torch.randn(prm.shape, generator=g) * (1.0 / math.sqrt(D)))
            else:
                prm.copy_(torch.randn(prm.shape, generator=g) * 0.05)
    m = m.to(DEV, torch.bfloat16)
    x = torch.randn(B, N, D, generator=g).to(torch.bfloat16)
    gy = torch.randn(B, N, D, generator=g).to(torch.bfloat16)
    xd = x.to(DEV).requires_grad_(True)
    y = m(xd, (T, H, W))
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
    offr = off_mod.float().cpu().requires_grad_(True)
    yr = dsa3d_module_ref(xr, params, (T, H, W), nh, offsets=offr)
    yr.backward(gy.float())
    predict_offsets_ref(xr, params, (T, H, W)).backward(offr.grad)
    errs = {"y": rel_err(y.detach().float().cpu(), yr.detach()),
            "dx": rel_err(xd.grad.float().cpu(), xr.grad)}
    for n, prm in m.named_parameters():
        if n == "k_proj.bias":  # zero by shift invariance of the softmax
            continue
        errs[n] = rel_err(prm.grad.float().cpu(), params[n].grad, floor=1e-2)
    print("  " + "  ".join(f"{k} {v:.1e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e < BF16_TOL, k
