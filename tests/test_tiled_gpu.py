"""Matrix-core (tiled) attention-core kernels: parity and invariants (GPU).

The tiled kernels serve bf16 and fp32, head_dim 32, 64, 96 and 128.  They must agree
with the fp32 oracle (relative to max|ref|: bf16 2e-2, fp32 1e-4) and with the
direct kernels; the log-sum-exp they return must match the oracle's to 1e-5.
"""

import pytest
import torch

from goldens import rel_err
from oracle.dsa3d_ref import dsa3d_core_ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16_TOL = 2e-2
FP32_TOL = 1e-4


def core():
    from megaslide_amd import dsa3d_core
    return dsa3d_core


def _inputs(B, T, H, W, nh, ks, off_std, seed, hd=64, dtype=torch.bfloat16):
    N, D = T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, N, D, generator=g).to(dtype) for _ in range(3))
    off = (torch.randn(B, N, C, generator=g) * off_std).to(dtype)
    return q, k, v, off


def test_tiled_single_tap_is_trilinear_sample():
    """Window 1x1x1: softmax over one tap is 1, so out = V sampled at the tap."""
    B, T, H, W, nh, ks = 1, 3, 6, 7, 1, (1, 1, 1)
    q, k, v, off = _inputs(B, T, H, W, nh, ks, 0.8, 5)
    ref = dsa3d_core_ref(q.float(), k.float(), v.float(), off.float(), (T, H, W), nh, ks, 1.0)
    with torch.no_grad():
        out = core()(*(t.to(DEV) for t in (q, k, v, off)), (T, H, W), nh, ks, algo="tiled")
    torch.cuda.synchronize()
    print("single tap err", rel_err(out.float().cpu(), ref), flush=True)
    assert rel_err(out.float().cpu(), ref) < BF16_TOL


def test_tiled_constant_values():
    """Constant V: out equals the constant whatever the scores are."""
    B, T, H, W, nh, ks = 1, 3, 8, 8, 2, (3, 7, 7)
    q, k, v, off = _inputs(B, T, H, W, nh, ks, 1.0, 6)
    const = torch.randn(nh * 64).to(torch.bfloat16)
    v = const.expand_as(v).contiguous()
    with torch.no_grad():
        out = core()(*(t.to(DEV) for t in (q, k, v, off)), (T, H, W), nh, ks, algo="tiled")
    torch.cuda.synchronize()
    err = rel_err(out.float().cpu(), const.float().expand_as(out))
    print("constant-V err", err, flush=True)
    if err >= 1e-2:
        o = out.float().cpu()
        print("const[:20]   ", [round(x, 3) for x in const.float()[:20].tolist()])
        print("out[0,0,:20] ", [round(x, 3) for x in o[0, 0, :20].tolist()])
        print("out[0,5,:20] ", [round(x, 3) for x in o[0, 5, :20].tolist()])
        print("ratio ch0 over tokens", [round(x, 3) for x in (o[0, :20, 0] / const.float()[0]).tolist()])
    assert err < 1e-2


@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, kernel, off_std, scale, head_dim
    (1, 3, 7, 9, 2, (3, 7, 7), 0.5, 1.0, 64),
    (2, 4, 8, 8, 1, (3, 5, 5), 1.5, 0.8, 64),
    (1, 5, 12, 40, 1, (3, 7, 7), 8.0, 1.0, 64),   # corner boxes span several chunks
    (1, 1, 4, 4, 2, (3, 3, 3), 1.0, 1.0, 64),     # T = 1
    (1, 3, 7, 9, 2, (3, 7, 7), 0.5, 1.0, 96),
    (1, 4, 13, 18, 1, (3, 7, 7), 4.0, 0.9, 96),   # non-tile-aligned grid, large offsets
    (1, 3, 8, 8, 2, (3, 7, 7), 0.5, 1.0, 128),
    (1, 5, 12, 40, 1, (3, 7, 7), 8.0, 1.0, 128),  # corner boxes span several chunks
    (1, 4, 1, 9, 2, (3, 7, 7), 1.0, 1.0, 64),     # H = 1: y slot dropped, base y divisor 1
    (1, 3, 6, 1, 1, (3, 7, 7), 1.0, 1.0, 64),     # W = 1: z slot dropped (slot/axis quirk)
    (2, 2, 3, 5, 2, (1, 3, 5), 3.0, 1.2, 96),     # B = 2, asymmetric window
    (1, 4, 9, 10, 3, (3, 7, 7), 1.0, 1.0, 32),
    (2, 5, 6, 7, 2, (3, 5, 5), 3.0, 0.8, 32),     # B = 2, large offsets
])
def test_tiled_backward_vs_oracle_and_direct(shape):
    B, T, H, W, nh, ks, off_std, scale, hd = shape
    print(f"[tiled bwd] {shape}", flush=True)
    q, k, v, off = _inputs(B, T, H, W, nh, ks, off_std, 300 + T * H * W + hd, hd=hd)
    g = torch.Generator().manual_seed(17)
    dout = torch.randn(q.shape, generator=g).to(torch.bfloat16)
    qq, kk, vv, oo = (t.float().requires_grad_(True) for t in (q, k, v, off))
    ref = dsa3d_core_ref(qq, kk, vv, oo, (T, H, W), nh, ks, scale)
    ref.backward(dout.float())
    grads, outs = {}, {}
    for algo in ("tiled", "direct"):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
        out = core()(*ts, (T, H, W), nh, ks, scale, algo=algo)
        out.backward(dout.to(DEV))
        outs[algo] = out.detach().float().cpu()
        grads[algo] = [t.grad.float().cpu() for t in ts]
    torch.cuda.synchronize()
    e_out = rel_err(outs["tiled"], ref.detach())
    print(f"  out: vs oracle {e_out:.2e}", flush=True)
    assert e_out < BF16_TOL
    for name, r, gt, gd in zip(("dq", "dk", "dv", "doff"), (qq.grad, kk.grad, vv.grad, oo.grad),
                               grads["tiled"], grads["direct"]):
        e_ref, e_dir = rel_err(gt, r), rel_err(gt, gd)
        print(f"  {name}: vs oracle {e_ref:.2e}  vs direct {e_dir:.2e}", flush=True)
        assert e_ref < BF16_TOL, name
        assert e_dir < BF16_TOL, name


def test_tiled_lse_matches_oracle():
    B, T, H, W, nh, ks = 1, 3, 8, 8, 2, (3, 7, 7)
    q, k, v, off = _inputs(B, T, H, W, nh, ks, 0.5, 7)
    _, ref_lse = dsa3d_core_ref(q.float(), k.float(), v.float(), off.float(), (T, H, W), nh, ks,
                                1.0, return_lse=True)
    with torch.no_grad():
        _, lse = core()(*(t.to(DEV) for t in (q, k, v, off)), (T, H, W), nh, ks,
                        return_lse=True, algo="tiled")
    torch.cuda.synchronize()
    err = rel_err(lse.cpu(), ref_lse.permute(0, 2, 1))
    print("lse err", err, flush=True)
    assert err < 1e-5


@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, kernel, off_std, scale, head_dim
    (1, 3, 7, 9, 2, (3, 7, 7), 0.5, 1.0, 64),
    (2, 4, 8, 8, 1, (3, 5, 5), 1.5, 0.8, 64),
    (1, 5, 12, 40, 1, (3, 7, 7), 8.0, 1.0, 64),   # corner boxes span several chunks
    (1, 4, 13, 18, 1, (3, 7, 7), 4.0, 0.9, 96),   # non-tile-aligned grid, large offsets
    (1, 3, 8, 8, 2, (3, 7, 7), 0.5, 1.0, 128),
    (1, 4, 1, 9, 2, (3, 7, 7), 1.0, 1.0, 64),     # H = 1
    (2, 2, 3, 5, 2, (1, 3, 5), 3.0, 1.2, 96),     # B = 2, asymmetric window
    (1, 4, 9, 10, 3, (3, 7, 7), 1.0, 1.0, 32),
])
def test_tiled_fp32_vs_oracle_and_direct(shape):
    """fp32 storage: the tiled kernels run the fp32 matrix-core instructions
    and must meet the fp32 tolerance against the oracle and the direct kernels."""
    B, T, H, W, nh, ks, off_std, scale, hd = shape
    print(f"[tiled fp32] {shape}", flush=True)
    q, k, v, off = _inputs(B, T, H, W, nh, ks, off_std, 700 + T * H * W + hd, hd=hd,
                           dtype=torch.float32)
    g = torch.Generator().manual_seed(23)
    dout = torch.randn(q.shape, generator=g)
    qq, kk, vv, oo = (t.clone().requires_grad_(True) for t in (q, k, v, off))
    ref, ref_lse = dsa3d_core_ref(qq, kk, vv, oo, (T, H, W), nh, ks, scale, return_lse=True)
    ref.backward(dout)
    grads, outs, lses = {}, {}, {}
    for algo in ("tiled", "direct"):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
        out, lse = core()(*ts, (T, H, W), nh, ks, scale, algo=algo, return_lse=True)
        out.backward(dout.to(DEV))
        outs[algo] = out.detach().cpu()
        lses[algo] = lse.detach().cpu()
        grads[algo] = [t.grad.cpu() for t in ts]
    torch.cuda.synchronize()
    assert outs["tiled"].dtype == torch.float32
    e_out = rel_err(outs["tiled"], ref.detach())
    e_lse = rel_err(lses["tiled"], ref_lse.detach().permute(0, 2, 1))
    print(f"  out: vs oracle {e_out:.2e}  lse {e_lse:.2e}", flush=True)
    assert e_out < FP32_TOL
    assert e_lse < 1e-5
    assert rel_err(outs["tiled"], outs["direct"]) < FP32_TOL
    for name, r, gt, gd in zip(("dq", "dk", "dv", "doff"), (qq.grad, kk.grad, vv.grad, oo.grad),
                               grads["tiled"], grads["direct"]):
        e_ref, e_dir = rel_err(gt, r), rel_err(gt, gd)
        print(f"  {name}: vs oracle {e_ref:.2e}  vs direct {e_dir:.2e}", flush=True)
        assert e_ref < FP32_TOL, name
        assert e_dir < FP32_TOL, name


@pytest.mark.parametrize("hd,dtype", [(64, torch.bfloat16), (96, torch.bfloat16),
                                      (128, torch.bfloat16), (64, torch.float32)])
def test_tiled_tap_shifted_offsets(hd, dtype):
    """Offsets that move whole taps apart, as an offset net's per-tap bias does
    (each (head, tap) shifted by U(-4, 4) voxels per axis, plus N(0, 0.1) per
    query): a tile's corners spread over a box of several chunks, part of whose
    (chunk, plane) steps no corner reaches.  Every output and gradient must
    match the oracle and the direct kernels."""
    B, T, H, W, nh, ks, scale = 1, 6, 24, 24, 2, (3, 7, 7), 1.0
    K = ks[0] * ks[1] * ks[2]
    print(f"[tiled tap-shifted] hd {hd} {dtype}", flush=True)
    q, k, v, _ = _inputs(B, T, H, W, nh, ks, 0.0, 900 + hd, hd=hd, dtype=dtype)
    g = torch.Generator().manual_seed(31 + hd)
    shift = torch.rand(nh, K, 3, generator=g) * 8.0 - 4.0
    off = (shift.reshape(1, 1, -1) + 0.1 * torch.randn(B, T * H * W, nh * K * 3, generator=g))
    off = off.to(dtype)
    dout = torch.randn(q.shape, generator=g).to(dtype)
    qq, kk, vv, oo = (t.float().clone().requires_grad_(True) for t in (q, k, v, off))
    ref = dsa3d_core_ref(qq, kk, vv, oo, (T, H, W), nh, ks, scale)
    ref.backward(dout.float())
    grads, outs = {}, {}
    for algo in ("tiled", "direct"):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
        out = core()(*ts, (T, H, W), nh, ks, scale, algo=algo)
        out.backward(dout.to(DEV))
        outs[algo] = out.detach().float().cpu()
        grads[algo] = [t.grad.float().cpu() for t in ts]
    torch.cuda.synchronize()
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    e_out = rel_err(outs["tiled"], ref.detach())
    print(f"  out: vs oracle {e_out:.2e}", flush=True)
    assert e_out < tol
    assert rel_err(outs["tiled"], outs["direct"]) < tol
    for name, r, gt, gd in zip(("dq", "dk", "dv", "doff"), (qq.grad, kk.grad, vv.grad, oo.grad),
                               grads["tiled"], grads["direct"]):
        e_ref, e_dir = rel_err(gt, r), rel_err(gt, gd)
        print(f"  {name}: vs oracle {e_ref:.2e}  vs direct {e_dir:.2e}", flush=True)
        assert e_ref < tol, name
        assert e_dir < tol, name


# Shapes where the column-streaming dq/dK/dV kernel (bf16, fp32 dK/dV sums) walks
# both columns of a pair at once: frames reach few planes (window depth 1, or
# small offsets) and the pair's box takes no more chunks than one column's, so
# one walk of four 32-query ring slots costs less than two of eight 16-query
# slots.  Odd column counts leave a last column to walk alone.
@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, kernel, off_std, scale, head_dim
    (1, 8, 8, 16, 2, (1, 7, 7), 0.3, 1.0, 64),    # frames reach 2 planes
    (1, 10, 8, 20, 1, (3, 5, 5), 0.2, 0.9, 96),   # 5 columns; frames share planes
    (2, 7, 5, 12, 2, (3, 5, 5), 0.4, 1.1, 128),   # 3 columns, B = 2, partial tiles
    (1, 9, 12, 8, 2, (2, 3, 3), 0.6, 1.0, 32),
])
def test_tiled_column_pairs_vs_oracle_and_direct(shape):
    B, T, H, W, nh, ks, off_std, scale, hd = shape
    print(f"[tiled column pairs] {shape}", flush=True)
    q, k, v, off = _inputs(B, T, H, W, nh, ks, off_std, 700 + T * H * W + hd, hd=hd)
    g = torch.Generator().manual_seed(19)
    dout = torch.randn(q.shape, generator=g).to(torch.bfloat16)
    qq, kk, vv, oo = (t.float().requires_grad_(True) for t in (q, k, v, off))
    ref = dsa3d_core_ref(qq, kk, vv, oo, (T, H, W), nh, ks, scale)
    ref.backward(dout.float())
    grads = {}
    for algo in ("tiled", "direct"):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, off)]
        out = core()(*ts, (T, H, W), nh, ks, scale, algo=algo)
        out.backward(dout.to(DEV))
        grads[algo] = [t.grad.float().cpu() for t in ts]
    torch.cuda.synchronize()
    for name, r, gt, gd in zip(("dq", "dk", "dv", "doff"), (qq.grad, kk.grad, vv.grad, oo.grad),
                               grads["tiled"], grads["direct"]):
        e_ref, e_dir = rel_err(gt, r), rel_err(gt, gd)
        print(f"  {name}: vs oracle {e_ref:.2e}  vs direct {e_dir:.2e}", flush=True)
        assert e_ref < BF16_TOL, name
        assert e_dir < BF16_TOL, name


# Shapes where the column-streaming kernel leaves columns to the tile kernel:
# offsets large enough that a tile's taps span more planes than its record
# header has bins, or that a frame starts before its ring slot's previous
# frame ends.
@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, kernel, off_std, scale, head_dim
    (1, 20, 8, 8, 1, (3, 5, 5), 6.0, 1.0, 64),
    (1, 14, 8, 12, 2, (3, 7, 7), 2.0, 0.8, 96),
])
def test_tiled_listed_columns_vs_oracle_and_direct(shape):
    test_tiled_column_pairs_vs_oracle_and_direct(shape)


# Corner boxes two chunks tall and one chunk wide (W <= 16, tall grids, large
# offsets): the column-streaming kernel's plane walk visits chunks (1, 0),
# (2, 0), ... whose records it must match by row chunk as well.
@pytest.mark.parametrize("shape", [
    # B, T, H, W, nh, kernel, off_std, scale, head_dim
    (1, 5, 24, 8, 1, (3, 7, 7), 4.0, 1.0, 64),
    (1, 7, 17, 6, 2, (3, 3, 3), 6.0, 1.2, 64),
    (2, 4, 20, 1, 2, (3, 5, 5), 8.0, 1.0, 96),
])
def test_tiled_tall_boxes_vs_oracle_and_direct(shape):
    test_tiled_column_pairs_vs_oracle_and_direct(shape)
