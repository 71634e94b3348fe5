"""msd_dsa3d_bwd_noalloc, the backward without a workspace argument, against
msd_dsa3d_bwd on the same inputs, through the C ABI (GPU).

Two calls in a row on each kernel family, the second smaller: the static
scratch keeps the first call's contents, so a second call that read stale
scratch would differ.  dq and the offset gradients are computed without
atomics and must match bit for bit; dK and dV are accumulated with global
atomics in an order that varies from run to run, so they are compared at the
parity tolerance (fp32 1e-4, bf16 2e-2, relative to max|ref|).
"""

import ctypes
import math

import pytest
import torch

from goldens import rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, T, H, W, nh, hd, ks, dtype, seed):
    N, D = T * H * W, nh * hd
    C = nh * ks[0] * ks[1] * ks[2] * 3
    g = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v, dout = (torch.randn(B, N, D, generator=g, device=DEV).to(dtype) for _ in range(4))
    off = (torch.randn(B, N, C, generator=g, device=DEV) * 1.2).to(dtype)
    return q, k, v, off, dout


def _both(shape, dtype, algo, seed):
    from megaslide_amd import _lib
    lib = _lib.load()
    B, T, H, W, nh, hd, ks = shape
    N, D = T * H * W, nh * hd
    q, k, v, off, dout = _inputs(B, T, H, W, nh, hd, ks, dtype, seed)
    desc = _lib.DsaDesc(B, T, H, W, nh, hd, *ks, _lib.dtype_code(dtype), D, D, D, 1.0,
                        1.0 / math.sqrt(hd), _lib.ALGOS[algo])
    need = lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(desc))
    assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
    out = torch.empty_like(q)
    lse = torch.empty(B, N, nh, device=DEV, dtype=torch.float32)
    sh = torch.cuda.current_stream().cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731
    _lib.check(lib.msd_dsa3d_fwd(ctypes.byref(desc), P(q), P(k), P(v), P(off), None, None, P(out),
                                 P(lse), sh), "fwd")
    res = []
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    for noalloc in (False, True):
        grads = [torch.full_like(t, float("nan")) for t in (q, k, v, off)]
        args = [ctypes.byref(desc), P(q), P(k), P(v), P(off), None, None, P(out), P(dout), P(lse),
                None, *(P(t) for t in grads), None, None]
        if noalloc:
            rc = lib.msd_dsa3d_bwd_noalloc(*args, sh)
        else:
            rc = lib.msd_dsa3d_bwd(*args, P(ws), need, sh)
        _lib.check(rc, "noalloc bwd" if noalloc else "bwd")
        res.append(grads)
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize("dtype,algo,hd", [(torch.bfloat16, "tiled", 64),
                                           (torch.float32, "tiled", 96),
                                           (torch.float32, "direct", 16)])
def test_noalloc_matches_workspace_entry_point(dtype, algo, hd):
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for shape, seed in (((2, 6, 16, 16, 4, hd, (3, 7, 7)), 1),   # 3,072 tokens
                        ((1, 3, 7, 9, 2, hd, (3, 5, 5)), 2)):    # then a smaller call
        print(f"[noalloc] {dtype} {algo} {shape}", flush=True)
        (dq0, dk0, dv0, do0), (dq1, dk1, dv1, do1) = _both(shape, dtype, algo, seed)
        for t in (dq1, dk1, dv1, do1):
            assert torch.isfinite(t.float()).all()
        if algo == "tiled":
            assert torch.equal(dq0, dq1) and torch.equal(do0, do1)
        else:
            assert rel_err(dq1.float().cpu(), dq0.float().cpu()) < tol
            assert rel_err(do1.float().cpu(), do0.float().cpu(), floor=1e-6) < tol
        assert rel_err(dk1.float().cpu(), dk0.float().cpu()) < tol
        assert rel_err(dv1.float().cpu(), dv0.float().cpu()) < tol


def test_noalloc_rejects_calls_beyond_its_scratch():
    from megaslide_amd import _lib
    lib = _lib.load()
    # 64 x 32 x 32 tokens x 16 heads x 147 taps x 8 bytes: ~1.2 GB of scratch
    desc = _lib.DsaDesc(1, 64, 32, 32, 16, 64, 3, 7, 7, _lib.MSD_BF16, 1024, 1024, 1024, 1.0, 0.125)
    x = torch.empty(16, dtype=torch.bfloat16, device=DEV)
    p = x.data_ptr()
    rc = lib.msd_dsa3d_bwd_noalloc(ctypes.byref(desc), *([p] * 4), None, None, *([p] * 3), None,
                                   *([p] * 4), None, None, torch.cuda.current_stream().cuda_stream)
    assert rc == -4
    assert b"maximum" in lib.msd_last_error()
