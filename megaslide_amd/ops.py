"""Autograd functions over the HIP kernels.

``dsa3d_core``   attention core (trilinear K/V sampling + local softmax attention)
                 replacing infinity/video/attention.py:106-186 of the reference,
                 as the custom operators megaslide::dsa3d_core (+ _bwd).
``dwconv3d``     depthwise 3-D conv (+ optional exact-erf GELU) replacing the
                 reference's nn.Conv3d(groups=D) terms (attention.py:58-74).

Both save their inputs and outputs for an explicit backward, the reference's
own idiom for custom autograd (infinity/ops/layers.py:16-62).  They run only on
ROCm device tensors; there is no CPU path.
"""

from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib

Tensor = torch.Tensor


def _require_device(*ts: Optional[Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "megaslide_amd kernels run on ROCm devices only; got a tensor on "
                f"{t.device} (there is no CPU implementation)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"megaslide_amd: tensors on different devices ({dev}, {t.device})")
    return dev


def _tokens_major(t: Tensor, B: int, N: int, D: int) -> Tensor:
    """[B, N, D] view with unit channel stride and a uniform token stride."""
    if t.shape != (B, N, D):
        raise ValueError(f"expected shape {(B, N, D)}, got {tuple(t.shape)}")
    if t.stride(2) == 1 and t.stride(0) == N * t.stride(1) and t.stride(1) >= D:
        return t
    return t.contiguous()


class _CoreCall:
    """Validated shapes of one attention-core call and its C descriptor."""

    def __init__(self, q, k, v, offsets, video_shape, num_heads, kernel_size, offset_scale, algo,
                 dropout=(0.0, 0, 0), extra_k=None, extra_v=None, dkv_accum="fp32"):
        self.dev = _require_device(q, k, v, offsets, extra_k, extra_v)
        B, N, D = q.shape
        T, H, W = (int(s) for s in video_shape)
        if N != T * H * W:
            raise ValueError(f"N={N} but T*H*W={T * H * W}")
        if D % num_heads != 0:
            raise ValueError(f"D={D} not divisible by num_heads={num_heads}")
        kt, kh, kw = (int(s) for s in kernel_size)
        C = num_heads * kt * kh * kw * 3
        dt = q.dtype
        for name, t in (("k", k), ("v", v), ("offsets", offsets)):
            if t.dtype != dt:
                raise TypeError(f"dsa3d_core: {name} is {t.dtype}, q is {dt}")
        if offsets.shape != (B, N, C):
            raise ValueError(f"offsets must be {(B, N, C)}, got {tuple(offsets.shape)}")
        if algo not in _lib.ALGOS:
            raise ValueError(f"algo must be one of {sorted(_lib.ALGOS)}")
        if dkv_accum not in _lib.ACCUMS:
            raise ValueError(f"dkv_accum must be one of {sorted(_lib.ACCUMS)}")
        if dkv_accum == "fp16" and dt != torch.bfloat16:
            raise ValueError("dkv_accum='fp16' needs bfloat16 tensors")
        self.q = _tokens_major(q, B, N, D)
        self.k = _tokens_major(k, B, N, D)
        self.v = _tokens_major(v, B, N, D)
        self.off = offsets.contiguous()
        self.B, self.N, self.D, self.T, self.H, self.W = B, N, D, T, H, W
        self.nh, self.hd = num_heads, D // num_heads
        self.ksz = (kt, kh, kw)
        self.dtype = dt
        self.offset_scale = float(offset_scale)
        self.algo = algo
        self.dkv_accum = dkv_accum
        p, seed, offset = dropout
        if not 0.0 <= float(p) < 1.0:
            raise ValueError(f"dropout probability must be in [0, 1), got {p}")
        self.dropout = (float(p), int(seed) & 0xFFFFFFFFFFFFFFFF, int(offset) & 0xFFFFFFFF)
        # extra keys / values shared by every query (attention.py:160-173)
        if (extra_k is None) != (extra_v is None):
            raise ValueError("extra_k and extra_v go together")
        self.G = 0
        self.ek = self.ev = None
        if extra_k is not None:
            G = extra_k.shape[1]
            for name, t in (("extra_k", extra_k), ("extra_v", extra_v)):
                if t.shape != (B, G, D):
                    raise ValueError(f"{name} must be {(B, G, D)}, got {tuple(t.shape)}")
                if t.dtype != dt:
                    raise TypeError(f"dsa3d_core: {name} is {t.dtype}, q is {dt}")
            self.G = G
            self.ek, self.ev = extra_k.contiguous(), extra_v.contiguous()

    def desc(self, qs=None, ks=None, vs=None) -> _lib.DsaDesc:
        kt, kh, kw = self.ksz
        return _lib.DsaDesc(
            self.B, self.T, self.H, self.W, self.nh, self.hd, kt, kh, kw,
            _lib.dtype_code(self.dtype),
            self.q.stride(1) if qs is None else qs,
            self.k.stride(1) if ks is None else ks,
            self.v.stride(1) if vs is None else vs,
            self.offset_scale, 1.0 / math.sqrt(self.hd), _lib.ALGOS[self.algo],
            self.dropout[2], self.dropout[1], self.dropout[0], self.G,
            _lib.ACCUMS[self.dkv_accum])

    def forward(self, want_lse: bool):
        out = torch.empty((self.B, self.N, self.D), dtype=self.dtype, device=self.dev)
        lse = (torch.empty((self.B, self.N, self.nh), dtype=torch.float32, device=self.dev)
               if want_lse else None)
        desc = self.desc()
        lib = _lib.load()
        with torch.cuda.device(self.dev):
            _lib.check(lib.msd_dsa3d_fwd(ctypes.byref(desc), self.q.data_ptr(), self.k.data_ptr(),
                                         self.v.data_ptr(), self.off.data_ptr(), _lib.ptr(self.ek),
                                         _lib.ptr(self.ev), out.data_ptr(), _lib.ptr(lse),
                                         _lib.stream_handle(self.dev)), "dsa3d_fwd")
        return out, lse


# The attention core is a torch.library custom operator (forward and
# backward), so the dispatcher sees it: torch.utils.checkpoint's selective
# policies can keep its outputs instead of recomputing it (keep_core_policy
# below), and torch.compile treats it as one opaque op.  The seed travels as a
# signed 64-bit int (the schema's int), the bits unchanged.

def _seed_in(seed: int) -> int:
    seed &= 0xFFFFFFFFFFFFFFFF
    return seed - (1 << 64) if seed >= (1 << 63) else seed


def _call(q, k, v, offsets, extra_k, extra_v, video_shape, num_heads, kernel_size,
          offset_scale, algo, dropout_p, dropout_seed, dropout_offset, dkv_accum) -> _CoreCall:
    return _CoreCall(q, k, v, offsets, video_shape, num_heads, kernel_size, offset_scale, algo,
                     (dropout_p, dropout_seed & 0xFFFFFFFFFFFFFFFF, dropout_offset), extra_k,
                     extra_v, dkv_accum)


@torch.library.custom_op("megaslide::dsa3d_core", mutates_args=(), device_types="cuda")
def _core_fwd_op(q: Tensor, k: Tensor, v: Tensor, offsets: Tensor, extra_k: Optional[Tensor],
                 extra_v: Optional[Tensor], video_shape: List[int], num_heads: int,
                 kernel_size: List[int], offset_scale: float, algo: str, dropout_p: float,
                 dropout_seed: int, dropout_offset: int,
                 dkv_accum: str) -> Tuple[Tensor, Tensor]:
    """out [B, N, D] and lse [B, N, num_heads] (fp32) of the attention core."""
    call = _call(q, k, v, offsets, extra_k, extra_v, video_shape, num_heads, kernel_size,
                 offset_scale, algo, dropout_p, dropout_seed, dropout_offset, dkv_accum)
    return call.forward(want_lse=True)


@_core_fwd_op.register_fake
def _(q, k, v, offsets, extra_k, extra_v, video_shape, num_heads, kernel_size, offset_scale, algo,
      dropout_p, dropout_seed, dropout_offset, dkv_accum):
    B, N, D = q.shape
    return q.new_empty((B, N, D)), q.new_empty((B, N, num_heads), dtype=torch.float32)


@torch.library.custom_op("megaslide::dsa3d_core_bwd", mutates_args=(), device_types="cuda")
def _core_bwd_op(q: Tensor, k: Tensor, v: Tensor, offsets: Tensor, extra_k: Optional[Tensor],
                 extra_v: Optional[Tensor], out: Tensor, lse: Tensor, dout: Tensor,
                 dlse: Optional[Tensor], video_shape: List[int], num_heads: int,
                 kernel_size: List[int], offset_scale: float, algo: str, dropout_p: float,
                 dropout_seed: int, dropout_offset: int,
                 dkv_accum: str) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """dq, dk, dv, d offsets and (empty without extra keys) d extra_k, d extra_v."""
    B, N, D = q.shape
    dt, dev = q.dtype, q.device
    dout = dout.to(dt).contiguous()
    if dlse is not None:
        dlse = dlse.to(torch.float32).contiguous()
    # gradients are written with the token strides of the desc: contiguous here
    qc, kc, vc = (t if t.stride(1) == D else t.contiguous() for t in (q, k, v))
    call = _call(qc, kc, vc, offsets, extra_k, extra_v, video_shape, num_heads, kernel_size,
                 offset_scale, algo, dropout_p, dropout_seed, dropout_offset, dkv_accum)
    desc = call.desc(D, D, D)
    dq = torch.empty((B, N, D), dtype=dt, device=dev)
    dk = torch.empty((B, N, D), dtype=dt, device=dev)
    dv = torch.empty((B, N, D), dtype=dt, device=dev)
    doff = torch.empty_like(call.off)
    has_extra = call.G > 0
    dek = torch.empty_like(call.ek) if has_extra else q.new_empty((0,))
    dev_ = torch.empty_like(call.ev) if has_extra else q.new_empty((0,))
    lib = _lib.load()
    ws_bytes = lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(desc))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.msd_dsa3d_bwd(
            ctypes.byref(desc), qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), call.off.data_ptr(),
            _lib.ptr(call.ek), _lib.ptr(call.ev), out.contiguous().data_ptr(), dout.data_ptr(),
            lse.contiguous().data_ptr(), _lib.ptr(dlse), dq.data_ptr(), dk.data_ptr(),
            dv.data_ptr(), doff.data_ptr(), _lib.ptr(dek if has_extra else None),
            _lib.ptr(dev_ if has_extra else None), ws.data_ptr(), ws_bytes,
            _lib.stream_handle(dev)), "dsa3d_bwd")
    return dq, dk, dv, doff, dek, dev_


@_core_bwd_op.register_fake
def _(q, k, v, offsets, extra_k, extra_v, out, lse, dout, dlse, video_shape, num_heads,
      kernel_size, offset_scale, algo, dropout_p, dropout_seed, dropout_offset, dkv_accum):
    e = q.new_empty((0,))
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            torch.empty_like(offsets), torch.empty_like(extra_k) if extra_k is not None else e,
            torch.empty_like(extra_v) if extra_v is not None else e)


_NON_TENSOR = ("video_shape", "num_heads", "kernel_size", "offset_scale", "algo", "dropout_p",
               "dropout_seed", "dropout_offset", "dkv_accum")


def _core_setup(ctx, inputs, output):
    q, k, v, offsets, extra_k, extra_v = inputs[:6]
    ctx.args = inputs[6:]
    ctx.has_extra = extra_k is not None
    out, lse = output
    ctx.save_for_backward(q, k, v, offsets, extra_k, extra_v, out, lse)


def _core_backward(ctx, dout, dlse):
    q, k, v, offsets, extra_k, extra_v, out, lse = ctx.saved_tensors
    if dout is None:
        dout = torch.zeros_like(out)
    dq, dk, dv, doff, dek, dev_ = _core_bwd_op(q, k, v, offsets, extra_k, extra_v, out, lse, dout,
                                               dlse, *ctx.args)
    if not ctx.has_extra:
        dek = dev_ = None
    return (dq, dk, dv, doff, dek, dev_) + (None,) * len(_NON_TENSOR)


_core_fwd_op.register_autograd(_core_backward, setup_context=_core_setup)


def keep_core_policy(ctx, op, *args, **kwargs):
    """Selective-checkpoint policy (torch.utils.checkpoint with
    create_selective_checkpoint_contexts): keep the attention core's outputs
    (out, lse: D + 4 nh / e bytes a token) from the forward, recompute the
    rest.  The backward's recomputed forward then skips the core, the costliest
    kernel of the recompute, while the projections, convolutions and norms are
    rerun as usual."""
    from torch.utils.checkpoint import CheckpointPolicy
    if op is torch.ops.megaslide.dsa3d_core.default:
        return CheckpointPolicy.MUST_SAVE
    return CheckpointPolicy.PREFER_RECOMPUTE


def keep_core_context():
    """context_fn for torch.utils.checkpoint.checkpoint(..., use_reentrant=False)
    that applies keep_core_policy."""
    from torch.utils.checkpoint import create_selective_checkpoint_contexts
    return create_selective_checkpoint_contexts(keep_core_policy)


def keep_gemms_policy(ctx, op, *args, **kwargs):
    """Selective-checkpoint policy that keeps the attention core's outputs and
    every GEMM's (the q/k/v, offset, output and MLP projections: aten mm /
    addmm), so the backward's recomputed forward reruns only elementwise work,
    the LayerNorms and the depthwise convolutions.  A DiT block at 46,800
    tokens, dim 1,536, then keeps ~2 GB of activations beyond its input."""
    from torch.utils.checkpoint import CheckpointPolicy
    if op in (torch.ops.megaslide.dsa3d_core.default, torch.ops.aten.mm.default,
              torch.ops.aten.addmm.default):
        return CheckpointPolicy.MUST_SAVE
    return CheckpointPolicy.PREFER_RECOMPUTE


def keep_gemms_context():
    """context_fn for torch.utils.checkpoint.checkpoint(..., use_reentrant=False)
    that applies keep_gemms_policy."""
    from torch.utils.checkpoint import create_selective_checkpoint_contexts
    return create_selective_checkpoint_contexts(keep_gemms_policy)


def dsa3d_core(q: Tensor, k: Tensor, v: Tensor, offsets: Tensor, video_shape: Sequence[int],
               num_heads: int, kernel_size: Sequence[int] = (3, 7, 7), offset_scale: float = 1.0,
               return_lse: bool = False, algo: str = "auto", dropout_p: float = 0.0,
               dropout_seed: Optional[int] = None, dropout_offset: int = 0,
               extra_k: Optional[Tensor] = None, extra_v: Optional[Tensor] = None,
               dkv_accum: str = "fp32"):
    """Attention core on device tensors.

    q, k, v: [B, N, D]; offsets: [B, N, num_heads*kt*kh*kw*3] unscaled, channel
    order [head][i][j][k][slot] (the reference's offsets.view order,
    attention.py:109).  Returns out [B, N, D] (and lse [B, N, num_heads]).
    ``algo``: "auto" (default), "direct" or "tiled" kernel family.

    ``dropout_p`` > 0 drops softmax weights as the reference's nn.Dropout does
    (attention.py:180): kept weights are scaled by 1 / (1 - p).  The keep mask
    comes from Philox4x32-10 keyed by ``dropout_seed`` (drawn from torch's
    default CPU generator when None, so torch.manual_seed makes it repeatable);
    the backward reuses the forward's mask.

    ``extra_k`` / ``extra_v`` ([B, G, D], already projected) are G keys and
    values shared by every query, appended to its taps before the softmax
    (the reference's ``extra_kv``, attention.py:160-173); extra key g is tap
    K + g for dropout.

    ``dkv_accum`` chooses how the backward sums dK / dV over query tiles:
    "fp32" (default, the reference's fp32 grid_sample backward precision) or,
    for bfloat16 tensors, "fp16" (power-of-two-scaled fp16 pairs: fewer atomic
    bytes, 11 significant bits per running sum, an fp32 redo on overflow).
    """
    p = float(dropout_p)
    if p > 0.0 and dropout_seed is None:
        dropout_seed = int(torch.randint(0, 2**63 - 1, (1,), dtype=torch.int64).item())
    dropout = (p, 0 if dropout_seed is None else int(dropout_seed), int(dropout_offset))
    grads = [t for t in (q, k, v, offsets, extra_k, extra_v) if t is not None]
    if torch.is_grad_enabled() and any(t.requires_grad for t in grads):
        out, lse = torch.ops.megaslide.dsa3d_core(
            q, k, v, offsets, extra_k, extra_v, [int(s) for s in video_shape], int(num_heads),
            [int(s) for s in kernel_size], float(offset_scale), algo, dropout[0],
            _seed_in(dropout[1]), dropout[2], dkv_accum)
        return (out, lse) if return_lse else out
    # forward only: nothing saved, no lse unless asked for
    call = _CoreCall(q, k, v, offsets, video_shape, num_heads, kernel_size, offset_scale, algo,
                     dropout, extra_k, extra_v, dkv_accum)
    out, lse = call.forward(want_lse=return_lse)
    return (out, lse) if return_lse else out


# ---------------------------------------------------------------------------
# depthwise conv
# ---------------------------------------------------------------------------

_ACT = {None: 0, "none": 0, "gelu": 1}


def _conv_desc(x: Tensor, video_shape, kernel: Tuple[int, int, int], act: int) -> _lib.ConvDesc:
    B, N, C = x.shape
    T, H, W = (int(s) for s in video_shape)
    if N != T * H * W:
        raise ValueError(f"N={N} but T*H*W={T * H * W}")
    kt, kh, kw = kernel
    return _lib.ConvDesc(B, T, H, W, C, kt, kh, kw, _lib.dtype_code(x.dtype), act)


class DwConv3dFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, video_shape, act, keep_preact):
        dev = _require_device(x, weight, bias)
        x = x.contiguous()
        C = x.shape[2]
        kernel = tuple(int(s) for s in weight.shape[-3:])
        if weight.numel() != C * kernel[0] * kernel[1] * kernel[2]:
            raise ValueError(f"weight {tuple(weight.shape)} does not match {C} channels")
        w = weight.to(x.dtype).contiguous()
        b = None if bias is None else bias.to(x.dtype).contiguous()
        desc = _conv_desc(x, video_shape, kernel, _ACT[act])
        y = torch.empty_like(x)
        # GELU: keep its input for the backward (what nn.GELU's autograd keeps)
        # when the caller will ask for a gradient (decided outside: autograd runs
        # this forward with gradients disabled)
        z = torch.empty_like(x) if (act == "gelu" and keep_preact) else None
        lib = _lib.load()
        with torch.cuda.device(dev):
            _lib.check(lib.msd_dwconv3d_fwd(ctypes.byref(desc), x.data_ptr(), w.data_ptr(),
                                            _lib.ptr(b), y.data_ptr(), _lib.ptr(z),
                                            _lib.stream_handle(dev)),
                       "dwconv3d_fwd")
        ctx.video_shape = tuple(video_shape)
        ctx.act = act
        ctx.kernel = kernel
        ctx.wdtype = weight.dtype
        ctx.bdtype = None if bias is None else bias.dtype
        ctx.save_for_backward(x, w, b, z)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, b, z = ctx.saved_tensors
        dev = x.device
        dy = dy.to(x.dtype).contiguous()
        need_x, need_w, need_b = ctx.needs_input_grad[:3]
        desc = _conv_desc(x, ctx.video_shape, ctx.kernel, _ACT[ctx.act])
        dx = torch.empty_like(x) if need_x else None
        dw = torch.empty_like(w) if need_w else None
        db = torch.empty_like(b) if (need_b and b is not None) else None
        lib = _lib.load()
        ws_bytes = lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(desc))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            _lib.check(lib.msd_dwconv3d_bwd(
                ctypes.byref(desc), x.data_ptr(), w.data_ptr(), _lib.ptr(b), _lib.ptr(z),
                dy.data_ptr(), _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(db), ws.data_ptr(), ws_bytes,
                _lib.stream_handle(dev)), "dwconv3d_bwd")
        if dw is not None:
            dw = dw.to(ctx.wdtype)
        if db is not None:
            db = db.to(ctx.bdtype)
        return dx, dw, db, None, None, None


def dwconv3d(x: Tensor, weight: Tensor, bias: Optional[Tensor], video_shape: Sequence[int],
             act: Optional[str] = None) -> Tensor:
    """Depthwise conv on channel-last tokens x [B, N, C]; weight [C, 1, kt, kh, kw]."""
    keep = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, weight, bias))
    return DwConv3dFunction.apply(x, weight, bias, tuple(video_shape), act, keep)
