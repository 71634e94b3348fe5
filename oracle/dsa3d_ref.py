"""PyTorch-CPU restatement of the reference 3D-DSA operator (oracle).

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  Never used by the product path.

Every function follows the reference op sequence of
``DeformableSlideAttention3D`` (infinity/video/attention.py) and cites the lines
it restates.  Tensors are channel-last at the interface, like the HIP kernels:

* ``q, k, v``            [B, N, D], N = T*H*W, token n = (t*H + h)*W + w
  (infinity/video/model.py:206), channel c = head*hd + d (attention.py:135-137).
* ``off``                [B, N, C], C = nh*kt*kh*kw*3, channel
  ((((m*kt + i)*kh + j)*kw + k)*3 + slot) -- the order of the reference's
  ``offsets.view(B, nh, kt, kh, kw, 3, T, H, W)`` (attention.py:109).
* dwconv weights         [D, 1, kt, kh, kw] as nn.Conv3d(groups=D) stores them.

Pinning (see tests/test_oracle_*.py): golden vectors written by the reference
module (tests/golden/make_golden.py), the numpy brute-force sampler in
``oracle.bruteforce``, closed-form invariants, and fp64 gradcheck.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor


# ---------------------------------------------------------------------------
# base grid and offset normalisation
# ---------------------------------------------------------------------------

def _axis_positions(S: int, k: int, device=None) -> Tensor:
    """Normalised tap positions along one axis, [S, k], computed in fp32.

    attention.py:209-230: ``arange`` in float32, centred kernel taps
    ``arange(k) - k//2``, absolute position p + c, then ``2*p/max(S-1,1) - 1``
    (the align_corners=True normalisation, sampled later with
    align_corners=False -- a reference quirk that parity keeps).
    """
    p = torch.arange(S, device=device, dtype=torch.float32).view(S, 1)
    c = torch.arange(k, device=device, dtype=torch.float32) - (k // 2)
    return 2 * (p + c.view(1, k)) / max(S - 1, 1) - 1


def base_grid(T: int, H: int, W: int, kernel_size: Sequence[int], device=None) -> Tensor:
    """[T, H, W, kt, kh, kw, 3] fp32 base sampling grid, components (x=w, y=h, z=t).

    attention.py:194-238 (``_get_base_grid``); stack order [w, h, t] at :236.
    """
    kt, kh, kw = kernel_size
    gz = _axis_positions(T, kt, device).view(T, 1, 1, kt, 1, 1)
    gy = _axis_positions(H, kh, device).view(1, H, 1, 1, kh, 1)
    gx = _axis_positions(W, kw, device).view(1, 1, W, 1, 1, kw)
    shape = (T, H, W, kt, kh, kw)
    return torch.stack([gx.expand(shape), gy.expand(shape), gz.expand(shape)], dim=-1)


def normalise_offsets(off: Tensor, T: int, H: int, W: int) -> Tensor:
    """Map raw offset slots to grid units, attention.py:118-124.

    Slot 0 is divided by (T-1) and slot 2 by (W-1) although slot 0 is added to
    grid component x (the W axis) and slot 2 to z (the T axis); a slot stays
    zero when its divisor dimension is 1.  ``off`` is [..., 3].
    """
    out = torch.zeros_like(off)
    if T > 1:
        out[..., 0] = off[..., 0] / (T - 1)
    if H > 1:
        out[..., 1] = off[..., 1] / (H - 1)
    if W > 1:
        out[..., 2] = off[..., 2] / (W - 1)
    return out


# ---------------------------------------------------------------------------
# attention core
# ---------------------------------------------------------------------------

def _heads_volume(t: Tensor, B: int, T: int, H: int, W: int, nh: int, hd: int) -> Tensor:
    """[B, N, D] -> [B, nh, hd, T, H, W] (attention.py:135-141)."""
    return t.reshape(B, T, H, W, nh, hd).permute(0, 4, 5, 1, 2, 3)


def _dropout_factors(dropout, B, N, Nq, nh, h0, h1, K, query_index, p) -> Tensor:
    """[B, h1-h0, Nq, K(+G)] factors 0 or 1/(1-p): tap k < K of the window, then
    extra key g as tap K + g (the counter the kernels draw for it)."""
    import numpy as np

    from .philox import dropout_scale, keep_mask

    prob, seed, offset = dropout
    n = (np.arange(Nq) if query_index is None
         else np.asarray(torch.as_tensor(query_index).cpu(), dtype=np.int64))
    rows = (np.arange(B, dtype=np.int64).reshape(B, 1) * N + n.reshape(1, -1)).reshape(-1)
    taps = p.shape[-1]
    keep = keep_mask(prob, seed, offset, rows, nh, taps).reshape(B, Nq, nh, taps)[:, :, h0:h1]
    f = torch.from_numpy(np.where(keep, dropout_scale(prob), np.float32(0.0)).astype(np.float32))
    return f.permute(0, 2, 1, 3).to(p.dtype)


def dsa3d_core_ref(q: Tensor, k: Tensor, v: Tensor, off: Tensor,
                   video_shape: Sequence[int], num_heads: int,
                   kernel_size: Sequence[int] = (3, 7, 7), offset_scale: float = 1.0,
                   head_chunk: Optional[int] = None, return_lse: bool = False,
                   extra_k: Optional[Tensor] = None, extra_v: Optional[Tensor] = None,
                   query_index: Optional[Tensor] = None,
                   dropout: Optional[Tuple[float, int, int]] = None):
    """Deformable local attention core, reference op sequence.

    Restates attention.py:106-186 without the projections: scale the offsets
    (:106), permute (:109-111), base grid + normalised offsets (:113-127),
    ``F.grid_sample`` of K and V (:144-145, :240-273), flatten taps in
    (i*kh + j)*kw + k order (:152-157), ``matmul / sqrt(hd)`` (:176),
    ``softmax`` (:179), weighted sum (:183), heads back to [B, N, D] (:186).

    ``extra_k``/``extra_v`` ([B, G, D], already projected) are appended to every
    query's tap list before the softmax, as attention.py:160-173 does with the
    projected ``extra_kv``.

    Heads are independent, so ``head_chunk`` splits them to bound memory; the
    result is identical.  ``query_index`` (1-D token indices) restricts the
    queries to a subset while K/V keep the full volume -- exact for those
    queries, since each query's output, dq and d offsets depend on its own taps
    only.  Returns out [B, Nq, D] (and the per-(b, head, token) log-sum-exp
    [B, nh, Nq] of the scores when ``return_lse``).

    ``dropout = (p, seed, offset)`` applies the reference's attention dropout
    (attention.py:180) to the local taps' softmax weights with the keep mask of
    ``oracle.philox.keep_mask`` (the generator the HIP kernels use) and the
    fp32 scale 1 / (1 - p); extra key g is dropped as tap K + g.
    """
    B, N, D = q.shape
    T, H, W = video_shape
    assert N == T * H * W
    nh = num_heads
    hd = D // nh
    kt, kh, kw = kernel_size
    K = kt * kh * kw
    hc = nh if head_chunk is None else max(1, min(nh, head_chunk))

    grid0 = base_grid(T, H, W, kernel_size, device=q.device).reshape(N, kt, kh, kw, 3)
    offs = (off * offset_scale).reshape(B, N, nh, kt, kh, kw, 3).permute(0, 2, 1, 3, 4, 5, 6)
    kvol = _heads_volume(k, B, T, H, W, nh, hd)
    vvol = _heads_volume(v, B, T, H, W, nh, hd)
    qh = q.reshape(B, N, nh, hd).permute(0, 2, 1, 3)  # [B, nh, N, hd]
    if query_index is not None:
        grid0 = grid0[query_index]
        offs = offs[:, :, query_index]
        qh = qh[:, :, query_index]
    Nq = grid0.shape[0]

    outs, lses = [], []
    for h0 in range(0, nh, hc):
        h1 = min(nh, h0 + hc)
        m = h1 - h0
        grid = grid0 + normalise_offsets(offs[:, h0:h1], T, H, W)  # [B,m,Nq,kt,kh,kw,3]
        g = grid.reshape(B * m, Nq, K, 1, 3)
        ks = F.grid_sample(kvol[:, h0:h1].reshape(B * m, hd, T, H, W), g,
                           mode="bilinear", padding_mode="border", align_corners=False)
        vs = F.grid_sample(vvol[:, h0:h1].reshape(B * m, hd, T, H, W), g,
                           mode="bilinear", padding_mode="border", align_corners=False)
        ks = ks.reshape(B, m, hd, Nq, K).permute(0, 1, 3, 2, 4)  # [B,m,Nq,hd,K]
        vs = vs.reshape(B, m, hd, Nq, K).permute(0, 1, 3, 2, 4)
        if extra_k is not None:
            G = extra_k.shape[1]
            ek = extra_k.reshape(B, G, nh, hd)[:, :, h0:h1].permute(0, 2, 3, 1)  # [B,m,hd,G]
            ev = extra_v.reshape(B, G, nh, hd)[:, :, h0:h1].permute(0, 2, 3, 1)
            ks = torch.cat([ks, ek.unsqueeze(2).expand(B, m, Nq, hd, G)], dim=-1)
            vs = torch.cat([vs, ev.unsqueeze(2).expand(B, m, Nq, hd, G)], dim=-1)
        qq = qh[:, h0:h1]  # [B,m,Nq,hd]
        scores = torch.matmul(qq.unsqueeze(-2), ks).squeeze(-2) / math.sqrt(hd)  # [B,m,N,K]
        p = F.softmax(scores, dim=-1)
        if dropout is not None and dropout[0] > 0:
            p = p * _dropout_factors(dropout, B, N, Nq, nh, h0, h1, K, query_index, p)
        o = torch.matmul(p.unsqueeze(-2), vs.transpose(-2, -1)).squeeze(-2)  # [B,m,N,hd]
        outs.append(o)
        if return_lse:
            lses.append(torch.logsumexp(scores, dim=-1))
    out = torch.cat(outs, dim=1).permute(0, 2, 1, 3).reshape(B, Nq, D)
    if return_lse:
        return out, torch.cat(lses, dim=1)
    return out


# ---------------------------------------------------------------------------
# depthwise convolutions and the offset predictor
# ---------------------------------------------------------------------------

def dwconv3d_ref(x: Tensor, weight: Tensor, bias: Optional[Tensor],
                 video_shape: Sequence[int], act: str = "none") -> Tensor:
    """Depthwise 3-D conv on channel-last tokens, zero padding k//2.

    attention.py:58-65 (``dw_conv``) and :71-72 (``offset_net[0:2]``, act="gelu",
    exact-erf GELU as nn.GELU() defaults).  x [B, N, D] -> [B, N, D].
    """
    B, N, D = x.shape
    T, H, W = video_shape
    kt, kh, kw = weight.shape[-3:]
    x5 = x.transpose(1, 2).reshape(B, D, T, H, W)
    y = F.conv3d(x5, weight, bias, padding=(kt // 2, kh // 2, kw // 2), groups=D)
    if act == "gelu":
        y = F.gelu(y)
    elif act != "none":
        raise ValueError(act)
    return y.reshape(B, D, N).transpose(1, 2)


def predict_offsets_ref(x: Tensor, params: Dict[str, Tensor], video_shape: Sequence[int]) -> Tensor:
    """``offset_net(x)`` as channel-last [B, N, C] (attention.py:70-74, :105)."""
    f = dwconv3d_ref(x, params["offset_net.0.weight"], params["offset_net.0.bias"],
                     video_shape, act="gelu")
    w2 = params["offset_net.2.weight"]
    return F.linear(f, w2.reshape(w2.shape[0], -1), params["offset_net.2.bias"])


# Parameter names, in registration order, of the reference module
# (attention.py:52-74); state_dict keys of the drop-in must match.
PARAM_NAMES = (
    "q_proj.weight", "q_proj.bias", "k_proj.weight", "k_proj.bias",
    "v_proj.weight", "v_proj.bias", "out_proj.weight", "out_proj.bias",
    "dw_conv.weight", "dw_conv.bias",
    "offset_net.0.weight", "offset_net.0.bias",
    "offset_net.2.weight", "offset_net.2.bias",
)


def param_shapes(D: int, nh: int, kernel_size: Sequence[int]) -> Dict[str, Tuple[int, ...]]:
    kt, kh, kw = kernel_size
    C = nh * kt * kh * kw * 3
    return {
        "q_proj.weight": (D, D), "q_proj.bias": (D,),
        "k_proj.weight": (D, D), "k_proj.bias": (D,),
        "v_proj.weight": (D, D), "v_proj.bias": (D,),
        "out_proj.weight": (D, D), "out_proj.bias": (D,),
        "dw_conv.weight": (D, 1, kt, kh, kw), "dw_conv.bias": (D,),
        "offset_net.0.weight": (D, 1, 3, 3, 3), "offset_net.0.bias": (D,),
        "offset_net.2.weight": (C, D, 1, 1, 1), "offset_net.2.bias": (C,),
    }


def dsa3d_module_ref(x: Tensor, params: Dict[str, Tensor], video_shape: Sequence[int],
                     num_heads: int, kernel_size: Sequence[int] = (3, 7, 7),
                     offset_scale: float = 1.0, head_chunk: Optional[int] = None,
                     offsets: Optional[Tensor] = None,
                     extra_kv: Optional[Tensor] = None) -> Tensor:
    """Whole-module forward, attention.py:82-192 (dropout p = 0).

    ``offsets`` ([B, N, C], unscaled) replaces ``offset_net(x)`` when given, the
    way the golden generator injects offsets into the reference module.
    """
    dw = dwconv3d_ref(x, params["dw_conv.weight"], params["dw_conv.bias"], video_shape)
    off = predict_offsets_ref(x, params, video_shape) if offsets is None else offsets
    q = F.linear(x, params["q_proj.weight"], params["q_proj.bias"])
    k = F.linear(x, params["k_proj.weight"], params["k_proj.bias"])
    v = F.linear(x, params["v_proj.weight"], params["v_proj.bias"])
    ek = ev = None
    if extra_kv is not None:
        ek = F.linear(extra_kv, params["k_proj.weight"], params["k_proj.bias"])
        ev = F.linear(extra_kv, params["v_proj.weight"], params["v_proj.bias"])
    a = dsa3d_core_ref(q, k, v, off, video_shape, num_heads, kernel_size, offset_scale,
                       head_chunk=head_chunk, extra_k=ek, extra_v=ev)
    return F.linear(a, params["out_proj.weight"], params["out_proj.bias"]) + dw


# ---------------------------------------------------------------------------
# DiT block around the module (the path's caller)
# ---------------------------------------------------------------------------

def dit_block_ref(x: Tensor, params: Dict[str, Tensor], video_shape: Sequence[int],
                  num_heads: int, kernel_size: Sequence[int] = (3, 7, 7),
                  offset_scale: float = 1.0, head_chunk: Optional[int] = None) -> Tensor:
    """DiTBlock.forward without text conditioning (infinity/video/model.py:83-117,
    dropout p = 0): ``x + attn(norm1(x))`` (:102), then ``x + mlp(norm2(x))``
    (:115) with the MLP fc1 -> exact-erf GELU -> fc2 (model.py:21-35) and both
    LayerNorms at eps 1e-6 (:51, :63).  ``params`` uses the block's own
    parameter names (``norm1.*``, ``attn.*``, ``norm2.*``, ``mlp.fc1.*``,
    ``mlp.fc2.*``)."""
    D = x.shape[-1]
    attn_p = {n[len("attn."):]: t for n, t in params.items() if n.startswith("attn.")}
    a = F.layer_norm(x, (D,), params["norm1.weight"], params["norm1.bias"], eps=1e-6)
    x = x + dsa3d_module_ref(a, attn_p, video_shape, num_heads, kernel_size, offset_scale,
                             head_chunk=head_chunk)
    h = F.layer_norm(x, (D,), params["norm2.weight"], params["norm2.bias"], eps=1e-6)
    h = F.gelu(F.linear(h, params["mlp.fc1.weight"], params["mlp.fc1.bias"]))
    return x + F.linear(h, params["mlp.fc2.weight"], params["mlp.fc2.bias"])
