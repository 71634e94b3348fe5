"""Drop-in ``DeformableSlideAttention3D`` running on the gfx950 HIP kernels.

Same constructor arguments, submodule names, parameter names/shapes/order,
default initialisation and ``forward(x, video_shape, extra_kv=None)`` signature
as the reference (infinity/video/attention.py:19-192), so ``DiTBlock``,
``MegaSlideDiT``, the hybrid wrappers and the CPU-master trainer can swap it in
and reference checkpoints load unchanged.

What runs where:
  * q/k/v/out projections and the 1x1 offset conv (offset_net[2]) are dense
    GEMMs and stay in PyTorch (hipBLASLt); the offset conv runs as a linear
    layer on channel-last features so offsets come out [B, N, C], and out_proj
    accumulates onto the dw_conv term in the same GEMM (torch.addmm), its bias
    folded into the conv's.
  * dw_conv (depthwise kt x kh x kw) and offset_net[0:2] (depthwise 3x3x3 +
    GELU) run as HIP depthwise-conv kernels on channel-last tokens.
  * offset scaling, base grid, trilinear K/V sampling with border clamp,
    scores, softmax and the weighted sum of V run fused in the HIP attention
    core, forward and backward.
  * ``extra_kv`` (attention.py:160-173) is merged exactly through the
    log-sum-exp: the HIP core returns the local output and its lse, the G extra
    keys shared by every query form a small dense attention in PyTorch, and the
    two softmax partitions are combined.

There is no CPU path: on CPU tensors ``forward`` raises.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .ops import dsa3d_core, dwconv3d


class DeformableSlideAttention3D(nn.Module):
    """3D Deformable Slide Attention (3D-DSA), HIP-kernel implementation.

    Args:
        hidden_size: Hidden dimension D.
        num_heads: Number of attention heads.
        kernel_size: Tuple (k_t, k_h, k_w) for the local neighbourhood.
        offset_scale: Scale factor for the learned offsets.
        dropout: Attention dropout rate on the softmax weights (training mode
            only, like nn.Dropout).  The kernels draw the keep mask from a
            Philox4x32-10 stream seeded from torch's default generator, so a
            fixed torch.manual_seed repeats it; it is not PyTorch's own stream.
    """

    def __init__(self, hidden_size: int, num_heads: int,
                 kernel_size: Tuple[int, int, int] = (3, 7, 7), offset_scale: float = 1.0,
                 dropout: float = 0.0):
        super().__init__()
        assert hidden_size % num_heads == 0, "hidden_size must be divisible by num_heads"
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = hidden_size // num_heads
        self.k_t, self.k_h, self.k_w = kernel_size
        self.offset_scale = offset_scale

        # registration order matches the reference (attention.py:52-80)
        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=True)
        self.k_proj = nn.Linear(hidden_size, hidden_size, bias=True)
        self.v_proj = nn.Linear(hidden_size, hidden_size, bias=True)
        self.out_proj = nn.Linear(hidden_size, hidden_size, bias=True)
        self.dw_conv = nn.Conv3d(hidden_size, hidden_size, kernel_size=kernel_size,
                                 padding=(self.k_t // 2, self.k_h // 2, self.k_w // 2),
                                 groups=hidden_size, bias=True)
        num_offsets = num_heads * self.k_t * self.k_h * self.k_w * 3
        self.offset_net = nn.Sequential(
            nn.Conv3d(hidden_size, hidden_size, 3, padding=1, groups=hidden_size),
            nn.GELU(),
            nn.Conv3d(hidden_size, num_offsets, 1, bias=True),
        )
        nn.init.zeros_(self.offset_net[-1].weight)
        nn.init.zeros_(self.offset_net[-1].bias)
        self.dropout = nn.Dropout(dropout)

    @property
    def kernel_size(self) -> Tuple[int, int, int]:
        return (self.k_t, self.k_h, self.k_w)

    def forward(self, x: Tensor, video_shape: Tuple[int, int, int],
                extra_kv: Optional[Tensor] = None) -> Tensor:
        B, N, D = x.shape
        T, H, W = video_shape
        assert N == T * H * W, f"Expected N={T*H*W} but got {N}"
        assert D == self.hidden_size
        if x.device.type != "cuda":
            raise RuntimeError("megaslide_amd.DeformableSlideAttention3D runs on ROCm devices "
                               "only (HIP kernels; no CPU implementation)")
        # attention dropout (attention.py:180): in training mode only, as nn.Dropout
        drop_p = self.dropout.p if self.training else 0.0

        # depthwise conv term and offset predictor, channel-last.  out_proj's bias
        # rides on the conv's, so the output projection below accumulates onto
        # the conv term in one GEMM (attention.py:187-192: out_proj(o) + dw_flat)
        dw = dwconv3d(x, self.dw_conv.weight, self.dw_conv.bias + self.out_proj.bias, video_shape)
        feat = dwconv3d(x, self.offset_net[0].weight, self.offset_net[0].bias, video_shape,
                        act="gelu")
        on2 = self.offset_net[2]
        off = F.linear(feat, on2.weight.view(on2.weight.shape[0], -1), on2.bias)

        q = self.q_proj(x)
        k = self.k_proj(x)
        v = self.v_proj(x)
        dt = q.dtype
        off = off.to(dt)
        if extra_kv is None:
            attn = dsa3d_core(q, k.to(dt), v.to(dt), off, video_shape, self.num_heads,
                              self.kernel_size, self.offset_scale, dropout_p=drop_p)
        else:
            attn = self._with_extra_kv(q, k.to(dt), v.to(dt), off, video_shape, extra_kv, drop_p)
        return torch.addmm(dw.reshape(B * N, D), attn.reshape(B * N, D),
                           self.out_proj.weight.t()).view(B, N, D)

    def _with_extra_kv(self, q, k, v, off, video_shape, extra_kv, drop_p=0.0):
        """Local taps + G shared extra keys, merged through the log-sum-exp.

        Exactly the reference's concatenation of the extra keys/values to every
        query's tap list followed by one softmax (attention.py:160-183).  With
        dropout, the merged weights of the local taps are a_l * p_local and of
        the extra keys a_e * p_extra; dropping them is dropping p_local (in the
        kernel) and p_extra (here), since the mask and scale commute with a_l
        and a_e.
        """
        B, N, D = q.shape
        nh, hd = self.num_heads, self.head_dim
        G = extra_kv.shape[1]
        loc, lse_loc = dsa3d_core(q, k, v, off, video_shape, nh, self.kernel_size,
                                  self.offset_scale, return_lse=True,
                                  dropout_p=drop_p)  # [B,N,D], [B,N,nh]
        ek = self.k_proj(extra_kv).float()
        ev = self.v_proj(extra_kv).float()
        qh = q.float().view(B, N, nh, hd).permute(0, 2, 1, 3).contiguous()      # [B,nh,N,hd]
        ekh = ek.view(B, G, nh, hd).permute(0, 2, 3, 1).contiguous()             # [B,nh,hd,G]
        evh = ev.view(B, G, nh, hd).permute(0, 2, 1, 3).contiguous()             # [B,nh,G,hd]
        s = torch.matmul(qh, ekh) * (1.0 / math.sqrt(hd))                       # [B,nh,N,G]
        lse_e = torch.logsumexp(s, dim=-1)                                       # [B,nh,N]
        pe = torch.softmax(s, dim=-1)
        if drop_p > 0:
            pe = F.dropout(pe, drop_p, training=True)
        o_e = torch.matmul(pe, evh)                                              # [B,nh,N,hd]
        lse_l = lse_loc.permute(0, 2, 1)                                         # [B,nh,N]
        lse = torch.logaddexp(lse_l, lse_e)
        a_l = torch.exp(lse_l - lse).unsqueeze(-1)
        a_e = torch.exp(lse_e - lse).unsqueeze(-1)
        loc_h = loc.float().view(B, N, nh, hd).permute(0, 2, 1, 3)
        out = loc_h * a_l + o_e * a_e
        return out.permute(0, 2, 1, 3).reshape(B, N, D).to(q.dtype)
