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
  * ``extra_kv`` (attention.py:160-173): its k_proj / v_proj projections are
    PyTorch GEMMs; the G extra keys and values join every query's taps in the
    HIP core's softmax (forward and backward, their gradients included).

There is no CPU path: on CPU tensors ``forward`` raises.
"""

from __future__ import annotations

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
        # How the backward sums dK / dV over query tiles (not a constructor
        # argument, so the reference's signature stays as it is): "fp32", the
        # reference's precision, or for bfloat16 weights "fp16" (scaled fp16
        # pairs, about half the atomic traffic).
        self.dkv_accum = "fp32"

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
        ek = ev = None
        if extra_kv is not None:  # attention.py:160-173: projected, appended to every query's taps
            ek = self.k_proj(extra_kv).to(dt)
            ev = self.v_proj(extra_kv).to(dt)
        attn = dsa3d_core(q, k.to(dt), v.to(dt), off, video_shape, self.num_heads,
                          self.kernel_size, self.offset_scale, dropout_p=drop_p, extra_k=ek,
                          extra_v=ev, dkv_accum=self.dkv_accum)
        return torch.addmm(dw.reshape(B * N, D), attn.reshape(B * N, D),
                           self.out_proj.weight.t()).view(B, N, D)
