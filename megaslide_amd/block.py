"""The DiT block around the attention module: drop-ins for the reference's
``MLP`` and ``DiTBlock`` (infinity/video/model.py:21-117).

Same constructor (a MegaSlideConfig, or any object with its fields), the same
submodules and parameter names in the same registration order (``norm1``,
``attn``, ``norm2``, ``mlp.fc1``, ``mlp.fc2``, and with text conditioning
``norm_cross`` and ``cross_attn``), so a reference checkpoint loads with
``load_state_dict(strict=True)`` and the trainer's parameter zip
(infinity/video/trainer.py:169-172) lines up.  The attention is the HIP
``DeformableSlideAttention3D``; LayerNorm, the MLP's GEMMs and exact-erf GELU
and the optional cross-attention stay in PyTorch.

Under gradient checkpointing (the C5 training configuration and
trainer.py:377-438's recompute pattern) the backward re-runs the block's
forward; ``checkpoint_keep_core`` runs it under torch.utils.checkpoint with a
selective policy that keeps the attention core's outputs (out and lse, about
D + 2 nh bytes a token in bf16) from the first forward, so the recompute skips
the core's forward kernel and reruns only the norms, GEMMs and convolutions;
``checkpoint_keep_gemms`` also keeps every GEMM's output (about 9 D more bytes
a token in bf16), so the recompute reruns only the norms, the elementwise work
and the depthwise convolutions.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from .attention import DeformableSlideAttention3D
from .ops import keep_core_context, keep_gemms_context


class MLP(nn.Module):
    """fc1 -> GELU (exact erf) -> dropout -> fc2 -> dropout (model.py:21-35)."""

    def __init__(self, hidden_size: int, intermediate_size: int, dropout: float = 0.0):
        super().__init__()
        self.fc1 = nn.Linear(hidden_size, intermediate_size)
        self.act = nn.GELU()
        self.fc2 = nn.Linear(intermediate_size, hidden_size)
        self.dropout = nn.Dropout(dropout)

    def forward(self, x: Tensor) -> Tensor:
        return self.dropout(self.fc2(self.dropout(self.act(self.fc1(x)))))


class DiTBlock(nn.Module):
    """Pre-LayerNorm 3D-DSA and MLP with residuals (model.py:40-117)."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.norm1 = nn.LayerNorm(config.hidden_size, eps=1e-6)
        self.attn = DeformableSlideAttention3D(
            hidden_size=config.hidden_size,
            num_heads=config.num_heads,
            kernel_size=tuple(config.dsa_kernel_size),
            offset_scale=config.offset_scale,
            dropout=config.dropout,
        )
        self.norm2 = nn.LayerNorm(config.hidden_size, eps=1e-6)
        self.mlp = MLP(config.hidden_size, config.mlp_hidden_size, dropout=config.dropout)
        if getattr(config, "use_text_conditioning", False):
            self.norm_cross = nn.LayerNorm(config.hidden_size, eps=1e-6)
            self.cross_attn = nn.MultiheadAttention(embed_dim=config.hidden_size,
                                                    num_heads=config.num_heads,
                                                    dropout=config.dropout, batch_first=True)

    def forward(self, x: Tensor, video_shape: Tuple[int, int, int],
                text_embeds: Optional[Tensor] = None,
                text_mask: Optional[Tensor] = None) -> Tensor:
        x = x + self.attn(self.norm1(x), video_shape)
        if text_embeds is not None and hasattr(self, "cross_attn"):
            x_normed = self.norm_cross(x)
            key_padding_mask = ~text_mask if text_mask is not None else None
            attn_out, _ = self.cross_attn(x_normed, text_embeds, text_embeds,
                                          key_padding_mask=key_padding_mask)
            x = x + attn_out
        return x + self.mlp(self.norm2(x))


def checkpoint_keep_core(block: nn.Module, x: Tensor, video_shape: Tuple[int, int, int],
                         *args, **kwargs) -> Tensor:
    """``block(x, video_shape, ...)`` under torch.utils.checkpoint (non-reentrant)
    keeping the attention core's outputs: activation memory of the block is
    its input plus the core's out and lse; the backward's recompute reruns
    everything else."""
    from torch.utils.checkpoint import checkpoint
    return checkpoint(block, x, video_shape, *args, use_reentrant=False,
                      context_fn=keep_core_context, **kwargs)


def checkpoint_keep_gemms(block: nn.Module, x: Tensor, video_shape: Tuple[int, int, int],
                          *args, **kwargs) -> Tensor:
    """``block(x, video_shape, ...)`` under torch.utils.checkpoint (non-reentrant)
    keeping the attention core's and every GEMM's outputs: the backward's
    recompute reruns the LayerNorms, GELU, residual adds and depthwise
    convolutions only."""
    from torch.utils.checkpoint import checkpoint
    return checkpoint(block, x, video_shape, *args, use_reentrant=False,
                      context_fn=keep_gemms_context, **kwargs)
