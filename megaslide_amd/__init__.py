"""megaslide_amd: MI355X (gfx950) HIP implementation of 3D Deformable Slide Attention.

Public surface:
  DeformableSlideAttention3D   drop-in for infinity/video/attention.py:19-273
  DiTBlock, MLP                drop-ins for infinity/video/model.py:21-117 around it
  dsa3d_core                   fused attention core (autograd; the custom
                               operator torch.ops.megaslide.dsa3d_core)
  dwconv3d                     depthwise 3-D conv (+GELU) on channel-last tokens (autograd)
  keep_core_policy, keep_core_context, checkpoint_keep_core
                               selective checkpointing that keeps the core's outputs
  keep_gemms_policy, keep_gemms_context, checkpoint_keep_gemms
                               ... and every GEMM's outputs
"""

from .attention import DeformableSlideAttention3D
from .block import MLP, DiTBlock, checkpoint_keep_core, checkpoint_keep_gemms
from .ops import (DwConv3dFunction, dsa3d_core, dwconv3d, keep_core_context, keep_core_policy,
                  keep_gemms_context, keep_gemms_policy)

__all__ = ["DeformableSlideAttention3D", "DiTBlock", "MLP", "DwConv3dFunction", "dsa3d_core",
           "dwconv3d", "keep_core_policy", "keep_core_context", "checkpoint_keep_core",
           "keep_gemms_policy", "keep_gemms_context", "checkpoint_keep_gemms"]
