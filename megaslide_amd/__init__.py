"""megaslide_amd: MI355X (gfx950) HIP implementation of 3D Deformable Slide Attention.

Public surface:
  DeformableSlideAttention3D   drop-in for infinity/video/attention.py:19-273
  dsa3d_core                   fused attention core (autograd)
  dwconv3d                     depthwise 3-D conv (+GELU) on channel-last tokens (autograd)
"""

from .attention import DeformableSlideAttention3D
from .ops import DSA3DCoreFunction, DwConv3dFunction, dsa3d_core, dwconv3d

__all__ = ["DeformableSlideAttention3D", "DSA3DCoreFunction", "DwConv3dFunction", "dsa3d_core",
           "dwconv3d"]
