"""CPU oracle for 3D Deformable Slide Attention (test infrastructure only).

This package is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``megaslide_amd``) never imports it and has no CPU
fallback.

Contents
--------
``dsa3d_ref``
    A PyTorch-CPU restatement of the reference operator
    ``DeformableSlideAttention3D`` (infinity/video/attention.py:19-273), op for
    op: depthwise convs, offset predictor, fp32 base grid, offset normalisation
    with the reference's slot/axis order, ``F.grid_sample`` (trilinear, border,
    align_corners=False), matmul/softmax/matmul.  Gradients come from autograd
    over that restatement.  Pinned by: golden vectors produced from the
    reference module itself (tests/golden/), the brute-force sampler below,
    closed-form invariants and fp64 ``gradcheck``.
``bruteforce``
    Pure-numpy loops restating the trilinear/border sampling rule and its
    coordinate gradient for tiny volumes; pins what ``F.grid_sample`` does.
"""
