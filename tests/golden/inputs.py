"""Seeded synthetic inputs shared by the golden generator and the tests.

Everything is drawn from ``numpy.random.Generator(PCG64(seed))`` so that the GPU
box regenerates bit-identical inputs without the reference being present.
Arrays are float64; callers cast.
"""

from __future__ import annotations

import math
from typing import Dict, Sequence

import numpy as np

PARAM_ORDER = (
    "q_proj.weight", "q_proj.bias", "k_proj.weight", "k_proj.bias",
    "v_proj.weight", "v_proj.bias", "out_proj.weight", "out_proj.bias",
    "dw_conv.weight", "dw_conv.bias",
    "offset_net.0.weight", "offset_net.0.bias",
    "offset_net.2.weight", "offset_net.2.bias",
)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def xavier(g: np.random.Generator, shape, fan_in: int, fan_out: int) -> np.ndarray:
    a = math.sqrt(6.0 / (fan_in + fan_out))
    return g.uniform(-a, a, size=shape)


def module_params(g: np.random.Generator, D: int, nh: int, kernel_size: Sequence[int],
                  on_std: float = 0.2, on0_std: float = 0.0, bias_std: float = 0.1,
                  on2_bias: str = "normal", on2_bias_scale: float = 0.1) -> Dict[str, np.ndarray]:
    """A full parameter set of the module, all entries non-trivial.

    Projections: Xavier-uniform weights, N(0, bias_std) biases.  ``dw_conv``:
    Xavier.  ``offset_net.0``: Xavier (or N(0, on0_std) when on0_std > 0).
    ``offset_net.2`` weight N(0, on_std); its bias N(0, on2_bias_scale) or
    U(-on2_bias_scale, on2_bias_scale) with on2_bias="uniform".
    """
    kt, kh, kw = kernel_size
    K = kt * kh * kw
    C = nh * K * 3
    p = {}
    for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
        p[f"{name}.weight"] = xavier(g, (D, D), D, D)
        p[f"{name}.bias"] = g.normal(0.0, bias_std, size=(D,))
    p["dw_conv.weight"] = xavier(g, (D, 1, kt, kh, kw), K, D * K)
    p["dw_conv.bias"] = g.normal(0.0, bias_std, size=(D,))
    if on0_std > 0:
        p["offset_net.0.weight"] = g.normal(0.0, on0_std, size=(D, 1, 3, 3, 3))
    else:
        p["offset_net.0.weight"] = xavier(g, (D, 1, 3, 3, 3), 27, D * 27)
    p["offset_net.0.bias"] = g.normal(0.0, bias_std, size=(D,))
    p["offset_net.2.weight"] = g.normal(0.0, on_std, size=(C, D, 1, 1, 1))
    if on2_bias == "uniform":
        p["offset_net.2.bias"] = g.uniform(-on2_bias_scale, on2_bias_scale, size=(C,))
    else:
        p["offset_net.2.bias"] = g.normal(0.0, on2_bias_scale, size=(C,))
    return p


def core_inputs(seed: int, B: int, T: int, H: int, W: int, D: int, nh: int,
                kernel_size: Sequence[int], off_std: float, qkv_std: float = 1.0):
    """q, k, v ~ N(0, qkv_std), raw offsets ~ N(0, off_std), dout ~ N(0, 1)."""
    g = rng(seed)
    kt, kh, kw = kernel_size
    N = T * H * W
    C = nh * kt * kh * kw * 3
    q = g.normal(0.0, qkv_std, size=(B, N, D))
    k = g.normal(0.0, qkv_std, size=(B, N, D))
    v = g.normal(0.0, qkv_std, size=(B, N, D))
    off = g.normal(0.0, off_std, size=(B, N, C))
    dout = g.normal(0.0, 1.0, size=(B, N, D))
    return q, k, v, off, dout


# Golden cases; tests/golden/make_golden.py runs the reference on each.
CASES = [
    # name, B, T, H, W, D, nh, kernel, offset_scale, mode, seed, dtype
    dict(name="k377_tiny", B=1, T=3, H=4, W=5, D=16, nh=2, kernel=(3, 7, 7), scale=1.0,
         mode="net", seed=11, on_std=0.3),
    dict(name="k377_inject", B=2, T=3, H=4, W=5, D=16, nh=2, kernel=(3, 7, 7), scale=0.75,
         mode="inject", seed=12, off_std=1.5, huge_frac=0.05),
    dict(name="k333_T1", B=1, T=1, H=4, W=5, D=8, nh=2, kernel=(3, 3, 3), scale=1.0,
         mode="inject", seed=13, off_std=1.0, huge_frac=0.0),
    dict(name="k333_H1", B=1, T=3, H=1, W=5, D=8, nh=2, kernel=(3, 3, 3), scale=1.0,
         mode="inject", seed=14, off_std=1.0, huge_frac=0.0),
    dict(name="k333_W1", B=1, T=3, H=4, W=1, D=8, nh=2, kernel=(3, 3, 3), scale=1.0,
         mode="inject", seed=15, off_std=1.0, huge_frac=0.0),
    dict(name="k333_111", B=1, T=1, H=1, W=1, D=4, nh=2, kernel=(3, 3, 3), scale=1.0,
         mode="net", seed=16, on_std=0.3),
    dict(name="k133", B=2, T=2, H=3, W=3, D=8, nh=2, kernel=(1, 3, 3), scale=1.0,
         mode="net", seed=17, on_std=0.5),
    dict(name="k311", B=1, T=2, H=1, W=1, D=2, nh=1, kernel=(3, 1, 1), scale=1.0,
         mode="net", seed=18, on_std=0.5),
    dict(name="k111", B=1, T=2, H=2, W=2, D=16, nh=4, kernel=(1, 1, 1), scale=1.0,
         mode="net", seed=19, on_std=0.5),
    dict(name="k355_b2", B=2, T=3, H=4, W=5, D=12, nh=3, kernel=(3, 5, 5), scale=0.5,
         mode="inject", seed=20, off_std=2.0, huge_frac=0.02),
    dict(name="k355_extra", B=2, T=3, H=4, W=5, D=12, nh=3, kernel=(3, 5, 5), scale=1.0,
         mode="net", seed=21, on_std=0.4, extra_g=4),
]

# The tiny forward configuration run on the reference CPU path: B=1, T=8,
# H=W=16, dim 256, 4 heads x 64, window 3x7x7, x ~ N(0,1), Xavier projections,
# both offset_net convs ~ N(0, 0.02), seed 0.  fp32; sampled rows are stored.
C1 = dict(name="c1_fwd_fp32", B=1, T=8, H=16, W=16, D=256, nh=4, kernel=(3, 7, 7), scale=1.0,
          mode="net", seed=0, rows=96)


def case_params(case):
    """Parameters, x, upstream grad and (for ``inject`` cases) raw offsets."""
    g = rng(case["seed"])
    if case["name"].startswith("c1"):
        p = module_params(g, case["D"], case["nh"], case["kernel"], on_std=0.02,
                          on0_std=0.02, bias_std=0.0, on2_bias_scale=0.0)
    else:
        p = module_params(g, case["D"], case["nh"], case["kernel"],
                          on_std=case.get("on_std", 0.3))
    x = g.normal(0.0, 1.0, size=(case["B"], case["T"] * case["H"] * case["W"], case["D"]))
    gy = g.normal(0.0, 1.0, size=x.shape)
    off = None
    if case["mode"] == "inject":
        kt, kh, kw = case["kernel"]
        C = case["nh"] * kt * kh * kw * 3
        off = g.normal(0.0, case["off_std"], size=(case["B"], x.shape[1], C))
        if case.get("huge_frac", 0.0) > 0:
            mask = g.uniform(size=off.shape) < case["huge_frac"]
            off = np.where(mask, np.sign(off) * 50.0, off)
    extra = None
    if case.get("extra_g", 0) > 0:
        extra = g.normal(0.0, 1.0, size=(case["B"], case["extra_g"], case["D"]))
    return p, x, gy, off, extra




# A tiny DiT block (infinity/video/model.py:40-117 with MegaSlideConfig): D=32,
# 2 heads, window 3x5x5, MLP ratio 4, on a 3x4x5 grid, B=2.  Parameters in the
# block's named_parameters() order; the offset net's last conv is non-zero
# (inside MegaSlideDiT every Conv3d is re-initialised, model.py:164-178).  The
# seed keeps every sampling coordinate at least 1.7e-5 voxel from a lattice line
# (where the trilinear gradient jumps), so an fp32 evaluation takes the same
# corners as the reference's float64 one.
BLOCK = dict(name="dit_block", B=2, T=3, H=4, W=5, D=32, nh=2, kernel=(3, 5, 5), scale=1.0,
             mlp_ratio=4.0, seed=40, on_std=0.3)


def block_params(case) -> Dict[str, np.ndarray]:
    g = rng(case["seed"])
    D = case["D"]
    M = int(D * case["mlp_ratio"])
    p = {"norm1.weight": 1.0 + g.normal(0.0, 0.1, size=(D,)),
         "norm1.bias": g.normal(0.0, 0.1, size=(D,))}
    for n, v in module_params(g, D, case["nh"], case["kernel"], on_std=case["on_std"]).items():
        p["attn." + n] = v
    p["norm2.weight"] = 1.0 + g.normal(0.0, 0.1, size=(D,))
    p["norm2.bias"] = g.normal(0.0, 0.1, size=(D,))
    p["mlp.fc1.weight"] = xavier(g, (M, D), D, M)
    p["mlp.fc1.bias"] = g.normal(0.0, 0.1, size=(M,))
    p["mlp.fc2.weight"] = xavier(g, (D, M), M, D)
    p["mlp.fc2.bias"] = g.normal(0.0, 0.1, size=(D,))
    return p


def block_inputs(case):
    """Parameters, x and upstream grad of the block case."""
    p = block_params(case)
    g = rng(case["seed"] + 1000)
    x = g.normal(0.0, 1.0, size=(case["B"], case["T"] * case["H"] * case["W"], case["D"]))
    gy = g.normal(0.0, 1.0, size=x.shape)
    return p, x, gy
