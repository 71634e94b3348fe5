"""Benchmark: 3D-DSA forward + backward through the HIP kernel set on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline] [--copy-calibration]
                    [--workload long-clip-65k|tiny-2k|fp32-32k|large-block-131k|dit-block-46k]
    python bench.py --summarize WORKLOAD TRACE_DIR FETCH_DIR WRITE_DIR
                    (rocprofv3 csv output -> markdown tables + profiles/traffic.json)
    python bench.py --counter-table PMC_DIR [PMC_DIR ...]
                    (rocprofv3 --pmc csv output -> per-kernel instruction/LDS table)

Workloads (one step = one pass of the hot path over one batch of synthetic
input, every buffer preallocated and resident in HBM):

  long-clip-65k    (default) B=1, T=64, H=W=32 (65,536 tokens), dim 1024,
                   16 heads x 64, bf16 storage with fp32 accumulation (dK / dV
                   summed over query tiles with fp32 atomics), raw offsets
                   ~ N(0, 0.5)
  long-clip-65k-f16acc  the same with dK / dV summed in power-of-two-scaled
                   fp16 pairs (MSD_ACCUM_F16; fp32 redo on overflow)
  long-clip-65k-g128  the same with 128 extra keys shared by every query
                   (the reference's extra_kv from HybridAttention3D's registers)
  tiny-2k          B=1, T=8, H=W=16 (2,048 tokens), dim 256, 4 x 64, fp32,
                   forward only, offsets from the offset net (depthwise 3x3x3
                   conv and 1x1 conv weights ~ N(0, 0.02))
  fp32-32k         B=2, T=16, H=W=32 (32,768 tokens), dim 512, 8 x 64, fp32,
                   raw offsets ~ N(0, 1.5)
  large-block-131k B=1, T=32, H=W=64 (131,072 tokens), dim 3072, 24 x 128,
                   bf16, offsets from the offset net (conv weights ~ N(0, 0.05))
  dit-block-46k    B=1, T=13, H=45, W=80 (46,800 tokens), dim 1536, 16 x 96,
                   bf16, offsets from the offset net with its bias ~ U(-4, 4)
                   voxels (weights ~ N(0, 0.02))

with window 3x7x7, x, q, k, v ~ N(0, 1) and upstream grads ~ N(0, 1).  A step
runs dw_conv 3x7x7 fwd, offset_net depthwise 3x3x3+GELU fwd, attention core
fwd, and (except tiny-2k, a forward config) attention core bwd, 3x3x3+GELU
bwd, 3x7x7 bwd: every HIP kernel of the module's forward and backward.  The
dense GEMMs (projections, 1x1 offset conv) stay in hipBLASLt and are not part
of the step; offsets from the offset net are computed once before timing.

Prints one JSON line.  `value` is tokens/s of the whole step.  `hbm_gbps` is the
step's algorithmic bytes over its time, with the byte model of `byte_model`
(each interface tensor once at its dtype: core fwd e(4D + C) + 4 nh, core bwd
e(8D + 2C) + 4 nh, depthwise pair 3eD fwd + 4eD bwd, per token).  `roofline`
is the dominant kernel's own compulsory bytes per launch over its average
duration, timed with events on the launch stream; `roofline.traffic` is the
measured L2<->fabric bytes per launch of that kernel from profiles/traffic.json
(two rocprofv3 --pmc runs, FETCH_SIZE and WRITE_SIZE, each scaled by the same
counter on a plain copy of known size -- see --copy-calibration), or null when
none is recorded for the workload; `cpu_baseline` is the float32 CPU oracle
(the reference op sequence) on a bounded slab of the same workload, median of
3 timed runs after a warm-up, its tokens/s taken as the workload's
(slab-extrapolated).

--copy-calibration first runs a plain 512 MiB -> 512 MiB bf16 copy (torch.neg)
twice, so a counter run of this script also measures the copy the counters
are scaled by, then a read-only pass over the same 512 MiB (torch.amax) as a
second FETCH_SIZE point.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "3D-DSA fwd+bwd tokens/sec at 65k tokens bf16; achieved HBM GB/s (% of peak)"
HBM_PEAK_GBPS = 8000.0
DEFAULT = "long-clip-65k"

# offsets: ("normal", std) raw offsets; ("net", conv std, 1x1 weight std, bias) from
# the offset net, bias ("uniform", a) ~ U(-a, a) or ("normal", std)
WORKLOADS = {
    "long-clip-65k": dict(
        B=1, T=64, H=32, W=32, D=1024, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("normal", 0.5), backward=True, metric=METRIC,
        workload="3D-DSA fwd+bwd HIP kernel set, long-clip 65,536 tokens",
        cpu_slab=dict(T=4)),
    "long-clip-65k-f16acc": dict(
        B=1, T=64, H=32, W=32, D=1024, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("normal", 0.5), backward=True, dkv_accum="fp16",
        metric="3D-DSA fwd+bwd tokens/sec at 65k tokens bf16, dK/dV summed in scaled fp16",
        workload="3D-DSA fwd+bwd HIP kernel set, long-clip 65,536 tokens, dK/dV accumulated in "
                 "scaled fp16 pairs",
        cpu_slab=dict(T=4)),
    "long-clip-65k-g128": dict(
        B=1, T=64, H=32, W=32, D=1024, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("normal", 0.5), backward=True, extra_g=128,
        metric="3D-DSA fwd+bwd tokens/sec at 65k tokens bf16, 128 extra keys",
        workload="3D-DSA fwd+bwd HIP kernel set, long-clip 65,536 tokens + 128 shared extra keys "
                 "(hybrid registers)",
        cpu_slab=dict(T=4)),
    "tiny-2k": dict(
        B=1, T=8, H=16, W=16, D=256, nh=4, kernel=(3, 7, 7), dtype="fp32",
        offsets=("net", 0.02, 0.02, ("normal", 0.02)), backward=False,
        metric="3D-DSA fwd tokens/sec at 2k tokens fp32",
        workload="3D-DSA fwd HIP kernel set, tiny 2,048 tokens", cpu_slab=dict()),
    "fp32-32k": dict(
        B=2, T=16, H=32, W=32, D=512, nh=8, kernel=(3, 7, 7), dtype="fp32",
        offsets=("normal", 1.5), backward=True,
        metric="3D-DSA fwd+bwd tokens/sec at 32k tokens fp32",
        workload="3D-DSA fwd+bwd HIP kernel set, fp32 32,768 tokens", cpu_slab=dict(B=1, T=4)),
    "large-block-131k": dict(
        B=1, T=32, H=64, W=64, D=3072, nh=24, kernel=(3, 7, 7), dtype="bf16",
        offsets=("net", 0.05, 0.05, ("normal", 0.05)), backward=True,
        metric="3D-DSA fwd+bwd tokens/sec at 131k tokens bf16",
        workload="3D-DSA fwd+bwd HIP kernel set, large-block 131,072 tokens, 24 x 128",
        cpu_slab=dict(T=2, H=24, W=24)),
    "long-clip-65k-module": dict(
        B=1, T=64, H=32, W=32, D=1024, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("module", 0.5), backward=True, module="attention",
        metric="3D-DSA module fwd+bwd tokens/sec at 65k tokens bf16, projections and offset "
               "GEMM included",
        workload="DeformableSlideAttention3D fwd+bwd (HIP kernels + PyTorch GEMMs), long-clip "
                 "65,536 tokens",
        cpu_slab=dict(T=4)),
    "dit-block-46k-ckpt": dict(
        B=1, T=13, H=45, W=80, D=1536, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("block", 4.0), backward=True, module="block", checkpoint="keep-gemms",
        metric="DiT block fwd+bwd tokens/sec at 46.8k tokens bf16, gradient checkpointing",
        workload="MegaSlideDiT block (pre-LN 3D-DSA + MLP x4) fwd+bwd under selective "
                 "gradient checkpointing that keeps the attention core's and every GEMM's "
                 "outputs, 46,800 tokens, 16 x 96",
        cpu_slab=dict(T=3, H=24, W=40)),
    "dit-block-46k-ckpt-core": dict(
        B=1, T=13, H=45, W=80, D=1536, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("block", 4.0), backward=True, module="block", checkpoint="keep-core",
        metric="DiT block fwd+bwd tokens/sec at 46.8k tokens bf16, gradient checkpointing",
        workload="MegaSlideDiT block (pre-LN 3D-DSA + MLP x4) fwd+bwd under gradient "
                 "checkpointing that keeps the attention core's outputs only, 46,800 tokens, "
                 "16 x 96",
        cpu_slab=dict(T=3, H=24, W=40)),
    "dit-block-46k-ckpt-plain": dict(
        B=1, T=13, H=45, W=80, D=1536, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("block", 4.0), backward=True, module="block", checkpoint="plain",
        metric="DiT block fwd+bwd tokens/sec at 46.8k tokens bf16, gradient checkpointing",
        workload="MegaSlideDiT block (pre-LN 3D-DSA + MLP x4) fwd+bwd under plain gradient "
                 "checkpointing (whole forward recomputed), 46,800 tokens, 16 x 96",
        cpu_slab=dict(T=3, H=24, W=40)),
    "dit-block-46k": dict(
        B=1, T=13, H=45, W=80, D=1536, nh=16, kernel=(3, 7, 7), dtype="bf16",
        offsets=("net", 0.02, 0.02, ("uniform", 4.0)), backward=True,
        metric="3D-DSA fwd+bwd tokens/sec at 46.8k tokens bf16 (DiT-block shape)",
        workload="3D-DSA fwd+bwd HIP kernel set, DiT-block 46,800 tokens, 16 x 96",
        cpu_slab=dict(T=3, H=24, W=40)),
}


def _sizes(cfg):
    N = cfg["B"] * cfg["T"] * cfg["H"] * cfg["W"]
    kt, kh, kw = cfg["kernel"]
    return N, cfg["D"], cfg["nh"], cfg["nh"] * kt * kh * kw * 3


def kernel_bytes(cfg, e):
    """Compulsory bytes per launch of each phase (each tensor once, at its dtype)."""
    N, D, nh, C = _sizes(cfg)
    return {
        "dwconv7_fwd": N * 2 * e * D,            # read x, write y
        "dwconv3_gelu_fwd": N * 2 * e * D,       # read x, write gelu(z)
        "dsa3d_fwd": N * (e * (4 * D + C) + 4 * nh),   # read q,k,v,off; write out, lse
        "dsa3d_bwd": N * (e * (8 * D + 2 * C) + 4 * nh),  # read q,k,v,off,out,dout,lse; write dq,dk,dv,doff
        "dwconv3_gelu_bwd": N * 3 * e * D,       # read x, dF; write dx
        "dwconv7_bwd": N * 3 * e * D,            # read x, dy; write dx
    }


def step_bytes(cfg, e):
    """Algorithmic bytes of one step with the depthwise pair counted as a unit:
    x read once for both convs (fwd 3eD: read x, write F and y; bwd 4eD: read
    x, dF, dy, write one dx)."""
    N, D, nh, C = _sizes(cfg)
    fwd = e * (4 * D + C) + 4 * nh + 3 * e * D
    bwd = e * (8 * D + 2 * C) + 4 * nh + 4 * e * D
    return N * (fwd + (bwd if cfg["backward"] else 0))


BYTE_MODEL = ("per token: core fwd e(4D+C)+4nh, core bwd e(8D+2C)+4nh, depthwise pair "
              "3eD fwd + 4eD bwd (x read once for both convs); each tensor once at its dtype")

COPY_BYTES = 512 * 2 ** 20  # read and written once each by the calibration copy


def copy_calibration(dev):
    """A plain 512 MiB -> 512 MiB copy (torch.neg), twice, which the traffic
    counters are scaled by, then a read-only pass over the same 512 MiB
    (torch.amax, a reduction writing one value) as a second FETCH_SIZE point."""
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    for _ in range(2):
        torch.amax(src)
    torch.cuda.synchronize()
    del src, dst


def measured_traffic(workload, kernel):
    """Traffic bytes per launch recorded for `kernel` of `workload` in
    profiles/traffic.json, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(workload, {}).get(kernel)
    except (OSError, ValueError, AttributeError):
        return None
    return None if rec is None else rec.get("bytes_per_launch")


def make_offsets(cfg, x, dev, dt, g):
    """Raw offsets [B, N, C] for the workload (outside the timed region)."""
    from megaslide_amd import dwconv3d

    B, T, H, W, D = cfg["B"], cfg["T"], cfg["H"], cfg["W"], cfg["D"]
    _, _, _, C = _sizes(cfg)
    N = T * H * W
    spec = cfg["offsets"]
    if spec[0] == "normal":
        return (torch.randn(B, N, C, generator=g, device=dev) * spec[1]).to(dt)
    _, conv_std, w_std, (bias_kind, bias_a) = spec
    w0 = (torch.randn(D, 1, 3, 3, 3, generator=g, device=dev) * conv_std).to(dt)
    b0 = (torch.randn(D, generator=g, device=dev) * conv_std).to(dt)
    w2 = (torch.randn(C, D, generator=g, device=dev) * w_std).to(dt)
    if bias_kind == "uniform":
        b2 = (torch.rand(C, generator=g, device=dev) * 2 * bias_a - bias_a).to(dt)
    else:
        b2 = (torch.randn(C, generator=g, device=dev) * bias_a).to(dt)
    with torch.no_grad():
        feat = dwconv3d(x, w0, b0, (T, H, W), act="gelu")
        return torch.nn.functional.linear(feat, w2, b2).contiguous()


def run_gpu(cfg, steps, warmup, calibrate=False):
    from megaslide_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if calibrate:
        copy_calibration(dev)
    B, T, H, W, D, nh = cfg["B"], cfg["T"], cfg["H"], cfg["W"], cfg["D"], cfg["nh"]
    hd = D // nh
    kt, kh, kw = cfg["kernel"]
    N = T * H * W
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
    mdt = _lib.MSD_BF16 if cfg["dtype"] == "bf16" else _lib.MSD_F32
    g = torch.Generator(device=dev).manual_seed(3)

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(dt)

    x = rnd(B, N, D)
    q, k, v = rnd(B, N, D), rnd(B, N, D), rnd(B, N, D)
    off = make_offsets(cfg, x, dev, dt, g)
    dout, dF, dY = rnd(B, N, D), rnd(B, N, D), rnd(B, N, D)
    w7, b7 = rnd(D, 1, kt, kh, kw, std=0.05), rnd(D, std=0.02)
    w3, b3 = rnd(D, 1, 3, 3, 3, std=0.1), rnd(D, std=0.02)
    y7, F = torch.empty_like(x), torch.empty_like(x)
    out = torch.empty_like(q)
    lse = torch.empty(B, N, nh, device=dev, dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    doff = torch.empty_like(off)
    dx3, dx7 = torch.empty_like(x), torch.empty_like(x)
    Z = torch.empty_like(x)  # the GELU conv's pre-activation, kept for its backward
    dw3, db3, dw7, db7 = (torch.empty_like(t) for t in (w3, b3, w7, b7))

    G = cfg.get("extra_g", 0)
    ek = rnd(B, G, D) if G else None
    ev = rnd(B, G, D) if G else None
    dek = torch.empty_like(ek) if G else None
    dev_ = torch.empty_like(ev) if G else None
    dsa = _lib.DsaDesc(B, T, H, W, nh, hd, kt, kh, kw, mdt, D, D, D, 1.0, 1.0 / math.sqrt(hd),
                       0, 0, 0, 0.0, G, _lib.ACCUMS[accumulation(cfg)])
    cv7 = _lib.ConvDesc(B, T, H, W, D, kt, kh, kw, mdt, 0)
    cv3 = _lib.ConvDesc(B, T, H, W, D, 3, 3, 3, mdt, 1)

    def ws(nbytes):
        return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=dev)

    ws_dsa = ws(lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(dsa)))
    ws7 = ws(lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(cv7)))
    ws3 = ws(lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(cv3)))
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731
    PX = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    phases = [
        ("dwconv7_fwd", lambda: lib.msd_dwconv3d_fwd(ctypes.byref(cv7), P(x), P(w7), P(b7), P(y7), None,
                                                     sh)),
        ("dwconv3_gelu_fwd", lambda: lib.msd_dwconv3d_fwd(ctypes.byref(cv3), P(x), P(w3), P(b3), P(F),
                                                          P(Z) if cfg["backward"] else None, sh)),
        ("dsa3d_fwd", lambda: lib.msd_dsa3d_fwd(ctypes.byref(dsa), P(q), P(k), P(v), P(off),
                                                PX(ek), PX(ev), P(out), P(lse), sh)),
    ]
    if cfg["backward"]:
        phases += [
            ("dsa3d_bwd", lambda: lib.msd_dsa3d_bwd(ctypes.byref(dsa), P(q), P(k), P(v), P(off),
                                                    PX(ek), PX(ev), P(out), P(dout), P(lse), None,
                                                    P(dq), P(dk), P(dv), P(doff), PX(dek), PX(dev_),
                                                    P(ws_dsa), ws_dsa.numel(), sh)),
            ("dwconv3_gelu_bwd", lambda: lib.msd_dwconv3d_bwd(ctypes.byref(cv3), P(x), P(w3), P(b3), P(Z),
                                                              P(dF), P(dx3), P(dw3), P(db3), P(ws3),
                                                              ws3.numel(), sh)),
            ("dwconv7_bwd", lambda: lib.msd_dwconv3d_bwd(ctypes.byref(cv7), P(x), P(w7), P(b7), None,
                                                         P(dY), P(dx7), P(dw7), P(db7), P(ws7),
                                                         ws7.numel(), sh)),
        ]

    def step(events=None):
        for i, (name, fn) in enumerate(phases):
            if events is not None:
                events[i][0].record(stream)
            rc = fn()
            if events is not None:
                events[i][1].record(stream)
            if rc != 0:
                raise RuntimeError(f"{name} failed: {lib.msd_last_error().decode()}")

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K steps, bracketed by device synchronisation
    evs = [[[torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
            for _ in phases] for _ in range(steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    for s in range(steps):
        step(evs[s])
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)
    per_phase = {name: sum(evs[s][i][0].elapsed_time(evs[s][i][1]) for s in range(steps)) / steps
                 for i, (name, _) in enumerate(phases)}
    return dict(total_ms=total_ms, wall_s=wall, per_phase_ms=per_phase, tokens=B * N)


class _BlockConfig:
    """The MegaSlideConfig fields a DiT block reads (MLP ratio 4, no dropout)."""

    def __init__(self, D, nh, kernel):
        self.hidden_size, self.num_heads, self.dsa_kernel_size = D, nh, kernel
        self.offset_scale, self.dropout, self.mlp_hidden_size = 1.0, 0.0, 4 * D


def _init_like_model(mod, g):
    """MegaSlideDiT._init_weights (model.py:164-178): Xavier-uniform weights and
    zero biases for every Linear and Conv3d (the offset net's last conv
    included), LayerNorms at their defaults."""
    for m in mod.modules():
        if isinstance(m, (torch.nn.Linear, torch.nn.Conv3d)):
            w = m.weight
            fan_out = w.shape[0] * (w[0][0].numel() if w.dim() > 2 else 1)
            fan_in = w[0].numel()
            a = math.sqrt(6.0 / (fan_in + fan_out))
            with torch.no_grad():
                w.copy_((torch.rand(w.shape, generator=g) * 2 - 1) * a)
                if m.bias is not None:
                    m.bias.zero_()


def build_module(cfg, dev):
    """The module of a module workload, in its dtype on `dev`, and its inputs:
    x (for the block: tokens plus a timestep embedding ~ N(0, 1), added at the
    model input as model.py:212-214 does) and an upstream gradient ~ N(0, 1)."""
    from megaslide_amd import DeformableSlideAttention3D, DiTBlock, dwconv3d

    B, T, H, W, D, nh = cfg["B"], cfg["T"], cfg["H"], cfg["W"], cfg["D"], cfg["nh"]
    N = T * H * W
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
    g = torch.Generator().manual_seed(11)
    if cfg["module"] == "attention":
        mod = DeformableSlideAttention3D(D, nh, kernel_size=cfg["kernel"])
    else:
        mod = DiTBlock(_BlockConfig(D, nh, cfg["kernel"]))
    _init_like_model(mod, g)
    attn = mod if cfg["module"] == "attention" else mod.attn
    gd = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn(B, N, D, generator=gd, device=dev)
    if cfg["module"] == "block":
        x = x + torch.randn(B, 1, D, generator=gd, device=dev)
        # offsets with a uniform per-tap voxel bias (config's U(-a, a))
        with torch.no_grad():
            on2 = attn.offset_net[2]
            a = cfg["offsets"][1]
            on2.bias.copy_(torch.rand(on2.bias.shape, generator=g) * 2 * a - a)
    mod = mod.to(dev, dt)
    x = x.to(dt)
    if cfg["module"] == "attention":
        # predicted offsets of the configured spread: the last conv's weights
        # scaled from the features they see
        with torch.no_grad():
            on0, on2 = attn.offset_net[0], attn.offset_net[2]
            feat = dwconv3d(x, on0.weight, on0.bias, (T, H, W), act="gelu").float()
            sd = cfg["offsets"][1] / (feat.std().item() * math.sqrt(D))
            on2.weight.copy_((torch.randn(on2.weight.shape, generator=g) * sd).to(dt))
    gy = torch.randn(B, N, D, generator=gd, device=dev).to(dt)
    return mod, attn, x, gy


def run_module(cfg, steps, warmup):
    """Module workloads: forward + backward of the whole module (the attention
    module with its PyTorch GEMMs, or the DiT block, optionally checkpointed),
    torch.autograd.grad over the input and every parameter, as the trainer
    takes them (infinity/video/trainer.py:431-438).  One more, untimed step
    brackets every call of the HIP library with events on the current stream
    (per-kernel-set times; the rest is PyTorch: GEMMs, norms, elementwise)."""
    from torch.utils.checkpoint import checkpoint

    from megaslide_amd import _lib, checkpoint_keep_core, checkpoint_keep_gemms

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, T, H, W = cfg["B"], cfg["T"], cfg["H"], cfg["W"]
    mod, attn, x, gy = build_module(cfg, dev)
    params = list(mod.parameters())
    ckpt = cfg.get("checkpoint")
    stream = torch.cuda.current_stream(dev)

    def step(ev=None):
        xi = x.detach().requires_grad_(True)
        if ckpt == "keep-gemms":
            y = checkpoint_keep_gemms(mod, xi, (T, H, W))
        elif ckpt == "keep-core":
            y = checkpoint_keep_core(mod, xi, (T, H, W))
        elif ckpt == "plain":
            y = checkpoint(mod, xi, (T, H, W), use_reentrant=False)
        else:
            y = mod(xi, (T, H, W))
        if ev is not None:
            ev.record(stream)
        return torch.autograd.grad(y, [xi] + params, grad_outputs=gy, allow_unused=True)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    for sidx in range(steps):
        marks[sidx][0].record(stream)
        step(marks[sidx][1])
        marks[sidx][2].record(stream)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)
    fwd = sum(m[0].elapsed_time(m[1]) for m in marks) / steps
    bwd = sum(m[1].elapsed_time(m[2]) for m in marks) / steps

    # instrumented step: events around each library call
    lib = _lib.load()
    names = ("msd_dsa3d_fwd", "msd_dsa3d_bwd", "msd_dwconv3d_fwd", "msd_dwconv3d_bwd")
    orig = {n: getattr(lib, n) for n in names}
    rec = {n: [] for n in names}

    def wrap(n):
        f = orig[n]

        def w(*a):
            s = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            rc = f(*a)
            e1.record(s)
            rec[n].append((e0, e1))
            return rc
        return w

    for n in names:
        setattr(lib, n, wrap(n))
    try:
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        step()
        e1.record(stream)
        torch.cuda.synchronize()
    finally:
        for n in names:
            setattr(lib, n, orig[n])
    inst_ms = e0.elapsed_time(e1)
    hip = {n[4:]: dict(calls=len(v), ms=round(sum(a.elapsed_time(b) for a, b in v), 4))
           for n, v in rec.items()}
    hip_total = sum(v["ms"] for v in hip.values())
    return dict(total_ms=total_ms, wall_s=wall, tokens=B * T * H * W, fwd_ms=fwd, bwd_ms=bwd,
                hip=hip, other_ms=inst_ms - hip_total, inst_ms=inst_ms,
                bwd_call_ms=hip["dsa3d_bwd"]["ms"] / max(1, hip["dsa3d_bwd"]["calls"]))


def module_flops(cfg):
    """Dense GEMM flops of one step (forward, backward's two products per GEMM,
    and the checkpoint's recomputed forward)."""
    N, D, nh, C = _sizes(cfg)
    per = 2 * N * (4 * D * D + D * C)          # q, k, v, out projections and the offset 1x1 conv
    if cfg["module"] == "block":
        per += 2 * N * 2 * D * 4 * D           # MLP fc1, fc2
    return per * (3 + (1 if cfg.get("checkpoint") else 0))


def cpu_baseline_module(cfg, runs=3):
    """float32 CPU oracle of the same module (the reference op sequence: the
    attention module restatement, or the DiT block around it) on a slab of the
    workload, forward + backward over the input and every parameter, one
    warm-up then the median of `runs`; its tokens/s stands for the workload's."""
    from oracle.dsa3d_ref import dit_block_ref, dsa3d_module_ref

    slab = dict(B=cfg["B"], T=cfg["T"], H=cfg["H"], W=cfg["W"])
    slab.update(cfg["cpu_slab"])
    B, T, H, W = slab["B"], slab["T"], slab["H"], slab["W"]
    from megaslide_amd import DeformableSlideAttention3D, DiTBlock
    D, nh = cfg["D"], cfg["nh"]
    g = torch.Generator().manual_seed(11)
    m = (DeformableSlideAttention3D(D, nh, kernel_size=cfg["kernel"]) if cfg["module"] == "attention"
         else DiTBlock(_BlockConfig(D, nh, cfg["kernel"])))
    _init_like_model(m, g)
    params = {n: p.detach().float().clone().requires_grad_(True) for n, p in m.named_parameters()}
    N = T * H * W
    x = torch.randn(B, N, D, requires_grad=True)
    gy = torch.randn(B, N, D)

    def one():
        if cfg["module"] == "attention":
            y = dsa3d_module_ref(x, params, (T, H, W), nh, cfg["kernel"], 1.0, head_chunk=4)
        else:
            y = dit_block_ref(x, params, (T, H, W), nh, cfg["kernel"], 1.0, head_chunk=4)
        torch.autograd.grad(y, [x] + list(params.values()), grad_outputs=gy, allow_unused=True)

    one()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return dict(
        value=B * N / med, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
        sample=(f"slab-extrapolated: float32 CPU oracle of the whole "
                f"{'attention module' if cfg['module'] == 'attention' else 'DiT block'} "
                f"(GEMMs, depthwise convs, grid_sample/matmul/softmax core"
                f"{', LayerNorms, MLP' if cfg['module'] == 'block' else ''}), fwd+bwd on a "
                f"B={B}, T={T}, H={H}, W={W} slab ({B * N} tokens, dim {D}, {nh}x{D // nh}); "
                f"median of {runs} runs after a warm-up: " + ", ".join(f"{t:.2f}" for t in times)
                + " s"),
        cpu_model=_cpu_model(), torch_version=torch.__version__, seconds=med)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, runs=3):
    """float32 CPU oracle (reference op sequence) on a slab of the workload: the
    same kernel set (both depthwise convs and the attention core, forward and,
    for a training workload, backward), one warm-up then `runs` timed runs; the
    median's tokens/s stands for the workload's (slab-extrapolated)."""
    from oracle.dsa3d_ref import dsa3d_core_ref, dwconv3d_ref

    slab = dict(B=cfg["B"], T=cfg["T"], H=cfg["H"], W=cfg["W"])
    full_cfg = dict(slab)
    slab.update(cfg["cpu_slab"])
    B, T, H, W = slab["B"], slab["T"], slab["H"], slab["W"]
    D, nh = cfg["D"], cfg["nh"]
    kt, kh, kw = cfg["kernel"]
    N = T * H * W
    C = nh * kt * kh * kw * 3
    torch.manual_seed(0)
    grad = cfg["backward"]
    x = torch.randn(B, N, D, requires_grad=grad)
    q, k, v = (torch.randn(B, N, D, requires_grad=grad) for _ in range(3))
    std = cfg["offsets"][1] if cfg["offsets"][0] == "normal" else 0.5
    off = (torch.randn(B, N, C) * std).requires_grad_(grad)
    w7 = (torch.randn(D, 1, kt, kh, kw) * 0.05).requires_grad_(grad)
    w3 = (torch.randn(D, 1, 3, 3, 3) * 0.1).requires_grad_(grad)
    b = torch.zeros(D, requires_grad=grad)
    gy = torch.randn(B, N, D)
    G = cfg.get("extra_g", 0)
    ek = torch.randn(B, G, D, requires_grad=grad) if G else None
    ev = torch.randn(B, G, D, requires_grad=grad) if G else None

    def one():
        with torch.set_grad_enabled(grad):
            y7 = dwconv3d_ref(x, w7, b, (T, H, W))
            f = dwconv3d_ref(x, w3, b, (T, H, W), act="gelu")
            o = dsa3d_core_ref(q, k, v, off, (T, H, W), nh, cfg["kernel"], 1.0, head_chunk=4,
                               extra_k=ek, extra_v=ev)
            if grad:
                torch.autograd.backward([y7, f, o], [gy, gy, gy])

    one()  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    what = "fwd+bwd" if grad else "fwd"
    return dict(
        value=N * B / med, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
        sample=(f"{'slab-extrapolated' if full_cfg != slab else 'whole workload'}: float32 CPU "
                f"oracle (grid_sample/matmul/softmax restatement + conv3d), {what} of the same "
                f"kernel set on a B={B}, T={T}, H={H}, W={W} slab "
                f"({B * N} tokens, dim {D}, {nh}x{D // nh}, window {kt}x{kh}x{kw}); median of "
                f"{runs} runs after a warm-up: " + ", ".join(f"{t:.2f}" for t in times) + " s"),
        cpu_model=_cpu_model(), torch_version=torch.__version__, seconds=med)


def accumulation(cfg):
    """How the workload's backward sums dK / dV over query tiles (msd_accum)."""
    return cfg.get("dkv_accum", "fp32")


def phase_kernels(dtype, accum="fp32", extra=0):
    """Bench phase -> the kernels its ABI call launches, in order (bf16 adds the
    conversion of the fp32 dK / dV rows to bf16; bf16 with fp32 accumulation and
    no extra keys runs the column-streaming dq/dK/dV kernel and the tile kernel
    over the columns it leaves; with fp16 accumulation the scale kernels before
    the dq/dK/dV kernel, the conversion, and the fp32 redo after an overflow,
    whose kernels return at once without one)."""
    if dtype != "bf16":
        return {"dsa3d_fwd": ["dsa3d_fwd_tiled_kernel"],
                "dsa3d_bwd": ["dsa3d_bwd_p1_kernel", "dsa3d_bwd_p2_kernel"]}
    if accum == "fp32" and extra:
        return {"dsa3d_fwd": ["dsa3d_fwd_tiled_kernel"],
                "dsa3d_bwd": ["dsa3d_bwd_p1_kernel", "dsa3d_bwd_extra_kernel",
                              "dsa3d_bwd_p2_kernel", "extra_grad_kernel",
                              "acc_to_bf16_kernel"]}
    if accum == "fp32":
        return {"dsa3d_fwd": ["dsa3d_fwd_tiled_kernel"],
                "dsa3d_bwd": ["dsa3d_bwd_p1_kernel", "dsa3d_bwd_p2s_kernel",
                              "dsa3d_bwd_p2_list_kernel", "acc_to_bf16_kernel"]}
    return {"dsa3d_fwd": ["dsa3d_fwd_tiled_kernel"],
            "dsa3d_bwd": ["dsa3d_bwd_p1_kernel", "h16_bounds_kernel", "h16_scales_kernel",
                          "dsa3d_bwd_p2_kernel", "h16_to_bf16_kernel", "fill_zero_if_flag",
                          "dsa3d_bwd_p2_redo_kernel", "acc_to_bf16_kernel"]}


def summarize(workload, trace_dir, fetch_dir, write_dir):
    """Per-kernel averages from a rocprofv3 --kernel-trace --stats run and the
    FETCH_SIZE / WRITE_SIZE runs of this script (--copy-calibration, one step);
    prints a markdown summary and records in profiles/traffic.json, under the
    workload, each bench phase's summed counters over the kernels of one ABI
    call, scaled by the copy."""
    import csv
    import glob

    cfg = WORKLOADS[workload]
    e = 2 if cfg["dtype"] == "bf16" else 4

    def one(pattern):
        hits = glob.glob(os.path.join(pattern))
        if not hits:
            raise FileNotFoundError(pattern)
        with open(hits[0]) as f:
            return list(csv.DictReader(f))

    stats = one(os.path.join(trace_dir, "*kernel_stats.csv"))
    print("| kernel | calls | avg ms | share |\n|---|---|---|---|")
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"])):
        print(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e6:.3f} | "
              f"{float(r['Percentage']):.1f}% |")

    def dispatches(rows, counter):
        acc = {}
        for r in rows:
            if r["Counter_Name"] != counter:
                continue
            key = (int(r["Dispatch_Id"]), r["Kernel_Name"])
            acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"])
        return sorted((d, name, v) for (d, name), v in acc.items())

    def phase_sum(seq, names):
        """Counter sum over the first run of consecutive dispatches matching `names`."""
        for i in range(len(seq) - len(names) + 1):
            if all(names[j] in seq[i + j][1] for j in range(len(names))):
                j, total = i, 0.0
                # a phase may launch a kernel more than once (channel windows)
                for name in names:
                    while j < len(seq) and name in seq[j][1]:
                        total += seq[j][2]
                        j += 1
                return total
        return None

    fetch = dispatches(one(os.path.join(fetch_dir, "*counter_collection.csv")), "FETCH_SIZE")
    write = dispatches(one(os.path.join(write_dir, "*counter_collection.csv")), "WRITE_SIZE")
    copy_f = [v for _, n, v in fetch if "neg_kernel" in n]
    copy_w = [v for _, n, v in write if "neg_kernel" in n]
    if not copy_f or not copy_w:
        raise RuntimeError("no calibration copy (neg_kernel) in the counter runs")
    kib = COPY_BYTES / 1024.0
    sf, sw = copy_f[0] / kib, copy_w[0] / kib  # counter KiB per true KiB
    print(f"\ncalibration copy {COPY_BYTES >> 20} MiB -> {COPY_BYTES >> 20} MiB: "
          f"FETCH_SIZE {copy_f[0]:.0f} KiB (x{sf:.3f}), WRITE_SIZE {copy_w[0]:.0f} KiB (x{sw:.3f})")
    # the read-only pass over the same 512 MiB (the largest reduction), a
    # second point for the FETCH_SIZE scale
    ro = [v for _, n, v in fetch if "reduce_kernel" in n]
    sf_ro = max(ro) / kib if ro else None
    if sf_ro is not None:
        print(f"read-only pass over {COPY_BYTES >> 20} MiB: FETCH_SIZE {max(ro):.0f} KiB "
              f"(x{sf_ro:.3f}; the copy's factor over it: {sf / sf_ro:.3f})")
    print()
    ab = kernel_bytes(cfg, e)
    rec = {}
    print("| phase (kernels) | FETCH KiB | WRITE KiB | traffic (scaled) | algorithmic | traffic / algorithmic |")
    print("|---|---|---|---|---|---|")
    for phase, names in phase_kernels(cfg["dtype"], accumulation(cfg),
                                      cfg.get("extra_g", 0)).items():
        f_kib, w_kib = phase_sum(fetch, names), phase_sum(write, names)
        if f_kib is None or w_kib is None:
            continue
        traffic = 1024.0 * (f_kib / sf + w_kib / sw)
        rec[phase] = {"kernels": names, "bytes_per_launch": int(traffic),
                      "fetch_kib": round(f_kib, 1), "write_kib": round(w_kib, 1),
                      "fetch_scale": round(sf, 4), "write_scale": round(sw, 4)}
        if sf_ro is not None:
            rec[phase]["fetch_scale_read_only"] = round(sf_ro, 4)
        print(f"| {phase} ({', '.join(names)}) | {f_kib:.0f} | {w_kib:.0f} | {traffic / 1e9:.3f} GB | "
              f"{ab[phase] / 1e9:.3f} GB | {traffic / ab[phase]:.2f} |")
    print("\nPer kernel (counter KiB, unscaled):\n\n| dispatch | kernel | FETCH | WRITE |\n|---|---|---|---|")
    wmap = {(d, n): v for d, n, v in write}
    for d, n, v in fetch:
        if "msd" in n:
            print(f"| {d} | `{n[:70]}` | {v:.0f} | {wmap.get((d, n), float('nan')):.0f} |")
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            allrec = json.load(f)
    except (OSError, ValueError):
        allrec = {}
    allrec[workload] = rec
    with open(path, "w") as f:
        json.dump(allrec, f, indent=1)


def counter_table(*dirs):
    """Per-kernel table from rocprofv3 --pmc runs of this script (one bench
    step each, counters split over passes): instructions per wave, LDS
    bank-conflict cycles per LDS instruction, wave-cycles per busy cycle.
    Counters are summed over every dispatch of a kernel name in a pass, then
    divided by the pass's SQ_WAVES for the same kernel name."""
    import csv
    import glob

    per = {}  # kernel -> counter -> (value summed over dispatches, dispatches)
    for d in dirs:
        for path in glob.glob(os.path.join(d, "*counter_collection.csv")):
            with open(path) as f:
                for r in csv.DictReader(f):
                    name = r["Kernel_Name"]
                    if "msd::" not in name:
                        continue
                    short = name.replace("(anonymous namespace)::", "").replace("msd::", "")
                    short = short.split("(")[0].replace("void ", "")
                    c = per.setdefault(short, {}).setdefault(d, {})
                    key = r["Counter_Name"]
                    c.setdefault(key, {})
                    c[key][r["Dispatch_Id"]] = c[key].get(r["Dispatch_Id"], 0.0) + \
                        float(r["Counter_Value"])
    cols = ["SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_MFMA",
            "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR"]
    print("| kernel | waves | VALU/wave | SALU/wave | LDS/wave | MFMA/wave | VMEM rd/wave | "
          "VMEM wr/wave | LDS bank-conflict cycles / LDS instr | wave-cycles / busy cycle | "
          "wait-any / wave-cycles |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for k in sorted(per):
        vals, waves = {}, None
        for d, cs in per[k].items():
            w = sum(cs.get("SQ_WAVES", {}).values()) or None
            for name, disp in cs.items():
                if name == "SQ_WAVES":
                    waves = w
                    continue
                tot = sum(disp.values())
                vals[name] = tot / w if w and name.startswith("SQ_INSTS") else tot
        if not waves:
            continue

        def f(x, p=0):
            return "—" if x is None else f"{x:.{p}f}"
        conf = vals.get("SQ_LDS_BANK_CONFLICT")
        lds = vals.get("SQ_INSTS_LDS")
        ratio = conf / (lds * waves) if conf is not None and lds else None
        wc, busy = vals.get("SQ_WAVE_CYCLES"), vals.get("SQ_BUSY_CYCLES")
        wait = vals.get("SQ_WAIT_ANY")
        print(f"| `{k[:60]}` | {waves:.0f} | " + " | ".join(f(vals.get(c)) for c in cols) +
              f" | {f(ratio, 2)} | {f(wc / busy if wc and busy else None, 1)} | "
              f"{f(wait / wc if wait and wc else None, 2)} |")


def module_line(args, cfg):
    """The JSON line of a module workload (the attention module with its GEMMs,
    or the DiT block)."""
    r = run_module(cfg, args.steps, args.warmup)
    e = 2 if cfg["dtype"] == "bf16" else 4
    kb = kernel_bytes(cfg, e)
    ms_step = r["total_ms"] / args.steps
    N, D, nh, C = _sizes(cfg)
    bwd_ms = r["bwd_call_ms"]
    achieved = kb["dsa3d_bwd"] / (bwd_ms / 1e3) / 1e9
    flops = module_flops(cfg)
    line = {
        "metric": cfg["metric"],
        "value": round(r["tokens"] / (ms_step / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic",
        "config": {
            "workload": cfg["workload"],
            "B": cfg["B"], "T": cfg["T"], "H": cfg["H"], "W": cfg["W"], "dim": D,
            "heads": nh, "head_dim": D // nh, "window": list(cfg["kernel"]),
            "offsets": (f"offset net's predictions, spread ~ N(0, {cfg['offsets'][1]})"
                        if cfg["module"] == "attention" else
                        f"offset net with its bias ~ U(-{cfg['offsets'][1]}, "
                        f"{cfg['offsets'][1]}) voxels, Xavier weights (model.py:164-178)"),
            "accumulation": "fp32 (dK/dV: fp32 atomics)",
            "pass": "fwd+bwd", "checkpoint": cfg.get("checkpoint", "none"),
            "init": "Xavier-uniform weights, zero biases (MegaSlideDiT._init_weights)",
        },
        "per_phase_ms": {"forward": round(r["fwd_ms"], 4), "backward": round(r["bwd_ms"], 4)},
        "hip_calls_one_step": r["hip"],
        "pytorch_ops_ms_one_step": round(r["other_ms"], 4),
        "gemm_tflops": round(flops / (ms_step / 1e3) / 1e12, 1),
        "gemm_flops_per_step": flops,
        "hbm_gbps_hip_set": round(step_bytes(cfg, e) / (ms_step / 1e3) / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "dsa3d_bwd",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(args.workload, "dsa3d_bwd"),
            "algorithmic_bytes_per_launch": kb["dsa3d_bwd"],
            "avg_launch_ms": round(bwd_ms, 4),
        },
        "wall_s_timed_region": round(r["wall_s"], 3),
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline_module(cfg)
        line["cpu_baseline"] = {k: (round(v, 2) if isinstance(v, float) else v)
                                for k, v in cb.items() if k != "seconds"}
    return line


def main():
    if len(sys.argv) == 6 and sys.argv[1] == "--summarize":
        summarize(*sys.argv[2:])
        return
    if len(sys.argv) >= 3 and sys.argv[1] == "--counter-table":
        counter_table(*sys.argv[2:])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 512 MiB copy first (scale for the FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default=DEFAULT)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the 3D-DSA kernels run on a single MI355X "
              "and no multi-GPU path is built.", file=sys.stderr)
        sys.exit(2)

    cfg = WORKLOADS[args.workload]
    if "module" in cfg:
        print(json.dumps(module_line(args, cfg)), flush=True)
        return
    r = run_gpu(cfg, args.steps, args.warmup, args.copy_calibration)
    e = 2 if cfg["dtype"] == "bf16" else 4
    kb = kernel_bytes(cfg, e)
    ms_step = r["total_ms"] / args.steps
    tokens_s = r["tokens"] / (ms_step / 1e3)
    sbytes = step_bytes(cfg, e)
    dom = max(r["per_phase_ms"], key=r["per_phase_ms"].get)
    dom_ms = r["per_phase_ms"][dom]
    achieved = kb[dom] / (dom_ms / 1e3) / 1e9
    N, D, nh, _ = _sizes(cfg)
    line = {
        "metric": cfg["metric"],
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic",
        "config": {
            "workload": cfg["workload"],
            "B": cfg["B"], "T": cfg["T"], "H": cfg["H"], "W": cfg["W"], "dim": D,
            "heads": nh, "head_dim": D // nh, "window": list(cfg["kernel"]),
            "offsets": (f"raw ~ N(0, {cfg['offsets'][1]})" if cfg["offsets"][0] == "normal" else
                        "offset net: depthwise 3x3x3 + GELU + 1x1, weights ~ N(0, {}) / N(0, {}), "
                        "bias {} {}".format(*cfg["offsets"][1:3], *cfg["offsets"][3])),
            "accumulation": ("fp32" if cfg["dtype"] == "fp32" or not cfg["backward"] else
                             {"fp32": "fp32 (dK/dV: fp32 atomics)",
                              "fp16": "fp32 except dK/dV: summed across query tiles in "
                                      "power-of-two-scaled fp16 atomics"}[accumulation(cfg)]),
            "pass": "fwd+bwd" if cfg["backward"] else "fwd",
            "extra_keys": cfg.get("extra_g", 0),
        },
        "hbm_gbps": round(sbytes / (ms_step / 1e3) / 1e9, 1),
        "hbm_frac_of_peak": round(sbytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
        "byte_model": BYTE_MODEL,
        "step_algorithmic_bytes": sbytes,
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(args.workload, dom),
            "algorithmic_bytes_per_launch": kb[dom],
            "avg_launch_ms": round(dom_ms, 4),
        },
        "per_kernel_ms": {k: round(v, 4) for k, v in r["per_phase_ms"].items()},
        "wall_s_timed_region": round(r["wall_s"], 3),
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline(cfg)
        line["cpu_baseline"] = {k: (round(v, 2) if isinstance(v, float) else v)
                                for k, v in cb.items() if k != "seconds"}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
