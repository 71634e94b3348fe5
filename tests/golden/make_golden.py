"""Write golden vectors for 3D-DSA from the reference module itself.

Run where the reference tree is present (the tests read only the committed
fixtures):

    python tests/golden/make_golden.py [--ref /root/reference]

The reference operator ``DeformableSlideAttention3D``
(infinity/video/attention.py:19-273) is loaded by file path -- only that file,
which imports nothing but ``math``, ``typing`` and ``torch`` -- so the package
``infinity/__init__.py`` with its LLM imports is never executed.  Each case
builds the module, loads a seeded parameter set (tests/golden/inputs.py), runs
forward and backward in float64 (the C1 case in float32, the configuration's
own dtype) and records, via hooks on the module's own submodules:

* ``y`` and the gradients of x and of every parameter for an upstream grad g;
* the intermediates at the operator boundary that the HIP kernels replace:
  the unscaled offsets ``offset_net(x)`` (channel-last [B, N, C]) and their
  gradient, q/k/v (``*_proj`` outputs) and their gradients, and the attention
  output fed to ``out_proj`` and its gradient.

Cases named ``*_inject`` replace ``offset_net`` by a module that returns a given
offsets tensor, so the reference path from ``offsets = self.offset_net(x_5d)``
(attention.py:105) on runs with chosen offsets, including large ones that hit
the border clamp.

Inputs are regenerated from their seeds by the tests; the fixture stores their
sums as a check that regeneration matches.

The ``dit_block`` case runs the reference DiT block around the operator
(infinity/video/model.py:40-117, built from a MegaSlideConfig): model.py,
attention.py and config.py are loaded by path as submodules of a stand-in
package, and y, dx and every parameter gradient are recorded in float64.
"""

from __future__ import annotations

import argparse
import hashlib
import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import inputs as gin  # noqa: E402
from inputs import C1, CASES, case_params  # noqa: E402

def load_reference(ref_root: str):
    path = os.path.join(ref_root, "infinity", "video", "attention.py")
    spec = importlib.util.spec_from_file_location("_ref_dsa_attention", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    with open(path, "rb") as f:
        digest = hashlib.sha256(f.read()).hexdigest()
    return mod.DeformableSlideAttention3D, digest


def load_reference_block(ref_root: str):
    """DiTBlock and MegaSlideConfig from infinity/video/model.py and config.py.

    model.py imports its siblings relatively (``from .attention import``,
    ``from .config import``), so the three files are loaded as submodules of a
    stand-in package whose search path is the infinity/video directory: the
    real package ``__init__`` files (and their LLM and data imports) never run.
    """
    import types
    vdir = os.path.join(ref_root, "infinity", "video")
    pkg = types.ModuleType("_ref_video")
    pkg.__path__ = [vdir]
    sys.modules["_ref_video"] = pkg
    mods = {}
    for name in ("config", "attention", "model"):
        path = os.path.join(vdir, name + ".py")
        spec = importlib.util.spec_from_file_location(f"_ref_video.{name}", path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    h = hashlib.sha256()
    for name in ("config", "attention", "model"):
        with open(os.path.join(vdir, name + ".py"), "rb") as f:
            h.update(f.read())
    return mods["model"].DiTBlock, mods["config"].MegaSlideConfig, h.hexdigest()


def run_block(Block, Config, case, dtype):
    """The reference DiTBlock on the seeded block case: y, dx and every
    parameter gradient for an upstream grad g."""
    p, x_np, gy_np = gin.block_inputs(case)
    B, T, H, W, D, nh = (case[k] for k in ("B", "T", "H", "W", "D", "nh"))
    cfg = Config(frames=T, height=16 * H, width=16 * W, patch_size=16, hidden_size=D,
                 num_layers=1, num_heads=nh, mlp_ratio=case["mlp_ratio"],
                 dsa_kernel_size=tuple(case["kernel"]), offset_scale=case["scale"], dropout=0.0)
    blk = Block(cfg).to(dtype)
    names = [n for n, _ in blk.named_parameters()]
    assert names == list(p), (names, list(p))
    with torch.no_grad():
        for n, prm in blk.named_parameters():
            prm.copy_(torch.from_numpy(p[n]).to(dtype))
    x = torch.from_numpy(x_np).to(dtype).requires_grad_(True)
    y = blk(x, (T, H, W))
    (y * torch.from_numpy(gy_np).to(dtype)).sum().backward()
    out = {"y": y.detach(), "dx": x.grad}
    for n, prm in blk.named_parameters():
        out["grad." + n] = prm.grad if prm.grad is not None else torch.zeros_like(prm)
    meta = dict(case, dtype=str(dtype).replace("torch.", ""), param_names=names,
                x_sum=float(x_np.sum()), gy_sum=float(gy_np.sum()),
                param_sums={k: float(v.sum()) for k, v in p.items()})
    return meta, {k: v.detach().contiguous().numpy() for k, v in out.items()}


class _Inject(torch.nn.Module):
    """Stands in for offset_net: returns the given channel-first offsets."""

    def __init__(self, off_cf: torch.Tensor):
        super().__init__()
        self.off_cf = off_cf

    def forward(self, x):  # noqa: D401 - x is ignored on purpose
        return self.off_cf


def run_case(Ref, case, dtype):
    p, x_np, gy_np, off_np, extra_np = case_params(case)
    B, T, H, W, D, nh = (case[k] for k in ("B", "T", "H", "W", "D", "nh"))
    N = T * H * W
    mod = Ref(D, nh, kernel_size=tuple(case["kernel"]), offset_scale=case["scale"], dropout=0.0)
    mod = mod.to(dtype)
    names = [n for n, _ in mod.named_parameters()]
    with torch.no_grad():
        sd = mod.state_dict()
        for n in names:
            sd[n].copy_(torch.from_numpy(p[n]).to(dtype))
    cap = {}

    def keep(name):
        def hook(grad):
            cap["d" + name] = grad.detach().clone()
        return hook

    def fwd_hook(name):
        def hook(module, inp, out):
            cap[name] = out.detach().clone()
            out.register_hook(keep(name))
        return hook

    if off_np is not None:
        off_cl = torch.from_numpy(off_np).to(dtype)
        off_cf = off_cl.transpose(1, 2).reshape(B, -1, T, H, W).contiguous().requires_grad_(True)
        mod.offset_net = _Inject(off_cf)
    else:
        mod.offset_net.register_forward_hook(fwd_hook("offsets_cf"))
    for nm in ("q_proj", "k_proj", "v_proj"):
        getattr(mod, nm).register_forward_hook(fwd_hook(nm[0]))

    def pre_hook(module, args):
        a = args[0]
        cap["attn"] = a.detach().clone()
        a.register_hook(keep("attn"))
    mod.out_proj.register_forward_pre_hook(pre_hook)

    x = torch.from_numpy(x_np).to(dtype).requires_grad_(True)
    gy = torch.from_numpy(gy_np).to(dtype)
    extra = None
    if extra_np is not None:
        extra = torch.from_numpy(extra_np).to(dtype).requires_grad_(True)
    y = mod(x, (T, H, W), extra_kv=extra)
    (y * gy).sum().backward()

    out = {}
    out["y"] = y.detach()
    out["dx"] = x.grad
    if extra is not None:
        out["dextra_kv"] = extra.grad
    for n, prm in mod.named_parameters():
        out["grad." + n] = prm.grad if prm.grad is not None else torch.zeros_like(prm)
    if off_np is not None:
        # injected offsets are inputs, regenerated from the seed by the tests
        d = off_cf.grad if off_cf.grad is not None else torch.zeros_like(off_cf)
        out["doffsets"] = d.reshape(B, -1, N).transpose(1, 2)
    else:
        out["offsets"] = cap["offsets_cf"].reshape(B, -1, N).transpose(1, 2)
        # no gradient reaches the offsets when every slot's divisor dim is 1
        d = cap.get("doffsets_cf", torch.zeros_like(cap["offsets_cf"]))
        out["doffsets"] = d.reshape(B, -1, N).transpose(1, 2)
    for nm in ("q", "k", "v", "attn"):
        out[nm] = cap[nm]
        out["d" + nm] = cap["d" + nm]
    meta = dict(case, dtype=str(dtype).replace("torch.", ""), param_names=names,
                x_sum=float(x_np.sum()), gy_sum=float(gy_np.sum()),
                param_sums={k: float(v.sum()) for k, v in p.items()},
                off_sum=None if off_np is None else float(off_np.sum()),
                extra_sum=None if extra_np is None else float(extra_np.sum()))
    return meta, {k: v.detach().contiguous().numpy() for k, v in out.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=HERE)
    ap.add_argument("--only", default=None, help="write just this case (e.g. dit_block)")
    args = ap.parse_args()
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    if args.only == gin.BLOCK["name"]:
        write_block(args)
        return
    Ref, digest = load_reference(args.ref)
    for case in CASES:
        if args.only is not None and case["name"] != args.only:
            continue
        meta, arrs = run_case(Ref, case, torch.float64)
        meta["reference_sha256"] = digest
        np.savez_compressed(os.path.join(args.out, f"{case['name']}.npz"),
                            meta=np.array(json.dumps(meta)), **arrs)
        print("wrote", case["name"], {k: v.shape for k, v in arrs.items() if k in ("y", "offsets")})
    if args.only is not None and args.only != C1["name"]:
        return
    meta, arrs = run_case(Ref, C1, torch.float32)
    g = gin.rng(1000)
    rows = np.sort(g.choice(arrs["y"].shape[1], size=C1["rows"], replace=False))
    keep = dict(rows=rows)
    for key in ("y", "attn", "offsets", "dx"):
        keep[key + "_rows"] = arrs[key][:, rows]
        keep[key + "_norm"] = np.array(np.linalg.norm(arrs[key].astype(np.float64)))
    meta["reference_sha256"] = digest
    np.savez_compressed(os.path.join(args.out, "c1_fwd_fp32.npz"), meta=np.array(json.dumps(meta)),
                        **keep)
    print("wrote c1_fwd_fp32")
    write_block(args)


def write_block(args):
    Block, Config, bdigest = load_reference_block(args.ref)
    meta, arrs = run_block(Block, Config, gin.BLOCK, torch.float64)
    meta["reference_sha256"] = bdigest
    np.savez_compressed(os.path.join(args.out, f"{gin.BLOCK['name']}.npz"),
                        meta=np.array(json.dumps(meta)), **arrs)
    print("wrote", gin.BLOCK["name"], arrs["y"].shape)


if __name__ == "__main__":
    main()
