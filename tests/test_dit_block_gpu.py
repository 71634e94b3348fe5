"""The drop-in DiTBlock (megaslide_amd.block) on the GPU.

* Against the reference DiTBlock's own float64 outputs (tests/golden/dit_block.npz,
  written by tests/golden/make_golden.py from infinity/video/model.py:40-117):
  y, dx and every parameter gradient at the fp32 tolerance 1e-4 relative to
  max|ref| (k_proj.bias, zero by the softmax's shift invariance, against the
  k_proj.weight gradient's scale).
* Selective checkpointing (checkpoint_keep_core, checkpoint_keep_gemms): the
  backward's recompute skips the attention core's forward kernel (and, keeping
  the GEMMs, every aten mm / addmm), and every gradient equals a plain (not
  checkpointed) run up to the fp32 atomics' summation order.
"""

import pytest
import torch

from goldens import load, rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"


class _Config:
    def __init__(self, hidden_size, num_heads, dsa_kernel_size, offset_scale=1.0, dropout=0.0,
                 mlp_ratio=4.0):
        self.hidden_size, self.num_heads = hidden_size, num_heads
        self.dsa_kernel_size, self.offset_scale, self.dropout = dsa_kernel_size, offset_scale, dropout
        self.mlp_ratio = mlp_ratio

    @property
    def mlp_hidden_size(self):
        return int(self.hidden_size * self.mlp_ratio)


def test_dit_block_matches_reference_golden():
    from inputs import BLOCK, block_inputs
    from megaslide_amd import DiTBlock

    print("[DiTBlock vs reference golden]", flush=True)
    meta, arrs = load(BLOCK["name"])
    p, x_np, gy_np = block_inputs(BLOCK)
    blk = DiTBlock(_Config(BLOCK["D"], BLOCK["nh"], BLOCK["kernel"], BLOCK["scale"],
                           mlp_ratio=BLOCK["mlp_ratio"]))
    blk.load_state_dict({n: torch.from_numpy(v).float() for n, v in p.items()}, strict=True)
    blk = blk.to(DEV)
    x = torch.from_numpy(x_np).float().to(DEV).requires_grad_(True)
    y = blk(x, (BLOCK["T"], BLOCK["H"], BLOCK["W"]))
    (y * torch.from_numpy(gy_np).float().to(DEV)).sum().backward()
    torch.cuda.synchronize()
    errs = {"y": rel_err(y.detach().cpu(), arrs["y"]), "dx": rel_err(x.grad.cpu(), arrs["dx"])}
    kw = float(abs(arrs["grad.attn.k_proj.weight"]).max())
    for n, prm in blk.named_parameters():
        ref = torch.from_numpy(arrs["grad." + n])
        if n == "attn.k_proj.bias":
            errs[n] = float((prm.grad.double().cpu() - ref).abs().max()) / kw
        else:
            errs[n] = rel_err(prm.grad.cpu(), ref, floor=1e-2)
    worst = max(errs, key=errs.get)
    print(f"  max rel err {errs[worst]:.2e} ({worst})", flush=True)
    bad = {k: v for k, v in errs.items() if not v < 1e-4}
    assert not bad, bad


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_selective_checkpoint_skips_core_recompute(dt):
    from megaslide_amd import DiTBlock, checkpoint_keep_core, checkpoint_keep_gemms
    from megaslide_amd import ops
    from torch.utils._python_dispatch import TorchDispatchMode
    from torch.utils.checkpoint import checkpoint

    print(f"[checkpoint keeping the core] {dt}", flush=True)
    B, T, H, W, D, nh = 1, 4, 8, 9, 128, 2
    N = T * H * W
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(3)
        blk = DiTBlock(_Config(D, nh, (3, 7, 7)))
    with torch.no_grad():
        blk.attn.offset_net[2].weight.normal_(0.0, 0.02, generator=torch.Generator().manual_seed(4))
        blk.attn.offset_net[2].bias.uniform_(-2.0, 2.0, generator=torch.Generator().manual_seed(5))
    blk = blk.to(DEV, dt)
    g = torch.Generator(device=DEV).manual_seed(6)
    x = torch.randn(B, N, D, generator=g, device=DEV).to(dt)
    gy = torch.randn(B, N, D, generator=g, device=DEV).to(dt)

    calls = []
    orig = ops._CoreCall.forward

    def counting(self, want_lse):
        calls.append(want_lse)
        return orig(self, want_lse)

    gemms = (torch.ops.aten.mm.default, torch.ops.aten.addmm.default)

    class CountGemms(TorchDispatchMode):
        """Counts the GEMMs of the forward, the backward and the backward's
        recompute (the checkpoint's own mode sits above this one, so a GEMM it
        answers from its saved outputs is not counted)."""
        n = 0

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            if func in gemms:
                CountGemms.n += 1
            return func(*args, **(kwargs or {}))

    def run(mode):
        xi = x.clone().requires_grad_(True)
        with CountGemms():
            if mode == "plain":
                y = blk(xi, (T, H, W))
            elif mode == "checkpoint":
                y = checkpoint(blk, xi, (T, H, W), use_reentrant=False)
            elif mode == "keep_core":
                y = checkpoint_keep_core(blk, xi, (T, H, W))
            else:
                y = checkpoint_keep_gemms(blk, xi, (T, H, W))
            gr = torch.autograd.grad(y, (xi, *blk.parameters()), grad_outputs=gy)
        return y.detach(), gr

    ops._CoreCall.forward = counting
    try:
        counts, mms, res = {}, {}, {}
        for mode in ("plain", "checkpoint", "keep_core", "keep_gemms"):
            calls.clear()
            CountGemms.n = 0
            res[mode] = run(mode)
            torch.cuda.synchronize()
            counts[mode], mms[mode] = len(calls), CountGemms.n
    finally:
        ops._CoreCall.forward = orig
    print(f"  core forward launches: {counts}; GEMMs: {mms}", flush=True)
    assert counts == {"plain": 1, "checkpoint": 2, "keep_core": 1, "keep_gemms": 1}
    # the plain checkpoint reruns the forward GEMMs up to the last one whose
    # inputs the backward needs (offset, q, k, v, out, fc1: not fc2), keeping
    # the GEMMs reruns none
    assert mms["checkpoint"] - mms["plain"] == 6, mms
    assert mms["keep_core"] == mms["checkpoint"], mms
    assert mms["keep_gemms"] == mms["plain"], mms
    y0, g0 = res["plain"]
    names = ["x"] + [n for n, _ in blk.named_parameters()]
    kw = g0[names.index("attn.k_proj.weight")].float().abs().max().item()
    tol = 1e-5 if dt == torch.float32 else 1e-2
    for mode in ("keep_core", "keep_gemms"):
        y1, g1 = res[mode]
        assert torch.equal(y0, y1), mode
        for n, a, b in zip(names, g0, g1):
            if n == "attn.k_proj.bias":  # rounding noise around zero
                assert (b.float() - a.float()).abs().max().item() < tol * kw, (mode, n)
            else:
                assert rel_err(b.float().cpu(), a.float().cpu(), floor=1e-6) < tol, (mode, n)
