"""Benchmark: 3D-DSA forward + backward through the HIP kernel set on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline] [--copy-calibration]
                    [--workload long-clip-65k|fp32-32k]
    python bench.py --summarize TRACE_DIR FETCH_DIR WRITE_DIR   (rocprofv3 csv output -> profiles/)

Workload (one step = one pass of the hot path over one batch): the 65,536-token
long-clip case -- B=1, T=64, H=W=32, dim 1024, 16 heads x 64, window 3x7x7,
bf16 storage with fp32 accumulation, raw offsets ~ N(0, 0.5), x ~ N(0, 1),
upstream grads ~ N(0, 1).  A step runs, on preallocated device buffers:
  dw_conv 3x7x7 fwd, offset_net depthwise 3x3x3+GELU fwd, attention core fwd,
  attention core bwd, 3x3x3+GELU bwd, 3x7x7 bwd
i.e. every HIP kernel of the module's forward and backward (the dense GEMMs of
the projections stay in hipBLASLt and are not part of the step).

--workload fp32-32k runs the same step on the fp32 32,768-token case instead
(B=2, T=16, H=W=32, dim 512, 8 heads x 64, raw offsets ~ N(0, 1.5)); its line
names that workload and carries no CPU baseline.

Prints one JSON line.  `value` is tokens/s of the whole step; `roofline` is the
dominant kernel's algorithmic HBM bytes per launch over its average duration,
timed with events on the launch stream; `roofline.traffic` is the measured
L2<->fabric bytes per launch of that kernel from profiles/traffic.json (two
rocprofv3 --pmc runs, FETCH_SIZE and WRITE_SIZE, each scaled by the same
counter on a plain copy of known size -- see --copy-calibration), or null when
no measurement for that kernel is recorded; `cpu_baseline` is the float32 CPU
oracle (the reference op sequence) on a bounded T-slab of the same workload.

--copy-calibration first runs a plain 512 MiB -> 512 MiB bf16 copy (torch.neg)
twice, so a counter run of this script also measures the copy the counters
are scaled by.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "3D-DSA fwd+bwd tokens/sec at 65k tokens bf16; achieved HBM GB/s (% of peak)"
HBM_PEAK_GBPS = 8000.0

CFG = dict(B=1, T=64, H=32, W=32, D=1024, nh=16, hd=64, kernel=(3, 7, 7), off_std=0.5,
           dtype="bf16", workload="3D-DSA fwd+bwd HIP kernel set, long-clip 65,536 tokens",
           metric=METRIC)
WORKLOADS = {
    "long-clip-65k": CFG,
    "fp32-32k": dict(B=2, T=16, H=32, W=32, D=512, nh=8, hd=64, kernel=(3, 7, 7), off_std=1.5,
                     dtype="fp32", workload="3D-DSA fwd+bwd HIP kernel set, fp32 32,768 tokens",
                     metric="3D-DSA fwd+bwd tokens/sec at 32k tokens fp32"),
}


def algorithmic_bytes(cfg, e):
    """Compulsory interface bytes per launch of each kernel (each tensor once)."""
    N = cfg["B"] * cfg["T"] * cfg["H"] * cfg["W"]
    D, nh = cfg["D"], cfg["nh"]
    kt, kh, kw = cfg["kernel"]
    C = nh * kt * kh * kw * 3
    return {
        "dwconv7_fwd": N * 2 * e * D,            # read x, write y
        "dwconv3_gelu_fwd": N * 2 * e * D,       # read x, write gelu(z)
        "dsa3d_fwd": N * (e * (4 * D + C) + 4 * nh),   # read q,k,v,off; write out, lse
        "dsa3d_bwd": N * (e * (8 * D + 2 * C) + 4 * nh),  # read q,k,v,off,out,dout,lse; write dq,dk,dv,doff
        "dwconv3_gelu_bwd": N * 3 * e * D,       # read x, dF; write dx
        "dwconv7_bwd": N * 3 * e * D,            # read x, dy; write dx
    }


COPY_BYTES = 512 * 2 ** 20  # read and written once each by the calibration copy


def copy_calibration(dev):
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def measured_traffic(kernel):
    """Traffic bytes per launch recorded for `kernel` in profiles/traffic.json, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("bytes_per_launch")


def run_gpu(steps, warmup, calibrate=False, cfg=CFG):
    from megaslide_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if calibrate:
        copy_calibration(dev)
    c = cfg
    B, T, H, W, D, nh, hd = c["B"], c["T"], c["H"], c["W"], c["D"], c["nh"], c["hd"]
    kt, kh, kw = c["kernel"]
    N = T * H * W
    C = nh * kt * kh * kw * 3
    dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    mdt = _lib.MSD_BF16 if c["dtype"] == "bf16" else _lib.MSD_F32
    g = torch.Generator(device=dev).manual_seed(3)

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(dt)

    x = rnd(B, N, D)
    q, k, v = rnd(B, N, D), rnd(B, N, D), rnd(B, N, D)
    off = rnd(B, N, C, std=c["off_std"])
    dout, dF, dY = rnd(B, N, D), rnd(B, N, D), rnd(B, N, D)
    w7, b7 = rnd(D, 1, kt, kh, kw, std=0.05), rnd(D, std=0.02)
    w3, b3 = rnd(D, 1, 3, 3, 3, std=0.1), rnd(D, std=0.02)
    y7, F = torch.empty_like(x), torch.empty_like(x)
    out = torch.empty_like(q)
    lse = torch.empty(B, N, nh, device=dev, dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    doff = torch.empty_like(off)
    dx3, dx7 = torch.empty_like(x), torch.empty_like(x)
    dw3, db3, dw7, db7 = (torch.empty_like(t) for t in (w3, b3, w7, b7))

    dsa = _lib.DsaDesc(B, T, H, W, nh, hd, kt, kh, kw, mdt, D, D, D, 1.0, 1.0 / math.sqrt(hd))
    cv7 = _lib.ConvDesc(B, T, H, W, D, kt, kh, kw, mdt, 0)
    cv3 = _lib.ConvDesc(B, T, H, W, D, 3, 3, 3, mdt, 1)
    ws_dsa = torch.empty(lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(dsa)), dtype=torch.uint8,
                         device=dev)
    ws7 = torch.empty(lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(cv7)), dtype=torch.uint8,
                      device=dev)
    ws3 = torch.empty(lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(cv3)), dtype=torch.uint8,
                      device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    phases = [
        ("dwconv7_fwd", lambda: lib.msd_dwconv3d_fwd(ctypes.byref(cv7), P(x), P(w7), P(b7), P(y7), sh)),
        ("dwconv3_gelu_fwd", lambda: lib.msd_dwconv3d_fwd(ctypes.byref(cv3), P(x), P(w3), P(b3), P(F), sh)),
        ("dsa3d_fwd", lambda: lib.msd_dsa3d_fwd(ctypes.byref(dsa), P(q), P(k), P(v), P(off), P(out),
                                                P(lse), sh)),
        ("dsa3d_bwd", lambda: lib.msd_dsa3d_bwd(ctypes.byref(dsa), P(q), P(k), P(v), P(off), P(out),
                                                P(dout), P(lse), None, P(dq), P(dk), P(dv), P(doff),
                                                P(ws_dsa), ws_dsa.numel(), sh)),
        ("dwconv3_gelu_bwd", lambda: lib.msd_dwconv3d_bwd(ctypes.byref(cv3), P(x), P(w3), P(b3), P(dF),
                                                          P(dx3), P(dw3), P(db3), P(ws3), ws3.numel(), sh)),
        ("dwconv7_bwd", lambda: lib.msd_dwconv3d_bwd(ctypes.byref(cv7), P(x), P(w7), P(b7), P(dY),
                                                     P(dx7), P(dw7), P(db7), P(ws7), ws7.numel(), sh)),
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
    ev = [[[torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
           for _ in phases] for _ in range(steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    for s in range(steps):
        step(ev[s])
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)
    per_phase = {name: sum(ev[s][i][0].elapsed_time(ev[s][i][1]) for s in range(steps)) / steps
                 for i, (name, _) in enumerate(phases)}
    return dict(total_ms=total_ms, wall_s=wall, per_phase_ms=per_phase, tokens=B * N)


def cpu_baseline(slab_T=6):
    """float32 CPU oracle (reference op sequence) on a T-slab of the workload
    (T=6: 6,144 tokens, ~10 s on 16 host threads)."""
    from oracle.dsa3d_ref import dsa3d_core_ref, dwconv3d_ref

    c = CFG
    B, H, W, D, nh = c["B"], c["H"], c["W"], c["D"], c["nh"]
    T = slab_T
    N = T * H * W
    C = nh * 147 * 3
    torch.manual_seed(0)
    x = torch.randn(B, N, D, requires_grad=True)
    q, k, v = (torch.randn(B, N, D, requires_grad=True) for _ in range(3))
    off = (torch.randn(B, N, C) * c["off_std"]).requires_grad_(True)
    w7 = (torch.randn(D, 1, 3, 7, 7) * 0.05).requires_grad_(True)
    w3 = (torch.randn(D, 1, 3, 3, 3) * 0.1).requires_grad_(True)
    b = torch.zeros(D, requires_grad=True)
    g = torch.randn(B, N, D)

    def one():
        y7 = dwconv3d_ref(x, w7, b, (T, H, W))
        f = dwconv3d_ref(x, w3, b, (T, H, W), act="gelu")
        o = dsa3d_core_ref(q, k, v, off, (T, H, W), nh, (3, 7, 7), 1.0, head_chunk=4)
        torch.autograd.backward([y7, f, o], [g, g, g])

    t0 = time.perf_counter()
    one()
    dt = time.perf_counter() - t0
    return dict(value=N / dt, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"float32 CPU oracle (grid_sample/matmul/softmax restatement + conv3d), "
                       f"fwd+bwd of the same kernel set on a T={T} slab "
                       f"({N} tokens, H=W=32, dim 1024, 16x64, window 3x7x7), one run of {dt:.1f} s",
                seconds=dt)


PHASE_KERNELS = {  # bench phase -> the kernels its ABI call launches, in order
    "dsa3d_fwd": ["dsa3d_fwd_tiled_kernel"],
    "dsa3d_bwd": ["fill_zero_f32", "dsa3d_bwd_p1_kernel", "dsa3d_bwd_p2_kernel",
                  "acc_to_out_kernel"],
}


def summarize(trace_dir, fetch_dir, write_dir):
    """Per-kernel averages from a rocprofv3 --kernel-trace --stats run and the
    FETCH_SIZE / WRITE_SIZE runs of this script (--copy-calibration, one step);
    prints a markdown summary and writes profiles/traffic.json (per bench phase:
    the summed counters of the kernels of one ABI call, scaled by the copy)."""
    import csv
    import glob

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
                return sum(seq[i + j][2] for j in range(len(names)))
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
          f"FETCH_SIZE {copy_f[0]:.0f} KiB (x{sf:.3f}), WRITE_SIZE {copy_w[0]:.0f} KiB (x{sw:.3f})\n")
    ab = algorithmic_bytes(CFG, 2)
    rec = {}
    print("| phase (kernels) | FETCH KiB | WRITE KiB | traffic (scaled) | algorithmic | traffic / algorithmic |")
    print("|---|---|---|---|---|---|")
    for phase, names in PHASE_KERNELS.items():
        f_kib, w_kib = phase_sum(fetch, names), phase_sum(write, names)
        if f_kib is None or w_kib is None:
            continue
        traffic = 1024.0 * (f_kib / sf + w_kib / sw)
        rec[phase] = {"kernels": names, "bytes_per_launch": int(traffic),
                      "fetch_kib": round(f_kib, 1), "write_kib": round(w_kib, 1),
                      "fetch_scale": round(sf, 4), "write_scale": round(sw, 4)}
        print(f"| {phase} ({', '.join(names)}) | {f_kib:.0f} | {w_kib:.0f} | {traffic / 1e9:.3f} GB | "
              f"{ab[phase] / 1e9:.3f} GB | {traffic / ab[phase]:.2f} |")
    print("\nPer kernel (counter KiB, unscaled):\n\n| dispatch | kernel | FETCH | WRITE |\n|---|---|---|---|")
    wmap = {(d, n): v for d, n, v in write}
    for d, n, v in fetch:
        if "msd::" in n:
            print(f"| {d} | `{n[:70]}` | {v:.0f} | {wmap.get((d, n), float('nan')):.0f} |")
    with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as f:
        json.dump(rec, f, indent=1)


def main():
    if len(sys.argv) == 5 and sys.argv[1] == "--summarize":
        summarize(*sys.argv[2:])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 512 MiB copy first (scale for the FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="long-clip-65k")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the 3D-DSA kernels run on a single MI355X "
              "and no multi-GPU path is built (see DESIGN.md for how it would shard).",
              file=sys.stderr)
        sys.exit(2)

    cfg = WORKLOADS[args.workload]
    r = run_gpu(args.steps, args.warmup, args.copy_calibration, cfg)
    e = 2 if cfg["dtype"] == "bf16" else 4
    ab = algorithmic_bytes(cfg, e)
    ms_step = r["total_ms"] / args.steps
    tokens_s = r["tokens"] / (ms_step / 1e3)
    step_bytes = sum(ab.values())
    dom = max(r["per_phase_ms"], key=r["per_phase_ms"].get)
    dom_ms = r["per_phase_ms"][dom]
    achieved = ab[dom] / (dom_ms / 1e3) / 1e9
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
            "B": cfg["B"], "T": cfg["T"], "H": cfg["H"], "W": cfg["W"], "dim": cfg["D"],
            "heads": cfg["nh"], "head_dim": cfg["hd"], "window": list(cfg["kernel"]),
            "offsets": f"raw ~ N(0, {cfg['off_std']})", "accumulation": "fp32",
        },
        "hbm_gbps": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
        "hbm_frac_of_peak": round(step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(dom) if cfg is CFG else None,
            "algorithmic_bytes_per_launch": ab[dom],
            "avg_launch_ms": round(dom_ms, 4),
        },
        "per_kernel_ms": {k: round(v, 4) for k, v in r["per_phase_ms"].items()},
        "wall_s_timed_region": round(r["wall_s"], 3),
    }
    if not args.no_cpu_baseline and cfg is CFG:
        cb = cpu_baseline()
        line["cpu_baseline"] = {k: (round(v, 2) if isinstance(v, float) else v)
                                for k, v in cb.items() if k != "seconds"}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
