"""Pure-numpy loop restatement of 3D-DSA for tiny inputs (oracle, test-only).

TEST INFRASTRUCTURE ONLY.  It pins two things that the torch restatement in
``oracle.dsa3d_ref`` takes from a library call:

* the sampling rule of ``F.grid_sample(mode='bilinear', padding_mode='border',
  align_corners=False)`` on a 5-D input (infinity/video/attention.py:262-268):
  unnormalise ``u = ((g + 1)*S - 1)/2``, clamp to [0, S-1], 8-corner trilinear
  weights, corners with an index >= S contribute nothing;
* the closed-form backward that the HIP kernels implement: softmax backward,
  scatter of dK/dV through the trilinear weights, and the coordinate gradient
  through the clamp (zero where u <= 0 or u >= S-1, as grid_sample's border mode
  defines it) and the unnormalisation (factor S/2), then back to the raw offset
  slots through the reference's slot/axis mapping (attention.py:118-127).

Loops are over (b, head, query, tap); channels are numpy vectors.  Only for
tiny shapes (a few hundred queries).
"""

from __future__ import annotations

import math
from typing import Sequence, Tuple

import numpy as np


def _axis_base(S: int, p: int, c: int) -> np.float32:
    # attention.py:209-230, evaluated in float32 like the reference
    num = np.float32(2.0) * (np.float32(p) + np.float32(c))
    return np.float32(num / np.float32(max(S - 1, 1))) - np.float32(1.0)


def tap_coords(T: int, H: int, W: int, t: int, h: int, w: int, ci: int, cj: int, ck: int,
               o: np.ndarray) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Grid value g, unnormalised u and clamped i for axes (x, y, z) of one tap.

    ``o`` holds the three raw (already offset_scale-multiplied) slots.  Slot 0
    goes to x divided by T-1, slot 1 to y by H-1, slot 2 to z by W-1
    (attention.py:118-127); a slot is dropped when its divisor dim is 1.
    """
    o = np.asarray(o, dtype=np.float64)
    base = np.array([_axis_base(W, w, ck), _axis_base(H, h, cj), _axis_base(T, t, ci)],
                    dtype=np.float64)
    add = np.zeros(3)
    if T > 1:
        add[0] = o[0] / (T - 1)
    if H > 1:
        add[1] = o[1] / (H - 1)
    if W > 1:
        add[2] = o[2] / (W - 1)
    g = base + add
    sizes = np.array([W, H, T], dtype=np.float64)
    u = ((g + 1.0) * sizes - 1.0) / 2.0
    i = np.minimum(np.maximum(u, 0.0), sizes - 1.0)
    return g, u, i


def corners(i: np.ndarray, sizes_xyz: Sequence[int]):
    """Yield (x, y, z, weight, dweight/d(ix,iy,iz)) for the in-bounds corners."""
    x0, y0, z0 = (int(math.floor(v)) for v in i)
    fx, fy, fz = i[0] - x0, i[1] - y0, i[2] - z0
    W, H, T = sizes_xyz
    for dz in (0, 1):
        wz = fz if dz else 1.0 - fz
        sz = 1.0 if dz else -1.0
        for dy in (0, 1):
            wy = fy if dy else 1.0 - fy
            sy = 1.0 if dy else -1.0
            for dx in (0, 1):
                wx = fx if dx else 1.0 - fx
                sx = 1.0 if dx else -1.0
                x, y, z = x0 + dx, y0 + dy, z0 + dz
                if 0 <= x < W and 0 <= y < H and 0 <= z < T:
                    yield x, y, z, wx * wy * wz, np.array([sx * wy * wz, sy * wx * wz, sz * wx * wy])


def dsa3d_core_bruteforce(q, k, v, off, video_shape, num_heads, kernel_size,
                          offset_scale=1.0, dout=None):
    """Forward (and, with ``dout``, backward) of the core by explicit loops.

    Shapes as ``oracle.dsa3d_ref.dsa3d_core_ref``.  Returns ``out`` or
    ``(out, dq, dk, dv, doff)``; ``doff`` is the gradient w.r.t. the unscaled
    offsets.  fp64 throughout.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    off = np.asarray(off, np.float64) * offset_scale
    B, N, D = q.shape
    T, H, W = video_shape
    nh = num_heads
    hd = D // nh
    kt, kh, kw = kernel_size
    K = kt * kh * kw
    scale = 1.0 / math.sqrt(hd)
    sizes = np.array([W, H, T], dtype=np.float64)
    div = np.array([(T - 1) if T > 1 else 0, (H - 1) if H > 1 else 0, (W - 1) if W > 1 else 0],
                   dtype=np.float64)
    out = np.zeros_like(q)
    if dout is not None:
        dout = np.asarray(dout, np.float64)
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        doff = np.zeros_like(off)
    for b in range(B):
        for m in range(nh):
            cs = slice(m * hd, (m + 1) * hd)
            for t in range(T):
                for h in range(H):
                    for w in range(W):
                        n = (t * H + h) * W + w
                        qv = q[b, n, cs]
                        taps = []
                        for i in range(kt):
                            for j in range(kh):
                                for kk in range(kw):
                                    kap = (i * kh + j) * kw + kk
                                    ch = (m * K + kap) * 3
                                    g, u, ic = tap_coords(T, H, W, t, h, w, i - kt // 2,
                                                          j - kh // 2, kk - kw // 2,
                                                          off[b, n, ch:ch + 3])
                                    cl = list(corners(ic, (W, H, T)))
                                    ks = sum((wt * k[b, (z * H + y) * W + x, cs]
                                              for x, y, z, wt, _ in cl), np.zeros(hd))
                                    vs = sum((wt * v[b, (z * H + y) * W + x, cs]
                                              for x, y, z, wt, _ in cl), np.zeros(hd))
                                    taps.append((ch, u, cl, ks, vs))
                        s = np.array([qv @ tp[3] for tp in taps]) * scale
                        p = np.exp(s - s.max())
                        p /= p.sum()
                        o = sum((p[a] * taps[a][4] for a in range(K)), np.zeros(hd))
                        out[b, n, cs] = o
                        if dout is None:
                            continue
                        go = dout[b, n, cs]
                        dp = np.array([go @ tp[4] for tp in taps])
                        delta = float(p @ dp)
                        ds = p * (dp - delta)
                        for a, (ch, u, cl, ks, vs) in enumerate(taps):
                            dq[b, n, cs] += ds[a] * scale * ks
                            dks = ds[a] * scale * qv
                            dvs = p[a] * go
                            gi = np.zeros(3)
                            for x, y, z, wt, dw in cl:
                                r = (z * H + y) * W + x
                                dk[b, r, cs] += wt * dks
                                dv[b, r, cs] += wt * dvs
                                gi += dw * (dks @ k[b, r, cs] + dvs @ v[b, r, cs])
                            inside = (u > 0.0) & (u < sizes - 1.0)
                            gg = gi * inside * sizes / 2.0
                            for a3 in range(3):
                                if div[a3] > 0:
                                    doff[b, n, ch + a3] = gg[a3] / div[a3] * offset_scale
    if dout is None:
        return out
    return out, dq, dk, dv, doff
