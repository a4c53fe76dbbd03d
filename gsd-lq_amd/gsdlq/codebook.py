"""A2 (hexagonal) lattice codebooks of GSD-LQ.

The codebook of radius R enumerates the integer pairs (r0, r1) with r0 in
-R..R (outer loop), r1 in -R..R (inner loop) and |r0 + r1| <= R; codeword i
is the plane point (r0 + r1/2, r1*sqrt(3)/2), evaluated in float64 and stored
as float32 (gsd_lq_v2/gsd_lq_cpu_runtime.py:111-118,
gsd_lq_v2/run_gpu_native_chat.py:26-33).  |T_6| = 127, |T_8| = 217.

Besides the float table the engine uses the integer fields (r0, r1) of each
codeword; they are what "unpacked integer fields" means in the parity tests.
"""
from __future__ import annotations

import numpy as np

SUPPORTED_RADII = (6, 8)


def n_points(radius: int) -> int:
    """Number of points of the radius-R hexagon: 3R^2 + 3R + 1."""
    return 3 * radius * radius + 3 * radius + 1


def integer_fields(radius: int) -> np.ndarray:
    """int8 array [n_pts, 2] of (r0, r1) in enumeration order."""
    out = []
    for r0 in range(-radius, radius + 1):
        lo = max(-radius, -radius - r0)
        hi = min(radius, radius - r0)
        for r1 in range(lo, hi + 1):
            out.append((r0, r1))
    return np.array(out, dtype=np.int8)


def xy_table(radius: int) -> np.ndarray:
    """float32 array [n_pts, 2]: the codebook points, computed in float64."""
    f = integer_fields(radius).astype(np.float64)
    s32 = np.sqrt(3.0) / 2.0
    pts = np.empty_like(f)
    pts[:, 0] = f[:, 0] + 0.5 * f[:, 1]
    pts[:, 1] = f[:, 1] * s32
    return pts.astype(np.float32)


def get_turbo_codebook(radius: int = 8):
    """Same return convention as the reference helper: (float32 [n,2], n)."""
    t = xy_table(radius)
    return t, int(t.shape[0])


def index_of(radius: int) -> np.ndarray:
    """int32 [2R+1, 2R+1] map (r0+R, r1+R) -> codeword index, -1 outside."""
    idx = np.full((2 * radius + 1, 2 * radius + 1), -1, dtype=np.int32)
    for i, (a, b) in enumerate(integer_fields(radius).astype(np.int64)):
        idx[a + radius, b + radius] = i
    return idx
