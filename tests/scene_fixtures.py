"""Small procedural scenes for the parity tests (dense numpy grids, float64 math).

A scene is a union of solids: the inside of a closed box room is free space
(its interior faces are the surface) and spheres / boxes are solid. Grid
samples sit on voxel corners ``bmin + i * voxel`` (projects/voxel-dag/src/
compiler.cpp:474-478) over a cube that pads the geometry's largest extent by
2 m (compiler.cpp:318-329); the value is the unsigned distance to the union's
surface, truncated.
"""

from __future__ import annotations

import numpy as np


def cube_for_extent(lo, hi, res):
    lo = np.asarray(lo, np.float64)
    hi = np.asarray(hi, np.float64)
    ext = float(np.max(hi - lo))
    side = np.float32(ext + 2.0)
    voxel = np.float32(side / np.float32(res))
    centre = (hi + lo) / 2.0
    bmin = (centre - (ext + 2.0) / 2.0).astype(np.float32)
    return bmin, voxel


def box_sdf(p, lo, hi):
    c = (lo + hi) / 2.0
    h = (hi - lo) / 2.0
    q = np.abs(p - c) - h
    outside = np.linalg.norm(np.maximum(q, 0.0), axis=-1)
    inside = np.minimum(np.max(q, axis=-1), 0.0)
    return outside + inside


def sphere_sdf(p, c, r):
    return np.linalg.norm(p - c, axis=-1) - r


def room_with_spheres(res=64, seed=1, n_spheres=16, trunc=0.5):
    """Config-1-like: 10 x 4 x 10 m room (y up) with seeded spheres."""
    rng = np.random.default_rng(seed)
    room_lo = np.array([-5.0, 0.0, -5.0])
    room_hi = np.array([5.0, 4.0, 5.0])
    radii = rng.uniform(0.3, 1.0, n_spheres)
    centres = rng.uniform(room_lo, room_hi, (n_spheres, 3))
    bmin, voxel = cube_for_extent(room_lo, room_hi, res)

    def sdf(p):
        d = -box_sdf(p, room_lo, room_hi)  # solid = outside the interior
        for c, r in zip(centres, radii):
            d = np.minimum(d, sphere_sdf(p, c, r))
        return d

    idx = np.arange(res, dtype=np.float64)
    zz, yy, xx = np.meshgrid(idx, idx, idx, indexing="ij")
    pts = np.stack([bmin[0] + xx * voxel, bmin[1] + yy * voxel, bmin[2] + zz * voxel], axis=-1)
    grid = np.minimum(np.abs(sdf(pts)), trunc).astype(np.float32)
    bmax = (bmin.astype(np.float64) + float(voxel) * res)
    return {
        "grid": grid,
        "bmin": [float(v) for v in bmin],
        "bmax": [float(v) for v in bmax],
        "voxel": float(voxel),
        "res": res,
        "sdf": sdf,
        "room": (room_lo, room_hi),
    }


def free_origin(scene, rng, clearance=0.3, lo=None, hi=None):
    lo = scene["room"][0] if lo is None else lo
    hi = scene["room"][1] if hi is None else hi
    for _ in range(10000):
        p = rng.uniform(lo, hi)
        if scene["sdf"](p[None])[0] > clearance:
            return p.astype(np.float32)
    raise RuntimeError("no free-space origin found")
