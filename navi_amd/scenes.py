"""Seeded procedural scenes compiled to ``.gmdag`` DAG words (host side).

Scene families (y is up; the sensor's elevation axis, sdfdag_backend.py:205-221):

* ``box_room``   — closed 10 x 4 x 10 m room (interior faces are the surface) with
  seeded spheres, radii U[0.3, 1.0] m (the reference's CPU-runnable case).
* ``cluttered``  — 20 x 5 x 20 m volume with 120 axis-aligned solid boxes (sides
  U[0.2, 2] m) and 80 spheres (r U[0.2, 1] m), centres uniform in the volume.
* ``rooms``      — seeded 10 x 10 grid of 4 m rooms: 0.2 m walls 3 m high,
  one door gap >= 0.9 m per interior wall segment, 0.2 m floor and ceiling slabs,
  1-3 furniture boxes (sides U[0.5, 1.5] m) per room.

Compilation follows the reference compiler's cube convention (the geometry's
largest extent plus 2 m, centred, voxel = side / resolution:
``projects/voxel-dag/src/compiler.cpp:313-329``) and its DAG rules (see
``navi_amd/csrc/scene_compiler.cpp``). Samples are the unsigned CSG distance,
truncated at ``trunc`` (0.5 m by default, the truncation the reference's CPU
case is quoted with).
"""

from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

SPHERE, SOLID_BOX, ROOM = 0, 1, 2

# NAVI_SCENE_LIB names another build (the sanitizer build of `make -C navi_amd/csrc asan`)
_LIB_PATH = Path(os.environ.get("NAVI_SCENE_LIB", Path(__file__).resolve().parent / "_lib" / "libnavi_scene.so"))
_lib: ctypes.CDLL | None = None


def _scene_lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise ImportError(f"{_LIB_PATH} is not built (run __graft_entry__.build())")
        so = ctypes.CDLL(str(_LIB_PATH))
        dp = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
        fp = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
        so.navi_scene_sample_dense.argtypes = [dp, ctypes.c_int32, dp, ctypes.c_double, ctypes.c_int32,
                                               ctypes.c_double, fp, ctypes.c_int32]
        so.navi_scene_sample_dense.restype = ctypes.c_int
        so.navi_dag_compile_dense.argtypes = [fp, ctypes.c_int32, ctypes.c_float, ctypes.c_int32,
                                              ctypes.POINTER(ctypes.c_void_p)]
        so.navi_dag_compile_dense.restype = ctypes.c_uint64
        so.navi_scene_compile.argtypes = [dp, ctypes.c_int32, dp, ctypes.c_double, ctypes.c_int32,
                                          ctypes.c_double, ctypes.c_float, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p),
                                          ctypes.POINTER(ctypes.c_uint64)]
        so.navi_scene_compile.restype = ctypes.c_uint64
        so.navi_scene_free.argtypes = [ctypes.c_void_p]
        so.navi_scene_last_error.restype = ctypes.c_char_p
        _lib = so
    return _lib


def _take_words(ptr: ctypes.c_void_p, count: int) -> np.ndarray:
    lib = _scene_lib()
    if count == 0:
        raise RuntimeError(f"scene compile failed: {lib.navi_scene_last_error().decode()}")
    buf = (ctypes.c_uint64 * count).from_address(ptr.value)
    words = np.frombuffer(buf, dtype=np.uint64).copy()
    lib.navi_scene_free(ptr)
    return words


@dataclass
class Scene:
    """A procedural scene and, once compiled, its DAG words and header."""

    name: str
    prims: np.ndarray  # [n, 7] float64: type, 6 parameters
    geometry_lo: np.ndarray
    geometry_hi: np.ndarray
    resolution: int
    trunc: float = 0.5
    free_lo: np.ndarray | None = None  # where free-space origins may be drawn
    free_hi: np.ndarray | None = None
    origin_height: float | None = None
    words: np.ndarray | None = None
    bbox_min: np.ndarray = field(default_factory=lambda: np.zeros(3, np.float32))
    voxel_size: np.float32 = np.float32(0)
    active_bricks: int = 0

    def __post_init__(self) -> None:
        self.bbox_min, self.voxel_size = cube_convention(self.geometry_lo, self.geometry_hi,
                                                         self.resolution)

    @property
    def bbox_max(self) -> list[float]:
        """``bbox_min + voxel * resolution`` as the reference loader derives it
        (``projects/environment/.../integration/voxel_dag.py:244-250``), in double."""
        ext = float(self.voxel_size) * int(self.resolution)
        return [float(self.bbox_min[k]) + ext for k in range(3)]

    @property
    def bbox_min_list(self) -> list[float]:
        return [float(v) for v in self.bbox_min]

    def sdf(self, points: np.ndarray) -> np.ndarray:
        """Signed union distance at points ``[..., 3]`` (float64, numpy)."""
        return union_sdf(self.prims, np.asarray(points, np.float64))

    def compile(self, threads: int = 8) -> np.ndarray:
        lib = _scene_lib()
        out = ctypes.c_void_p()
        active = ctypes.c_uint64()
        bmin = self.bbox_min.astype(np.float64)
        count = lib.navi_scene_compile(
            np.ascontiguousarray(self.prims, np.float64), int(self.prims.shape[0]), bmin,
            float(self.voxel_size), int(self.resolution), float(self.trunc),
            float(self.voxel_size), 0, int(threads), ctypes.byref(out), ctypes.byref(active),
        )
        self.words = _take_words(out, int(count))
        self.active_bricks = int(active.value)
        return self.words

    def dense_grid(self, threads: int = 8) -> np.ndarray:
        """Dense ``[z, y, x]`` float32 samples (only for small resolutions)."""
        n = int(self.resolution)
        grid = np.empty((n, n, n), np.float32)
        code = _scene_lib().navi_scene_sample_dense(
            np.ascontiguousarray(self.prims, np.float64), int(self.prims.shape[0]),
            self.bbox_min.astype(np.float64), float(self.voxel_size), n, float(self.trunc),
            grid.reshape(-1), int(threads))
        if code != 0:
            raise RuntimeError(_scene_lib().navi_scene_last_error().decode())
        return grid

    def free_origins(self, rng: np.random.Generator, count: int, clearance: float = 0.3) -> np.ndarray:
        """Seeded rejection samples with union distance > clearance (float32 ``[count, 3]``)."""
        lo = self.geometry_lo if self.free_lo is None else self.free_lo
        hi = self.geometry_hi if self.free_hi is None else self.free_hi
        out = np.empty((count, 3), np.float32)
        got = 0
        while got < count:
            cand = rng.uniform(lo, hi, (max(64, 4 * (count - got)), 3))
            if self.origin_height is not None:
                cand[:, 1] = self.origin_height
            ok = cand[self.sdf(cand) > clearance]
            take = min(len(ok), count - got)
            out[got:got + take] = ok[:take]
            got += take
        return out


def cube_convention(lo, hi, resolution: int) -> tuple[np.ndarray, np.float32]:
    """Cube of side ``max_extent + 2`` centred on the geometry, float32 arithmetic
    (``compiler.cpp:313-329``)."""
    lo = np.asarray(lo, np.float32)
    hi = np.asarray(hi, np.float32)
    ext = hi - lo
    max_extent = np.float32(max(ext))
    side = np.float32(max_extent + np.float32(2.0))
    voxel = np.float32(side / np.float32(resolution))
    centre = (hi + lo) / np.float32(2.0)
    bmin = (centre - side / np.float32(2.0)).astype(np.float32)
    return bmin, voxel


def union_sdf(prims: np.ndarray, p: np.ndarray) -> np.ndarray:
    d = np.full(p.shape[:-1], np.inf)
    for row in prims:
        t = int(row[0])
        a = row[1:7]
        if t == SPHERE:
            s = np.linalg.norm(p - a[:3], axis=-1) - a[3]
        else:
            c = (a[:3] + a[3:]) / 2.0
            h = (a[3:] - a[:3]) / 2.0
            q = np.abs(p - c) - h
            s = np.linalg.norm(np.maximum(q, 0.0), axis=-1) + np.minimum(q.max(axis=-1), 0.0)
            if t == ROOM:
                s = -s
        d = np.minimum(d, s)
    return d


def _prim(t, *a) -> list[float]:
    a = list(a) + [0.0] * (6 - len(a))
    return [float(t)] + [float(v) for v in a]


def box_room(seed: int = 1, resolution: int = 64, n_spheres: int = 16, trunc: float = 0.5) -> Scene:
    rng = np.random.default_rng(seed)
    lo = np.array([-5.0, 0.0, -5.0])
    hi = np.array([5.0, 4.0, 5.0])
    prims = [_prim(ROOM, *lo, *hi)]
    radii = rng.uniform(0.3, 1.0, n_spheres)
    centres = rng.uniform(lo, hi, (n_spheres, 3))
    prims += [_prim(SPHERE, *c, r) for c, r in zip(centres, radii)]
    return Scene("box_room", np.array(prims), lo, hi, resolution, trunc, lo, hi)


def cluttered(seed: int = 2, resolution: int = 128, n_boxes: int = 120, n_spheres: int = 80,
              trunc: float = 0.5) -> Scene:
    rng = np.random.default_rng(seed)
    lo = np.array([-10.0, 0.0, -10.0])
    hi = np.array([10.0, 5.0, 10.0])
    prims = []
    for _ in range(n_boxes):
        c = rng.uniform(lo, hi)
        s = rng.uniform(0.2, 2.0, 3)
        prims.append(_prim(SOLID_BOX, *(c - s / 2), *(c + s / 2)))
    for _ in range(n_spheres):
        c = rng.uniform(lo, hi)
        prims.append(_prim(SPHERE, *c, rng.uniform(0.2, 1.0)))
    arr = np.array(prims)
    glo, ghi = _prims_bounds(arr)
    return Scene("cluttered", arr, glo, ghi, resolution, trunc, lo, hi)


def rooms(seed: int = 3, resolution: int = 512, grid: int = 10, room: float = 4.0, wall: float = 0.2,
          height: float = 3.0, trunc: float = 0.5) -> Scene:
    rng = np.random.default_rng(seed)
    size = grid * room
    half_w = wall / 2.0
    prims = []
    # floor and ceiling slabs
    prims.append(_prim(SOLID_BOX, 0.0, -wall, 0.0, size, 0.0, size))
    prims.append(_prim(SOLID_BOX, 0.0, height, 0.0, size, height + wall, size))

    def wall_x(x, z0, z1, door):  # wall in the plane x = const, spanning z
        segs = [(z0, z1)]
        if door:
            w = rng.uniform(0.9, 1.4)
            c = rng.uniform(z0 + 0.3 + w / 2, z1 - 0.3 - w / 2)
            segs = [(z0, c - w / 2), (c + w / 2, z1)]
        for a, b in segs:
            prims.append(_prim(SOLID_BOX, x - half_w, 0.0, a, x + half_w, height, b))

    def wall_z(z, x0, x1, door):
        segs = [(x0, x1)]
        if door:
            w = rng.uniform(0.9, 1.4)
            c = rng.uniform(x0 + 0.3 + w / 2, x1 - 0.3 - w / 2)
            segs = [(x0, c - w / 2), (c + w / 2, x1)]
        for a, b in segs:
            prims.append(_prim(SOLID_BOX, a, 0.0, z - half_w, b, height, z + half_w))

    for i in range(grid + 1):
        for j in range(grid):
            interior = 0 < i < grid
            wall_x(i * room, j * room, (j + 1) * room, interior)
            wall_z(i * room, j * room, (j + 1) * room, interior)
    for i in range(grid):
        for j in range(grid):
            for _ in range(int(rng.integers(1, 4))):
                s = rng.uniform(0.5, 1.5, 3)
                s[1] = min(s[1], height - 0.5)
                cx = rng.uniform(i * room + wall + s[0] / 2, (i + 1) * room - wall - s[0] / 2)
                cz = rng.uniform(j * room + wall + s[2] / 2, (j + 1) * room - wall - s[2] / 2)
                prims.append(_prim(SOLID_BOX, cx - s[0] / 2, 0.0, cz - s[2] / 2, cx + s[0] / 2, s[1],
                                   cz + s[2] / 2))
    arr = np.array(prims)
    glo, ghi = _prims_bounds(arr)
    sc = Scene("rooms", arr, glo, ghi, resolution, trunc, np.array([0.0, 0.0, 0.0]),
               np.array([size, height, size]))
    sc.origin_height = 1.5
    return sc


def _prims_bounds(prims: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    lo = np.full(3, np.inf)
    hi = np.full(3, -np.inf)
    for row in prims:
        a = row[1:7]
        if int(row[0]) == SPHERE:
            lo = np.minimum(lo, a[:3] - a[3])
            hi = np.maximum(hi, a[:3] + a[3])
        else:
            lo = np.minimum(lo, a[:3])
            hi = np.maximum(hi, a[3:])
    return lo, hi


def corpus_scene(seed: int, resolution: int = 1024) -> Scene:
    """Multi-scene corpus member: even seeds are cluttered volumes, odd seeds room grids."""
    if seed % 2 == 0:
        return cluttered(seed=seed, resolution=resolution)
    return rooms(seed=seed, resolution=resolution)


def canonical_directions(azimuth_bins: int, elevation_bins: int) -> np.ndarray:
    """Local sensor directions ``[Az*El, 3]`` float32 in the canonical order
    ``az * El + el`` (``sdfdag_backend.py:205-221``)."""
    az = np.linspace(0.0, 2.0 * math.pi, azimuth_bins, endpoint=False, dtype=np.float32)
    el = np.linspace(math.pi / 2.0, -math.pi / 2.0, elevation_bins, endpoint=True, dtype=np.float32)
    az_grid, el_grid = np.meshgrid(az, el, indexing="ij")
    az_flat = az_grid.reshape(-1)
    el_flat = el_grid.reshape(-1)
    cos_el = np.cos(el_flat)
    return np.stack([cos_el * np.sin(az_flat), np.sin(el_flat), -cos_el * np.cos(az_flat)],
                    axis=-1).astype(np.float32)


def world_directions(local: np.ndarray, yaw: np.ndarray) -> np.ndarray:
    """``[B, R, 3]`` = R_y(yaw) · local (``sdfdag_backend.py:1300-1310``), float32."""
    yaw = np.asarray(yaw, np.float32).reshape(-1, 1)
    c = np.cos(yaw).astype(np.float32)
    s = np.sin(yaw).astype(np.float32)
    out = np.empty((yaw.shape[0], local.shape[0], 3), np.float32)
    out[..., 0] = local[None, :, 0] * c + local[None, :, 2] * s
    out[..., 1] = local[None, :, 1]
    out[..., 2] = -local[None, :, 0] * s + local[None, :, 2] * c
    return out
