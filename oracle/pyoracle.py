"""ctypes front end of ``liboracle.so`` plus numpy/torch-CPU restatements.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Functions and what pins each one (the pinning tests in brackets, ``tests/<file>::<test>``):

* ``trace`` / ``trace_multi`` — restate ``projects/torch-sdf/cpp_src/kernel.cu:9-309``.
  Pinned by the ten known answers of ``projects/torch-sdf/tests/test_sphere_tracing.py:683-949``
  [test_oracle_tracer::test_known_answers], hand-derived void exits and leaf accumulation
  [::test_void_cell_exit_closed_form, ::test_leaf_accumulation_closed_form], the slab distance of
  ``projects/contracts/src/navi_contracts/testing/oracle_box.py:115-160``
  [::test_unit_box_rays_within_reference_tolerance] and a cache-free brute-force march
  [::test_cache_free_march_agrees_off_faces]; a planted mistake must fail them
  [::test_planted_mistake_is_caught].
* ``point_query`` — build-defined clearance query (no reference kernel). Pinned by answers
  derived by hand on the reference's fixture DAGs (outside / faces / popcount child choice /
  void octants) [test_oracle_tracer::test_point_query_closed_forms], by the pinned tracer's
  first step at the same point (leaf distance, 1000 outside, void side = sum of the +x and
  -x exits) [::test_point_query_agrees_with_one_step_trace], and by the compiler's pruning
  guarantee on the dense grid (every sample of a void block exceeds the bound; the parent's
  side, a planted mistake, violates it) [::test_point_query_void_bound_holds_on_the_grid].
* ``half_to_float`` / ``float_to_half`` — IEEE binary16, pinned exhaustively against numpy's
  float16 [test_oracle_codecs::test_half_decode_exhaustive, ::test_half_encode_rne_matches_numpy].
  ``float_to_half(quirk=True)`` restates ``projects/voxel-dag/src/compiler.cpp:542-560``, pinned by
  hand-derived bit patterns [test_oracle_codecs::test_reference_quirk_encoder].
* ``compile_dense`` — restates ``compiler.cpp:563-674``, pinned by hand-built DAGs of tiny grids
  and the reference's contract tests [test_compiler::test_two_voxel_grid_by_hand and neighbours].
* ``ray_directions`` / ``yaw_rotate`` — restate ``projects/environment/src/navi_environment/
  backends/sdfdag_backend.py:205-221,1300-1310``; pinned by the cardinal directions, unit norms,
  poles and index map of ``projects/environment/tests/unit/test_ray_direction_oracle.py``
  [test_caller_side::test_cardinal_directions and neighbours]. Exact float32 bits of numpy's
  sin/cos are parity unpinned (atol 1e-6).
* ``postprocess`` / ``fp16_depth_obs`` — restate ``sdfdag_backend.py:408-473``; pinned by the known
  values of ``projects/environment/tests/unit/test_postprocessing_oracle.py`` and the horizon cases
  of ``test_sdfdag_conventions.py:604-730`` [test_caller_side::test_postpass_known_values,
  ::test_postpass_horizon_cases]. torch CPU ``log1p`` bits versus the reference's CUDA ``log1p``
  are parity unpinned (atol 1e-6 in the reference's tests).
* ``observation_ratios`` / ``observe`` — restate ``sdfdag_backend.py:366-405`` and the collision
  test of ``:1340``; pinned by the known answer of ``test_sdfdag_conventions.py:123-142`` and
  counts built by hand [test_caller_side::test_observation_ratios_known_answer,
  ::test_observation_ratios_by_hand].
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

__all__ = [
    "HIT_EPSILON",
    "OUTSIDE_DOMAIN",
    "lib",
    "trace",
    "trace_multi",
    "trace_nocache",
    "point_query",
    "half_to_float",
    "float_to_half",
    "compile_dense",
    "ray_directions",
    "yaw_rotate",
    "postprocess",
    "fp16_depth_obs",
    "observation_ratios",
    "observe",
]

HIT_EPSILON = 0.01  # kernel.cuh:7
OUTSIDE_DOMAIN = 1000.0  # kernel.cuh:8

_HERE = Path(__file__).resolve().parent
_LIB: ctypes.CDLL | None = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p


def lib() -> ctypes.CDLL:
    """Load (building with ``make`` if needed) ``oracle/liboracle.so``."""
    global _LIB
    if _LIB is not None:
        return _LIB
    # NAVI_ORACLE_LIB names another build (the sanitizer build of `make -C oracle asan`)
    path = Path(os.environ.get("NAVI_ORACLE_LIB", _HERE / "liboracle.so"))
    if not path.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE), "liboracle.so"], check=True)
    so = ctypes.CDLL(str(path))
    so.oracle_trace.argtypes = [
        _u64p, ctypes.c_uint64, _f32p, _f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
        _f32p, _f32p, ctypes.c_float, _f32p, _i32p, _vp, _vp, _vp, ctypes.c_int32,
    ]
    so.oracle_trace_multi.argtypes = [
        _u64p, _u64p, _u64p, _f32p, _i32p, ctypes.c_int64, ctypes.c_int64, _f32p, _f32p,
        ctypes.c_int32, ctypes.c_float, ctypes.c_float, _f32p, _i32p, _vp, _vp, _vp, ctypes.c_int32,
    ]
    so.oracle_trace_nocache.argtypes = [
        _u64p, ctypes.c_uint64, _f32p, _f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
        _f32p, _f32p, ctypes.c_float, _f32p, _i32p, _vp, _vp,
    ]
    so.oracle_point_query.argtypes = [
        _u64p, ctypes.c_uint64, _f32p, ctypes.c_int64, _f32p, _f32p, _f32p, _i32p, _i32p, _vp,
    ]
    so.oracle_half_encode.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int32, _u16p]
    so.oracle_half_decode.argtypes = [_u16p, ctypes.c_int64, _f32p]
    so.oracle_compile_dense.argtypes = [
        _f32p, ctypes.c_int32, ctypes.c_float, ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p),
    ]
    so.oracle_compile_dense.restype = ctypes.c_uint64
    so.oracle_free.argtypes = [ctypes.c_void_p]
    _LIB = so
    return so


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def _bounds(b) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(b, dtype=np.float32).reshape(3))


def _as_words(dag) -> np.ndarray:
    arr = np.asarray(dag)
    if arr.dtype == np.int64:
        arr = arr.view(np.uint64)
    return np.ascontiguousarray(arr, dtype=np.uint64).reshape(-1)


def trace(dag, origins, dirs, max_steps: int, max_distance: float, bbox_min, bbox_max,
          hit_epsilon: float = HIT_EPSILON, threads: int = 1) -> dict[str, np.ndarray]:
    """Trace rays ``[..., 3]``; returns dict of ``distance, semantic, steps, words, fault``
    shaped like ``origins[..., 0]``."""
    words = _as_words(dag)
    o = np.ascontiguousarray(origins, dtype=np.float32)
    d = np.ascontiguousarray(dirs, dtype=np.float32)
    shape = o.shape[:-1]
    n = int(np.prod(shape)) if shape else 1
    out_d = np.empty(n, np.float32)
    out_s = np.empty(n, np.int32)
    steps = np.empty(n, np.int32)
    wcount = np.empty(n, np.uint64)
    fault = np.empty(n, np.uint8)
    lib().oracle_trace(
        words, words.size, o.reshape(-1), d.reshape(-1), n, int(max_steps), float(max_distance),
        _bounds(bbox_min), _bounds(bbox_max), float(hit_epsilon), out_d, out_s, _ptr(steps),
        _ptr(wcount), _ptr(fault), int(threads),
    )
    return {
        "distance": out_d.reshape(shape),
        "semantic": out_s.reshape(shape),
        "steps": steps.reshape(shape),
        "words": wcount.reshape(shape),
        "fault": fault.reshape(shape),
    }


def trace_multi(pool, scene_base, scene_words, scene_bounds, env_scene, origins, dirs,
                max_steps: int, max_distance: float, hit_epsilon: float = HIT_EPSILON,
                threads: int = 1) -> dict[str, np.ndarray]:
    """Multi-scene trace: origins/dirs ``[E, R, 3]``, env ``e`` traces scene ``env_scene[e]``."""
    words = _as_words(pool)
    o = np.ascontiguousarray(origins, dtype=np.float32)
    d = np.ascontiguousarray(dirs, dtype=np.float32)
    n_env, rays = int(o.shape[0]), int(o.shape[1])
    n = n_env * rays
    out_d = np.empty(n, np.float32)
    out_s = np.empty(n, np.int32)
    steps = np.empty(n, np.int32)
    wcount = np.empty(n, np.uint64)
    fault = np.empty(n, np.uint8)
    lib().oracle_trace_multi(
        words, np.ascontiguousarray(scene_base, dtype=np.uint64),
        np.ascontiguousarray(scene_words, dtype=np.uint64),
        np.ascontiguousarray(scene_bounds, dtype=np.float32).reshape(-1),
        np.ascontiguousarray(env_scene, dtype=np.int32), n_env, rays, o.reshape(-1), d.reshape(-1),
        int(max_steps), float(max_distance), float(hit_epsilon), out_d, out_s, _ptr(steps),
        _ptr(wcount), _ptr(fault), int(threads),
    )
    shape = (n_env, rays)
    return {
        "distance": out_d.reshape(shape),
        "semantic": out_s.reshape(shape),
        "steps": steps.reshape(shape),
        "words": wcount.reshape(shape),
        "fault": fault.reshape(shape),
    }


def trace_nocache(dag, origins, dirs, max_steps: int, max_distance: float, bbox_min, bbox_max,
                  hit_epsilon: float = HIT_EPSILON) -> dict[str, np.ndarray]:
    words = _as_words(dag)
    o = np.ascontiguousarray(origins, dtype=np.float32)
    d = np.ascontiguousarray(dirs, dtype=np.float32)
    shape = o.shape[:-1]
    n = int(np.prod(shape)) if shape else 1
    out_d = np.empty(n, np.float32)
    out_s = np.empty(n, np.int32)
    steps = np.empty(n, np.int32)
    touch = np.empty(n, np.uint8)
    lib().oracle_trace_nocache(
        words, words.size, o.reshape(-1), d.reshape(-1), n, int(max_steps), float(max_distance),
        _bounds(bbox_min), _bounds(bbox_max), float(hit_epsilon), out_d, out_s, _ptr(steps),
        _ptr(touch),
    )
    return {
        "distance": out_d.reshape(shape),
        "semantic": out_s.reshape(shape),
        "steps": steps.reshape(shape),
        "touch": touch.reshape(shape),
    }


def point_query(dag, points, bbox_min, bbox_max) -> dict[str, np.ndarray]:
    words = _as_words(dag)
    p = np.ascontiguousarray(points, dtype=np.float32)
    shape = p.shape[:-1]
    n = int(np.prod(shape)) if shape else 1
    out_d = np.empty(n, np.float32)
    out_s = np.empty(n, np.int32)
    kind = np.empty(n, np.int32)
    wcount = np.empty(n, np.uint64)
    lib().oracle_point_query(
        words, words.size, p.reshape(-1), n, _bounds(bbox_min), _bounds(bbox_max), out_d, out_s,
        kind, _ptr(wcount),
    )
    return {
        "distance": out_d.reshape(shape),
        "semantic": out_s.reshape(shape),
        "kind": kind.reshape(shape),
        "words": wcount.reshape(shape),
    }


def half_to_float(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    out = np.empty(b.size, np.float32)
    lib().oracle_half_decode(b, b.size, out)
    return out


def float_to_half(values, quirk: bool = False) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    lib().oracle_half_encode(v, v.size, 1 if quirk else 0, out)
    return out


def compile_dense(grid: np.ndarray, voxel_size: float, quirk_half: bool = False) -> np.ndarray:
    """Naive ``build_recursive`` over a dense ``[z, y, x]`` float32 grid → u64 words."""
    g = np.ascontiguousarray(grid, dtype=np.float32)
    n = int(g.shape[0])
    assert g.shape == (n, n, n)
    out = ctypes.c_void_p()
    count = lib().oracle_compile_dense(g.reshape(-1), n, float(voxel_size), 1 if quirk_half else 0,
                                       ctypes.byref(out))
    if count == 0:
        raise MemoryError("oracle_compile_dense failed")
    buf = (ctypes.c_uint64 * count).from_address(out.value)
    words = np.frombuffer(buf, dtype=np.uint64).copy()
    lib().oracle_free(out)
    return words


# ---------------------------------------------------------------------------
# Caller-side restatements (numpy / torch CPU).
# ---------------------------------------------------------------------------

def ray_directions(azimuth_bins: int, elevation_bins: int) -> np.ndarray:
    """``build_spherical_ray_directions`` (sdfdag_backend.py:205-221): ``[Az*El, 3]`` f32,
    flat index ``az * El + el``; az in [0, 2π) without endpoint, el from +π/2 to −π/2."""
    az = np.linspace(0.0, 2.0 * math.pi, azimuth_bins, endpoint=False, dtype=np.float32)
    el = np.linspace(math.pi / 2.0, -math.pi / 2.0, elevation_bins, endpoint=True, dtype=np.float32)
    az_grid, el_grid = np.meshgrid(az, el, indexing="ij")
    az_flat = az_grid.reshape(-1)
    el_flat = el_grid.reshape(-1)
    cos_el = np.cos(el_flat)
    return np.stack(
        [cos_el * np.sin(az_flat), np.sin(el_flat), -cos_el * np.cos(az_flat)], axis=-1
    ).astype(np.float32)


def yaw_rotate(dirs_local: np.ndarray, yaw: np.ndarray) -> np.ndarray:
    """World directions ``[B, R, 3]`` = R_y(yaw) · local (sdfdag_backend.py:1300-1310):
    x' = x cosψ + z sinψ, y' = y, z' = −x sinψ + z cosψ (float32 arithmetic)."""
    yaw = np.asarray(yaw, dtype=np.float32).reshape(-1, 1)
    c = np.cos(yaw).astype(np.float32)
    s = np.sin(yaw).astype(np.float32)
    x = dirs_local[None, :, 0]
    y = dirs_local[None, :, 1]
    z = dirs_local[None, :, 2]
    out = np.empty((yaw.shape[0], dirs_local.shape[0], 3), dtype=np.float32)
    out[..., 0] = x * c + z * s
    out[..., 1] = np.broadcast_to(y, out[..., 1].shape)
    out[..., 2] = -x * s + z * c
    return out


def postprocess(out_distances, out_semantics, az_bins: int, el_bins: int, max_distance: float):
    """``_postprocess_cast_outputs_tensor`` (sdfdag_backend.py:408-452) core, torch CPU:
    returns ``(depth, semantic, valid, min_distance, clamped)`` shaped ``(B, Az, El)``."""
    import torch

    d = torch.as_tensor(np.asarray(out_distances, dtype=np.float32))
    s = torch.as_tensor(np.asarray(out_semantics, dtype=np.int32))
    b = int(d.shape[0])
    metric = d.reshape(b, az_bins, el_bins)
    sem = s.reshape(b, az_bins, el_bins).to(torch.int32)
    valid = torch.isfinite(metric)
    clamped = metric.clamp(min=0.0, max=max_distance)
    depth = (torch.log1p(clamped) / math.log1p(max_distance)).clamp(min=0.0, max=1.0)
    min_d = clamped.amin(dim=(1, 2))
    return depth, sem, valid, min_d, clamped


def fp16_depth_obs(out_distances, az_bins: int, el_bins: int, max_distance: float) -> np.ndarray:
    """North-star observation layout: depth of ``postprocess`` transposed to
    ``(B, 1, El, Az)`` and rounded to float16."""
    depth = postprocess(out_distances, np.zeros(np.shape(out_distances), np.int32), az_bins,
                        el_bins, max_distance)[0]
    return depth.permute(0, 2, 1).unsqueeze(1).contiguous().numpy().astype(np.float16)


def observation_ratios(clamped, valid, max_distance: float, band_min: float, band_max: float,
                       proximity: float) -> np.ndarray:
    """``_compute_observation_ratios_tensor`` (sdfdag_backend.py:366-405) on ``(B, Az, El)``
    clamped distances and validity: ``[B, 4]`` float32 = starvation, proximity,
    structure-band and forward-structure ratios. Python-float thresholds are rounded to
    float32 before comparing, as torch does with scalars; means are float32 count / size."""
    c = np.asarray(clamped, dtype=np.float32)
    v = np.asarray(valid, dtype=bool)
    b, az, el = c.shape
    with np.errstate(invalid="ignore"):
        sat = c >= np.float32(max_distance - 1e-3)
        out = np.zeros((b, 4), np.float32)
        out[:, 0] = sat.reshape(b, -1).sum(1).astype(np.float32) / np.float32(az * el)
        if band_max > band_min:
            band = v & (c >= np.float32(band_min)) & (c <= np.float32(band_max))
            out[:, 2] = band.reshape(b, -1).sum(1).astype(np.float32) / np.float32(az * el)
            half = max(1, az // 6)
            sector = np.concatenate((band[:, :half, :], band[:, az - half:, :]), axis=1)
            out[:, 3] = sector.reshape(b, -1).sum(1).astype(np.float32) / np.float32(2 * half * el)
        if proximity > 0.0:
            near = v & (c <= np.float32(proximity))
            out[:, 1] = near.reshape(b, -1).sum(1).astype(np.float32) / np.float32(az * el)
    return np.clip(out, 0.0, 1.0)


def observe(out_distances, az_bins: int, el_bins: int, max_distance: float, band_min: float = 1.5,
            band_max: float = 30.0, proximity: float = 2.0, clearance: float = 0.15, semantics=None,
            prev_depth=None) -> dict[str, np.ndarray]:
    """The observation step after a trace: ``depth16 (B, 1, El, Az)`` float16 (north-star
    layout of ``postprocess``'s depth), ``stats [B, 5]`` = min clamped distance and the four
    ``observation_ratios``, ``collision [B]`` = min < clearance (sdfdag_backend.py:1340); with
    ``semantics``, ``obs (B, 3, Az, El)`` = stack(depth, semantic, valid) float32, and with
    ``prev_depth (B, Az, El)``, ``delta`` = depth - prev_depth, zero for envs whose
    prev_depth sums below 1e-6 in absolute value (``_consume_observation_batch``,
    sdfdag_backend.py:1501-1526)."""
    import torch

    d = np.asarray(out_distances, dtype=np.float32)
    sem = np.zeros(d.shape, np.int32) if semantics is None else np.asarray(semantics, np.int32)
    depth, sem_t, valid, min_d, clamped = postprocess(d, sem, az_bins, el_bins, max_distance)
    ratios = observation_ratios(clamped.numpy(), valid.numpy(), max_distance, band_min, band_max, proximity)
    stats = np.concatenate([min_d.numpy()[:, None].astype(np.float32), ratios], axis=1)
    with np.errstate(invalid="ignore"):
        collision = (stats[:, 0] < np.float32(clearance)).astype(np.int32)
    out = {
        "depth16": depth.permute(0, 2, 1).unsqueeze(1).contiguous().numpy().astype(np.float16),
        "depth": depth.numpy(),
        "stats": stats,
        "collision": collision,
    }
    if semantics is not None:
        out["obs"] = torch.stack((depth, sem_t.to(torch.float32), valid.to(torch.float32)), dim=1).numpy()
    if prev_depth is not None:
        prev = torch.as_tensor(np.asarray(prev_depth, np.float32))
        first = prev.abs().sum(dim=(1, 2)) < 1e-6
        delta = depth - prev
        out["delta"] = torch.where(first.view(-1, 1, 1), torch.zeros_like(delta), delta).numpy()
    return out


if os.environ.get("NAVI_ORACLE_EAGER"):
    lib()
