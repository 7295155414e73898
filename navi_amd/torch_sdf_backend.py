"""MI355X replacement of the native module ``torch_sdf_backend``.

Mirrors the pybind11 surface of ``projects/torch-sdf/cpp_src/bindings.cpp:112-120``
(same name, same 11 arguments, same ``skip_direction_validation`` default) and
the argument contract of ``cast_rays_forward`` (``bindings.cpp:43-110``): the
same checks in the same order with the same messages, raised as
``RuntimeError`` (what a failed ``TORCH_CHECK`` becomes in Python). The launch
goes through the C ABI ``navi_cast_rays`` (``include/navi_trace.h``) on
PyTorch's *current* HIP stream — the reference launches on the legacy default
stream (``kernel.cu:320``) although its trainer calls it under side streams.

Additions, all keyword-only so the positional contract is unchanged:
``hit_epsilon`` (the reference's compile-time ``kHitEpsilon``, ``kernel.cuh:7``),
``out_steps`` (an int32 ``[B, R]`` tensor receiving per-ray step counts),
``elevation_bins`` (declares the canonical ``az * El + el`` ray order so rays are
traced in angular tiles) and ``kernel``. ``out_distances`` may also be bfloat16 or
float16, the reference roadmap's T2 item (``docs/FUTURE_HARDWARE_ROADMAP.md:140-222``):
the march accumulates in float32 and each finished ray's distance is rounded to nearest
even (record-layout tracer only; a call that would take the word-layout kernel raises).

Kernels. ``kernel="auto"`` (default) traces with the record-layout tracer
(``navi_trace_relaid``) over a record-layout copy of the DAG tensor: its words
copied to the host once, converted (``navi_relayout``, ``navi_build_cell_table``)
and uploaded, keyed by the tensor object, its version counter (in-place tensor
ops invalidate it), its address and the bbox. ``prepare(dag_tensor, bbox_min,
bbox_max)`` does that at scene load (the reference's ``_load_scene``,
``sdfdag_backend.py:1893-1900``); otherwise the first ``cast_rays`` with the
tensor does it, with a device-to-host copy that waits for the device, and warns
(``LayoutConversionWarning``, once per call site under Python's default warning
filter; ``conversion_counts()`` counts every conversion). Writes
that bypass the version counter (through ``.data``, or from outside PyTorch)
need ``invalidate(dag_tensor)``. Leaves of semantic 0x7fff or above (the
format's field is 16 bits) go to a leaf table beside the records. DAGs the
record layout cannot hold (more than 65536 distinct such leaves, or 2^27
records) and batches above 2^30 rays use the word-layout kernel
(``navi_cast_rays``), as does ``kernel="raw"``. Results are identical either
way. Once prepared, a call with ``skip_direction_validation=True`` allocates
nothing and never waits for the device, as the reference's
(``bindings.cpp:91-109``).
"""

from __future__ import annotations

import ctypes

import math
from typing import Any

import numpy as np
import torch

import threading
import warnings
import weakref

from . import _native

_DIRECTION_NORM_EPS = 1e-4  # kernel.cuh:9
HIT_EPSILON = 0.01  # kernel.cuh:7
_INT32_MAX = 0x7FFFFFFF
RELAID_MAX_RAYS = 1 << 30  # rays per navi_trace_relaid launch; larger batches take navi_cast_rays
_DISTANCE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

__all__ = ["cast_rays", "prepare", "invalidate", "conversion_counts", "LayoutConversionWarning", "HIT_EPSILON"]


class LayoutConversionWarning(RuntimeWarning):
    """``cast_rays`` converted a DAG tensor to the record layout inside the call: a
    device-to-host copy that waits for the device, a host relayout and an upload.
    ``prepare()`` at scene load moves that work out of the step."""


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _f32(value) -> float:
    # pybind11 converts to C++ float before any check (bindings.cpp:50,51,84).
    with np.errstate(over="ignore"):
        return float(np.float32(float(value)))


def _validate_bounds(bbox_min, bbox_max) -> None:  # bindings.cpp:10-21
    _check(len(bbox_min) == 3, "bbox_min must contain exactly 3 floats")
    _check(len(bbox_max) == 3, "bbox_max must contain exactly 3 floats")
    for idx in range(3):
        lo = _f32(bbox_min[idx])
        hi = _f32(bbox_max[idx])
        _check(math.isfinite(lo), "bbox_min must contain only finite floats")
        _check(math.isfinite(hi), "bbox_max must contain only finite floats")
        _check(lo < hi, "bbox_min entries must be strictly less than bbox_max entries")


def _validate_direction_norms(dirs: torch.Tensor) -> None:  # bindings.cpp:23-34
    norms = torch.sqrt(torch.sum(dirs * dirs, -1))
    _check(bool(torch.isfinite(norms).all().item()), "dirs must contain only finite direction vectors")
    max_error = float(torch.abs(norms - 1.0).amax().item())
    _check(
        max_error <= _DIRECTION_NORM_EPS,
        f"dirs must be normalized within tolerance {_DIRECTION_NORM_EPS:g}; max error was {max_error:g}",
    )


def validate_cast_inputs(dag_tensor, origins, dirs, out_distances, out_semantics, max_steps,
                         max_distance, bbox_min, bbox_max, resolution) -> None:
    """The TORCH_CHECK block of ``cast_rays_forward`` (bindings.cpp:57-86)."""
    _check(dag_tensor.is_cuda, "dag_tensor must be a CUDA tensor")
    _check(origins.is_cuda, "origins must be a CUDA tensor")
    _check(dirs.is_cuda, "dirs must be a CUDA tensor")
    _check(out_distances.is_cuda, "out_distances must be a CUDA tensor")
    _check(out_semantics.is_cuda, "out_semantics must be a CUDA tensor")

    _check(origins.is_contiguous(), "origins must be contiguous")
    _check(dirs.is_contiguous(), "dirs must be contiguous")
    _check(out_distances.is_contiguous(), "out_distances must be contiguous")
    _check(out_semantics.is_contiguous(), "out_semantics must be contiguous")
    # The reference C++ layer does not check this one (its Python layer does,
    # backend.py:64-65); the kernel reads the words as one flat array.
    _check(dag_tensor.is_contiguous(), "dag_tensor must be contiguous")

    _check(dag_tensor.dtype == torch.int64, "dag_tensor must be int64")
    _check(origins.dtype == torch.float32, "origins must be float32")
    _check(dirs.dtype == torch.float32, "dirs must be float32")
    # float32 as bindings.cpp:71; bfloat16 and float16 are the reference roadmap's
    # extension of this check (docs/FUTURE_HARDWARE_ROADMAP.md:157-176)
    _check(out_distances.dtype in _DISTANCE_DTYPES, "out_distances must be float32 or bfloat16 (or float16)")
    _check(out_semantics.dtype == torch.int32, "out_semantics must be int32")

    _check(origins.dim() == 3 and origins.size(2) == 3, "origins must be [Batch, Rays, 3]")
    _check(dirs.dim() == 3 and dirs.size(2) == 3, "dirs must be [Batch, Rays, 3]")
    _check(tuple(dirs.shape) == tuple(origins.shape), "dirs must match origins shape")
    _check(out_distances.dim() == 2, "out_distances must be [Batch, Rays]")
    _check(out_semantics.dim() == 2, "out_semantics must be [Batch, Rays]")
    _check(
        out_distances.size(0) == origins.size(0) and out_distances.size(1) == origins.size(1),
        "out_distances must match the [Batch, Rays] shape of origins",
    )
    _check(
        out_semantics.size(0) == origins.size(0) and out_semantics.size(1) == origins.size(1),
        "out_semantics must match the [Batch, Rays] shape of origins",
    )
    # int max_steps and int resolution in the native call (bindings.cpp:49,53)
    _check(0 < int(max_steps) <= _INT32_MAX, "max_steps must be a positive integer")
    _check(
        math.isfinite(_f32(max_distance)) and _f32(max_distance) > 0.0,
        "max_distance must be a finite positive float",
    )
    _check(0 < int(resolution) <= _INT32_MAX, "resolution must be a positive integer")
    _validate_bounds(bbox_min, bbox_max)
    # One device for every operand: the kernel dereferences all of them.
    dev = dag_tensor.device
    for name, t in (("origins", origins), ("dirs", dirs), ("out_distances", out_distances),
                    ("out_semantics", out_semantics)):
        _check(t.device == dev, f"{name} must be on the same device as dag_tensor ({dev})")


class _RecordLayout:
    """The record-layout copy of one DAG tensor (see the module docstring)."""

    def __init__(self, dag_tensor: torch.Tensor, bounds: tuple[tuple[float, ...], tuple[float, ...]]) -> None:
        from .multiscene import ResidentScenes

        self.ref = weakref.ref(dag_tensor)
        self.version = dag_tensor._version
        self.data_ptr = dag_tensor.data_ptr()
        self.bounds = bounds
        words = dag_tensor.detach().cpu().numpy().view(np.uint64)
        scenes = ResidentScenes([(words, bounds[0], bounds[1])], dag_tensor.device, keep_words=False)
        self.scenes = scenes if scenes.relaid_ok else None

    def valid_for(self, dag_tensor: torch.Tensor, bounds) -> bool:
        return (self.ref() is dag_tensor and self.version == dag_tensor._version
                and self.data_ptr == dag_tensor.data_ptr() and self.bounds == bounds)


_layout_lock = threading.Lock()
_layouts: dict[int, _RecordLayout] = {}
_conversions = {"prepare": 0, "cast_rays": 0}


def _record_layout(dag_tensor: torch.Tensor, bbox_min, bbox_max, caller: str):
    bounds = (tuple(_f32(v) for v in bbox_min), tuple(_f32(v) for v in bbox_max))
    with _layout_lock:
        entry = _layouts.get(id(dag_tensor))
        if entry is None or not entry.valid_for(dag_tensor, bounds):
            for key in [k for k, e in _layouts.items() if e.ref() is None]:
                del _layouts[key]
            entry = _RecordLayout(dag_tensor, bounds)
            _layouts[id(dag_tensor)] = entry
            _conversions[caller] += 1
            if caller == "cast_rays":
                warnings.warn(
                    f"cast_rays converted a {dag_tensor.numel()}-word DAG tensor to the record layout inside the "
                    "call (a device-to-host copy that waits for the device); call torch_sdf.prepare(dag_tensor, "
                    "bbox_min, bbox_max) when the scene is loaded", LayoutConversionWarning, stacklevel=4)
        return entry.scenes


def conversion_counts() -> dict[str, int]:
    """How many record-layout conversions ``prepare`` and ``cast_rays`` have done in this
    process (a conversion inside ``cast_rays`` waits for the device)."""
    with _layout_lock:
        return dict(_conversions)


def prepare(dag_tensor: torch.Tensor, bbox_min, bbox_max) -> bool:
    """Convert ``dag_tensor`` (int64 words on a CUDA device) to the record layout now,
    so that ``cast_rays`` calls with it neither copy, allocate nor wait. Synchronous.
    Returns whether the record layout holds the DAG (else ``kernel="auto"`` traces it
    with the word-layout kernel, which needs no preparation)."""
    _check(dag_tensor.is_cuda, "dag_tensor must be a CUDA tensor")
    _check(dag_tensor.dtype == torch.int64, "dag_tensor must be int64")
    _check(dag_tensor.is_contiguous(), "dag_tensor must be contiguous")
    _validate_bounds(bbox_min, bbox_max)
    _native.device_init(dag_tensor.device)
    return _record_layout(dag_tensor, bbox_min, bbox_max, "prepare") is not None


def invalidate(dag_tensor: torch.Tensor | None = None) -> None:
    """Drop the record-layout copy of ``dag_tensor`` (of every tensor when None). In-place
    tensor ops bump the version counter and need no call; writes through ``.data`` or a
    raw pointer do."""
    with _layout_lock:
        if dag_tensor is None:
            _layouts.clear()
        else:
            _layouts.pop(id(dag_tensor), None)


def cast_rays(
    dag_tensor: torch.Tensor,
    origins: torch.Tensor,
    dirs: torch.Tensor,
    out_distances: torch.Tensor,
    out_semantics: torch.Tensor,
    max_steps: int,
    max_distance: float,
    bbox_min: list[float],
    bbox_max: list[float],
    resolution: int,
    skip_direction_validation: bool = False,
    *,
    hit_epsilon: float = HIT_EPSILON,
    out_steps: Any | None = None,
    elevation_bins: int = 0,
    kernel: str = "auto",
) -> None:
    """Batched bounded stackless sphere tracing (bindings.cpp:112-120 surface)."""
    validate_cast_inputs(dag_tensor, origins, dirs, out_distances, out_semantics, max_steps,
                         max_distance, bbox_min, bbox_max, resolution)
    if out_steps is not None:
        _check(out_steps.is_cuda and out_steps.dtype == torch.int32 and out_steps.is_contiguous()
               and tuple(out_steps.shape) == tuple(out_distances.shape)
               and out_steps.device == dag_tensor.device,
               "out_steps must be a contiguous int32 CUDA tensor shaped like out_distances")
    if not skip_direction_validation:
        _validate_direction_norms(dirs)

    _check(kernel in ("auto", "raw"), f"kernel must be 'auto' or 'raw'; got {kernel!r}")
    n_envs, rays = int(origins.size(0)), int(origins.size(1))
    n_rays = n_envs * rays
    dev = dag_tensor.device
    scenes = (_record_layout(dag_tensor, bbox_min, bbox_max, "cast_rays")
              if kernel == "auto" and n_rays <= RELAID_MAX_RAYS else None)
    dist_dtype = scenes._distance_dtype(out_distances) if scenes is not None else _native.DIST_F32
    if out_distances.dtype != torch.float32 and scenes is None:
        raise RuntimeError("bfloat16 and float16 distances need the record-layout tracer (kernel='auto', a DAG "
                           "the record layout holds, at most 2^30 rays); this call would take the word-layout "
                           "kernel, which writes float32")
    if scenes is not None:
        # one scene, no scene table or env order (navi_trace_relaid_ex, leaf table included)
        L = scenes._launch_args(None, None, n_envs, rays, elevation_bins, out_distances.data_ptr(),
                                out_semantics.data_ptr(), out_steps, max_steps, max_distance, hit_epsilon,
                                dist_dtype)
        L.origins, L.dirs = origins.data_ptr(), dirs.data_ptr()
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            code = _native.lib().navi_trace_relaid_ex(ctypes.byref(L), stream)
        _native.check(code)
        return
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        code = _native.lib().navi_cast_rays(
            dag_tensor.data_ptr(), int(dag_tensor.numel()), origins.data_ptr(), dirs.data_ptr(),
            out_distances.data_ptr(), out_semantics.data_ptr(), n_rays, int(max_steps),
            float(max_distance), _native.float3(bbox_min), _native.float3(bbox_max),
            int(resolution), float(hit_epsilon),
            out_steps.data_ptr() if out_steps is not None else None, None, stream,
        )
    _native.check(code)
