"""MI355X drop-in for ``torch_sdf.backend`` (``projects/torch-sdf/torch_sdf/backend.py``).

Same module-level names (``HAS_CUDA_BACKEND``, ``torch_sdf_backend``,
``_validate_*``), the same validation order and messages (pinned by
``projects/torch-sdf/tests/test_sphere_tracing.py:294-680``), and the same
11-positional-argument native call (``backend.py:185-197``). The native module
is :mod:`navi_amd.torch_sdf_backend`, which launches the HIP tracer through the
C ABI. As in the reference there is no CPU fallback (``backend.py:158-169``).
"""

from __future__ import annotations

import math
from typing import Any

import torch

torch_sdf_backend: Any | None = None
try:
    from .. import torch_sdf_backend as _torch_sdf_backend

    torch_sdf_backend = _torch_sdf_backend
    HAS_CUDA_BACKEND = True
except ImportError:
    HAS_CUDA_BACKEND = False

_DAG_DTYPE = torch.int64
_DISTANCE_DTYPE = torch.float32
_DISTANCE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)  # out_distances
_SEMANTIC_DTYPE = torch.int32
_HIT_EPSILON = 0.01  # kernel.cuh:7
_DIRECTION_NORM_EPS = 1e-4  # kernel.cuh:9


def _shape_tuple(tensor: Any) -> tuple[int, ...]:
    return tuple(int(dim) for dim in tensor.shape)


def _validate_cuda_tensor(tensor: Any, *, name: str, dtype: torch.dtype,
                          shape: tuple[int, ...] | None = None) -> None:
    # backend.py:28-46
    if not tensor.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor. CPU tensors are not supported.")
    if tensor.dtype != dtype:
        raise RuntimeError(f"{name} must have dtype {dtype}; got {tensor.dtype}.")
    if not tensor.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous.")
    if shape is not None and _shape_tuple(tensor) != shape:
        raise RuntimeError(f"{name} must have shape {shape}; got {_shape_tuple(tensor)}.")


def _validate_direction_norms(dirs: torch.Tensor, *, eps: float = _DIRECTION_NORM_EPS) -> None:
    # backend.py:101-111
    norms = torch.linalg.vector_norm(dirs, dim=-1)
    if bool((~torch.isfinite(norms)).any().item()):
        raise RuntimeError("dirs must contain only finite direction vectors.")
    max_error = float(torch.abs(norms - 1.0).amax().detach().cpu().item())
    if max_error > eps:
        raise RuntimeError(
            f"dirs must be normalized within tolerance {eps}; max error was {max_error:.6g}."
        )


def _validate_cast_rays_inputs(dag_tensor: Any, origins: Any, dirs: Any, out_distances: Any,
                               out_semantics: Any, *, skip_direction_validation: bool = False) -> None:
    # backend.py:49-98
    if not dag_tensor.is_cuda:
        raise RuntimeError("dag_tensor must be on CUDA. CPU tensors are not supported.")
    if dag_tensor.dtype != _DAG_DTYPE:
        raise RuntimeError(f"dag_tensor must have dtype {_DAG_DTYPE}; got {dag_tensor.dtype}.")
    if not dag_tensor.is_contiguous():
        raise RuntimeError("dag_tensor must be contiguous.")
    if origins.dim() != 3 or origins.size(2) != 3:
        raise RuntimeError(f"origins must have shape [batch, rays, 3]; got {_shape_tuple(origins)}.")
    if dirs.dim() != 3 or dirs.size(2) != 3:
        raise RuntimeError(f"dirs must have shape [batch, rays, 3]; got {_shape_tuple(dirs)}.")
    batch = int(origins.size(0))
    rays = int(origins.size(1))
    if _shape_tuple(dirs) != (batch, rays, 3):
        raise RuntimeError(
            f"dirs must match origins shape {(batch, rays, 3)}; got {_shape_tuple(dirs)}."
        )
    _validate_cuda_tensor(origins, name="origins", dtype=_DISTANCE_DTYPE)
    _validate_cuda_tensor(dirs, name="dirs", dtype=_DISTANCE_DTYPE)
    # float32, or the reference roadmap's bfloat16 / float16 distances
    # (docs/FUTURE_HARDWARE_ROADMAP.md:157-176): validated against the tensor's own dtype
    # when it is one of those, so any other dtype gets the float32 message
    _validate_cuda_tensor(out_distances, name="out_distances",
                          dtype=out_distances.dtype if getattr(out_distances, "dtype", None) in _DISTANCE_DTYPES
                          else _DISTANCE_DTYPE,
                          shape=(batch, rays))
    _validate_cuda_tensor(out_semantics, name="out_semantics", dtype=_SEMANTIC_DTYPE,
                          shape=(batch, rays))
    if not skip_direction_validation and torch.is_tensor(dirs):
        _validate_direction_norms(dirs)


def _validate_bounds(bbox_min: list[float], bbox_max: list[float]) -> None:
    # backend.py:114-123
    if len(bbox_min) != 3 or len(bbox_max) != 3:
        raise RuntimeError("bbox_min and bbox_max must each contain exactly 3 floats.")
    for index, (lower, upper) in enumerate(zip(bbox_min, bbox_max)):
        if not math.isfinite(lower) or not math.isfinite(upper):
            raise RuntimeError("bbox_min and bbox_max must contain only finite floats.")
        if lower >= upper:
            raise RuntimeError(
                f"bbox_min[{index}] must be strictly less than bbox_max[{index}]; got {lower} >= {upper}."
            )


def _validate_runtime_parameters(*, max_steps: int, max_distance: float, bbox_min: list[float],
                                 bbox_max: list[float], resolution: int) -> None:
    # backend.py:126-142
    if max_steps <= 0:
        raise RuntimeError(f"max_steps must be a positive integer; got {max_steps}.")
    if not math.isfinite(max_distance) or max_distance <= 0.0:
        raise RuntimeError(f"max_distance must be a finite positive float; got {max_distance}.")
    if resolution <= 0:
        raise RuntimeError(f"resolution must be a positive integer; got {resolution}.")
    _validate_bounds(bbox_min, bbox_max)


def cast_rays(
    dag_tensor: Any,
    origins: Any,
    dirs: Any,
    out_distances: Any,
    out_semantics: Any,
    max_steps: int,
    max_distance: float,
    bbox_min: list[float],
    bbox_max: list[float],
    resolution: int,
    skip_direction_validation: bool = False,
    *,
    hit_epsilon: float = _HIT_EPSILON,
    out_steps: Any | None = None,
    elevation_bins: int = 0,
    kernel: str = "auto",
) -> None:
    """Batched sphere tracing of a device-resident ``.gmdag`` DAG on the MI355X.

    Drop-in for ``torch_sdf.cast_rays`` (``backend.py:145-197``): writes every
    element of ``out_distances`` / ``out_semantics`` in place, asynchronously on
    PyTorch's current stream. Keyword-only extensions: ``hit_epsilon``,
    ``out_steps`` (int32 ``[B, R]`` per-ray step counts), ``elevation_bins``
    (the rays are in the canonical ``az * El + el`` order with this ``El``) and
    ``kernel`` (``"auto"``: record-layout tracer with a cached conversion of the
    DAG tensor; ``"raw"``: the word-layout kernel). GPU only.
    """
    if not HAS_CUDA_BACKEND:
        raise RuntimeError(
            "torch_sdf_backend is not available. Build the HIP tracer library "
            "(navi_amd/_lib/libnavi_trace.so) before running TopoNav."
        )
    if not torch.cuda.is_available():
        raise RuntimeError(
            "CUDA is not available. TopoNav requires a ROCm GPU and does not support CPU fallback."
        )
    _validate_cast_rays_inputs(dag_tensor, origins, dirs, out_distances, out_semantics,
                               skip_direction_validation=skip_direction_validation)
    _validate_runtime_parameters(max_steps=max_steps, max_distance=max_distance, bbox_min=bbox_min,
                                 bbox_max=bbox_max, resolution=resolution)
    backend = torch_sdf_backend
    if backend is None:
        raise RuntimeError("torch_sdf_backend import unexpectedly resolved to None.")
    extra: dict[str, Any] = {}
    if hit_epsilon != _HIT_EPSILON:
        extra["hit_epsilon"] = hit_epsilon
    if out_steps is not None:
        extra["out_steps"] = out_steps
    if elevation_bins:
        extra["elevation_bins"] = int(elevation_bins)
    if kernel != "auto":
        extra["kernel"] = kernel
    backend.cast_rays(
        dag_tensor,
        origins,
        dirs,
        out_distances,
        out_semantics,
        max_steps,
        max_distance,
        bbox_min,
        bbox_max,
        resolution,
        skip_direction_validation,
        **extra,
    )


def prepare(dag_tensor: torch.Tensor, bbox_min: list[float], bbox_max: list[float]) -> bool:
    """Scene-load step (an extension; the reference converts nothing): builds the
    record-layout copy of ``dag_tensor`` that ``cast_rays(kernel="auto")`` traces, so
    the calls that follow neither copy, allocate nor wait. See
    :func:`navi_amd.torch_sdf_backend.prepare`."""
    if not HAS_CUDA_BACKEND or torch_sdf_backend is None:
        raise RuntimeError("torch_sdf_backend is not available. Build the HIP tracer library "
                           "(navi_amd/_lib/libnavi_trace.so) first.")
    return torch_sdf_backend.prepare(dag_tensor, bbox_min, bbox_max)


def invalidate(dag_tensor: torch.Tensor | None = None) -> None:
    """Drop the record-layout copy of ``dag_tensor`` (all copies when None); needed
    after writes that bypass its version counter (``.data``, raw pointers)."""
    if HAS_CUDA_BACKEND and torch_sdf_backend is not None:
        torch_sdf_backend.invalidate(dag_tensor)
