"""ctypes binding of ``libnavi_trace.so`` (the C ABI declared in ``include/navi_trace.h``).

Importing this module loads the HIP library and raises ``ImportError`` when it
has not been built — there is no fallback: the tracer runs on the GPU or not at
all (the reference's own stance, ``projects/torch-sdf/torch_sdf/backend.py:158-169``).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIB_PATH = Path(os.environ.get("NAVI_TRACE_LIB", LIB_DIR / "libnavi_trace.so"))

NAVI_OK = 0
NAVI_E_ARG = -1
NAVI_E_LAUNCH = -2
NAVI_E_LAYOUT = -3
NAVI_E_NOMEM = -4

if not LIB_PATH.exists():
    raise ImportError(
        f"libnavi_trace.so not found at {LIB_PATH}; build it with "
        "`python -c 'import __graft_entry__ as g; g.build()'` (or `make -C navi_amd/csrc`)."
    )

_lib = ctypes.CDLL(str(LIB_PATH))

_vp = ctypes.c_void_p
_f3 = ctypes.POINTER(ctypes.c_float)

_lib.navi_last_error.restype = ctypes.c_char_p
_lib.navi_last_error.argtypes = []
_lib.navi_version.restype = ctypes.c_char_p
_lib.navi_version.argtypes = []

_lib.navi_device_init.restype = ctypes.c_int
_lib.navi_device_init.argtypes = []
_lib.navi_set_wide_min_rays.restype = ctypes.c_uint64
_lib.navi_set_wide_min_rays.argtypes = [ctypes.c_uint64]

_lib.navi_cast_rays.restype = ctypes.c_int
_lib.navi_cast_rays.argtypes = [
    _vp, ctypes.c_uint64, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
    _f3, _f3, ctypes.c_int32, ctypes.c_float, _vp, _vp, _vp,
]
_lib.navi_cast_rays_multi.restype = ctypes.c_int
_lib.navi_cast_rays_multi.argtypes = [
    _vp, _vp, ctypes.c_int32, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp, _vp, _vp,
    ctypes.c_int32, ctypes.c_float, ctypes.c_float, _vp, _vp, _vp,
]

_u64p = ctypes.POINTER(ctypes.c_uint64)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_lib.navi_relayout.restype = ctypes.c_int
_lib.navi_relayout.argtypes = [_vp, ctypes.c_uint64, _vp, ctypes.c_uint64, _u64p, _u32p, _vp]
_lib.navi_trace_relaid.restype = ctypes.c_int
_lib.navi_build_cell_table.restype = ctypes.c_int
_lib.navi_build_cell_table.argtypes = [_vp, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int32, _vp]
_lib.navi_record_depth.restype = ctypes.c_int
_lib.navi_record_depth.argtypes = [_vp, ctypes.c_uint64, ctypes.c_uint32, _u32p]
_lib.navi_trace_relaid.argtypes = [
    _vp, ctypes.c_uint64, _vp, ctypes.c_int32, _vp, ctypes.c_int32, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
    ctypes.c_int32, _vp, _vp, _vp, _vp, ctypes.c_int32, ctypes.c_float, ctypes.c_float, _vp, _vp,
]

_lib.navi_trace_relaid_noalloc.restype = ctypes.c_int
_lib.navi_trace_relaid_noalloc.argtypes = _lib.navi_trace_relaid.argtypes

_lib.navi_trace_relaid_poses.restype = ctypes.c_int
_lib.navi_trace_relaid_poses.argtypes = [
    _vp, ctypes.c_uint64, _vp, ctypes.c_int32, _vp, ctypes.c_int32, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
    ctypes.c_int32, _vp, _vp, _vp, _vp, _vp, ctypes.c_int32, ctypes.c_float, ctypes.c_float, _vp, _vp,
]


class PointQueries(ctypes.Structure):
    """navi_point_queries (include/navi_trace.h)."""

    _fields_ = [("records", _vp), ("n_records", ctypes.c_uint64), ("scenes", _vp), ("n_scenes", ctypes.c_int32),
                ("cell_tables", _vp), ("table_depth", ctypes.c_int32), ("point_scene", _vp), ("points", _vp),
                ("n_points", ctypes.c_int64),
                ("out_distances", _vp), ("out_semantics", _vp), ("out_kind", _vp)]


class Observation(ctypes.Structure):
    """navi_observation (include/navi_trace.h)."""

    _fields_ = [("distances", _vp), ("semantics", _vp), ("n_envs", ctypes.c_int64),
                ("azimuth_bins", ctypes.c_int32), ("elevation_bins", ctypes.c_int32),
                ("max_distance", ctypes.c_float), ("structure_band_min", ctypes.c_float),
                ("structure_band_max", ctypes.c_float), ("proximity_threshold", ctypes.c_float),
                ("collision_clearance", ctypes.c_float), ("depth_f16", _vp), ("obs", _vp), ("prev_depth", _vp),
                ("delta", _vp), ("stats", _vp), ("collision", _vp)]


_lib.navi_point_query.restype = ctypes.c_int
_lib.navi_point_query.argtypes = [ctypes.POINTER(PointQueries), _vp]
_lib.navi_observe.restype = ctypes.c_int
_lib.navi_observe.argtypes = [ctypes.POINTER(Observation), ctypes.POINTER(PointQueries), _vp]

# Layout of navi_relaid_scene (include/navi_trace.h), 48 bytes.
RELAID_SCENE_DTYPE = [("rec_offset", "<u8"), ("n_records", "<u4"), ("root_slot", "<u4"),
                      ("bbox_min", "<f4", (3,)), ("bbox_max", "<f4", (3,)), ("max_depth", "<u4"),
                      ("flags", "<u4")]
SCENE_NONNEG_LEAVES = 1  # navi_relaid_scene.flags bit (include/navi_trace.h)


def nonneg_leaves(records, root_slot) -> bool:
    """Whether no leaf slot of ``records`` (uint32 [n, 8]) nor an inlined root leaf has
    its fp16 sign bit set (``NAVI_SCENE_NONNEG_LEAVES``)."""
    import numpy as np

    rec = np.asarray(records, dtype=np.uint32)
    leaf_neg = (rec >> np.uint32(31)).astype(bool) & ((rec >> np.uint32(15)) & np.uint32(1)).astype(bool)
    root = int(root_slot)
    return not bool(leaf_neg.any()) and not (root >> 31 and (root >> 15) & 1)


def relayout(words):
    """Host conversion to the device record layout: returns
    ``(records uint32 [n, 8], root_slot, levels_prefix[8])``; raises RuntimeError
    (NAVI_E_LAYOUT) for DAGs the layout cannot hold."""
    import numpy as np

    w = np.ascontiguousarray(np.asarray(words).view(np.uint64).reshape(-1))
    n = ctypes.c_uint64()
    root = ctypes.c_uint32()
    levels = np.zeros(8, np.uint64)
    check(_lib.navi_relayout(w.ctypes.data, w.size, None, 0, ctypes.byref(n), ctypes.byref(root),
                             levels.ctypes.data))
    rec = np.zeros((max(1, n.value), 8), np.uint32)
    check(_lib.navi_relayout(w.ctypes.data, w.size, rec.ctypes.data, n.value, ctypes.byref(n),
                             ctypes.byref(root), levels.ctypes.data))
    return rec[: n.value], int(root.value), levels


def cell_table(records, root_slot, depth):
    """Host cell table of one scene at ``depth`` in [4, 7] (``navi_build_cell_table``):
    uint64 [8**depth]."""
    import numpy as np

    rec = np.ascontiguousarray(records, dtype=np.uint32).reshape(-1, 8)
    out = np.zeros(8 ** int(depth) if 4 <= int(depth) <= 7 else 1, np.uint64)
    check(_lib.navi_build_cell_table(rec.ctypes.data if rec.size else None, rec.shape[0], int(root_slot),
                                     int(depth), out.ctypes.data))
    return out


def record_depth(records, root_slot):
    """Longest record chain below ``root_slot`` (``navi_record_depth``); 0xffffffff on a cycle."""
    import numpy as np

    rec = np.ascontiguousarray(records, dtype=np.uint32).reshape(-1, 8)
    out = ctypes.c_uint32()
    check(_lib.navi_record_depth(rec.ctypes.data if rec.size else None, rec.shape[0], int(root_slot),
                                 ctypes.byref(out)))
    return int(out.value)


# Layout of navi_scene_desc (include/navi_trace.h), 40 bytes.
SCENE_DESC_DTYPE = [("word_offset", "<u8"), ("n_words", "<u8"), ("bbox_min", "<f4", (3,)),
                    ("bbox_max", "<f4", (3,))]


def lib() -> ctypes.CDLL:
    return _lib


def set_wide_min_rays(n_rays: int) -> int:
    """Launches of the record-layout tracer with at least ``n_rays`` rays run in
    1024-thread workgroups when their split planes fit (results are identical);
    returns the previous threshold."""
    if not 0 <= int(n_rays) < (1 << 64):
        raise ValueError("n_rays must fit an unsigned 64-bit integer")
    return int(_lib.navi_set_wide_min_rays(int(n_rays)))


def version() -> str:
    return _lib.navi_version().decode()


def last_error() -> str:
    return _lib.navi_last_error().decode(errors="replace")


def check(code: int) -> None:
    """Raise ``RuntimeError`` (the exception type TORCH_CHECK surfaces) for a failed call."""
    if code != NAVI_OK:
        raise RuntimeError(last_error() or f"navi_trace call failed with code {code}")


_initialised: set[int] = set()


def device_init(device) -> None:
    """``navi_device_init`` on ``device`` (a CUDA ``torch.device`` or index), once per
    process: the tracers' work-queue counters, so that no launch allocates or waits."""
    import torch

    index = torch.device(device).index if not isinstance(device, int) else device
    if index is None:
        index = torch.cuda.current_device()
    if index in _initialised:
        return
    with torch.cuda.device(index):
        check(_lib.navi_device_init())
    _initialised.add(index)


def float3(values) -> ctypes.Array:
    return (ctypes.c_float * 3)(*[float(v) for v in values])
