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



class _HostOnly:
    """A host-only build of the library's host code (the sanitizer build of
    ``make -C navi_amd/csrc asan``, named by ``NAVI_HOST_LIB``): the record-layout
    helpers are there, the device entry points are not (calling one raises)."""

    class _Absent:
        def __init__(self, name: str) -> None:
            self.__dict__["name"] = name
            self.__dict__["argtypes"] = []
            self.__dict__["restype"] = None

        def __setattr__(self, key, value) -> None:  # argtypes / restype of an absent entry point
            pass

        def __call__(self, *args):
            raise RuntimeError(f"{self.name} is not in the host-only library {HOST_LIB_PATH}")

    def __init__(self, path: str) -> None:
        self._so = ctypes.CDLL(path)

    def __getattr__(self, name: str):
        try:
            return getattr(self._so, name)
        except AttributeError:
            return _HostOnly._Absent(name)


HOST_LIB_PATH = os.environ.get("NAVI_HOST_LIB")
if HOST_LIB_PATH:
    _lib = _HostOnly(HOST_LIB_PATH)
else:
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
_lib.navi_relayout_leaves.restype = ctypes.c_int
_lib.navi_relayout_leaves.argtypes = [_vp, ctypes.c_uint64, _vp, ctypes.c_uint64, _u64p, _u32p, _vp, _vp,
                                      ctypes.c_uint32, _u32p]
_lib.navi_scene_flags.restype = ctypes.c_int
_lib.navi_scene_flags.argtypes = [_vp, ctypes.c_uint64, ctypes.c_uint32, _vp, ctypes.c_uint32, _u32p]


class PointQueries(ctypes.Structure):
    """navi_point_queries (include/navi_trace.h)."""

    _fields_ = [("records", _vp), ("n_records", ctypes.c_uint64), ("scenes", _vp), ("n_scenes", ctypes.c_int32),
                ("cell_tables", _vp), ("table_depth", ctypes.c_int32), ("point_scene", _vp), ("points", _vp),
                ("n_points", ctypes.c_int64),
                ("out_distances", _vp), ("out_semantics", _vp), ("out_kind", _vp),
                ("leaves", _vp), ("n_leaves", ctypes.c_uint32)]


class RelaidLaunch(ctypes.Structure):
    """navi_relaid_launch (include/navi_trace.h)."""

    _fields_ = [("records", _vp), ("n_records", ctypes.c_uint64), ("leaves", _vp), ("n_leaves", ctypes.c_uint32),
                ("scenes", _vp), ("n_scenes", ctypes.c_int32), ("cell_tables", _vp), ("table_depth", ctypes.c_int32),
                ("env_scene", _vp), ("env_order", _vp), ("n_envs", ctypes.c_int64), ("rays_per_env", ctypes.c_int64),
                ("elevation_bins", ctypes.c_int32), ("origins", _vp), ("dirs", _vp), ("local_dirs", _vp),
                ("env_pos", _vp), ("env_rot", _vp), ("out_distances", _vp), ("out_semantics", _vp),
                ("out_steps", _vp), ("max_steps", ctypes.c_int32), ("max_distance", ctypes.c_float),
                ("hit_epsilon", ctypes.c_float), ("distance_dtype", ctypes.c_int32)]


class LaunchInfo(ctypes.Structure):
    """navi_launch_info (include/navi_trace.h)."""

    _fields_ = [("kernels", ctypes.c_uint32), ("queue", ctypes.c_uint32), ("pair", ctypes.c_int32),
                ("fast_planes", ctypes.c_uint32), ("planes", ctypes.c_uint32), ("staged", ctypes.c_uint32),
                ("waves", ctypes.c_uint32), ("n_rays", ctypes.c_uint64)]


_lib.navi_trace_relaid_ex.restype = ctypes.c_int
_lib.navi_trace_relaid_ex.argtypes = [ctypes.POINTER(RelaidLaunch), _vp]
_lib.navi_last_launch.restype = ctypes.c_int
_lib.navi_last_launch.argtypes = [ctypes.POINTER(LaunchInfo)]

# navi_launch_info bits and kinds (include/navi_trace.h)
KERNEL_FAST, KERNEL_FAST_WIDE, KERNEL_COMBINED, KERNEL_RAW = 1, 2, 4, 8
QUEUE_NONE, QUEUE_STREAM, QUEUE_CAPTURE, QUEUE_LEASE, QUEUE_SCRATCH = 0, 1, 2, 3, 4
QUEUE_NAMES = {0: "none", 1: "stream", 2: "capture", 3: "lease", 4: "scratch"}


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
DIST_F32, DIST_BF16, DIST_F16 = 0, 1, 2  # navi_relaid_launch.distance_dtype


def scene_flags(records, root_slot, leaves=None) -> int:
    """``navi_scene_flags``: the NAVI_SCENE_* bits the records reachable from
    ``root_slot`` support (``records`` uint32 [n, 8] as navi_build_cell_table takes them,
    ``leaves`` the pool's leaf table or None)."""
    import numpy as np

    rec = np.ascontiguousarray(records, dtype=np.uint32).reshape(-1, 8)
    lv = np.ascontiguousarray(leaves if leaves is not None else np.zeros(0, np.uint32), dtype=np.uint32)
    out = ctypes.c_uint32()
    check(_lib.navi_scene_flags(rec.ctypes.data if rec.size else None, rec.shape[0], int(root_slot),
                                lv.ctypes.data if lv.size else None, lv.size, ctypes.byref(out)))
    return int(out.value)


def nonneg_leaves(records, root_slot, leaves=None) -> bool:
    """Whether no reachable leaf has its fp16 sign bit set (``NAVI_SCENE_NONNEG_LEAVES``)."""
    return bool(scene_flags(records, root_slot, leaves) & SCENE_NONNEG_LEAVES)


def last_launch() -> dict:
    """``navi_last_launch``: what the calling thread's last tracer launch enqueued."""
    info = LaunchInfo()
    check(_lib.navi_last_launch(ctypes.byref(info)))
    k = info.kernels
    return {"fast": bool(k & KERNEL_FAST), "fast_wide": bool(k & KERNEL_FAST_WIDE),
            "combined": bool(k & KERNEL_COMBINED), "raw": bool(k & KERNEL_RAW),
            "queue": QUEUE_NAMES.get(info.queue, str(info.queue)), "pair": info.pair,
            "fast_planes": info.fast_planes, "planes": info.planes, "staged": bool(info.staged),
            "waves": info.waves, "n_rays": info.n_rays}


def relayout_leaves(words):
    """``navi_relayout_leaves``: ``(records uint32 [n, 8], root_slot, levels_prefix[8],
    leaves uint32 [m])``; leaves of semantic 0x7fff or above go to the leaf table (slot
    0xffff0000 | entry). Raises RuntimeError (NAVI_E_LAYOUT) beyond 65536 entries."""
    import numpy as np

    w = np.ascontiguousarray(np.asarray(words).view(np.uint64).reshape(-1))
    n = ctypes.c_uint64()
    root = ctypes.c_uint32()
    n_leaves = ctypes.c_uint32()
    levels = np.zeros(8, np.uint64)
    check(_lib.navi_relayout_leaves(w.ctypes.data, w.size, None, 0, ctypes.byref(n), ctypes.byref(root),
                                    levels.ctypes.data, None, 0, ctypes.byref(n_leaves)))
    rec = np.zeros((max(1, n.value), 8), np.uint32)
    leaves = np.zeros(max(1, n_leaves.value), np.uint32)
    check(_lib.navi_relayout_leaves(w.ctypes.data, w.size, rec.ctypes.data, n.value, ctypes.byref(n),
                                    ctypes.byref(root), levels.ctypes.data, leaves.ctypes.data, leaves.size,
                                    ctypes.byref(n_leaves)))
    return rec[: n.value], int(root.value), levels, leaves[: n_leaves.value]


TABLE_LEAF = 0xFFFF0000  # a leaf slot of the leaf table; the low 16 bits index it


def rebase_leaves(records, root_slot, offset):
    """Records and root slot with every leaf-table slot's entry moved by ``offset`` (a
    scene's place in a pool's concatenated leaf table)."""
    import numpy as np

    rec = np.asarray(records, np.uint32).copy()
    table = (rec & np.uint32(TABLE_LEAF)) == np.uint32(TABLE_LEAF)
    if offset and table.any():
        idx = (rec[table] & np.uint32(0xFFFF)) + np.uint32(offset)
        if int(idx.max()) > 0xFFFF:
            raise RuntimeError("leaf table of the pool exceeds 65536 entries")
        rec[table] = np.uint32(TABLE_LEAF) | idx
    root = int(root_slot)
    if offset and (root & TABLE_LEAF) == TABLE_LEAF:
        if (root & 0xFFFF) + offset > 0xFFFF:
            raise RuntimeError("leaf table of the pool exceeds 65536 entries")
        root = TABLE_LEAF | ((root & 0xFFFF) + offset)
    return rec, root


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
