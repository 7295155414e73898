"""Several ``.gmdag`` scenes resident on one GPU, traced in one launch.

The reference keeps one DAG tensor per backend and swaps it on scene rotation
(``projects/environment/src/navi_environment/backends/sdfdag_backend.py:864-886,
1897-1905``); a batch over envs in different scenes costs one ``cast_rays`` per
scene. Here all scenes live in one device word pool with a 40-byte descriptor
each (``navi_scene_desc`` in ``include/navi_trace.h``) and an int32 scene id
per env selects the DAG inside the kernel.

Work order. The record-layout tracer hands out rays in env order, and a launch
lasts until its slowest wave ends: a scene whose rays run long (rooms with flat
floors give grazing rays of hundreds of steps) should start first, not last.
``ResidentScenes`` therefore sorts envs by scene, with the scenes in descending
order of their measured cost (mean steps per ray) once it knows them: the first
multi-scene launch also counts steps per ray, reduces them per scene on the
device and copies the sums back asynchronously; a later launch that finds the
copy complete adopts the order (longest-processing-time-first scheduling).
Results do not depend on the order.
"""

from __future__ import annotations

import ctypes
import math
from typing import Any, Sequence

import numpy as np
import torch

from . import _native


# The tracer stages each scene's split planes in LDS when the scene table and
# planes of a launch fit in this many bytes (kPlaneLds in trace_relaid.hip:
# 7 waves per SIMD), else in the wider budget (kPlaneLdsWide: 5 waves):
# 32 bytes per scene plus scene_stride(P) floats, P the planes' depth.
PLANE_LDS_BYTES = 22528
PLANE_LDS_BYTES_WIDE = 32512


def _plane_bytes(depth: int) -> int:
    # scene_stride in trace_relaid.hip: 8 header floats, then 2^depth + 2 per axis
    return 4 * ((8 + 3 * ((1 << depth) + 2) + 3) & ~3)


def plane_depth(n_scenes: int, table_depth: int) -> int:
    """The split-plane depth the tracer uses for ``n_scenes`` scenes and cell tables of
    ``table_depth`` (launch_relaid in trace_relaid.hip): the deepest P <= min(D, 6), at
    most two levels above the tables, whose planes fit ``PLANE_LDS_BYTES``, else
    ``PLANE_LDS_BYTES_WIDE``; 0 for none."""
    for budget in (PLANE_LDS_BYTES, PLANE_LDS_BYTES_WIDE):
        for p in range(min(table_depth, 6), max(4, table_depth - 2) - 1, -1):
            if n_scenes * (32 + _plane_bytes(p)) <= budget:
                return p
    return 0


WIDE_PLANE_LDS_BYTES = 81920  # kFastLdsWide: two 1024-thread workgroups per CU


def wide_plane_depth(n_scenes: int, table_depth: int) -> int:
    """The split-plane depth of the 1024-thread fast kernel (launch_relaid's
    ``plane_depth_wide``): the deepest P in [max(4, D - 2), min(D + 2, 8)] whose planes
    and scene table fit ``WIDE_PLANE_LDS_BYTES``; 0 when none does (such launches take
    the 256-thread workgroups). Launches of fewer rays than ``navi_set_wide_min_rays``
    (default 2^19) take the 256-thread workgroups whatever this says."""
    for p in range(min(table_depth + 2, 8), max(4, table_depth - 2) - 1, -1):
        if n_scenes * (32 + _plane_bytes(p)) <= WIDE_PLANE_LDS_BYTES:
            return p
    return 0


# Cell tables take 8 bytes per cell: 2 MiB per scene at depth 6, 16 MiB at 7.
TABLE_BYTES_BUDGET = 256 << 20


def default_table_depth(n_scenes: int) -> int:
    """The deepest cell table, at most 6, whose tables stay within
    ``TABLE_BYTES_BUDGET``: 6 up to 128 scenes, 5 up to 1024. Depth 7 (16 MiB per
    scene) measured no faster than 6 on the 16-scene 1024^3 batch (3.51 against
    3.47 ms), and its tables do not fit the 256 MB MALL beside the records."""
    for depth in (6, 5):
        if n_scenes * 8 ** depth * 8 <= TABLE_BYTES_BUDGET:
            return depth
    return 4


class ResidentScenes:
    """Concatenated word pool + scene table on one device.

    ``scenes`` is a sequence of ``(words, bbox_min, bbox_max)`` with ``words`` a
    uint64 (or int64-viewed) array in the reference word layout; child pointers
    stay relative to each scene's first word.
    """

    def __init__(self, scenes: Sequence[tuple[np.ndarray, Sequence[float], Sequence[float]]],
                 device: str | torch.device = "cuda", *, keep_words: bool = True,
                 table_depth: int | None = None, order_by_cost: bool = True) -> None:
        if not scenes:
            raise ValueError("at least one scene is required")
        if table_depth is not None and not 4 <= int(table_depth) <= 7:
            raise ValueError("table_depth must be in [4, 7]")
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        table = np.zeros(len(scenes), dtype=_native.SCENE_DESC_DTYPE)
        offset = 0
        chunks = []
        for i, (words, lo, hi) in enumerate(scenes):
            w = np.ascontiguousarray(np.asarray(words).view(np.uint64).reshape(-1))
            if w.size == 0:
                raise ValueError(f"scene {i} has no words")
            for k in range(3):
                if not (math.isfinite(float(lo[k])) and math.isfinite(float(hi[k])) and float(lo[k]) < float(hi[k])):
                    raise ValueError(f"scene {i}: bbox_min must be finite and strictly below bbox_max")
            table[i]["word_offset"] = offset
            table[i]["n_words"] = w.size
            table[i]["bbox_min"] = np.asarray(lo, np.float32)
            table[i]["bbox_max"] = np.asarray(hi, np.float32)
            chunks.append(w)
            offset += w.size
        self.n_scenes = len(scenes)
        self.word_counts = [int(c.size) for c in chunks]
        self.host_table = table
        # the word pool serves kernel="raw"; callers that keep their own word tensor skip it
        self.pool = torch.from_numpy(np.concatenate(chunks).view(np.int64)).to(self.device) if keep_words else None
        self.table = torch.from_numpy(table.view(np.uint8).copy()).to(self.device)

        # device record layout (one 32-byte record per internal node); leaves of
        # semantic 0x7fff or above go to one leaf table shared by the pool
        rtable = np.zeros(len(scenes), dtype=_native.RELAID_SCENE_DTYPE)
        recs = []
        leaf_tables = []
        roff = 0
        loff = 0
        self.relaid_ok = True
        for i, w in enumerate(chunks):
            try:
                rec, root, _levels, leaves = _native.relayout_leaves(w)
                rec, root = _native.rebase_leaves(rec, root, loff)
            except RuntimeError:
                self.relaid_ok = False
                break
            leaf_tables.append(leaves)
            loff += int(leaves.size)
            rtable[i]["rec_offset"] = roff
            rtable[i]["n_records"] = rec.shape[0]
            # child record slots become absolute pool indices
            rec = rec.copy()
            child = rec < 0x7FFFFFFD
            rec[child] += np.uint32(roff)
            rtable[i]["root_slot"] = root if root & 0x80000000 else roff + root
            rtable[i]["bbox_min"] = table[i]["bbox_min"]
            rtable[i]["bbox_max"] = table[i]["bbox_max"]
            recs.append(rec)
            roff += rec.shape[0]
        if self.relaid_ok:
            # navi_trace_relaid reads the pool through a buffer resource whose
            # 32-bit byte size must not wrap: fewer than 2^27 records
            if roff >= (1 << 27):
                self.relaid_ok = False
        self.n_leaves = 0
        self.leaves = None
        if self.relaid_ok:
            allrec = np.concatenate(recs) if roff else np.zeros((1, 8), np.uint32)
            all_leaves = np.concatenate(leaf_tables) if loff else np.zeros(0, np.uint32)
            for i in range(len(scenes)):
                rtable[i]["max_depth"] = _native.record_depth(allrec[:roff], int(rtable[i]["root_slot"]))
                rtable[i]["flags"] = _native.scene_flags(allrec[:roff], int(rtable[i]["root_slot"]), all_leaves)
            if loff:
                self.n_leaves = loff
                self.leaves = torch.from_numpy(all_leaves.view(np.int32).copy()).to(self.device)
            if table_depth is not None:
                self.table_depth = int(table_depth)
            else:
                # no deeper than one level below the deepest record: such a table
                # already answers every descent
                deepest = max(int(d) for d in rtable["max_depth"])  # 0xffffffff for a cycle
                self.table_depth = max(4, min(default_table_depth(len(scenes)), deepest + 1))
            tables = np.concatenate([_native.cell_table(allrec[:roff], int(rtable[i]["root_slot"]), self.table_depth)
                                     for i in range(len(scenes))])
            self.cell_tables = torch.from_numpy(tables.view(np.int64)).to(self.device)
            self.n_records = int(roff)
            self.records = torch.from_numpy(allrec.view(np.int32).reshape(-1).copy()).to(self.device)
            self.relaid_table = torch.from_numpy(rtable.view(np.uint8).copy()).to(self.device)
            self.record_counts = [int(r.shape[0]) for r in recs]
        self._order_key = None
        self._order = None
        # scene order by measured cost (module docstring)
        self.order_by_cost = bool(order_by_cost) and self.n_scenes > 1
        self.scene_cost: np.ndarray | None = None  # mean steps per ray, once measured
        self._scene_rank: torch.Tensor | None = None  # [n_scenes + 1] position of each scene; unknown ids last
        self._cost_pending = False  # a measurement is queued behind _cost_event
        self._cost_version = 0
        # Everything a launch needs is allocated here, at scene load: the
        # tracer's work-queue counters, and the buffers of the cost measurement
        # and its readback. A launch then allocates nothing and never waits
        # (the measuring launch aside, which takes a steps buffer when the
        # caller passes none, and launches that sort envs for a new env_scene).
        cuda = self.device.type == "cuda"
        n1 = self.n_scenes + 1
        self._cost_dev = torch.zeros((2, n1), dtype=torch.int64, device=self.device)
        self._cost_host = torch.zeros((2, n1), dtype=torch.int64, pin_memory=cuda)
        self._rank_host = torch.zeros(n1, dtype=torch.int64, pin_memory=cuda)
        self._rank_dev = torch.zeros(n1, dtype=torch.int64, device=self.device)
        self._cost_event = None
        if cuda:
            _native.device_init(self.device)
            with torch.cuda.device(self.device):
                self._cost_event = torch.cuda.Event()

    @property
    def pool_bytes(self) -> int:
        return int(self.pool.numel()) * 8 if self.pool is not None else 0

    @property
    def record_bytes(self) -> int:
        return int(self.records.numel()) * 4 if self.relaid_ok else 0

    def env_order(self, env_scene: torch.Tensor) -> torch.Tensor:
        """Envs sorted (stably) by scene: by scene id, or, once the scenes' costs are
        measured, by descending cost. Cached per env_scene contents/version."""
        key = (env_scene.data_ptr(), env_scene._version, tuple(env_scene.shape), self._cost_version)
        if self._order_key != key:
            if self._scene_rank is None:
                sort_key = env_scene.to(torch.int64)
            else:
                n = self.n_scenes
                known = (env_scene >= 0) & (env_scene < n)
                sort_key = self._scene_rank[torch.where(known, env_scene, n).to(torch.int64)]
            self._order = torch.sort(sort_key, stable=True).indices.to(torch.int32)
            self._order_key = key
        return self._order

    def _capturing(self) -> bool:
        return self.device.type == "cuda" and torch.cuda.is_current_stream_capturing()

    def _cost_steps(self, out_steps: Any, e: int, r: int, sort_by_scene: bool) -> tuple[Any, bool]:
        """The steps tensor for a launch and whether the launch measures the scenes' costs
        (never inside a graph capture: its readback belongs to one eager launch)."""
        if (not (self.order_by_cost and sort_by_scene) or self.scene_cost is not None
                or self._cost_pending or e * r == 0 or self._capturing()):
            return out_steps, False
        if out_steps is None:
            out_steps = torch.empty((e, r), dtype=torch.int32, device=self.device)
        return out_steps, True

    def _start_cost_readback(self, steps: torch.Tensor, env_scene: torch.Tensor) -> None:
        """Per-scene step sums and ray counts of the launch just queued, copied to pinned
        host memory behind an event on the current stream (no wait here)."""
        n = self.n_scenes
        with torch.cuda.device(self.device):
            idx = torch.where((env_scene >= 0) & (env_scene < n), env_scene, n).to(torch.int64)
            self._cost_dev.zero_()
            self._cost_dev[0].index_add_(0, idx, steps.sum(dim=1, dtype=torch.int64))
            self._cost_dev[1].index_add_(0, idx, torch.full_like(idx, int(steps.shape[1])))
            self._cost_host.copy_(self._cost_dev, non_blocking=True)
            self._cost_event.record()
        self._cost_pending = True

    def _poll_cost(self) -> None:
        """Adopt the measured scene costs if their copy has completed (never waits; never
        inside a graph capture, where an event query is not allowed)."""
        if not self._cost_pending or self._capturing():
            return
        if self._cost_event is not None and not self._cost_event.query():
            return
        host = self._cost_host.numpy()
        self._cost_pending = False
        n = self.n_scenes
        sums, rays = host[0, :n].astype(np.float64), host[1, :n]
        if not np.any(rays > 0):  # no ray of a known scene: measure on a later launch
            return
        cost = np.full(n, np.nan)
        np.divide(sums, rays, out=cost, where=rays > 0)
        cost[np.isnan(cost)] = np.nanmean(cost) if np.any(rays > 0) else 0.0  # unmeasured scenes
        rank = np.empty(n + 1, np.int64)
        rank[np.argsort(-cost, kind="stable")] = np.arange(n)
        rank[n] = n
        self.scene_cost = cost
        # written once: the pinned source of the asynchronous copy is never reused
        self._rank_host.copy_(torch.from_numpy(rank))
        if self.device.type == "cuda":
            with torch.cuda.device(self.device):
                self._rank_dev.copy_(self._rank_host, non_blocking=True)
        else:
            self._rank_dev.copy_(self._rank_host)
        self._scene_rank = self._rank_dev
        self._cost_version += 1

    def cast_rays(self, env_scene: torch.Tensor, origins: torch.Tensor, dirs: torch.Tensor,
                  out_distances: torch.Tensor, out_semantics: torch.Tensor, max_steps: int,
                  max_distance: float, *, hit_epsilon: float = 0.01, out_steps: Any | None = None,
                  out_words: Any | None = None, kernel: str = "relaid",
                  elevation_bins: int | None = None, sort_by_scene: bool = True) -> None:
        """Trace ``origins``/``dirs`` ``[E, R, 3]``; env ``e`` uses scene ``env_scene[e]``.
        Outputs ``[E, R]`` are written in place on the current stream.

        ``kernel="relaid"`` (default) runs the device-layout tracer; ``"raw"`` walks the
        reference word layout (and is the one that can fill ``out_words``). Both give
        identical per-ray results. ``out_distances`` may be float32, bfloat16 or float16
        (``docs/FUTURE_HARDWARE_ROADMAP.md:140-222`` of the reference: the march keeps float32,
        a finished ray's distance is rounded to nearest even; record-layout tracer only).
        ``elevation_bins`` declares the canonical
        ``az * El + el`` ray layout for angular tiling. ``sort_by_scene`` hands the
        envs to the kernel grouped by scene, costliest scenes first once their costs
        are measured (the first such launch counts steps per ray for that)."""
        self._require_gpu()
        e, r = int(origins.shape[0]), int(origins.shape[1])
        dist_dtype = self._distance_dtype(out_distances)
        for name, t, dt, shape in (("origins", origins, torch.float32, (e, r, 3)),
                                   ("dirs", dirs, torch.float32, (e, r, 3)),
                                   ("out_distances", out_distances, out_distances.dtype, (e, r)),
                                   ("out_semantics", out_semantics, torch.int32, (e, r)),
                                   ("env_scene", env_scene, torch.int32, (e,))):
            if t.device != self.device or t.dtype != dt or not t.is_contiguous() or tuple(t.shape) != shape:
                raise RuntimeError(f"{name} must be a contiguous {dt} tensor of shape {shape} on {self.device}")
        for name, t, dt in (("out_steps", out_steps, torch.int32), ("out_words", out_words, torch.int32)):
            if t is not None and (t.device != self.device or t.dtype != dt or not t.is_contiguous()
                                  or tuple(t.shape) != (e, r)):
                raise RuntimeError(f"{name} must be a contiguous {dt} tensor of shape {(e, r)}")
        if not 0 < int(max_steps) <= 0x7FFFFFFF:  # an int32 in the C ABI
            raise RuntimeError("max_steps must be a positive integer")
        if not (math.isfinite(float(max_distance)) and float(max_distance) > 0.0):
            raise RuntimeError("max_distance must be a finite positive float")
        if kernel == "relaid" and out_words is None and self.relaid_ok:
            self._poll_cost()
            order = self.env_order(env_scene) if sort_by_scene else None
            out_steps, measure = self._cost_steps(out_steps, e, r, sort_by_scene)
            L = self._launch_args(env_scene.data_ptr(), order, e, r, elevation_bins, out_distances.data_ptr(),
                                  out_semantics.data_ptr(), out_steps, max_steps, max_distance, hit_epsilon,
                                  dist_dtype)
            L.origins, L.dirs = origins.data_ptr(), dirs.data_ptr()
            self._launch(L, e, r, elevation_bins, order)
            if measure:
                self._start_cost_readback(out_steps, env_scene)
            return
        if kernel not in ("relaid", "raw"):
            raise ValueError(f"unknown kernel {kernel!r}")
        if dist_dtype != _native.DIST_F32:
            raise RuntimeError("bfloat16 and float16 distances need the record-layout tracer "
                               "(kernel='relaid' without out_words, on scenes the record layout holds)")
        if self.pool is None:
            raise RuntimeError("this ResidentScenes keeps no word pool (keep_words=False)")
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            code = _native.lib().navi_cast_rays_multi(
                self.pool.data_ptr(), self.table.data_ptr(), self.n_scenes, env_scene.data_ptr(), e, r,
                origins.data_ptr(), dirs.data_ptr(), out_distances.data_ptr(), out_semantics.data_ptr(),
                int(max_steps), float(max_distance), float(hit_epsilon),
                out_steps.data_ptr() if out_steps is not None else None,
                out_words.data_ptr() if out_words is not None else None, stream)
        _native.check(code)

    # ---- pose-driven tracing, point queries and the observation post-pass ----

    def _require_gpu(self) -> None:
        # the kernels dereference every pointer on the GPU: host tensors never reach them
        if self.device.type != "cuda":
            raise RuntimeError(f"tracing needs the scenes on a GPU device, not {self.device}")

    def _require_relaid(self) -> None:
        self._require_gpu()
        if not self.relaid_ok:
            raise RuntimeError("these scenes do not fit the device record layout "
                               "(more than 65536 distinct leaves of semantic 0x7fff or above, or 2^27 records)")

    @staticmethod
    def _distance_dtype(out_distances: Any) -> int:
        """``navi_relaid_launch.distance_dtype`` of a distance output tensor: float32,
        bfloat16 or float16 (the march accumulates in float32 either way)."""
        code = {torch.float32: _native.DIST_F32, torch.bfloat16: _native.DIST_BF16,
                torch.float16: _native.DIST_F16}.get(getattr(out_distances, "dtype", None))
        if code is None:
            raise RuntimeError(f"out_distances must be float32, bfloat16 or float16; got "
                               f"{getattr(out_distances, 'dtype', None)}")
        return code

    def _check(self, name: str, t: Any, dtype: Any, shape: tuple[int, ...], optional: bool = False) -> int | None:
        if t is None:
            if optional:
                return None
            raise RuntimeError(f"{name} is required")
        if t.device != self.device or t.dtype != dtype or not t.is_contiguous() or tuple(t.shape) != shape:
            raise RuntimeError(f"{name} must be a contiguous {dtype} tensor of shape {shape} on {self.device}")
        return t.data_ptr()

    def cast_rays_poses(self, env_scene: torch.Tensor, local_dirs: torch.Tensor, env_pos: torch.Tensor,
                        env_rot: torch.Tensor, out_distances: torch.Tensor, out_semantics: torch.Tensor,
                        max_steps: int, max_distance: float, *, hit_epsilon: float = 0.01,
                        out_steps: Any | None = None, elevation_bins: int | None = None,
                        sort_by_scene: bool = True) -> None:
        """Trace with rays generated in the kernel: env ``e`` casts ``local_dirs`` ``[R, 3]``
        rotated by its yaw (``env_rot[e] = (cos, sin)``) from ``env_pos[e]``, the ray layout
        of ``sdfdag_backend.py:1300-1312``. Outputs ``[E, R]`` as ``cast_rays`` (distances
        float32, bfloat16 or float16)."""
        self._require_relaid()
        if not 0 < int(max_steps) <= 0x7FFFFFFF:  # an int32 in the C ABI
            raise RuntimeError("max_steps must be a positive integer")
        e, r = int(env_pos.shape[0]), int(local_dirs.shape[0])
        dist_dtype = self._distance_dtype(out_distances)
        ptrs = [self._check("env_scene", env_scene, torch.int32, (e,)),
                self._check("local_dirs", local_dirs, torch.float32, (r, 3)),
                self._check("env_pos", env_pos, torch.float32, (e, 3)),
                self._check("env_rot", env_rot, torch.float32, (e, 2)),
                self._check("out_distances", out_distances, out_distances.dtype, (e, r)),
                self._check("out_semantics", out_semantics, torch.int32, (e, r)),
                self._check("out_steps", out_steps, torch.int32, (e, r), optional=True)]
        self._poll_cost()
        order = self.env_order(env_scene) if sort_by_scene else None
        steps, measure = self._cost_steps(out_steps, e, r, sort_by_scene)
        L = self._launch_args(ptrs[0], order, e, r, elevation_bins, ptrs[4], ptrs[5], steps, max_steps,
                              max_distance, hit_epsilon, dist_dtype)
        L.local_dirs, L.env_pos, L.env_rot = ptrs[1], ptrs[2], ptrs[3]
        self._launch(L, e, r, elevation_bins, order)
        if measure:
            self._start_cost_readback(steps, env_scene)

    # ---- launches ----

    def _launch_args(self, env_scene_ptr, order, e, r, elevation_bins, out_d_ptr, out_s_ptr, steps, max_steps,
                     max_distance, hit_epsilon, dist_dtype: int = 0) -> Any:
        L = _native.RelaidLaunch()
        L.records, L.n_records = self.records.data_ptr(), self.n_records
        if self.n_leaves:
            L.leaves, L.n_leaves = self.leaves.data_ptr(), self.n_leaves
        L.scenes, L.n_scenes = self.relaid_table.data_ptr(), self.n_scenes
        L.cell_tables, L.table_depth = self.cell_tables.data_ptr(), self.table_depth
        L.env_scene = env_scene_ptr
        L.env_order = order.data_ptr() if order is not None else None
        L.n_envs, L.rays_per_env, L.elevation_bins = e, r, int(elevation_bins or 0)
        L.out_distances, L.out_semantics = out_d_ptr, out_s_ptr
        L.out_steps = steps.data_ptr() if steps is not None else None
        L.max_steps, L.max_distance, L.hit_epsilon = int(max_steps), float(max_distance), float(hit_epsilon)
        L.distance_dtype = int(dist_dtype)
        return L

    def _launch(self, L, e: int, r: int, elevation_bins, order) -> None:
        """Enqueues ``navi_trace_relaid_ex`` on the current stream."""
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            code = _native.lib().navi_trace_relaid_ex(ctypes.byref(L), stream)
        _native.check(code)

    def _point_queries(self, points, out_distances, out_semantics, point_scene, out_kind, prefix=""):
        self._require_relaid()
        p = int(points.shape[0])
        q = _native.PointQueries()
        q.records, q.n_records = self.records.data_ptr(), self.n_records
        q.scenes, q.n_scenes, q.cell_tables = self.relaid_table.data_ptr(), self.n_scenes, self.cell_tables.data_ptr()
        q.table_depth = self.table_depth
        q.points = self._check("points", points, torch.float32, (p, 3))
        q.n_points = p
        q.point_scene = self._check(prefix + "point_scene", point_scene, torch.int32, (p,), optional=True)
        q.out_distances = self._check(prefix + "distances", out_distances, torch.float32, (p,))
        q.out_semantics = self._check(prefix + "semantics", out_semantics, torch.int32, (p,))
        q.out_kind = self._check(prefix + "kind", out_kind, torch.int32, (p,), optional=True)
        if self.n_leaves:
            q.leaves, q.n_leaves = self.leaves.data_ptr(), self.n_leaves
        return q

    def point_query(self, points: torch.Tensor, out_distances: torch.Tensor, out_semantics: torch.Tensor, *,
                    point_scene: torch.Tensor | None = None, out_kind: torch.Tensor | None = None) -> None:
        """Point-SDF queries ``points [P, 3]`` (scene ``point_scene[i]``, default 0); see
        ``navi_point_query`` in ``include/navi_trace.h`` for the result kinds."""
        q = self._point_queries(points, out_distances, out_semantics, point_scene, out_kind)
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            code = _native.lib().navi_point_query(ctypes.byref(q), stream)
        _native.check(code)

    def observe(self, distances: torch.Tensor, azimuth_bins: int, elevation_bins: int, max_distance: float, *,
                structure_band_min: float = 1.5, structure_band_max: float = 30.0,
                proximity_threshold: float = 2.0, collision_clearance: float = 0.15,
                out_depth_f16: torch.Tensor | None = None, out_stats: torch.Tensor | None = None,
                out_collision: torch.Tensor | None = None, semantics: torch.Tensor | None = None,
                out_obs: torch.Tensor | None = None, prev_depth: torch.Tensor | None = None,
                out_delta: torch.Tensor | None = None, points: torch.Tensor | None = None,
                point_scene: torch.Tensor | None = None, point_distances: torch.Tensor | None = None,
                point_semantics: torch.Tensor | None = None, point_kind: torch.Tensor | None = None) -> None:
        """The observation post-pass of ``sdfdag_backend.py:366-473,1340,1501-1526`` in one
        launch, with optional point queries fused in. ``distances [E, Az*El]``; writes any of
        ``out_depth_f16 [E, 1, El, Az]`` (float16), ``out_obs [E, 3, Az, El]`` (depth,
        semantic, valid; needs ``semantics [E, Az*El]``), ``out_delta [E, Az, El]`` (against
        ``prev_depth``, which then holds the depth), ``out_stats [E, 5]`` (min distance,
        starvation, proximity, structure-band and forward-structure ratios) and
        ``out_collision [E]`` (int32). Defaults are the reference's
        (``sdfdag_backend.py:38,48-51``)."""
        self._require_gpu()
        e = int(distances.shape[0])
        az, el = int(azimuth_bins), int(elevation_bins)
        o = _native.Observation()
        o.distances = self._check("distances", distances, torch.float32, (e, az * el))
        o.semantics = self._check("semantics", semantics, torch.int32, (e, az * el), optional=out_obs is None)
        o.n_envs, o.azimuth_bins, o.elevation_bins = e, az, el
        o.max_distance = float(max_distance)
        o.structure_band_min, o.structure_band_max = float(structure_band_min), float(structure_band_max)
        o.proximity_threshold, o.collision_clearance = float(proximity_threshold), float(collision_clearance)
        o.depth_f16 = self._check("out_depth_f16", out_depth_f16, torch.float16, (e, 1, el, az), optional=True)
        o.obs = self._check("out_obs", out_obs, torch.float32, (e, 3, az, el), optional=True)
        o.prev_depth = self._check("prev_depth", prev_depth, torch.float32, (e, az, el), optional=out_delta is None)
        o.delta = self._check("out_delta", out_delta, torch.float32, (e, az, el), optional=True)
        o.stats = self._check("out_stats", out_stats, torch.float32, (e, 5), optional=True)
        o.collision = self._check("out_collision", out_collision, torch.int32, (e,), optional=True)
        q = None
        if points is not None:
            q = self._point_queries(points, point_distances, point_semantics, point_scene, point_kind, "point_")
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            code = _native.lib().navi_observe(ctypes.byref(o), ctypes.byref(q) if q is not None else None, stream)
        _native.check(code)
