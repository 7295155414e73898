"""Observation-path benchmark with the command-line surface of the reference's
``bench-sdfdag`` (projects/environment/src/navi_environment/cli.py:88-159,724-830).

The reference times whole ``SdfDagBackend.batch_step_tensor_actions`` steps
(sdfdag_backend.py:1196-1464). This harness times the part of such a step that
is the tracing path, on the MI355X kernels:

1. the step's kinematics for the benchmark actions of
   ``_benchmark_actions_tensor`` (cli.py:75-85: forward 1.5, yaw +-0.15
   alternating by actor), as ``_step_kinematics_tensor`` and
   ``_step_kinematics_indexed`` compute them (sdfdag_backend.py:560-617,
   2055-2094): a speed factor from the previous frame's nearest forward depth
   (the first and last Az/8 azimuth bins, expm1 of the log-normalised depth
   over the speed-limiter distance, clamped to [0.05, 1]), commands scaled by
   the drone speeds, velocity smoothing 0.15 against the previous command,
   position and yaw integrated over physics_dt, yaw wrapped to [0, 2 pi),
   position clamped to the scene box (config.py:94-105 defaults);
2. rays generated in the tracer from each actor's pose (sdfdag_backend.py:
   1300-1312) and traced on the device record layout;
3. one post-pass launch: the (actors, 3, Az, El) observation, delta depth and
   its previous-frame state, per-actor minimum distance and ratios, the
   collision flag (sdfdag_backend.py:1325-1368,1501-1526);
4. colliding actors return to their previous pose (sdfdag_backend.py:
   1340-1346); their smoothed velocities stay, as in the reference.

Rewards, resets and episode bookkeeping are the trainer's control plane and
are not part of it. Several ``.gmdag`` files may be given: they are resident
together and actor i traces scene i mod n, all in one launch (the reference
traces one scene per call and rotates scenes). Actors spawn at seeded positions
whose point-SDF clearance is at least 0.5 m. Output keys follow the reference's
summary (``measured_sps`` = actor steps per second over the timed steps,
``avg_batch_ms`` ...). Usage::

    python -m navi_amd.bench_sdfdag --gmdag-file a.gmdag [b.gmdag ...] --actors 64 --json
"""

from __future__ import annotations

import argparse
import json
import math
import statistics
import sys
import time
from pathlib import Path
from typing import Any

import numpy as np

ACTION_FWD, ACTION_YAW = 1.5, 0.15  # cli.py:82-84
DT = 0.02  # config.py:94 physics_dt
SPEED_FWD, SPEED_VERT, SPEED_LAT, SPEED_YAW = 5.0, 2.0, 3.0, 3.0  # config.py:96-99
SMOOTHING = 0.15  # sdfdag_backend.py:826
SPEED_LIMITER_DISTANCE = 0.8  # config.py:105-109
COLLISION_CLEARANCE = 0.15  # config.py:100, sdfdag_backend.py:38
SPAWN_CLEARANCE = 0.5


class ObservationHarness:
    """Resident scenes + per-actor state + preallocated outputs for the step loop.

    ``scenes``: a sequence of ``(words, bbox_min, bbox_max)``; actor i traces scene
    i mod len(scenes)."""

    def __init__(self, scenes, actors: int, azimuth_bins: int = 256, elevation_bins: int = 48,
                 max_distance: float = 30.0, sdf_max_steps: int = 256, device: str = "cuda",
                 seed: int = 0) -> None:
        import torch

        from . import scenes as S
        from .multiscene import ResidentScenes

        self.torch = torch
        scenes = list(scenes)
        self.res = ResidentScenes(scenes, device, keep_words=False)
        if not self.res.relaid_ok:
            raise RuntimeError("a DAG does not fit the device record layout")
        dev = self.res.device
        self.dev = dev
        self.actors, self.az, self.el = int(actors), int(azimuth_bins), int(elevation_bins)
        self.max_distance, self.max_steps = float(max_distance), int(sdf_max_steps)
        r = self.az * self.el
        self.local = torch.from_numpy(S.canonical_directions(self.az, self.el)).to(dev)
        scene_of = np.arange(self.actors) % len(scenes)
        self.env_scene = torch.from_numpy(scene_of.astype(np.int32)).to(dev)
        lo = np.array([np.asarray(sc[1], np.float32) for sc in scenes])
        hi = np.array([np.asarray(sc[2], np.float32) for sc in scenes])
        self.bmin = torch.from_numpy(np.ascontiguousarray(lo[scene_of])).to(dev)  # [A, 3] per actor
        self.bmax = torch.from_numpy(np.ascontiguousarray(hi[scene_of])).to(dev)
        self.pos = self._spawn(seed, scene_of, lo, hi)
        self.yaw = torch.zeros(self.actors, device=dev)
        act = torch.zeros(self.actors, 4, device=dev)  # cli.py:75-85: [fwd, vert, lat, yaw]
        act[:, 0] = ACTION_FWD
        act[::2, 3] = ACTION_YAW
        act[1::2, 3] = -ACTION_YAW
        self.actions = act
        self.prev_linear = torch.zeros((self.actors, 3), device=dev)
        self.prev_angular = torch.zeros((self.actors, 3), device=dev)
        self.rot = torch.empty((self.actors, 2), device=dev)
        self.out_d = torch.empty((self.actors, r), device=dev)
        self.out_s = torch.empty((self.actors, r), device=dev, dtype=torch.int32)
        self.obs = torch.empty((self.actors, 3, self.az, self.el), device=dev)
        self.prev_depth = torch.zeros((self.actors, self.az, self.el), device=dev)
        self.delta = torch.empty((self.actors, self.az, self.el), device=dev)
        self.stats = torch.empty((self.actors, 5), device=dev)
        self.collision = torch.empty((self.actors,), device=dev, dtype=torch.int32)

    def _spawn(self, seed: int, scene_of: np.ndarray, lo: np.ndarray, hi: np.ndarray):
        """Seeded rejection sampling of free positions in each actor's scene (batched
        point queries)."""
        torch = self.torch
        rng = np.random.default_rng(seed)
        out = np.empty((self.actors, 3), np.float32)
        for s in range(lo.shape[0]):
            want = np.flatnonzero(scene_of == s)
            found = np.empty((0, 3), np.float32)
            for _ in range(64):
                if len(found) >= want.size:
                    break
                n = max(256, 4 * want.size)
                cand = rng.uniform(lo[s].astype(np.float64), hi[s].astype(np.float64), (n, 3)).astype(np.float32)
                tp = torch.from_numpy(cand).to(self.dev)
                ps = torch.full((n,), s, dtype=torch.int32, device=self.dev)
                d = torch.empty(n, device=self.dev)
                sem = torch.empty(n, device=self.dev, dtype=torch.int32)
                k = torch.empty(n, device=self.dev, dtype=torch.int32)
                self.res.point_query(tp, d, sem, point_scene=ps, out_kind=k)
                ok = ((d >= SPAWN_CLEARANCE) & ((k == 1) | (k == 2))).cpu().numpy()
                found = np.concatenate([found, cand[ok]])
            if len(found) < want.size:
                raise RuntimeError(f"could not find free spawn positions in scene {s}")
            out[want] = found[: want.size]
        return torch.from_numpy(out).to(self.dev)

    def kinematics(self) -> None:
        """sdfdag_backend.py:560-617 (``_step_kinematics_tensor``) and the box clamp of
        :2087-2094, on every actor, with the previous frame's log-normalised depth."""
        torch = self.torch
        a = self.actors
        span = max(1, self.az // 8)
        front_left = self.prev_depth[:, :span, :].reshape(a, -1).amin(dim=1)
        front_right = self.prev_depth[:, -span:, :].reshape(a, -1).amin(dim=1)
        min_front = torch.minimum(front_left, front_right)
        min_front_metric = torch.expm1(min_front * math.log1p(self.max_distance))
        speed_factors = (min_front_metric / SPEED_LIMITER_DISTANCE).clamp(min=0.05, max=1.0).unsqueeze(1)
        linear_cmd = self.actions[:, :3].clone()
        linear_cmd[:, 0] *= SPEED_FWD
        linear_cmd[:, 1] *= SPEED_VERT
        linear_cmd[:, 2] *= SPEED_LAT
        linear_cmd *= speed_factors
        angular_cmd = torch.zeros((a, 3), device=self.dev)
        angular_cmd[:, 2] = self.actions[:, 3]
        angular_cmd[:, 2] *= SPEED_YAW
        smooth_linear = (1.0 - SMOOTHING) * linear_cmd + SMOOTHING * self.prev_linear
        smooth_angular = (1.0 - SMOOTHING) * angular_cmd + SMOOTHING * self.prev_angular
        cos_yaw = torch.cos(self.yaw)
        sin_yaw = torch.sin(self.yaw)
        fwd = smooth_linear[:, 0]
        lat = smooth_linear[:, 2]
        # yaw 0 faces -z: forward (-sin, 0, -cos), right (cos, 0, -sin)
        dx = -fwd * sin_yaw + lat * cos_yaw
        dz = -fwd * cos_yaw - lat * sin_yaw
        pos = self.pos.clone()
        pos[:, 0] += dx * DT
        pos[:, 1] += smooth_linear[:, 1] * DT
        pos[:, 2] += dz * DT
        self.yaw.copy_((self.yaw + smooth_angular[:, 2] * DT) % (2.0 * math.pi))
        self.prev_linear.copy_(smooth_linear)
        self.prev_angular.copy_(smooth_angular)
        self.pos.copy_(pos.clamp(min=self.bmin, max=self.bmax))

    def step(self) -> None:
        """One batched step: kinematics, rays from poses, trace, post-pass, collision revert."""
        torch = self.torch
        prev_pos = self.pos.clone()
        prev_yaw = self.yaw.clone()
        self.kinematics()
        torch.stack((torch.cos(self.yaw), torch.sin(self.yaw)), 1, out=self.rot)
        self.res.cast_rays_poses(self.env_scene, self.local, self.pos, self.rot, self.out_d, self.out_s,
                                 self.max_steps, self.max_distance, elevation_bins=self.el)
        self.res.observe(self.out_d, self.az, self.el, self.max_distance, semantics=self.out_s,
                         out_obs=self.obs, prev_depth=self.prev_depth, out_delta=self.delta,
                         out_stats=self.stats, out_collision=self.collision,
                         collision_clearance=COLLISION_CLEARANCE)
        hit = (self.collision != 0).unsqueeze(1)
        self.pos.copy_(torch.where(hit, prev_pos, self.pos))
        self.yaw.copy_(torch.where(hit[:, 0], prev_yaw, self.yaw))


def run_iteration(scenes, *, actors: int, steps: int, warmup_steps: int, azimuth_bins: int,
                  elevation_bins: int, max_distance: float, sdf_max_steps: int, seed: int) -> dict[str, Any]:
    h = ObservationHarness(scenes, actors, azimuth_bins, elevation_bins, max_distance, sdf_max_steps, seed=seed)
    torch = h.torch
    for _ in range(warmup_steps):
        h.step()
    torch.cuda.synchronize()
    batch_ms = []
    started = time.perf_counter()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        h.step()
        ev[i + 1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - started
    batch_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    rays = actors * azimuth_bins * elevation_bins
    return {
        "measured_sps": actors * steps / elapsed if elapsed > 0 else 0.0,
        "last_batch_ms": batch_ms[-1],
        "avg_batch_ms": statistics.fmean(batch_ms),
        "avg_actor_ms": statistics.fmean(batch_ms) / actors,
        "rays_per_s": rays * steps / (sum(batch_ms) / 1e3),
        "total_batches": steps + warmup_steps,
        "total_actor_steps": (steps + warmup_steps) * actors,
        "collisions_last_step": int(h.collision.sum().item()),
        "mean_min_distance": float(h.stats[:, 0].mean().item()),
    }


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="Benchmark the batched SDF/DAG observation path (MI355X).")
    ap.add_argument("--gmdag-file", required=True, nargs="+",
                    help="Path to compiled .gmdag world cache (several: resident together, actor i in scene i mod n)")
    ap.add_argument("--actors", type=int, default=4, help="Number of actors to benchmark in one batch")
    ap.add_argument("--steps", type=int, default=200, help="Measured batch steps after warmup")
    ap.add_argument("--warmup-steps", type=int, default=25, help="Unmeasured warmup batch steps")
    ap.add_argument("--repeats", type=int, default=1, help="Independent runs aggregated by median")
    ap.add_argument("--azimuth-bins", type=int, default=256)
    ap.add_argument("--elevation-bins", type=int, default=48)
    ap.add_argument("--max-distance", type=float, default=30.0)
    ap.add_argument("--sdf-max-steps", type=int, default=256)
    ap.add_argument("--seed", type=int, default=0, help="spawn positions")
    ap.add_argument("--json", action="store_true", help="Emit a JSON benchmark summary instead of text")
    args = ap.parse_args(argv)
    if min(args.actors, args.steps, args.repeats) < 1 or args.warmup_steps < 0:
        ap.error("actors, steps and repeats must be >= 1, warmup-steps >= 0")

    from .gmdag import load_gmdag_asset

    assets = [load_gmdag_asset(p) for p in args.gmdag_file]
    scenes = [(a.nodes, a.bbox_min, a.bbox_max) for a in assets]
    runs = [run_iteration(scenes, actors=args.actors, steps=args.steps,
                          warmup_steps=args.warmup_steps, azimuth_bins=args.azimuth_bins,
                          elevation_bins=args.elevation_bins, max_distance=args.max_distance,
                          sdf_max_steps=args.sdf_max_steps, seed=args.seed + r)
            for r in range(args.repeats)]
    sps = [r["measured_sps"] for r in runs]
    best = runs[sorted(range(len(runs)), key=lambda i: sps[i])[len(runs) // 2]]
    summary = {
        "profile": "bench-sdfdag",
        "gmdag_file": (str(Path(args.gmdag_file[0]).expanduser()) if len(args.gmdag_file) == 1
                       else [str(Path(f).expanduser()) for f in args.gmdag_file]),
        "scenes": len(args.gmdag_file),
        "actors": args.actors, "steps": args.steps, "warmup_steps": args.warmup_steps,
        "repeats": args.repeats, "azimuth_bins": args.azimuth_bins, "elevation_bins": args.elevation_bins,
        "max_distance": args.max_distance, "sdf_max_steps": args.sdf_max_steps,
        "aggregation": "median" if args.repeats > 1 else "single",
        **best,
    }
    if args.repeats > 1:
        summary.update(measured_sps_min=min(sps), measured_sps_max=max(sps), measured_sps_mean=statistics.fmean(sps))
    if args.json:
        print(json.dumps(summary, indent=2))
    else:
        print("bench-sdfdag - " + ", ".join(
            f"{k}={v:.2f}" if isinstance(v, float) else f"{k}={v}" for k, v in summary.items()
            if k not in ("profile", "gmdag_file")))
    return 0


if __name__ == "__main__":
    sys.exit(main())
