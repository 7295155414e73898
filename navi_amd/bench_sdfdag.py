"""Observation-path benchmark with the command-line surface of the reference's
``bench-sdfdag`` (projects/environment/src/navi_environment/cli.py:88-159,724-830).

The reference times whole ``SdfDagBackend.batch_step_tensor_actions`` steps
(sdfdag_backend.py:1196-1464). This harness times the part of such a step that
is the tracing path, on the MI355X kernels:

1. kinematics for the benchmark actions of ``_benchmark_actions_tensor``
   (cli.py:75-85: forward 1.5, yaw +-0.15 alternating by actor), integrated
   plainly with the environment defaults (physics_dt 0.02, drone_max_speed 5,
   drone_yaw_rate 3; projects/environment/src/navi_environment/config.py:
   94-99): position += dt * speed * action * forward, yaw += dt * rate *
   action, clamped to the scene box; the velocity smoothing, action limits and
   depth-based speed limiter of ``_step_kinematics_tensor`` are not reproduced;
2. rays generated in the tracer from each actor's pose (sdfdag_backend.py:
   1300-1312) and traced on the device record layout;
3. one post-pass launch: the (actors, 3, Az, El) observation, delta depth and
   its previous-frame state, per-actor minimum distance and ratios, the
   collision flag (sdfdag_backend.py:1325-1368,1501-1526);
4. colliding actors return to their previous pose (sdfdag_backend.py:
   1340-1346).

Actors spawn at seeded positions whose point-SDF clearance is at least 0.5 m.
Output keys follow the reference's summary (``measured_sps`` = actor steps per
second over the timed steps, ``avg_batch_ms`` ...). Usage::

    python -m navi_amd.bench_sdfdag --gmdag-file scene.gmdag --actors 64 --json
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import time
from pathlib import Path
from typing import Any

import numpy as np

ACTION_FWD, ACTION_YAW = 1.5, 0.15  # cli.py:82-84
DT, MAX_SPEED, YAW_RATE = 0.02, 5.0, 3.0  # config.py:94,96,99
COLLISION_CLEARANCE = 0.15  # config.py:100, sdfdag_backend.py:38
SPAWN_CLEARANCE = 0.5


class ObservationHarness:
    """Resident scene + per-actor state + preallocated outputs for the step loop."""

    def __init__(self, words: np.ndarray, bbox_min, bbox_max, actors: int, azimuth_bins: int = 256,
                 elevation_bins: int = 48, max_distance: float = 30.0, sdf_max_steps: int = 256,
                 device: str = "cuda", seed: int = 0) -> None:
        import torch

        from . import scenes as S
        from .multiscene import ResidentScenes

        self.torch = torch
        self.res = ResidentScenes([(words, bbox_min, bbox_max)], device, keep_words=False)
        if not self.res.relaid_ok:
            raise RuntimeError("the DAG does not fit the device record layout")
        dev = self.res.device
        self.dev = dev
        self.actors, self.az, self.el = int(actors), int(azimuth_bins), int(elevation_bins)
        self.max_distance, self.max_steps = float(max_distance), int(sdf_max_steps)
        r = self.az * self.el
        self.local = torch.from_numpy(S.canonical_directions(self.az, self.el)).to(dev)
        self.bmin = torch.tensor(np.asarray(bbox_min, np.float32), device=dev)
        self.bmax = torch.tensor(np.asarray(bbox_max, np.float32), device=dev)
        self.env_scene = torch.zeros(self.actors, dtype=torch.int32, device=dev)
        self.pos = self._spawn(seed)
        self.yaw = torch.zeros(self.actors, device=dev)
        act = torch.zeros(self.actors, 4, device=dev)  # cli.py:75-85
        act[:, 0] = ACTION_FWD
        act[::2, 3] = ACTION_YAW
        act[1::2, 3] = -ACTION_YAW
        self.actions = act
        self.rot = torch.empty((self.actors, 2), device=dev)
        self.out_d = torch.empty((self.actors, r), device=dev)
        self.out_s = torch.empty((self.actors, r), device=dev, dtype=torch.int32)
        self.obs = torch.empty((self.actors, 3, self.az, self.el), device=dev)
        self.prev_depth = torch.zeros((self.actors, self.az, self.el), device=dev)
        self.delta = torch.empty((self.actors, self.az, self.el), device=dev)
        self.stats = torch.empty((self.actors, 5), device=dev)
        self.collision = torch.empty((self.actors,), device=dev, dtype=torch.int32)

    def _spawn(self, seed: int):
        """Seeded rejection sampling of free positions with point queries (batched)."""
        torch = self.torch
        rng = np.random.default_rng(seed)
        lo = self.bmin.cpu().numpy().astype(np.float64)
        hi = self.bmax.cpu().numpy().astype(np.float64)
        found = np.empty((0, 3), np.float32)
        for _ in range(64):
            cand = rng.uniform(lo, hi, (max(256, 4 * self.actors), 3)).astype(np.float32)
            tp = torch.from_numpy(cand).to(self.dev)
            d = torch.empty(len(cand), device=self.dev)
            s = torch.empty(len(cand), device=self.dev, dtype=torch.int32)
            k = torch.empty(len(cand), device=self.dev, dtype=torch.int32)
            self.res.point_query(tp, d, s, out_kind=k)
            ok = ((d >= SPAWN_CLEARANCE) & ((k == 1) | (k == 2))).cpu().numpy()
            found = np.concatenate([found, cand[ok]])
            if len(found) >= self.actors:
                return torch.from_numpy(np.ascontiguousarray(found[: self.actors])).to(self.dev)
        raise RuntimeError("could not find free spawn positions")

    def step(self) -> None:
        """One batched step: kinematics, rays from poses, trace, post-pass, collision revert."""
        torch = self.torch
        prev_pos = self.pos.clone()
        prev_yaw = self.yaw.clone()
        # forward of yaw psi: R_y(psi) (0, 0, -1) = (-sin psi, 0, -cos psi)
        self.yaw.add_(self.actions[:, 3] * (DT * YAW_RATE))
        fwd = torch.stack((-torch.sin(self.yaw), torch.zeros_like(self.yaw), -torch.cos(self.yaw)), 1)
        self.pos.add_(fwd * (self.actions[:, 0:1] * (DT * MAX_SPEED)))
        torch.maximum(self.pos, self.bmin, out=self.pos)
        torch.minimum(self.pos, self.bmax, out=self.pos)
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


def run_iteration(words, bbox_min, bbox_max, *, actors: int, steps: int, warmup_steps: int, azimuth_bins: int,
                  elevation_bins: int, max_distance: float, sdf_max_steps: int, seed: int) -> dict[str, Any]:
    h = ObservationHarness(words, bbox_min, bbox_max, actors, azimuth_bins, elevation_bins, max_distance,
                           sdf_max_steps, seed=seed)
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
    ap.add_argument("--gmdag-file", required=True, help="Path to compiled .gmdag world cache")
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

    asset = load_gmdag_asset(args.gmdag_file)
    runs = [run_iteration(asset.nodes, asset.bbox_min, asset.bbox_max, actors=args.actors, steps=args.steps,
                          warmup_steps=args.warmup_steps, azimuth_bins=args.azimuth_bins,
                          elevation_bins=args.elevation_bins, max_distance=args.max_distance,
                          sdf_max_steps=args.sdf_max_steps, seed=args.seed + r)
            for r in range(args.repeats)]
    sps = [r["measured_sps"] for r in runs]
    best = runs[sorted(range(len(runs)), key=lambda i: sps[i])[len(runs) // 2]]
    summary = {
        "profile": "bench-sdfdag",
        "gmdag_file": str(Path(args.gmdag_file).expanduser()),
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
