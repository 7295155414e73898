"""The benchmark's workloads, shared by ``bench.py`` and the GPU parity tests.

Five workloads, each a seeded procedural scene set with seeded rays:

* ``box_room``  — one 10 x 4 x 10 m room with 16 spheres at 64^3; 1 env x 64 x 16
  rays, max 64 steps, traced at hit epsilon 0.01 (the reference's compile-time
  ``kHitEpsilon``, ``projects/torch-sdf/cpp_src/kernel.cuh:7``) and 1e-3;
* ``cluttered`` — a 20 x 5 x 20 m volume with 120 boxes and 80 spheres at 128^3;
  4 envs x 256 x 48 rays, max 128 steps;
* ``rooms``     — a 10 x 10 grid of 4 m rooms at 512^3; 64 envs x 256 x 48 rays
  from 1.5 m height, max 256 steps;
* ``corpus``    — 16 scenes at 1024^3 (seeds 100..115, even: cluttered, odd:
  rooms), all resident; 1024 envs with seeded scene ids x 256 x 48 rays
  (12,582,912 per step), max 256 steps;
* ``observation walk`` — the corpus traced from per-env poses, fused with the
  post-pass (fp16 ``(env, 1, 48, 256)`` depth, per-env statistics) and four point
  queries per env, for 128 seeded random-walk steps.

Rays follow the reference's sensor layout (``build_spherical_ray_directions``,
``projects/environment/src/navi_environment/backends/sdfdag_backend.py:205-221``,
yaw-rotated as at ``:1300-1312``). Max distance is 30 m throughout.
"""

from __future__ import annotations

import concurrent.futures as cf
import math
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import scenes as S

AZ, EL = 256, 48
MAX_DISTANCE = 30.0
CORPUS_SEEDS = tuple(range(100, 116))
CORPUS_RESOLUTION = 1024
CORPUS_ENVS = 1024
CORPUS_MAX_STEPS = 256
CORPUS_RAY_SEED = 4
WALK_SEED = 5
WALK_STEPS = 128
POINTS_PER_ENV = 4  # the proposed move and three probes
CLEARANCE = 0.15    # the reference's collision clearance (sdfdag_backend.py:38)


@dataclass(frozen=True)
class SingleSceneConfig:
    """One scene, ``envs`` envs of ``az x el`` rays from seeded free-space origins."""

    name: str
    family: str  # box_room | cluttered | rooms
    seed: int
    resolution: int
    envs: int
    az: int
    el: int
    max_steps: int
    hit_epsilons: tuple[float, ...] = (0.01,)

    def scene(self) -> S.Scene:
        return getattr(S, self.family)(seed=self.seed, resolution=self.resolution)

    def describe(self) -> str:
        return (f"{self.envs} env{'s' if self.envs > 1 else ''} x {self.az}x{self.el} rays, {self.family} "
                f"@{self.resolution}^3 (seed {self.seed}), max {self.max_steps} steps")


SMALL_CONFIGS = (
    SingleSceneConfig("box_room_64", "box_room", 1, 64, 1, 64, 16, 64, (0.01, 1e-3)),
    SingleSceneConfig("cluttered_128", "cluttered", 2, 128, 4, 256, 48, 128),
    SingleSceneConfig("rooms_512", "rooms", 3, 512, 64, 256, 48, 256),
)


def single_scene_rays(cfg: SingleSceneConfig, scene: S.Scene) -> tuple[np.ndarray, np.ndarray]:
    """Origins and directions ``[envs, az*el, 3]`` float32 (rng seeded by the env count)."""
    rng = np.random.default_rng(cfg.envs)
    origins = scene.free_origins(rng, cfg.envs)
    dirs = S.world_directions(S.canonical_directions(cfg.az, cfg.el), rng.uniform(0, 2 * math.pi, cfg.envs))
    o = np.ascontiguousarray(np.broadcast_to(origins[:, None, :], dirs.shape))
    return o, dirs


def scene_cache_dir(root: Path) -> Path | None:
    """Where compiled corpus scenes are kept (``NAVI_SCENE_CACHE``; "off" disables)."""
    d = os.environ.get("NAVI_SCENE_CACHE", str(root / ".scene_cache"))
    if d in ("", "0", "off"):
        return None
    p = Path(d)
    p.mkdir(parents=True, exist_ok=True)
    return p


def build_corpus(seeds=CORPUS_SEEDS, resolution: int = CORPUS_RESOLUTION, threads_total: int = 8,
                 cache: Path | None = None) -> list[S.Scene]:
    """Compile the corpus scenes (four at a time, the threads split among them)."""
    corpus = [S.corpus_scene(int(s), resolution) for s in seeds]
    per = max(1, threads_total // 4)

    def work(sc_seed):
        sc, seed = sc_seed
        path = cache / f"{sc.name}_{seed}_{resolution}.npy" if cache else None
        if path is not None and path.exists():
            sc.words = np.load(path)
        else:
            sc.compile(threads=per)
            if path is not None:
                np.save(path, sc.words)
        return sc

    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        return list(ex.map(work, zip(corpus, seeds)))


def corpus_rays(corpus: list[S.Scene], n_envs: int = CORPUS_ENVS, seed: int = CORPUS_RAY_SEED):
    """Seeded scene ids ``[E]`` int32, free-space origins ``[E, 3]`` (room grids at 1.5 m),
    yaws ``[E]`` and the local direction table ``[AZ*EL, 3]``."""
    rng = np.random.default_rng(seed)
    env_scene = rng.integers(0, len(corpus), n_envs).astype(np.int32)
    yaw = rng.uniform(0.0, 2.0 * math.pi, n_envs)
    origins = np.empty((n_envs, 3), np.float32)
    for s in range(len(corpus)):
        idx = np.flatnonzero(env_scene == s)
        if idx.size:
            origins[idx] = corpus[s].free_origins(rng, idx.size)
    return env_scene, origins, yaw, S.canonical_directions(AZ, EL)


def corpus_oracle_inputs(corpus: list[S.Scene]):
    """The corpus as the oracle's multi-scene call takes it: word pool, per-scene
    word offsets and counts, and bounds ``[n, 6]``."""
    pool = np.concatenate([c.words for c in corpus])
    base = np.cumsum([0] + [c.words.size for c in corpus[:-1]]).astype(np.uint64)
    nw = np.array([c.words.size for c in corpus], np.uint64)
    bounds = np.array([c.bbox_min_list + c.bbox_max for c in corpus], np.float32)
    return pool, base, nw, bounds


class ObservationWalk:
    """The observation step, repeated for seeded random-walk poses: each env's rays are
    generated in the tracer from its pose (``navi_trace_relaid_poses``), then one launch
    (``navi_observe``) packs the fp16 ``(env, 1, El, Az)`` depth, reduces the per-env
    clearance, ratios and collision flag, and answers four point-SDF queries per env (the
    proposed move, position + N(0, 0.05 m), and three probes jittered +-0.3 m). A move is
    kept when its point SDF is at least 0.15 m; yaw walks by N(0, 0.1 rad). Seeded with a
    device generator. All buffers are allocated here: a step allocates nothing in the
    tracer or the post-pass."""

    def __init__(self, res, env_scene, origins_env, yaw_env, steps: int = WALK_STEPS, *,
                 max_steps: int = CORPUS_MAX_STEPS, max_distance: float = MAX_DISTANCE, seed: int = WALK_SEED):
        import torch

        dev = res.device
        self.res, self.steps, self.max_steps, self.max_distance = res, steps, max_steps, max_distance
        E = int(np.asarray(origins_env).shape[0])
        self.E, self.R = E, AZ * EL
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.env_scene = env_scene if isinstance(env_scene, torch.Tensor) else torch.from_numpy(
            np.asarray(env_scene, np.int32)).to(dev)
        self.pos = torch.from_numpy(np.ascontiguousarray(origins_env, np.float32)).to(dev)
        self.yaw = torch.from_numpy(np.asarray(yaw_env, np.float32)).to(dev)
        self.local = torch.from_numpy(S.canonical_directions(AZ, EL)).to(dev)
        n = max(1, steps)
        self.dpos = torch.randn((n, E, 3), generator=gen, device=dev) * 0.05
        self.dyaw = torch.randn((n, E), generator=gen, device=dev) * 0.1
        self.jitter = torch.rand((n, E, 3, 3), generator=gen, device=dev) * 0.6 - 0.3
        self.pscene = self.env_scene.repeat_interleave(POINTS_PER_ENV)
        self.rot = torch.empty((E, 2), device=dev)
        self.pts = torch.empty((E, POINTS_PER_ENV, 3), device=dev)
        self.out_d = torch.empty((E, self.R), device=dev)
        self.out_s = torch.empty((E, self.R), device=dev, dtype=torch.int32)
        self.depth16 = torch.empty((E, 1, EL, AZ), device=dev, dtype=torch.float16)
        self.stats = torch.empty((E, 5), device=dev)
        self.collision = torch.empty((E,), device=dev, dtype=torch.int32)
        self.pd = torch.empty((POINTS_PER_ENV * E,), device=dev)
        self.ps = torch.empty((POINTS_PER_ENV * E,), device=dev, dtype=torch.int32)
        self.pk = torch.empty((POINTS_PER_ENV * E,), device=dev, dtype=torch.int32)

    def trace(self) -> None:
        import torch

        torch.stack((torch.cos(self.yaw), torch.sin(self.yaw)), 1, out=self.rot)
        self.res.cast_rays_poses(self.env_scene, self.local, self.pos, self.rot, self.out_d, self.out_s,
                                 self.max_steps, self.max_distance, elevation_bins=EL)

    def observe(self) -> None:
        self.res.observe(self.out_d, AZ, EL, self.max_distance, out_depth_f16=self.depth16, out_stats=self.stats,
                         out_collision=self.collision, points=self.pts.view(-1, 3), point_scene=self.pscene,
                         point_distances=self.pd, point_semantics=self.ps, point_kind=self.pk)

    def step(self, k: int) -> None:
        import torch

        self.trace()
        self.pts[:, 0] = self.pos + self.dpos[k]
        self.pts[:, 1:] = self.pos[:, None, :] + self.jitter[k]
        self.observe()
        keep = self.pd.view(self.E, POINTS_PER_ENV)[:, 0] >= CLEARANCE
        self.pos.copy_(torch.where(keep[:, None], self.pts[:, 0], self.pos))
        self.yaw.add_(self.dyaw[k])

    def explicit_rays(self) -> tuple[np.ndarray, np.ndarray]:
        """The rays of the current poses as origins / directions ``[E, R, 3]`` (host),
        built with the tracer's own operation order from the same cos / sin values."""
        c = self.rot[:, 0].cpu().numpy()[:, None]
        s = self.rot[:, 1].cpu().numpy()[:, None]
        loc = self.local.cpu().numpy()
        d = np.empty((self.E, self.R, 3), np.float32)
        d[..., 0] = loc[None, :, 0] * c + loc[None, :, 2] * s
        d[..., 1] = loc[None, :, 1]
        d[..., 2] = (-loc[None, :, 0]) * s + loc[None, :, 2] * c
        o = np.ascontiguousarray(np.broadcast_to(self.pos.cpu().numpy()[:, None, :], d.shape))
        return o, d
