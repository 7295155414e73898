"""GPU parity at the benchmark's full workloads (navi_amd/workloads.py), on the timed
kernels' own outputs: the 512^3 room grid, the 16-scene 1024^3 corpus batch and the
observation step after its 128-step random walk. Launches without step counts (the
timed ones) stage their outputs per tile in LDS; their distances and semantics are
checked as well as those of the launch that also returns step counts.

Bar: hit/miss, semantic and step count bit-exact for every ray, distance bit-exact
(the north star allows 1e-4 * max_distance; the tests assert that bound and bit
equality), and the per-ray DAG-word counts of the word-layout counting kernel
bit-exact. Observation outputs: fp16 depth within one binary16 ulp (the oracle's
torch-CPU log1p against the device's, parity of the last bit unpinned), minimum
distance and collision flag exact, ratios within 1e-6, point queries bit-exact.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

MAX_DD = 1e-4 * 30.0


def _threads() -> int:
    return min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1)


def _say(msg: str) -> None:
    print(f"[test_gpu_configs] {msg}", file=sys.stderr, flush=True)


def _assert_parity(gd, gs, gn, ref, what):
    both_nan = np.isnan(gd) & np.isnan(ref["distance"])
    assert np.array_equal(gs != 0, ref["semantic"] != 0), f"{what}: hit mask"
    assert np.array_equal(gs, ref["semantic"]), f"{what}: semantics"
    assert np.array_equal(gn, ref["steps"]), f"{what}: step counts"
    dd = np.where(both_nan, 0.0, np.abs(gd.astype(np.float64) - ref["distance"]))
    assert float(np.max(dd, initial=0.0)) <= MAX_DD, f"{what}: max |dd| {np.max(dd)}"
    bits = (gd.view(np.uint32) == ref["distance"].view(np.uint32)) | both_nan
    assert bits.all(), f"{what}: {int((~bits).sum())} distances differ in their bits"


@pytest.fixture(scope="module")
def corpus():
    from navi_amd import workloads as W

    _say("compiling the 16-scene corpus at 1024^3")
    return W.build_corpus(threads_total=_threads())


@pytest.fixture(scope="module")
def resident(gpu, corpus):
    import torch

    from navi_amd.multiscene import ResidentScenes

    return ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus], torch.device("cuda:0"))


def _small_cases():
    from navi_amd import workloads as W

    return [(c.name, eps) for c in W.SMALL_CONFIGS for eps in c.hit_epsilons]


@pytest.mark.parametrize("name,eps", _small_cases(), ids=lambda v: str(v))
def test_small_config_every_ray(gpu, name, eps):
    """The benchmark's smaller workloads with their own seeded ray sets
    (navi_amd.workloads.single_scene_rays, as bench.py times them): the 64^3 box room
    (1 env x 64x16 rays, max 64 steps) at hit epsilon 0.01 and 1e-3, the 128^3 cluttered
    volume (4 envs x 256x48, max 128) and the 512^3 room grid (64 envs x 256x48, max
    256): every ray of the timed launch shape (staged outputs where the launch stages)
    and of the launch that returns step counts, and the word counts."""
    import torch

    from navi_amd import workloads as W
    from navi_amd.multiscene import ResidentScenes

    cfg = next(c for c in W.SMALL_CONFIGS if c.name == name)
    sc = cfg.scene()
    sc.compile(threads=_threads())
    o_np, d_np = W.single_scene_rays(cfg, sc)
    E, R = d_np.shape[:2]
    dev = torch.device("cuda:0")
    res = ResidentScenes([(sc.words, sc.bbox_min_list, sc.bbox_max)], dev)
    o, d = torch.from_numpy(o_np).to(dev), torch.from_numpy(d_np).to(dev)
    es = torch.zeros(E, dtype=torch.int32, device=dev)
    out_d = torch.full((E, R), -1.0, device=dev)
    out_s = torch.full((E, R), -1, device=dev, dtype=torch.int32)
    out_n = torch.full((E, R), -1, device=dev, dtype=torch.int32)
    out_w = torch.zeros((E, R), device=dev, dtype=torch.int32)
    what = f"{name} eps {eps:g}"
    _say(f"{what}: {E * R} rays, relaid kernel")
    for _ in range(3):  # the timed launch shape: no step counts (outputs staged where the launch stages)
        res.cast_rays(es, o, d, out_d, out_s, cfg.max_steps, W.MAX_DISTANCE, hit_epsilon=eps, elevation_bins=cfg.el)
    torch.cuda.synchronize()
    staged_d, staged_s = out_d.cpu().numpy(), out_s.cpu().numpy()
    res.cast_rays(es, o, d, out_d, out_s, cfg.max_steps, W.MAX_DISTANCE, hit_epsilon=eps, out_steps=out_n,
                  elevation_bins=cfg.el)
    torch.cuda.synchronize()
    ref = oracle.trace(sc.words, o_np, d_np, cfg.max_steps, W.MAX_DISTANCE, sc.bbox_min_list, sc.bbox_max,
                       hit_epsilon=eps, threads=_threads())
    _assert_parity(out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(), ref, what)
    _assert_parity(staged_d, staged_s, out_n.cpu().numpy(), ref, what + ", timed launch shape")
    _say(f"{what}: word-layout counting kernel")
    res.cast_rays(es, o, d, out_d, out_s, cfg.max_steps, W.MAX_DISTANCE, hit_epsilon=eps, out_words=out_w,
                  kernel="raw")
    torch.cuda.synchronize()
    assert np.array_equal(out_w.cpu().numpy().astype(np.uint64), ref["words"]), f"{what}: word counts"
    _assert_parity(out_d.cpu().numpy(), out_s.cpu().numpy(), ref["steps"], ref, what + ", word-layout kernel")
    assert (ref["semantic"] != 0).any()  # rays hit


def test_corpus_batch_every_ray(gpu, corpus, resident):
    """The benchmark batch itself: 1024 envs x 256x48 rays over the 16 resident scenes
    (12,582,912 rays), cost-ordered as the bench runs it, every ray against the oracle."""
    import torch

    from navi_amd import scenes as S
    from navi_amd import workloads as W

    env_scene, origins_env, yaw, local = W.corpus_rays(corpus)
    dirs = S.world_directions(local, yaw)
    origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))
    E, R = dirs.shape[:2]
    dev = resident.device
    t_es = torch.from_numpy(env_scene).to(dev)
    t_o, t_d = torch.from_numpy(origins).to(dev), torch.from_numpy(dirs).to(dev)
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    out_n = torch.full((E, R), -1, device=dev, dtype=torch.int32)
    _say(f"corpus batch: {E * R} rays; first launch measures the scene costs")
    for _ in range(3):  # the first launch measures costs, a later one adopts the order
        resident.cast_rays(t_es, t_o, t_d, out_d, out_s, W.CORPUS_MAX_STEPS, W.MAX_DISTANCE, elevation_bins=W.EL)
        torch.cuda.synchronize()
    assert resident.scene_cost is not None
    # the timed launch as the bench runs it (no step counts: outputs staged per tile)
    out_d.fill_(-1.0)
    out_s.fill_(-1)
    resident.cast_rays(t_es, t_o, t_d, out_d, out_s, W.CORPUS_MAX_STEPS, W.MAX_DISTANCE, elevation_bins=W.EL)
    torch.cuda.synchronize()
    staged_d, staged_s = out_d.cpu().numpy(), out_s.cpu().numpy()
    out_d.fill_(-1.0)
    out_s.fill_(-1)
    resident.cast_rays(t_es, t_o, t_d, out_d, out_s, W.CORPUS_MAX_STEPS, W.MAX_DISTANCE, out_steps=out_n,
                       elevation_bins=W.EL)
    torch.cuda.synchronize()
    pool, base, nw, bounds = W.corpus_oracle_inputs(corpus)
    _say("corpus batch: oracle")
    ref = oracle.trace_multi(pool, base, nw, bounds, env_scene, origins, dirs, W.CORPUS_MAX_STEPS, W.MAX_DISTANCE,
                             threads=_threads())
    _assert_parity(out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(), ref, "corpus batch")
    _assert_parity(staged_d, staged_s, out_n.cpu().numpy(), ref, "corpus batch, staged outputs")
    assert set(np.unique(env_scene).tolist()) == set(range(len(corpus)))


def test_observation_walk_last_step(gpu, corpus, resident):
    """The observation step after the 128-step random walk: the last step's rays (from
    poses), fp16 depth, per-env statistics and collision flags, and its 4096 point
    queries, each against the oracle."""
    import torch

    from navi_amd import workloads as W

    env_scene, origins_env, yaw, _local = W.corpus_rays(corpus)
    walk = W.ObservationWalk(resident, env_scene, origins_env, yaw)
    _say(f"observation walk: {walk.steps} steps")
    for k in range(walk.steps):
        walk.step(k)
    walk.trace()
    walk.pts[:, 0] = walk.pos
    walk.pts[:, 1:] = walk.pos[:, None, :] + walk.jitter[-1]
    walk.observe()
    torch.cuda.synchronize()
    E, R = walk.E, walk.R
    o_np, d_np = walk.explicit_rays()
    # rays from poses, steps from the same kernel (pose entry point) with out_steps
    out_n = torch.full((E, R), -1, device=resident.device, dtype=torch.int32)
    cd = torch.empty((E, R), device=resident.device)
    cs = torch.empty((E, R), device=resident.device, dtype=torch.int32)
    resident.cast_rays_poses(walk.env_scene, walk.local, walk.pos, walk.rot, cd, cs, W.CORPUS_MAX_STEPS,
                             W.MAX_DISTANCE, out_steps=out_n, elevation_bins=W.EL)
    torch.cuda.synchronize()
    gd, gs = walk.out_d.cpu().numpy(), walk.out_s.cpu().numpy()
    assert np.array_equal(cd.cpu().numpy().view(np.uint32), gd.view(np.uint32))
    pool, base, nw, bounds = W.corpus_oracle_inputs(corpus)
    _say("observation walk: oracle")
    ref = oracle.trace_multi(pool, base, nw, bounds, env_scene, o_np, d_np, W.CORPUS_MAX_STEPS, W.MAX_DISTANCE,
                             threads=_threads())
    _assert_parity(gd, gs, out_n.cpu().numpy(), ref, "observation step trace")

    want = oracle.observe(ref["distance"], W.AZ, W.EL, W.MAX_DISTANCE)
    got16 = walk.depth16.cpu().numpy().view(np.uint16).astype(np.int32)
    ulps = np.abs(got16 - want["depth16"].view(np.uint16).astype(np.int32))
    assert int(ulps.max()) <= 1, f"fp16 depth off by {int(ulps.max())} ulps"
    stats = walk.stats.cpu().numpy()
    assert np.array_equal(stats[:, 0].view(np.uint32), want["stats"][:, 0].view(np.uint32)), "min distance"
    assert float(np.abs(stats[:, 1:] - want["stats"][:, 1:]).max()) <= 1e-6, "ratios"
    assert np.array_equal(walk.collision.cpu().numpy(), want["collision"]), "collision flags"

    pts = walk.pts.view(-1, 3).cpu().numpy()
    pscene = walk.pscene.cpu().numpy()
    pd, ps, pk = walk.pd.cpu().numpy(), walk.ps.cpu().numpy(), walk.pk.cpu().numpy()
    assert pts.shape[0] == W.POINTS_PER_ENV * E == 4096
    for s, c in enumerate(corpus):
        idx = np.flatnonzero(pscene == s)
        if idx.size == 0:
            continue
        q = oracle.point_query(c.words, pts[idx], c.bbox_min_list, c.bbox_max)
        same = (pd[idx].view(np.uint32) == q["distance"].view(np.uint32)) | (np.isnan(pd[idx]) & np.isnan(q["distance"]))
        assert same.all(), f"scene {s}: point distances"
        assert np.array_equal(ps[idx], q["semantic"]) and np.array_equal(pk[idx], q["kind"]), f"scene {s}"
    # the walk moved most envs and kept them in free space
    assert (pk == 1).any() or (pk == 2).any()
