"""The reference's own call patterns of ``torch_sdf.cast_rays``, driven through
``navi_amd.dropin.install()`` (``import torch_sdf`` then resolves to this package), each
checked ray for ray against the oracle:

* spawn probing (``SdfDagBackend._find_spawn_poses``,
  ``projects/environment/src/navi_environment/backends/sdfdag_backend.py:2564-2699``):
  a candidate grid over the scene box, repeated probe directions, direction validation
  left on, a step budget of max(32, min(steps, 128)), ``.cpu()`` readback;
* indexed per-actor casts into preallocated scratch slots
  (``_cast_actor_batch_tensors`` / ``_cast_actor_batch_indexed_tensors``, ``:2229-2319``,
  slots as at ``:750-769``): rays built with the reference's tensor expressions into
  views of ``[slot, :k]``, the other slot left untouched;
* a ``batch_step_tensor_actions``-shaped sequence (``:1196-1464``) on a PyTorch side
  stream: kinematics, rays into the step's scratch slot, the cast, the tensor post-pass
  and the collision revert, several steps queued back to back before one synchronize;
  once through the drop-in on one scene, once through ``ResidentScenes`` over two.

The callers' code here is a minimal restatement of those call sites (tensor shapes,
dtypes, stream use and the arguments they pass), not the reference's Python.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SPAWN_PER_AXIS, SPAWN_HEIGHTS = 5, 7            # sdfdag_backend.py:63-64
SPAWN_PROBE_AZ, SPAWN_PROBE_EL = 48, 12         # :65-66
SCRATCH_SLOTS = 2                               # :69


def _say(msg: str) -> None:
    print(f"[test_gpu_dropin_patterns] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def torch_sdf(gpu):
    import importlib

    from navi_amd import dropin

    dropin.install(force=True)
    return importlib.import_module("torch_sdf")


@pytest.fixture(scope="module")
def scene():
    from navi_amd import scenes as S

    sc = S.rooms(seed=3, resolution=128)
    sc.compile()
    return sc


def _check(sc, origins, dirs, out_d, out_s, max_steps, what):
    ref = oracle.trace(sc.words, origins, dirs, max_steps, 30.0, sc.bbox_min_list, sc.bbox_max, threads=8)
    gd = out_d.cpu().numpy()
    both_nan = np.isnan(gd) & np.isnan(ref["distance"])
    assert np.array_equal(out_s.cpu().numpy(), ref["semantic"]), f"{what}: semantics"
    assert ((gd.view(np.uint32) == ref["distance"].view(np.uint32)) | both_nan).all(), f"{what}: distances"


def test_spawn_probe_pattern(torch_sdf, scene):
    import torch

    from navi_amd import scenes as S

    dev = torch.device("cuda:0")
    sc = scene
    bmin = np.array(sc.bbox_min_list, np.float32)
    bmax = np.array(sc.bbox_max, np.float32)
    ext = bmax - bmin
    xs = np.linspace(bmin[0] + 0.2 * ext[0], bmax[0] - 0.2 * ext[0], SPAWN_PER_AXIS, dtype=np.float32)
    zs = np.linspace(bmin[2] + 0.2 * ext[2], bmax[2] - 0.2 * ext[2], SPAWN_PER_AXIS, dtype=np.float32)
    ys = np.linspace(bmin[1] + 0.2 * ext[1], bmax[1] - 0.2 * ext[1], SPAWN_HEIGHTS, dtype=np.float32)
    cand = np.array([[x, y, z] for x in xs for y in ys for z in zs], np.float32)
    probe = S.canonical_directions(SPAWN_PROBE_AZ, SPAWN_PROBE_EL)
    origins_np = np.repeat(cand[:, None, :], probe.shape[0], axis=1)
    dirs_np = np.repeat(probe[None], cand.shape[0], axis=0)
    origins = torch.from_numpy(origins_np).to(dev)
    dirs = torch.from_numpy(dirs_np).to(dev)
    out_d = torch.empty((cand.shape[0], probe.shape[0]), device=dev)
    out_s = torch.empty((cand.shape[0], probe.shape[0]), device=dev, dtype=torch.int32)
    dag = torch.from_numpy(sc.words.view(np.int64)).to(dev)
    steps = max(32, min(256, 128))
    _say(f"spawn probe: {cand.shape[0]} candidates x {probe.shape[0]} rays")
    torch_sdf.cast_rays(dag, origins, dirs, out_d, out_s, steps, 30.0, sc.bbox_min_list, list(sc.bbox_max),
                        sc.resolution)  # direction validation on, as the caller leaves it
    metric = out_d.detach().cpu().numpy().astype(np.float32, copy=False)
    metric = metric.reshape(cand.shape[0], SPAWN_PROBE_AZ, SPAWN_PROBE_EL)
    _check(sc, origins_np, dirs_np, out_d, out_s, steps, "spawn probe")
    # candidates inside walls see a hit at once; free ones see at least one open direction
    assert np.isfinite(metric).any() and (metric.reshape(cand.shape[0], -1).max(1) > 1.0).any()


def _dirs_world(torch, base, yaw, out):
    """The caller's yaw rotation into a preallocated view (sdfdag_backend.py:2246-2249)."""
    cos_yaw = torch.cos(yaw).unsqueeze(1)
    sin_yaw = torch.sin(yaw).unsqueeze(1)
    out[..., 0] = base[..., 0] * cos_yaw + base[..., 2] * sin_yaw
    out[..., 1] = base[..., 1]
    out[..., 2] = -base[..., 0] * sin_yaw + base[..., 2] * cos_yaw


def test_indexed_actor_casts_into_scratch_slots(torch_sdf, scene):
    import torch

    from navi_amd import scenes as S

    dev = torch.device("cuda:0")
    sc = scene
    A, az, el = 8, 64, 16
    R = az * el
    rng = np.random.default_rng(21)
    positions = torch.from_numpy(sc.free_origins(rng, A)).to(dev)
    yaws = torch.from_numpy(rng.uniform(0, 2 * math.pi, A).astype(np.float32)).to(dev)
    local = torch.from_numpy(S.canonical_directions(az, el)).to(dev)
    ray_origins = torch.empty((SCRATCH_SLOTS, A, R, 3), device=dev)
    ray_dirs = torch.empty_like(ray_origins)
    out_dist = torch.full((SCRATCH_SLOTS, A, R), -5.0, device=dev)
    out_sem = torch.full((SCRATCH_SLOTS, A, R), -5, device=dev, dtype=torch.int32)
    dag = torch.from_numpy(sc.words.view(np.int64)).to(dev)
    torch_sdf.prepare(dag, sc.bbox_min_list, list(sc.bbox_max))
    for slot, idx in ((0, [0, 1, 2, 3, 4, 5, 6, 7]), (1, [6, 2, 5])):
        actor_indices = torch.tensor(idx, device=dev, dtype=torch.int64)
        k = int(actor_indices.shape[0])
        yaw = yaws.index_select(0, actor_indices)
        pos = positions.index_select(0, actor_indices)
        origins, dirs_world = ray_origins[slot, :k], ray_dirs[slot, :k]
        out_d, out_s = out_dist[slot, :k], out_sem[slot, :k]
        _dirs_world(torch, local.unsqueeze(0).expand(k, -1, -1), yaw, dirs_world)
        origins.copy_(pos.unsqueeze(1).expand(-1, R, -1))
        torch_sdf.cast_rays(dag, origins, dirs_world, out_d, out_s, 128, 30.0, sc.bbox_min_list,
                            list(sc.bbox_max), sc.resolution, skip_direction_validation=True)
        torch.cuda.synchronize()
        _check(sc, origins.cpu().numpy(), dirs_world.cpu().numpy(), out_d, out_s, 128, f"slot {slot}")
    # slot 1 held 3 actors: its other rows were never written
    assert bool((out_dist[1, 3:] == -5.0).all()) and bool((out_sem[1, 3:] == -5).all())


def _post_pass(torch, out_d, az, el, max_distance):
    """The tensor post-pass core of sdfdag_backend.py:408-452: clamp, log1p depth, amin."""
    metric = out_d.reshape(-1, az, el)
    clamped = metric.clamp(min=0.0, max=max_distance)
    depth = (torch.log1p(clamped) / math.log1p(max_distance)).clamp(0.0, 1.0)
    return depth, clamped.amin(dim=(1, 2))


@pytest.mark.parametrize("resident", [False, True], ids=["dropin", "resident_scenes"])
def test_side_stream_step_sequence(torch_sdf, scene, resident):
    import torch

    from navi_amd import scenes as S
    from navi_amd.multiscene import ResidentScenes

    dev = torch.device("cuda:0")
    scenes = [scene]
    if resident:
        other = S.cluttered(seed=2, resolution=128)
        other.compile()
        scenes.append(other)
    A, az, el, steps = 6, 64, 16, 5
    R = az * el
    rng = np.random.default_rng(31)
    env_scene = np.arange(A, dtype=np.int32) % len(scenes)
    pos0 = np.concatenate([scenes[s].free_origins(rng, 1) for s in env_scene])
    positions = torch.from_numpy(pos0).to(dev)
    yaws = torch.from_numpy(rng.uniform(0, 2 * math.pi, A).astype(np.float32)).to(dev)
    local = torch.from_numpy(S.canonical_directions(az, el)).to(dev)
    ray_origins = torch.empty((SCRATCH_SLOTS, A, R, 3), device=dev)
    ray_dirs = torch.empty_like(ray_origins)
    out_dist = torch.empty((SCRATCH_SLOTS, A, R), device=dev)
    out_sem = torch.empty((SCRATCH_SLOTS, A, R), device=dev, dtype=torch.int32)
    dag = torch.from_numpy(scene.words.view(np.int64)).to(dev)
    res = None
    if resident:
        res = ResidentScenes([(s.words, s.bbox_min_list, s.bbox_max) for s in scenes], dev)
        t_es = torch.from_numpy(env_scene).to(dev)
    else:
        torch_sdf.prepare(dag, scene.bbox_min_list, list(scene.bbox_max))
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    side = torch.cuda.Stream()
    record = []
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(steps):
            slot = k % SCRATCH_SLOTS
            prev_pos, prev_yaw = positions.clone(), yaws.clone()
            # kinematics: a small seeded move and turn per actor
            positions += torch.randn((A, 3), generator=gen, device=dev) * 0.1
            yaws += torch.randn((A,), generator=gen, device=dev) * 0.2
            origins, dirs_world = ray_origins[slot], ray_dirs[slot]
            out_d, out_s = out_dist[slot], out_sem[slot]
            _dirs_world(torch, local.unsqueeze(0).expand(A, -1, -1), yaws, dirs_world)
            origins.copy_(positions.unsqueeze(1).expand(-1, R, -1))
            if resident:
                res.cast_rays(t_es, origins, dirs_world, out_d, out_s, 128, 30.0, elevation_bins=el)
            else:
                torch_sdf.cast_rays(dag, origins, dirs_world, out_d, out_s, 128, 30.0, scene.bbox_min_list,
                                    list(scene.bbox_max), scene.resolution, skip_direction_validation=True)
            _depth, min_d = _post_pass(torch, out_d, az, el, 30.0)
            collided = min_d < 0.15
            record.append((origins.clone(), dirs_world.clone(), out_d.clone(), out_s.clone(), collided.clone()))
            positions.copy_(torch.where(collided.unsqueeze(1), prev_pos, positions))
            yaws.copy_(torch.where(collided, prev_yaw, yaws))
    side.synchronize()
    _say(f"{'resident' if resident else 'drop-in'}: {steps} side-stream steps queued, checking")
    for k, (o, d, od, os_, _coll) in enumerate(record):
        o_np, d_np = o.cpu().numpy(), d.cpu().numpy()
        for s, sc in enumerate(scenes):
            envs = np.flatnonzero(env_scene == s)
            _check(sc, o_np[envs], d_np[envs], od[envs], os_[envs], 128, f"step {k} scene {s}")


def test_conversion_inside_a_call_warns(torch_sdf, scene):
    """A DAG tensor that was not prepared is converted inside ``cast_rays`` (a
    device-to-host copy that waits): the call warns and counts it; later calls with the
    same tensor, and calls with a prepared tensor, convert nothing and do not warn."""
    import warnings

    import torch

    from navi_amd import scenes as S
    from navi_amd import torch_sdf_backend as B

    dev = torch.device("cuda:0")
    sc = scene
    dirs_np = np.repeat(S.canonical_directions(16, 4)[None], 3, axis=0)
    lo, hi = np.array(sc.bbox_min_list, np.float32), np.array(sc.bbox_max, np.float32)
    pts = (lo + (hi - lo) * np.array([[0.3, 0.4, 0.5], [0.5, 0.5, 0.5], [0.7, 0.6, 0.4]], np.float32))
    origins_np = np.ascontiguousarray(np.repeat(pts.astype(np.float32)[:, None, :], dirs_np.shape[1], axis=1))
    origins = torch.from_numpy(origins_np).to(dev)
    dirs = torch.from_numpy(dirs_np).to(dev)
    out_d = torch.empty(dirs.shape[:2], device=dev)
    out_s = torch.empty(dirs.shape[:2], device=dev, dtype=torch.int32)

    def cast(dag):
        torch_sdf.cast_rays(dag, origins, dirs, out_d, out_s, 96, 30.0, sc.bbox_min_list, list(sc.bbox_max),
                            sc.resolution)

    before = B.conversion_counts()
    unprepared = torch.from_numpy(sc.words.view(np.int64).copy()).to(dev)
    with pytest.warns(B.LayoutConversionWarning, match="prepare"):
        cast(unprepared)
    _check(sc, origins_np, dirs_np, out_d, out_s, 96, "converted in the call")
    prepared = torch.from_numpy(sc.words.view(np.int64).copy()).to(dev)
    assert torch_sdf.prepare(prepared, sc.bbox_min_list, list(sc.bbox_max))
    with warnings.catch_warnings():
        warnings.simplefilter("error", B.LayoutConversionWarning)
        cast(unprepared)
        cast(prepared)
    _check(sc, origins_np, dirs_np, out_d, out_s, 96, "prepared")
    after = B.conversion_counts()
    assert after["cast_rays"] - before["cast_rays"] == 1 and after["prepare"] - before["prepare"] == 1
