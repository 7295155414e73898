"""Output staging of the fast march: a launch without step counts collects finished
rays per 64-ray tile in LDS and the wave writes each tile out in whole sectors; a
launch with step counts stores each ray's outputs itself. Both must give the same
distances and semantics bit for bit, and leave what the tracer must not write (rays
of skipped envs) untouched. Called through the C ABI on a pool of monotone scenes (the
fast march's launches), for 8x8 tiles and for linear ray order, explicit rays and
rays from poses, env orders with skipped entries, unknown scene ids, a batch with
many tiles per wave (slots evicted while rays of their tile still march) and the
no-allocation entry point; one staged launch is checked against the oracle too. Every
test runs in both launch shapes (256- and 1024-thread workgroups).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

DEPTH = 6
SENTINEL_D = -7.0


def _say(msg: str) -> None:
    print(f"[test_gpu_staging] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module", params=["wg256", "wg1024"])
def pool(gpu, request):
    """The scene pool; the module runs twice: the default launch shape for these
    small batches (256-thread workgroups, planes above the tables) and the wide one
    (1024-thread workgroups, planes two levels below the tables), forced through
    navi_set_wide_min_rays."""
    import torch

    from navi_amd import _native
    from navi_amd import scenes as S

    prev = _native.set_wide_min_rays(0 if request.param == "wg1024" else 1 << 19)
    request.addfinalizer(lambda: _native.set_wide_min_rays(prev))

    scenes = [S.rooms(seed=3, resolution=128), S.cluttered(seed=2, resolution=128), S.box_room(seed=4, resolution=64)]
    for sc in scenes:
        sc.compile()
    rtable = np.zeros(len(scenes), dtype=_native.RELAID_SCENE_DTYPE)
    recs, roff = [], 0
    for i, sc in enumerate(scenes):
        rec, root, _ = _native.relayout(sc.words)
        rec = rec.copy()
        rec[rec < 0x7FFFFFFD] += np.uint32(roff)
        rtable[i]["rec_offset"], rtable[i]["n_records"] = roff, rec.shape[0]
        rtable[i]["root_slot"] = root if root & 0x80000000 else roff + root
        rtable[i]["bbox_min"], rtable[i]["bbox_max"] = sc.bbox_min_list, sc.bbox_max
        recs.append(rec)
        roff += rec.shape[0]
    allrec = np.concatenate(recs)
    for i in range(len(scenes)):
        rtable[i]["max_depth"] = _native.record_depth(allrec, int(rtable[i]["root_slot"]))
        assert _native.nonneg_leaves(allrec, int(rtable[i]["root_slot"]))
        rtable[i]["flags"] = _native.SCENE_NONNEG_LEAVES
    tables = np.concatenate([_native.cell_table(allrec, int(rtable[i]["root_slot"]), DEPTH)
                             for i in range(len(scenes))])
    dev = torch.device("cuda:0")
    _native.device_init(dev)
    return {
        "scenes": scenes, "n_records": allrec.shape[0], "dev": dev,
        "records": torch.from_numpy(allrec.view(np.int32).reshape(-1).copy()).to(dev),
        "table": torch.from_numpy(rtable.view(np.uint8).copy()).to(dev),
        "cells": torch.from_numpy(tables.view(np.int64)).to(dev),
    }


def _rays(pool, E, az, el, seed, env_scene=None):
    from navi_amd import scenes as S

    rng = np.random.default_rng(seed)
    scenes = pool["scenes"]
    if env_scene is None:
        env_scene = rng.integers(0, len(scenes), E).astype(np.int32)
    origins_env = np.concatenate([scenes[min(int(s), len(scenes) - 1) % len(scenes)].free_origins(rng, 1)
                                  for s in env_scene])
    yaw = rng.uniform(0, 2 * np.pi, E)
    local = S.canonical_directions(az, el)
    dirs = S.world_directions(local, yaw)
    origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))
    return env_scene, origins, dirs, origins_env, yaw, local


def _launch(pool, name, env_scene, env_order, E, R, el, a, b, c=None, steps=False, max_steps=128):
    """One tracer call through the C ABI; returns (distances, semantics, steps or None)."""
    import torch

    from navi_amd import _native

    dev = pool["dev"]
    od = torch.full((E, R), SENTINEL_D, device=dev)
    os_ = torch.full((E, R), -7, device=dev, dtype=torch.int32)
    on = torch.full((E, R), -7, device=dev, dtype=torch.int32) if steps else None
    es = torch.from_numpy(np.ascontiguousarray(env_scene, np.int32)).to(dev)
    eo = torch.from_numpy(np.ascontiguousarray(env_order, np.int32)).to(dev) if env_order is not None else None
    stream = torch.cuda.current_stream(dev).cuda_stream
    lib = _native.lib()
    head = (pool["records"].data_ptr(), pool["n_records"], pool["table"].data_ptr(), len(pool["scenes"]),
            pool["cells"].data_ptr(), DEPTH, es.data_ptr(), eo.data_ptr() if eo is not None else None, E, R, el)
    tail = (od.data_ptr(), os_.data_ptr(), max_steps, 30.0, 0.01, on.data_ptr() if steps else None, stream)
    if name == "navi_trace_relaid_poses":
        args = head + (a.data_ptr(), b.data_ptr(), c.data_ptr()) + tail
    else:
        args = head + (a.data_ptr(), b.data_ptr()) + tail
    _native.check(getattr(lib, name)(*args))
    torch.cuda.synchronize()
    return od.cpu().numpy(), os_.cpu().numpy(), (on.cpu().numpy() if steps else None)


def _same(staged, direct, what):
    assert np.array_equal(staged[0].view(np.uint32), direct[0].view(np.uint32)), f"{what}: distances"
    assert np.array_equal(staged[1], direct[1]), f"{what}: semantics"


@pytest.mark.parametrize("el_arg", [16, 0], ids=["tiles_8x8", "linear"])
def test_staged_equals_direct_explicit_rays(pool, el_arg):
    import torch

    E, az, el = 24, 64, 16
    env_scene, origins, dirs, *_ = _rays(pool, E, az, el, seed=5)
    o = torch.from_numpy(origins).to(pool["dev"])
    d = torch.from_numpy(dirs).to(pool["dev"])
    _say(f"explicit rays, elevation_bins={el_arg}")
    staged = _launch(pool, "navi_trace_relaid", env_scene, None, E, az * el, el_arg, o, d)
    direct = _launch(pool, "navi_trace_relaid", env_scene, None, E, az * el, el_arg, o, d, steps=True)
    _same(staged, direct, f"el={el_arg}")
    assert (direct[2] > 0).all()
    if el_arg:
        # the staged launch against the oracle itself
        sc = pool["scenes"]
        pool_w = np.concatenate([s.words for s in sc])
        base = np.cumsum([0] + [s.words.size for s in sc[:-1]]).astype(np.uint64)
        nw = np.array([s.words.size for s in sc], np.uint64)
        bounds = np.array([s.bbox_min_list + s.bbox_max for s in sc], np.float32)
        ref = oracle.trace_multi(pool_w, base, nw, bounds, env_scene, origins, dirs, 128, 30.0, threads=8)
        assert np.array_equal(staged[0].view(np.uint32), ref["distance"].view(np.uint32))
        assert np.array_equal(staged[1], ref["semantic"])


def test_staged_equals_direct_poses(pool):
    import torch

    E, az, el = 20, 64, 16
    env_scene, _o, _d, origins_env, yaw, local = _rays(pool, E, az, el, seed=6)
    dev = pool["dev"]
    ld = torch.from_numpy(local).to(dev)
    pos = torch.from_numpy(origins_env).to(dev)
    rot = torch.from_numpy(np.stack([np.cos(yaw), np.sin(yaw)], 1).astype(np.float32)).to(dev)
    _say("rays from poses")
    staged = _launch(pool, "navi_trace_relaid_poses", env_scene, None, E, az * el, el, ld, pos, rot)
    direct = _launch(pool, "navi_trace_relaid_poses", env_scene, None, E, az * el, el, ld, pos, rot, steps=True)
    _same(staged, direct, "poses")


def test_staged_skips_and_unknown_scenes(pool):
    """env_order entries outside [0, n_envs) skip their envs: those rays keep what the
    caller put there; an unknown scene id gives NaN and semantic 0, as unstaged."""
    import torch

    E, az, el = 16, 32, 16
    env_scene, origins, dirs, *_ = _rays(pool, E, az, el, seed=7)
    env_scene = env_scene.copy()
    env_scene[[3, 11]] = [7, -2]  # unknown scenes
    order = np.arange(E, dtype=np.int32)[::-1].copy()
    order[[2, 9]] = [-1, E + 4]  # envs 13 and 6 are never traced
    o = torch.from_numpy(origins).to(pool["dev"])
    d = torch.from_numpy(dirs).to(pool["dev"])
    _say("env_order with skipped entries, unknown scene ids")
    staged = _launch(pool, "navi_trace_relaid", env_scene, order, E, az * el, el, o, d)
    direct = _launch(pool, "navi_trace_relaid", env_scene, order, E, az * el, el, o, d, steps=True)
    _same(staged, direct, "skips")
    skipped = [E - 1 - 2, E - 1 - 9]
    for e in skipped:
        assert (staged[0][e] == SENTINEL_D).all() and (staged[1][e] == -7).all(), f"env {e} was written"
    for e in (3, 11):
        assert np.isnan(staged[0][e]).all() and (staged[1][e] == 0).all()
    traced = [e for e in range(E) if e not in skipped + [3, 11]]
    assert not np.isnan(staged[0][traced]).any() and (staged[0][traced] != SENTINEL_D).all()


def test_staged_many_tiles_per_wave(pool):
    """A batch of ~11 tiles per resident wave, 256 steps: each wave's four slots are
    evicted over and over, often while long rays of the evicted tile still march."""
    import torch

    E, az, el = 400, 256, 48
    env_scene, origins, dirs, *_ = _rays(pool, E, az, el, seed=8)
    o = torch.from_numpy(origins).to(pool["dev"])
    d = torch.from_numpy(dirs).to(pool["dev"])
    _say(f"{E * az * el} rays, 256 steps")
    staged = _launch(pool, "navi_trace_relaid", env_scene, None, E, az * el, el, o, d, max_steps=256)
    direct = _launch(pool, "navi_trace_relaid", env_scene, None, E, az * el, el, o, d, steps=True, max_steps=256)
    _same(staged, direct, "many tiles")
    assert (direct[2] > 64).any()


def test_noalloc_staged_equals_direct(pool):
    import torch

    E, az, el = 12, 64, 16
    env_scene, origins, dirs, *_ = _rays(pool, E, az, el, seed=9)
    o = torch.from_numpy(origins).to(pool["dev"])
    d = torch.from_numpy(dirs).to(pool["dev"])
    _say("no-allocation entry point")
    staged = _launch(pool, "navi_trace_relaid_noalloc", env_scene, None, E, az * el, el, o, d)
    direct = _launch(pool, "navi_trace_relaid", env_scene, None, E, az * el, el, o, d, steps=True)
    _same(staged, direct, "noalloc")
