"""GPU parity of the drop-in tracer (navi_cast_rays via navi_amd.torch_sdf.cast_rays)
against the CPU oracle and the reference's known answers.

Bar: hit/miss and step counts bit-exact; distance within 1e-4 * max_distance
(the tests also count bit-exact distances, expected to be all of them).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests import scene_fixtures as sf

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).with_name("golden") / "known_answers.json"


def _cuda(x, dtype=None):
    import torch

    return torch.as_tensor(np.ascontiguousarray(x), dtype=dtype).cuda()


def gpu_trace(words, origins, dirs, max_steps, max_distance, bmin, bmax, res=1, hit_epsilon=0.01,
              skip=True, stream=None, kernel="auto"):
    """Run the drop-in cast_rays; returns numpy (distance, semantic, steps)."""
    import torch
    from navi_amd import torch_sdf

    o = np.asarray(origins, np.float32)
    if o.ndim == 2:
        o = o[None]
    d = np.asarray(dirs, np.float32).reshape(o.shape)
    dag = _cuda(np.asarray(words, np.uint64).view(np.int64))
    to = _cuda(o)
    td = _cuda(d)
    out_d = torch.full(o.shape[:2], -7.0, device="cuda", dtype=torch.float32)
    out_s = torch.full(o.shape[:2], -7, device="cuda", dtype=torch.int32)
    out_n = torch.full(o.shape[:2], -7, device="cuda", dtype=torch.int32)
    if stream is None:
        torch_sdf.cast_rays(dag, to, td, out_d, out_s, max_steps, max_distance, list(bmin), list(bmax),
                            res, skip, hit_epsilon=hit_epsilon, out_steps=out_n, kernel=kernel)
        torch.cuda.synchronize()
    else:
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            torch_sdf.cast_rays(dag, to, td, out_d, out_s, max_steps, max_distance, list(bmin),
                                list(bmax), res, skip, hit_epsilon=hit_epsilon, out_steps=out_n, kernel=kernel)
        stream.synchronize()
    return out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy()


def assert_parity(words, origins, dirs, max_steps, max_distance, bmin, bmax, hit_epsilon=0.01,
                  label="", kernel="auto"):
    o = np.asarray(origins, np.float32)
    d = np.asarray(dirs, np.float32)
    gd, gs, gn = gpu_trace(words, o, d, max_steps, max_distance, bmin, bmax, hit_epsilon=hit_epsilon,
                           kernel=kernel)
    ref = oracle.trace(words, o.reshape(gd.shape + (3,)), d.reshape(gd.shape + (3,)), max_steps,
                       max_distance, bmin, bmax, hit_epsilon=hit_epsilon, threads=8)
    rd, rs, rn = ref["distance"], ref["semantic"], ref["steps"]
    hit_g = gs != 0
    hit_r = rs != 0
    assert np.array_equal(hit_g, hit_r), f"{label}: hit mask differs on {np.sum(hit_g != hit_r)} rays"
    assert np.array_equal(gs, rs), f"{label}: semantics differ on {np.sum(gs != rs)} rays"
    assert np.array_equal(gn, rn), f"{label}: step counts differ on {np.sum(gn != rn)} rays"
    both_nan = np.isnan(gd) & np.isnan(rd)
    diff = np.where(both_nan, 0.0, np.abs(gd.astype(np.float64) - rd.astype(np.float64)))
    assert np.all(np.isnan(gd) == np.isnan(rd)), f"{label}: NaN pattern differs"
    tol = 1e-4 * max_distance
    assert float(np.nanmax(diff, initial=0.0)) <= tol, f"{label}: max |dd| {np.nanmax(diff)} > {tol}"
    exact = np.sum((gd.view(np.uint32) == rd.view(np.uint32)) | both_nan)
    return {"rays": gd.size, "bit_exact_distance": int(exact), "hits": int(hit_g.sum())}


def _words(case):
    return np.array([int(w, 16) for w in case["words"]], dtype=np.uint64)


@pytest.mark.parametrize("kernel", ["auto", "raw"])
@pytest.mark.parametrize("case", json.loads(GOLDEN.read_text())["cases"], ids=lambda c: c["name"])
def test_known_answers(gpu, case, kernel):
    gd, gs, gn = gpu_trace(_words(case), case["origins"], case["dirs"], case["max_steps"],
                           case["max_distance"], case["bbox_min"], case["bbox_max"], case["resolution"],
                           skip=False, kernel=kernel)
    for i, e in enumerate(case["expect"]):
        assert int(gs[0, i]) == e["semantic"], (case["name"], i)
        if "atol" in e:
            assert abs(float(gd[0, i]) - e["distance"]) <= e["atol"], (case["name"], i, gd[0, i])
        else:
            assert float(gd[0, i]) > e["distance_gt"], (case["name"], i, gd[0, i])
    assert_parity(_words(case), np.array(case["origins"])[None], np.array(case["dirs"])[None],
                  case["max_steps"], case["max_distance"], case["bbox_min"], case["bbox_max"],
                  label=case["name"], kernel=kernel)


def test_overwrites_preallocated_outputs_between_calls(gpu):
    import torch
    from navi_amd import torch_sdf

    cases = {c["name"]: c for c in json.loads(GOLDEN.read_text())["cases"]}
    first, second = cases["overwrite_first_call"], cases["overwrite_second_call"]
    o = _cuda(np.array([first["origins"]], np.float32))
    d = _cuda(np.array([first["dirs"]], np.float32))
    out_d = torch.full((1, 1), -7.0, device="cuda")
    out_s = torch.full((1, 1), -7, device="cuda", dtype=torch.int32)
    for case, want_d, want_s in ((first, 0.0, 3), (second, 0.5, 0)):
        dag = _cuda(_words(case).view(np.int64))
        torch_sdf.cast_rays(dag, o, d, out_d, out_s, case["max_steps"], case["max_distance"],
                            case["bbox_min"], case["bbox_max"], 1)
        torch.cuda.synchronize()
        assert abs(float(out_d.item()) - want_d) <= 1e-5
        assert int(out_s.item()) == want_s


@pytest.fixture(scope="module")
def room_scene():
    scene = sf.room_with_spheres(res=64, seed=1)
    scene["words"] = oracle.compile_dense(scene["grid"], scene["voxel"])
    return scene


@pytest.mark.parametrize("kernel", ["auto", "raw"])
@pytest.mark.parametrize("hit_epsilon", [0.01, 1e-3])
def test_room_scene_panorama_parity(gpu, room_scene, hit_epsilon, kernel):
    """Config-1 shape: 1 env x 64 az x 16 el from a free-space origin, 64 steps, 30 m."""
    rng = np.random.default_rng(1)
    origin = sf.free_origin(room_scene, rng)
    dirs = oracle.yaw_rotate(oracle.ray_directions(64, 16), rng.uniform(0, 2 * math.pi, 1))
    origins = np.broadcast_to(origin, dirs.shape).copy()
    stats = assert_parity(room_scene["words"], origins, dirs, 64, 30.0, room_scene["bmin"],
                          room_scene["bmax"], hit_epsilon=hit_epsilon, label="room", kernel=kernel)
    assert stats["hits"] > 0


def test_room_scene_many_envs_parity(gpu, room_scene):
    rng = np.random.default_rng(7)
    n_env = 24
    local = oracle.ray_directions(32, 12)
    dirs = oracle.yaw_rotate(local, rng.uniform(0, 2 * math.pi, n_env))
    origins = np.stack([np.broadcast_to(sf.free_origin(room_scene, rng), local.shape)
                        for _ in range(n_env)])
    stats = assert_parity(room_scene["words"], origins, dirs, 128, 30.0, room_scene["bmin"],
                          room_scene["bmax"], label="room-multi")
    assert stats["bit_exact_distance"] == stats["rays"]


def test_random_rays_including_outside_starts(gpu, room_scene):
    """Origins anywhere in a box 20% larger than the cube, random unit directions."""
    rng = np.random.default_rng(11)
    lo = np.array(room_scene["bmin"]) - 2.0
    hi = np.array(room_scene["bmax"]) + 2.0
    n = 4096
    o = rng.uniform(lo, hi, (1, n, 3)).astype(np.float32)
    d = rng.normal(size=(1, n, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    assert_parity(room_scene["words"], o, d, 96, 30.0, room_scene["bmin"], room_scene["bmax"],
                  label="random")


def _full_octree_words(depth, leaf_bits):
    """Full octree of the given depth, leaves carrying the given fp16 bit patterns."""
    words = [0]
    level = [0]
    for _ in range(depth):
        nxt = []
        for node in level:
            base = len(words)
            words[node] = (0xFF << 55) | base
            words.extend([0] * 8)
            for k in range(8):
                words[base + k] = len(words)
                words.append(0)
                nxt.append(len(words) - 1)
        level = nxt
    for i, node in enumerate(level):
        words[node] = (1 << 63) | (int(leaf_bits[i % len(leaf_bits)]) & 0xFFFF)
    return np.array(words, dtype=np.uint64), level


def test_exhaustive_fp16_leaf_decode(gpu):
    """Every binary16 pattern as a leaf distance: one step from the leaf's centre
    returns t = 0 + decode(bits) (semantic 0, so never a hit)."""
    depth = 6  # 8^6 = 262144 leaves >= 65536 patterns
    bits = np.arange(65536, dtype=np.uint32)
    words, _ = _full_octree_words(depth, bits)
    n = 1 << depth
    cells = np.arange(65536)
    # leaf order of the construction is breadth-first over octants: recover each
    # leaf's cell by replaying octant digits (x bit0, y bit1, z bit2, most significant first)
    ix = np.zeros(65536, np.int64)
    iy = np.zeros(65536, np.int64)
    iz = np.zeros(65536, np.int64)
    for lvl in range(depth):
        digit = (cells // (8 ** (depth - 1 - lvl))) % 8
        ix = ix * 2 + (digit & 1)
        iy = iy * 2 + ((digit >> 1) & 1)
        iz = iz * 2 + ((digit >> 2) & 1)
    centres = (np.stack([ix, iy, iz], -1) + 0.5) / n
    dirs = np.tile(np.array([1.0, 0.0, 0.0], np.float32), (65536, 1))
    gd, gs, gn = gpu_trace(words, centres[None], dirs[None], 1, 3e38,
                           [0, 0, 0], [1, 1, 1])
    want = oracle.half_to_float(bits.astype(np.uint16))
    want = want + np.float32(0.0)  # t = 0 + d
    same = (gd[0].view(np.uint32) == want.view(np.uint32)) | (np.isnan(gd[0]) & np.isnan(want))
    assert same.all(), f"{(~same).sum()} patterns decode differently, first {np.flatnonzero(~same)[:5]}"
    assert (gn == 1).all() and (gs == 0).all()


def test_out_of_range_pointer_reports_nan(gpu):
    """Malformed DAG: the child table points past the array. The reference reads
    out of bounds (undefined); the tracer reports NaN / semantic 0, like the oracle."""
    words = np.array([(0xFF << 55) | 1] + [50] * 8, dtype=np.uint64)
    o = np.array([[[0.25, 0.25, 0.25], [0.75, 0.75, 0.75]]], np.float32)
    d = np.array([[[1.0, 0.0, 0.0], [0.0, 1.0, 0.0]]], np.float32)
    gd, gs, _ = gpu_trace(words, o, d, 8, 10.0, [0, 0, 0], [1, 1, 1])
    assert np.isnan(gd).all() and (gs == 0).all()
    assert_parity(words, o, d, 8, 10.0, [0, 0, 0], [1, 1, 1], label="oob")


def test_cyclic_dag_exhausts_descent_depth(gpu):
    """A self-referencing node never reaches a leaf: after 32 levels the query
    leaves distance/semantic stale (kernel.cu:136-199); with distance 0 the ray
    never advances and runs all max_steps."""
    words = np.array([(0xFF << 55) | 1] + [0] * 8, dtype=np.uint64)
    o = np.array([[[0.3, 0.6, 0.2]]], np.float32)
    d = np.array([[[0.0, 0.0, 1.0]]], np.float32)
    gd, gs, gn = gpu_trace(words, o, d, 5, 10.0, [0, 0, 0], [1, 1, 1])
    assert gn[0, 0] == 5 and gs[0, 0] == 0 and gd[0, 0] == 0.0
    assert_parity(words, o, d, 5, 10.0, [0, 0, 0], [1, 1, 1], label="cycle")


def test_launches_on_current_stream(gpu, room_scene):
    import torch

    rng = np.random.default_rng(3)
    origin = sf.free_origin(room_scene, rng)
    dirs = oracle.ray_directions(64, 16)[None]
    origins = np.broadcast_to(origin, dirs.shape).copy()
    side = torch.cuda.Stream()
    gd, gs, gn = gpu_trace(room_scene["words"], origins, dirs, 64, 30.0, room_scene["bmin"],
                           room_scene["bmax"], stream=side)
    ref = oracle.trace(room_scene["words"], origins, dirs, 64, 30.0, room_scene["bmin"],
                       room_scene["bmax"])
    assert np.array_equal(gs, ref["semantic"]) and np.array_equal(gn, ref["steps"])


@pytest.mark.parametrize("shape", [(0, 5), (3, 0)])
def test_empty_batches(gpu, shape):
    import torch
    from navi_amd import torch_sdf

    dag = _cuda(np.array([(1 << 63)], np.uint64).view(np.int64))
    o = torch.zeros(shape + (3,), device="cuda")
    d = torch.zeros(shape + (3,), device="cuda")
    d[..., 0] = 1.0
    out_d = torch.zeros(shape, device="cuda")
    out_s = torch.zeros(shape, device="cuda", dtype=torch.int32)
    torch_sdf.cast_rays(dag, o, d, out_d, out_s, 4, 10.0, [0, 0, 0], [1, 1, 1], 1,
                        skip_direction_validation=True)
    torch.cuda.synchronize()


def test_dropin_layout_cache_follows_the_tensor(gpu, room_scene):
    """The record-layout copy behind kernel="auto" is rebuilt when the DAG tensor is
    written in place, replaced, or traced with another bbox."""
    import torch
    from navi_amd import torch_sdf

    rng = np.random.default_rng(5)
    words = room_scene["words"].copy()
    origin = sf.free_origin(room_scene, rng)
    dirs = oracle.ray_directions(32, 8)[None]
    origins = np.broadcast_to(origin, dirs.shape).copy()
    dag = _cuda(words.view(np.int64))
    o, d = _cuda(origins), _cuda(dirs)
    out_d = torch.empty((1, dirs.shape[1]), device="cuda")
    out_s = torch.empty((1, dirs.shape[1]), device="cuda", dtype=torch.int32)

    def check(w, bmin, bmax):
        torch_sdf.cast_rays(dag, o, d, out_d, out_s, 64, 30.0, bmin, bmax, 1, True)
        torch.cuda.synchronize()
        ref = oracle.trace(w, origins, dirs, 64, 30.0, bmin, bmax)
        assert np.array_equal(out_d.cpu().numpy().view(np.uint32), ref["distance"].view(np.uint32))
        assert np.array_equal(out_s.cpu().numpy(), ref["semantic"])

    bmin, bmax = list(room_scene["bmin"]), list(room_scene["bmax"])
    check(words, bmin, bmax)
    check(words, bmin, bmax)  # cached
    # every leaf of the DAG gets distance 0.25 and semantic 9: different results
    leaf = (words >> np.uint64(63)) == 1
    words[leaf] = np.uint64((1 << 63) | (9 << 16) | 0x3400)
    dag.copy_(_cuda(words.view(np.int64)))  # in-place write bumps the version counter
    check(words, bmin, bmax)
    check(words, [v - 1.0 for v in bmin], [v + 1.0 for v in bmax])
    dag = _cuda(room_scene["words"].view(np.int64))  # a new tensor
    check(room_scene["words"], bmin, bmax)
