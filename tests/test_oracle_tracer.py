"""Pins of the CPU tracer oracle (oracle/trace_oracle.c), no GPU.

* the ten known answers held by projects/torch-sdf/tests/test_sphere_tracing.py:683-949
  (tests/golden/known_answers.json);
* closed forms: void-cell exits derived by hand, leaf accumulation k * fp16(d), the slab
  distance of projects/contracts/src/navi_contracts/testing/oracle_box.py:115-160 within
  the reference's tolerance 5h + 0.02 (test_analytical_raycasting.py:116);
* a cache-free brute-force march (semantics of test_sphere_tracing.py:121-178), which must
  agree with the cached march on every ray whose samples never land on a cached box face;
* invariants: determinism, thread-count independence, hit => last distance < eps,
  outside start => distance >= 1000.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests import scene_fixtures as sf

GOLDEN = Path(__file__).with_name("golden") / "known_answers.json"
CASES = json.loads(GOLDEN.read_text())["cases"]


def _words(case):
    return np.array([int(w, 16) for w in case["words"]], dtype=np.uint64)


@pytest.mark.parametrize("case", CASES, ids=lambda c: c["name"])
def test_known_answers(case):
    r = oracle.trace(_words(case), np.array(case["origins"], np.float32),
                     np.array(case["dirs"], np.float32), case["max_steps"], case["max_distance"],
                     case["bbox_min"], case["bbox_max"])
    for i, e in enumerate(case["expect"]):
        assert int(r["semantic"][i]) == e["semantic"]
        if "atol" in e:
            assert abs(float(r["distance"][i]) - e["distance"]) <= e["atol"]
        else:
            assert float(r["distance"][i]) > e["distance_gt"]


def test_planted_mistake_is_caught():
    """A wrong octant bit order in a DAG (x and z swapped) must fail the octant case:
    the known answers discriminate octant layouts."""
    case = next(c for c in CASES if c["name"] == "octant_selection")
    words = _words(case).copy()
    # swap children 1 and 4 (x-bit vs z-bit) in the pointer table
    words[1 + 1], words[1 + 4] = words[1 + 4], words[1 + 1]
    r = oracle.trace(words, np.array(case["origins"], np.float32), np.array(case["dirs"], np.float32),
                     case["max_steps"], case["max_distance"], case["bbox_min"], case["bbox_max"])
    assert list(r["semantic"]) != [e["semantic"] for e in case["expect"]]


def _leaf(d, s=0):
    bits = int(np.asarray([d], np.float16).view(np.uint16)[0])
    return (1 << 63) | (s << 16) | bits


def test_leaf_accumulation_closed_form():
    """One leaf covering the domain: t = k * fp16(d) after k steps (exact in binary32
    for these values)."""
    for d in (0.25, 0.125, 0.0625, 0.375):
        for k in (1, 2, 3, 5):
            r = oracle.trace(np.array([_leaf(d, 0)], np.uint64), np.array([[0.0, 0.5, 0.5]], np.float32),
                             np.array([[1.0, 0.0, 0.0]], np.float32), k, 100.0, [0, 0, 0], [8, 8, 8])
            assert float(r["distance"][0]) == pytest.approx(k * d, abs=0)
            # the root leaf is loaded once; later samples stay inside its box (the domain)
            assert int(r["steps"][0]) == k and int(r["words"][0]) == 1


def test_void_cell_exit_closed_form():
    """Root with only octant 7 present; a ray from (0.25,0.1,0.3) along +x crosses the void
    octants 0 -> 1 (both void, exits at x=0.5 then x=1.0) and leaves the unit cube."""
    words = np.array([(1 << 7) << 55 | 1, 2, _leaf(0.005, 17)], np.uint64)
    o = np.array([[0.25, 0.1, 0.3]], np.float32)
    d = np.array([[1.0, 0.0, 0.0]], np.float32)
    r1 = oracle.trace(words, o, d, 1, 10.0, [0, 0, 0], [1, 1, 1])
    assert float(r1["distance"][0]) == np.float32(0.25)  # (0.5 - 0.25) / 1
    r2 = oracle.trace(words, o, d, 2, 10.0, [0, 0, 0], [1, 1, 1])
    assert float(r2["distance"][0]) == np.float32(0.75)  # + (1.0 - 0.5) / 1
    r3 = oracle.trace(words, o, d, 3, 10.0, [0, 0, 0], [1, 1, 1])
    # at x = 1.0 (on the cube face, inclusive) the void box's exit is 0 -> clamped to 1e-5
    assert float(r3["distance"][0]) == np.float32(np.float32(0.75) + np.float32(1e-5))
    # diagonal: exit is the nearest face; direction (0.6, 0.8, 0) from (0.1, 0.1, 0.2)
    o = np.array([[0.1, 0.1, 0.2]], np.float32)
    d = np.array([[0.6, 0.8, 0.0]], np.float32)
    r = oracle.trace(words, o, d, 1, 10.0, [0, 0, 0], [1, 1, 1])
    want = min((np.float32(0.5) - np.float32(0.1)) / np.float32(0.6),
               (np.float32(0.5) - np.float32(0.1)) / np.float32(0.8))
    assert float(r["distance"][0]) == float(np.float32(want))


def test_axis_epsilon_excludes_tiny_direction_components():
    """kernel.cu:66-82: components within +-1e-4 do not bound the exit."""
    words = np.array([(1 << 7) << 55 | 1, 2, _leaf(0.005, 17)], np.uint64)
    o = np.array([[0.25, 0.25, 0.25]], np.float32)
    for tiny in (1e-4, -1e-4, 5e-5):
        dv = np.array([[1.0, tiny, 0.0]], np.float32)
        r = oracle.trace(words, o, dv, 1, 10.0, [0, 0, 0], [1, 1, 1])
        assert float(r["distance"][0]) == np.float32(0.25)
    dv = np.array([[0.0, 0.0, 0.0]], np.float32)  # no axis: exit stays 1000
    r = oracle.trace(words, o, dv, 1, 1e4, [0, 0, 0], [1, 1, 1])
    assert float(r["distance"][0]) == 1000.0


def test_outside_start_reports_at_least_1000():
    scene = sf.room_with_spheres(res=32, seed=4, n_spheres=4)
    words = oracle.compile_dense(scene["grid"], scene["voxel"])
    rng = np.random.default_rng(0)
    o = rng.uniform(-50, -20, (200, 3)).astype(np.float32)
    d = rng.normal(size=(200, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    r = oracle.trace(words, o, d, 64, 30.0, scene["bmin"], scene["bmax"])
    assert (r["distance"] >= 1000.0).all() and (r["semantic"] == 0).all()


def _box_dag(res=64):
    """Unit-box fixture: box [-1,1] x [0,2] x [-1,1] (oracle_box.py:25-60), unsigned
    distance to its faces, no truncation, semantic 1 for every near-surface leaf."""
    lo = np.array([-1.0, 0.0, -1.0])
    hi = np.array([1.0, 2.0, 1.0])
    bmin, voxel = sf.cube_for_extent(lo, hi, res)
    idx = np.arange(res, dtype=np.float64)
    zz, yy, xx = np.meshgrid(idx, idx, idx, indexing="ij")
    pts = np.stack([bmin[0] + xx * voxel, bmin[1] + yy * voxel, bmin[2] + zz * voxel], -1)
    grid = np.abs(sf.box_sdf(pts, lo, hi)).astype(np.float32)
    words = oracle.compile_dense(grid, float(voxel))
    bmax = (bmin.astype(np.float64) + float(voxel) * res).tolist()
    return words, [float(v) for v in bmin], bmax, float(voxel)


def _slab_distance(o, d, lo, hi):
    """oracle_box.py:115-160 semantics: exit distance of a ray starting inside the box."""
    t_exit = math.inf
    for a in range(3):
        if abs(d[a]) < 1e-12:
            continue
        t1 = (lo[a] - o[a]) / d[a]
        t2 = (hi[a] - o[a]) / d[a]
        t_exit = min(t_exit, max(t1, t2))
    return t_exit


def test_unit_box_rays_within_reference_tolerance():
    """Centre (0,1,0): axis and diagonal rays agree with the slab distance within
    5h + 0.01 + 0.01 (test_analytical_raycasting.py:108-206) whenever they hit."""
    words, bmin, bmax, h = _box_dag()
    lo, hi = (-1.0, 0.0, -1.0), (1.0, 2.0, 1.0)
    raw = [(1, 0, 0), (-1, 0, 0), (0, 1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1),
           (1, 0, 1), (1, 0, -1), (-1, 0, 1), (-1, 0, -1), (0, 1, 1), (0, -1, -1)]
    dirs = np.array([np.array(v) / np.linalg.norm(v) for v in raw], np.float32)
    o = np.tile(np.array([0.0, 1.0, 0.0], np.float32), (len(raw), 1))
    r = oracle.trace(words, o, dirs, 128, 20.0, bmin, bmax)
    tol = 5 * h + 0.02
    hits = 0
    for i, dv in enumerate(dirs):
        if r["semantic"][i] != 0:
            hits += 1
            assert abs(float(r["distance"][i]) - _slab_distance(o[i], dv, lo, hi)) < tol
    assert hits >= len(raw) // 2


def test_cache_free_march_agrees_off_faces():
    """Every ray whose samples never touch a cached box face gives identical results
    with and without the traversal caches (kernel.cu:114,120,265)."""
    scene = sf.room_with_spheres(res=64, seed=2)
    words = oracle.compile_dense(scene["grid"], scene["voxel"])
    rng = np.random.default_rng(5)
    n = 3000
    o = rng.uniform(np.array(scene["bmin"]) + 0.5, np.array(scene["bmax"]) - 0.5, (n, 3)).astype(np.float32)
    d = rng.normal(size=(n, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    a = oracle.trace(words, o, d, 96, 30.0, scene["bmin"], scene["bmax"])
    b = oracle.trace_nocache(words, o, d, 96, 30.0, scene["bmin"], scene["bmax"])
    clean = b["touch"] == 0
    assert clean.sum() > n // 4
    same = (a["semantic"] == b["semantic"]) & (a["steps"] == b["steps"]) & (
        a["distance"].view(np.uint32) == b["distance"].view(np.uint32))
    assert same[clean].all()


def test_invariants_and_thread_independence():
    scene = sf.room_with_spheres(res=64, seed=3)
    words = oracle.compile_dense(scene["grid"], scene["voxel"])
    rng = np.random.default_rng(8)
    origin = sf.free_origin(scene, rng)
    dirs = oracle.yaw_rotate(oracle.ray_directions(64, 16), [0.7])[0]
    o = np.broadcast_to(origin, dirs.shape).copy()
    r1 = oracle.trace(words, o, dirs, 64, 30.0, scene["bmin"], scene["bmax"], threads=1)
    r8 = oracle.trace(words, o, dirs, 64, 30.0, scene["bmin"], scene["bmax"], threads=8)
    for k in ("distance", "semantic", "steps", "words"):
        assert np.array_equal(r1[k], r8[k])
    hit = r1["semantic"] != 0
    # a hit stops at the sample whose leaf distance was below eps: one more step with
    # max_steps = steps reproduces the same (t, sem)
    assert (r1["steps"][hit] >= 1).all()
    assert (r1["steps"] <= 64).all()


def _case(name):
    return next(c for c in CASES if c["name"] == name)


def _half(bits):
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def test_point_query_closed_forms():
    """Answers derived by hand on the reference's own fixture DAGs
    (test_sphere_tracing.py:783-877,926-949): outside the box (1000, 0, kind 0), the
    faces themselves inside (inclusive test, kernel.cu:108-112); a pruned octant is a
    void of side 0.5 (bound 0.5 * 1.7321, kind 2); present octants are their leaves'
    fp16 distance and semantic (kind 1), the child chosen by popcount of the lower mask
    bits (kernel.cu:192-198)."""
    box = ([0.0, 0.0, 0.0], [1.0, 1.0, 1.0])
    octants = np.array([[0.25 + 0.5 * (k & 1), 0.25 + 0.5 * ((k >> 1) & 1), 0.25 + 0.5 * (k >> 2)]
                        for k in range(8)], np.float32)
    # octant_selection: all eight octants present, leaf k has semantic k + 1, distance 0x1d1f
    r = oracle.point_query(_words(_case("octant_selection")), octants, *box)
    assert r["kind"].tolist() == [1] * 8 and r["semantic"].tolist() == list(range(1, 9))
    assert (r["distance"] == np.float32(_half(0x1D1F))).all()
    # void_macro_cells: only octant 7 present (mask 0x80), its leaf semantic 0x11
    r = oracle.point_query(_words(_case("void_macro_cells")), octants, *box)
    assert r["kind"].tolist() == [2] * 7 + [1]
    assert (r["distance"][:7] == np.float32(0.5 * 1.7321)).all() and (r["semantic"][:7] == 0).all()
    assert r["semantic"][7] == 0x11 and r["distance"][7] == np.float32(_half(0x1D1F))
    # sparse_mask_popcount: top byte 0x25, so bits 62..55 hold mask 0x4a = octants 1, 3, 6
    # -> child slots 0, 1, 2 (semantics 11, 33, 66)
    r = oracle.point_query(_words(_case("sparse_mask_popcount")), octants, *box)
    assert r["kind"].tolist() == [2, 1, 2, 1, 2, 2, 1, 2]
    assert r["semantic"].tolist() == [0, 11, 0, 33, 0, 0, 66, 0]
    # outside the box by a hair on each side, far outside, and on the faces
    words = _words(_case("octant_selection"))
    eps = np.float32(1e-6)
    out = []
    for a in range(3):
        for v in (np.float32(0) - eps, np.float32(1) + eps, np.float32(-50), np.float32(50)):
            q = np.full(3, 0.5, np.float32)
            q[a] = v
            out.append(q)
    r = oracle.point_query(words, np.array(out), *box)
    assert (r["kind"] == 0).all() and (r["distance"] == 1000.0).all() and (r["semantic"] == 0).all()
    faces = np.array([[0, 0, 0], [1, 1, 1], [1, 0, 0.25], [0.5, 1, 0.5]], np.float32)
    r = oracle.point_query(words, faces, *box)
    assert (r["kind"] == 1).all()
    # the >= rule: on a midplane the upper octant is taken (kernel.cu:165-176)
    assert r["semantic"].tolist() == [1, 8, 2, 8]


def _query_scene():
    # truncation 2 m so that void octants of 1, 2 and 4 voxels occur (bound 1.7321 * side)
    scene = sf.room_with_spheres(res=64, seed=6, n_spheres=10, trunc=2.0)
    words = oracle.compile_dense(scene["grid"], scene["voxel"])
    rng = np.random.default_rng(3)
    lo = np.array(scene["bmin"], np.float32)
    hi = np.array(scene["bmax"], np.float32)
    pts = rng.uniform(lo - 0.5, hi + 0.5, (6000, 3)).astype(np.float32)
    return scene, words, pts


def test_point_query_agrees_with_one_step_trace():
    """The pinned tracer (known answers of test_sphere_tracing.py) at max_steps = 1 starts
    with the same fresh descent as a point query: outside the box it reports 1000; at a
    leaf its distance t = 0 + d is the leaf's distance (or a hit at t = 0); in a void cell
    the exits along +x and -x add up to the cell's side, which the query's bound divided
    by 1.7321 must equal (both cell sides are one float subtraction from exact)."""
    scene, words, pts = _query_scene()
    q = oracle.point_query(words, pts, scene["bmin"], scene["bmax"])
    assert {0, 1, 2} <= set(q["kind"].tolist())

    def one_step(direction):
        d = np.broadcast_to(np.array(direction, np.float32), pts.shape)
        return oracle.trace(words, pts, d, 1, 3000.0, scene["bmin"], scene["bmax"])

    px, mx = one_step([1, 0, 0]), one_step([-1, 0, 0])
    out = q["kind"] == 0
    assert (px["distance"][out] == 1000.0).all()
    leaf = q["kind"] == 1
    hit = leaf & (q["semantic"] != 0) & (q["distance"] < oracle.HIT_EPSILON)
    assert np.array_equal(px["distance"][leaf & ~hit], q["distance"][leaf & ~hit])
    assert (px["semantic"][leaf & ~hit] == 0).all()
    assert (px["distance"][hit] == 0.0).all() and np.array_equal(px["semantic"][hit], q["semantic"][hit])
    void = q["kind"] == 2
    side = px["distance"][void].astype(np.float64) + mx["distance"][void]
    bound_side = q["distance"][void].astype(np.float64) / np.float32(1.7321)
    assert void.sum() > 100
    assert np.allclose(side, bound_side, rtol=1e-5, atol=2e-5)
    assert set(np.round(bound_side / scene["voxel"]).astype(int).tolist()) == {1, 2, 4}


def _void_bound_violations(scene, words, pts, scale):
    """Void points whose returned bound (times ``scale``) is not below every grid sample
    of their void block: the compiler prunes an octant only when its smallest sample
    exceeds 1.7321 x its side (compiler.cpp:626,639-643)."""
    q = oracle.point_query(words, pts, scene["bmin"], scene["bmax"])
    grid, voxel = scene["grid"], scene["voxel"]
    bmin = np.array(scene["bmin"], np.float64)
    bad = checked = 0
    for i in np.flatnonzero(q["kind"] == 2):
        bound = float(q["distance"][i]) * scale
        half = int(round(float(q["distance"][i]) / 1.7321 / voxel))
        u = (pts[i].astype(np.float64) - bmin) / voxel / half
        if np.any(np.abs(u - np.round(u)) < 1e-4):  # too close to a block face to place it
            continue
        x0, y0, z0 = (np.floor(u).astype(int) * half).tolist()
        block = grid[z0:z0 + half, y0:y0 + half, x0:x0 + half]
        checked += 1
        bad += int(float(block.min()) < bound * (1.0 - 1e-5))
    return bad, checked


def test_point_query_void_bound_holds_on_the_grid():
    """Every void point's bound lies below every sample of its block in the dense grid
    the DAG was compiled from (the compiler's pruning rule, compiler.cpp:626,639-643);
    the parent's side, a plausible mistake, breaks it."""
    scene, words, pts = _query_scene()
    bad, checked = _void_bound_violations(scene, words, pts, 1.0)
    assert checked > 100 and bad == 0
    bad, checked = _void_bound_violations(scene, words, pts, 2.0)
    assert bad > 0
