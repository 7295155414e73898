"""DAG compiler: the naive oracle restatement of projects/voxel-dag/src/compiler.cpp:563-674
pinned by hand-built DAGs, and the product compiler (dense and sparse-brick paths)
checked word-for-word against it. No GPU.

Note (reference discrepancy): projects/voxel-dag/tests/test_compiler_contracts.cpp:48-78
expects a uniform 4^3 grid to compile to a root with 8 identical children, but
compiler.cpp:600-622 collapses any uniform block into one leaf before subdividing; these
tests follow compiler.cpp.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from navi_amd import scenes as S


def _half(v):
    return int(np.asarray([v], np.float16).view(np.uint16)[0])


def _leaf(v, sem):
    return (1 << 63) | (sem << 16) | _half(v)


def test_uniform_grid_collapses_to_one_leaf():
    words = oracle.compile_dense(np.full((4, 4, 4), 1.0, np.float32), 0.25)
    # index 0 reserved then overwritten by the root copy; the leaf itself at index 1
    assert list(words) == [_leaf(1.0, 0), _leaf(1.0, 0)]
    words = oracle.compile_dense(np.full((4, 4, 4), 0.1, np.float32), 0.25)
    assert list(words) == [_leaf(0.1, 1), _leaf(0.1, 1)]  # 0.1 < 2 * voxel: semantic 1


def test_two_voxel_grid_by_hand():
    """2^3 grid with distinct values: root internal with 8 leaves; each leaf dedups
    exactly (two equal samples share one word); post-order pool, root copied to 0."""
    g = np.array([0.5, 0.25, 0.25, 2.0, 0.125, 0.5, 3.0, 0.0625], np.float32).reshape(2, 2, 2)
    voxel = 0.5  # semantic iff d < 1.0; void extent 1 * 0.5 * 1.7321 = 0.866 -> 2.0, 3.0 void
    words = oracle.compile_dense(g, voxel)
    flat = g.reshape(-1)  # z-major: index = z*4 + y*2 + x = octant x|y<<1|z<<2
    expect = [0]
    leaves = {}
    kids = []
    mask = 0
    for octant in range(8):
        v = float(flat[octant])
        if v > 0.5 * 1.7321:
            continue
        mask |= 1 << octant
        w = _leaf(v, 1 if v < 1.0 else 0)
        if w not in leaves:
            leaves[w] = len(expect)
            expect.append(w)
        kids.append(leaves[w])
    node_at = len(expect)
    expect.append((mask << 55) | (node_at + 1))
    expect.extend(kids)
    expect[0] = expect[node_at]
    assert list(words) == expect


def test_all_void_node_becomes_far_leaf():
    g = np.full((2, 2, 2), 5.0, np.float32)
    g[1, 1, 1] = 6.0  # not uniform, every octant void
    words = oracle.compile_dense(g, 0.5)
    assert list(words) == [(1 << 63) | _half(5.0), (1 << 63) | _half(5.0)]


def test_quirk_fp16_encoder_maps_zero_to_infinity():
    g = np.zeros((2, 2, 2), np.float32)
    g[0, 0, 1] = 0.25
    w = oracle.compile_dense(g, 1.0, quirk_half=True)
    zero_leaf = [x for x in w if (int(x) >> 63) and (int(x) & 0xFFFF) == 0x7C00]
    assert zero_leaf, "compiler.cpp:542-560 encodes 0.0 as +inf"


def _product_dense(grid, voxel):
    lib = S._scene_lib()
    out = ctypes.c_void_p()
    n = lib.navi_dag_compile_dense(np.ascontiguousarray(grid).reshape(-1), grid.shape[0], float(voxel), 0,
                                   ctypes.byref(out))
    return S._take_words(out, int(n))


@pytest.mark.parametrize("family,res", [("box_room", 32), ("box_room", 64), ("cluttered", 64),
                                        ("rooms", 64), ("cluttered", 128)])
def test_product_compiler_matches_oracle(family, res):
    scene = getattr(S, family)(resolution=res)
    sparse = scene.compile(threads=4)
    grid = scene.dense_grid(threads=4)
    naive = oracle.compile_dense(grid, float(scene.voxel_size))
    assert np.array_equal(sparse, naive)
    assert np.array_equal(_product_dense(grid, scene.voxel_size), naive)


def test_sparse_grid_samples_match_closed_form():
    scene = S.cluttered(resolution=32)
    grid = scene.dense_grid()
    idx = np.arange(32, dtype=np.float64)
    zz, yy, xx = np.meshgrid(idx, idx, idx, indexing="ij")
    pts = np.stack([scene.bbox_min[0] + xx * float(scene.voxel_size),
                    scene.bbox_min[1] + yy * float(scene.voxel_size),
                    scene.bbox_min[2] + zz * float(scene.voxel_size)], -1)
    want = np.minimum(np.abs(scene.sdf(pts)), scene.trunc)
    assert np.max(np.abs(grid - want)) < 1e-6


def test_compile_is_deterministic_and_dedup_is_structural():
    scene = S.rooms(resolution=64)
    a = scene.compile(threads=1)
    b = scene.compile(threads=8)
    assert np.array_equal(a, b)
    # no two identical leaf words, no two identical internal nodes (mask + child list)
    seen = set()
    i = 1
    reach = [0]
    internal = {}
    while reach:
        n = reach.pop()
        w = int(a[n])
        if w >> 63 or n in internal:
            continue
        mask = (w >> 55) & 0xFF
        base = w & 0xFFFFFFFF
        kids = tuple(int(a[base + k]) for k in range(bin(mask).count("1")))
        internal[n] = (mask, kids)
        reach.extend(kids)
    keys = [v for k, v in internal.items() if k != 0]
    assert len(keys) == len(set(keys))
    leaves = [int(w) for w in a[1:] if int(w) >> 63]
    assert len(leaves) == len(set(leaves))
    del seen, i


def test_cube_convention():
    lo = np.array([-5.0, 0.0, -5.0])
    hi = np.array([5.0, 4.0, 5.0])
    bmin, voxel = S.cube_convention(lo, hi, 64)
    assert voxel == np.float32(12.0 / 64)
    assert list(bmin) == [np.float32(-6.0), np.float32(-4.0), np.float32(-6.0)]
