"""Leaf tables of the device record layout (leaves of semantic 0x7fff or above; the
format's semantic field is 16 bits, docs/GMDAG.md:215,223) and navi_scene_flags, on the
host. The record walk is checked against the oracle's word-layout point query, which
reads the reference's 16-bit field directly (kernel.cu:43-52).
"""

from __future__ import annotations

import numpy as np
import pytest

from navi_amd import _native

LEAF = np.uint64(1 << 63)


def wide_semantics(words: np.ndarray, seed: int = 5) -> np.ndarray:
    """The DAG with every non-zero leaf semantic replaced by a seeded value in
    [0x7ff0, 0xffff] (a valid DAG: only leaf words change)."""
    w = np.asarray(words, np.uint64).copy()
    leaf = (w & LEAF) != 0
    sem = (w >> np.uint64(16)) & np.uint64(0xFFFF)
    rng = np.random.default_rng(seed)
    new = rng.integers(0x7FF0, 0x10000, w.size).astype(np.uint64)
    sel = leaf & (sem != 0)
    w[sel] = (w[sel] & ~np.uint64(0xFFFF << 16)) | (new[sel] << np.uint64(16))
    return w


def walk(rec, root, leaves, p, lo, hi):
    """(kind, distance bits, semantic) of a point by record reads from the root, leaf
    words decoded through the leaf table (kernel.cu:136-199 on the record layout)."""
    slot = root
    while True:
        if slot >> 31:
            word = leaves[slot & 0xFFFF] if (slot & 0xFFFF0000) == 0xFFFF0000 else slot & 0x7FFFFFFF
            return 1, word & 0xFFFF, word >> 16
        if slot == 0x7FFFFFFF:
            return 2, None, 0
        mid = ((lo + hi) * np.float32(0.5)).astype(np.float32)
        ge = p >= mid
        o = int(ge[0]) | int(ge[1]) << 1 | int(ge[2]) << 2
        lo, hi = np.where(ge, mid, lo), np.where(ge, hi, mid)
        slot = int(rec[slot][o])


def test_leaf_table_walk_matches_the_word_layout():
    import oracle
    from navi_amd import scenes as S

    scene = S.box_room(resolution=32)
    words = wide_semantics(scene.compile())
    with pytest.raises(RuntimeError, match="leaf table"):
        _native.relayout(words)
    rec, root, _, leaves = _native.relayout_leaves(words)
    assert leaves.size > 0 and len(set(leaves.tolist())) == leaves.size  # deduplicated entries
    assert ((leaves >> 16) >= 0x7FFF).all()
    table_slots = rec[(rec & 0xFFFF0000) == 0xFFFF0000]
    assert table_slots.size > 0 and int((table_slots & 0xFFFF).max()) < leaves.size
    inline = rec[((rec >> 31) == 1) & ((rec & 0xFFFF0000) != 0xFFFF0000)]
    assert (((inline >> 16) & 0x7FFF) < 0x7FFF).all()
    rng = np.random.default_rng(3)
    lo0 = np.array(scene.bbox_min_list, np.float32)
    hi0 = np.array(scene.bbox_max, np.float32)
    pts = rng.uniform(lo0, hi0, (600, 3)).astype(np.float32)
    ref = oracle.point_query(words, pts, scene.bbox_min_list, scene.bbox_max)
    n_wide = 0
    for i, p in enumerate(pts):
        kind, dbits, sem = walk(rec, root, leaves, p, lo0.copy(), hi0.copy())
        assert kind == ref["kind"][i]
        if kind == 1:
            assert sem == ref["semantic"][i]
            assert np.array([dbits], np.uint16).view(np.float16)[0] == ref["distance"][i]
            n_wide += sem >= 0x8000
    assert n_wide > 0


def test_leaf_table_boundary_values_and_root_leaf():
    # one internal root with eight leaves: semantics around the inline limit
    sems = [0, 1, 0x7FFE, 0x7FFF, 0x8000, 0xFFFF, 0x8000, 0x7FFF]
    dists = [0x3C00, 0x3800, 0x3400, 0x3000, 0x2C00, 0x2800, 0x2C00, 0x3000]
    root = (0xFF << 55) | 1
    words = np.array([root] + [9 + k for k in range(8)]
                     + [(1 << 63) | (s << 16) | d for s, d in zip(sems, dists)], np.uint64)
    rec, root_slot, _, leaves = _native.relayout_leaves(words)
    assert root_slot == 0 and rec.shape == (1, 8)
    slots = [int(v) for v in rec[0]]
    for k in range(3):  # inline below 0x7fff
        assert slots[k] == 0x80000000 | (sems[k] << 16) | dists[k]
    for k in range(3, 8):
        assert slots[k] & 0xFFFF0000 == 0xFFFF0000
        assert int(leaves[slots[k] & 0xFFFF]) == (sems[k] << 16) | dists[k]
    assert leaves.size == 3  # (0x7fff, 0x3000), (0x8000, 0x2c00), (0xffff, 0x2800): repeats share entries
    # a one-leaf DAG of a wide semantic: the root slot is a table slot
    rec1, root1, _, leaves1 = _native.relayout_leaves(np.array([(1 << 63) | (0xABCD << 16) | 0x3C00], np.uint64))
    assert rec1.shape[0] == 0 and root1 == 0xFFFF0000 and leaves1.tolist() == [(0xABCD << 16) | 0x3C00]
    # rebasing into a pool's table moves the entry indices only
    rb, rr = _native.rebase_leaves(rec, root_slot, 10)
    assert [int(v) for v in rb[0][:3]] == slots[:3]
    assert [int(v) & 0xFFFF for v in rb[0][3:]] == [(v & 0xFFFF) + 10 for v in slots[3:]] and rr == 0


def test_leaf_table_limit():
    """More than 65536 distinct wide leaves do not fit a table: NAVI_E_LAYOUT."""
    # a full octree of depth 6 (262,144 leaves), built level by level
    levels = 6
    words: list[int] = []
    n_internal = sum(8 ** k for k in range(levels))
    first_leaf = n_internal + 8 * n_internal  # internal nodes, their child tables, then leaves
    table = n_internal
    for node in range(n_internal):
        words.append((0xFF << 55) | (table + 8 * node))
    for node in range(n_internal):
        for k in range(8):
            child = 8 * node + k + 1
            words.append(child if child < n_internal else first_leaf + child - n_internal)
    n_leaves = 8 ** levels
    i = np.arange(n_leaves, dtype=np.uint64)
    leaf_words = LEAF | ((np.uint64(0x8000) + (i >> np.uint64(16))) << np.uint64(16)) | (i & np.uint64(0xFFFF))
    w = np.concatenate([np.array(words, np.uint64), leaf_words])
    with pytest.raises(RuntimeError, match="65536"):
        _native.relayout_leaves(w)
    # 65536 distinct entries fit
    leaf_words = LEAF | (np.uint64(0x8000) << np.uint64(16)) | (i & np.uint64(0xFFFF))
    rec, root, _, leaves = _native.relayout_leaves(np.concatenate([np.array(words, np.uint64), leaf_words]))
    assert leaves.size == 65536 and rec.shape[0] == n_internal


def test_scene_flags():
    """NAVI_SCENE_NONNEG_LEAVES: set when no reachable leaf (inline or table) has its fp16
    sign bit set; unreachable records are not examined."""
    NN = _native.SCENE_NONNEG_LEAVES
    pos, neg = 0x3C00, 0xBC00  # +1.0, -1.0
    rec = np.full((3, 8), 0x7FFFFFFF, np.uint32)
    rec[0][0] = 1                                   # root -> record 1
    rec[1][3] = 0x80000000 | (5 << 16) | pos        # inline positive leaf
    rec[1][4] = 0xFFFF0000                          # table leaf 0
    rec[2][0] = 0x80000000 | (5 << 16) | neg        # unreachable negative leaf
    leaves_pos = np.array([(0x9000 << 16) | pos], np.uint32)
    leaves_neg = np.array([(0x9000 << 16) | neg], np.uint32)
    assert _native.scene_flags(rec, 0, leaves_pos) == NN
    assert _native.scene_flags(rec, 0, leaves_neg) == 0
    assert _native.scene_flags(rec, 2, leaves_pos) == 0          # from record 2 the negative leaf is reachable
    assert _native.scene_flags(rec, 0x80000000 | neg, None) == 0  # a negative one-leaf root
    assert _native.scene_flags(rec, 0xFFFF0000, leaves_pos) == NN  # a table root leaf
    rec[1][5] = 7                                   # an out-of-range record ends its branch
    assert _native.scene_flags(rec, 0, leaves_pos) == NN
    rec[1][6] = 0                                   # a cycle back to the root
    assert _native.scene_flags(rec, 0, leaves_pos) == NN
    # agrees with the compiler's scenes: every RNE-fp16 distance is non-negative
    from navi_amd import scenes as S

    scene = S.box_room(resolution=32)
    r, root, _, lv = _native.relayout_leaves(scene.compile())
    assert _native.scene_flags(r, root, lv) == NN
