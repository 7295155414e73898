"""The device record layout built on the host (relayout.cpp, part of libnavi_trace.so):
record walks against the word layout's point queries, cell tables against record walks
at every depth, record depths against brute force, and malformed, cyclic, one-leaf and
out-of-range DAGs. Imports neither torch nor a GPU runtime path, so the sanitizer run
(tests/test_sanitizers.py) executes it against an AddressSanitizer / UBSan build.
"""

from __future__ import annotations

import numpy as np
import pytest

from navi_amd import _native


def test_relayout_on_the_host():
    """The device record layout answers every point query exactly like the word layout."""
    import oracle
    from navi_amd import scenes as S

    scene = S.box_room(resolution=32)
    words = scene.compile()
    rec, root, levels = _native.relayout(words)
    assert root == 0 and levels[0] == 1 and (np.diff(levels) >= 0).all()
    rng = np.random.default_rng(3)
    pts = rng.uniform(scene.bbox_min, np.array(scene.bbox_max), (400, 3)).astype(np.float32)
    ref = oracle.point_query(words, pts, scene.bbox_min_list, scene.bbox_max)
    for i, p in enumerate(pts):
        lo = np.array(scene.bbox_min_list, np.float32)
        hi = np.array(scene.bbox_max, np.float32)
        slot = root
        while True:
            mid = ((lo + hi) * np.float32(0.5)).astype(np.float32)
            ge = p >= mid
            o = int(ge[0]) | int(ge[1]) << 1 | int(ge[2]) << 2
            lo, hi = np.where(ge, mid, lo), np.where(ge, hi, mid)
            slot = int(rec[slot][o])
            if slot == 0x7FFFFFFF:
                assert ref["kind"][i] == 2
                break
            if slot >> 31:
                assert ref["kind"][i] == 1 and ref["semantic"][i] == (slot >> 16) & 0x7FFF
                assert ref["distance"][i] == np.array([slot & 0xFFFF], np.uint16).view(np.float16)[0]
                break
    # a semantic beyond the inline slot's 15 bits needs a leaf table (navi_relayout_leaves)
    with pytest.raises(RuntimeError, match="leaf table"):
        _native.relayout(np.array([(1 << 63) | (0x9000 << 16) | 0x3C00], np.uint64))


def _walk(rec, root, cell, depth=4):
    """`depth` levels of record reads from the root along the octants of `cell`
    (x bits low, then y, then z, `depth` bits each)."""
    if root >> 31:
        return root, 0
    r = root
    m = (1 << depth) - 1
    ix, iy, iz = cell & m, (cell >> depth) & m, cell >> (2 * depth)
    for lvl in range(depth):
        b = depth - 1 - lvl
        oct_ = ((ix >> b) & 1) | ((iy >> b) & 1) << 1 | ((iz >> b) & 1) << 2
        slot = int(rec[r][oct_]) if r < rec.shape[0] else 0x7FFFFFFE
        if slot >= 0x7FFFFFFD or lvl == depth - 1:
            return (0x7FFFFFFE if slot == 0x7FFFFFFD else slot), lvl + 1
        r = slot


@pytest.mark.parametrize("case", ["room", "shallow", "malformed", "one_leaf", "offset"])
def test_depth4_cell_table_matches_record_walks(case):
    from navi_amd import scenes as S

    if case in ("room", "offset"):
        rec, root, _ = _native.relayout(S.box_room(resolution=32).compile())
    elif case == "shallow":  # leaves at depth 2: every entry ends above depth 4
        w = [(0xFF << 55) | 1] + list(range(9, 17)) + [(0xFF << 55) | 17] * 8
        w += [(1 << 63) | ((i + 1) << 16) | 0x3C00 for i in range(8)]
        rec, root, _ = _native.relayout(np.array(w, np.uint64))
    elif case == "malformed":  # child table points past the words: fault slots at depth 1
        rec, root, _ = _native.relayout(np.array([(0xFF << 55) | 5, 1, 2], np.uint64))
    else:
        rec, root, _ = _native.relayout(np.array([(1 << 63) | (3 << 16) | 0x3C00], np.uint64))
    if case == "offset":  # the scene sits at record 7 of a pool
        rec = np.concatenate([np.full((7, 8), 0x7FFFFFFF, np.uint32), np.where(rec < 0x7FFFFFFD, rec + 7, rec)])
        root += 7
    table = _native.cell_table(rec, root, 4)
    slots = table & 0xFFFFFFFF
    depths = table >> 32
    for cell in range(4096):
        slot, d = _walk(rec, root, cell)
        assert (int(slots[cell]), int(depths[cell])) == (slot, d), cell
    if case == "shallow":
        assert set(depths.tolist()) == {2}
    if case == "one_leaf":
        assert set(depths.tolist()) == {0} and set(slots.tolist()) == {root}
    if case in ("room", "offset"):
        assert (depths == 4).any() and (slots[depths == 4] < 0x7FFFFFFD).any()


@pytest.mark.parametrize("depth", [4, 5, 6, 7])
def test_cell_table_matches_record_walks(depth):
    """navi_build_cell_table at every depth against record walks (every cell up to
    depth 5, a seeded sample deeper), on a scene whose leaves lie at depths 5 to 7,
    with a pool offset."""
    from navi_amd import scenes as S

    rec, root, _ = _native.relayout(S.box_room(resolution=128, seed=3).compile())
    rec = np.concatenate([np.full((5, 8), 0x7FFFFFFF, np.uint32), np.where(rec < 0x7FFFFFFD, rec + 5, rec)])
    root += 5
    table = _native.cell_table(rec, root, depth)
    assert table.size == 8 ** depth
    cells = range(table.size) if depth <= 5 else np.random.default_rng(depth).integers(0, table.size, 20000)
    for cell in cells:
        slot, d = _walk(rec, root, int(cell), depth)
        assert (int(table[cell] & 0xFFFFFFFF), int(table[cell] >> 32)) == (slot, d), cell
    depths = table >> 32
    assert (depths == depth).any() and (depths < depth).any()
    with pytest.raises(RuntimeError, match="table depth"):
        _native.cell_table(rec, root, 8)


def _longest_chain(rec, root):
    """Brute force: longest record chain below root, None on a cycle."""
    import functools
    import sys

    sys.setrecursionlimit(10000)
    on_path = set()

    @functools.lru_cache(maxsize=None)
    def h(r):
        if r in on_path:
            raise RecursionError
        on_path.add(r)
        best = 0
        for s in rec[r]:
            s = int(s)
            if s < 0x7FFFFFFD:
                best = max(best, h(s) + 1)
        on_path.discard(r)
        return best

    try:
        return h(root)
    except RecursionError:
        return None


def _chain_words(n):
    """A chain of n internal nodes, each with one child in octant 7, ending in a leaf."""
    w = []
    for i in range(n):
        w += [(1 << 62) | (2 * i + 1), 2 * i + 2]
    w[-1] = len(w)
    return np.array(w + [(1 << 63) | (5 << 16) | 0x3C00], np.uint64)


@pytest.mark.parametrize("case", ["room", "chain31", "chain32", "shared", "cycle", "one_leaf"])
def test_record_depth(case):
    from navi_amd import scenes as S

    if case == "room":
        words = S.box_room(resolution=64).compile()
    elif case.startswith("chain"):
        words = _chain_words(int(case[5:]))
    elif case == "shared":  # a DAG whose shared child is reached at depths 1 and 2
        words = np.array([(0x03 << 55) | 1, 3, 4, (0x01 << 55) | 5, (0x01 << 55) | 6, 4, (1 << 63) | 0x3C00],
                         np.uint64)
    elif case == "cycle":
        words = np.array([(0xFF << 55) | 1] + [0] * 8, np.uint64)
    else:
        words = np.array([(1 << 63) | 0x3C00], np.uint64)
    rec, root, _ = _native.relayout(words)
    got = _native.record_depth(rec, root)
    if case == "one_leaf":
        assert got == 0
        return
    want = _longest_chain(rec, root)
    assert got == (0xFFFFFFFF if want is None else want)
    if case.startswith("chain"):
        assert got == int(case[5:]) - 1
    if case == "shared":
        assert got == 2


@pytest.mark.parametrize("n,kept", [(31, False), (32, True)])
def test_relayout_resolves_bad_children_of_shallow_scenes(n, kept):
    """A child index past the words is a fault wherever it is examined above the
    32-level limit: in a graph at most 30 records deep that is everywhere, so the
    relayout writes it as a plain fault; deeper graphs keep the distinct code."""
    words = _chain_words(n)
    words[2 * n - 1] = words.size + 5
    rec, root, _ = _native.relayout(words)
    assert _native.record_depth(rec, root) == n - 1
    assert bool((rec == 0x7FFFFFFD).any()) == kept
    assert bool((rec == 0x7FFFFFFE).any()) == (not kept)
    table = _native.cell_table(rec, root, 4)
    assert not ((table & 0xFFFFFFFF) == 0x7FFFFFFD).any()
