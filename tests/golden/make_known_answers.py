"""Writes ``known_answers.json``: the tracer known-answer cases that
``projects/torch-sdf/tests/test_sphere_tracing.py:683-949`` holds.

Each case is data only — hand-packed DAG words, rays, call parameters and the
expected outputs with the tolerance the reference test asserts. The word
builders below construct the same DAGs the reference tests describe
(leaf word :26-28, internal word :36-37, single-path DAG :75-91, prefixed
uniform-leaf DAG :94-118, octant-path centre :45-72).

Run: ``python tests/golden/make_known_answers.py`` (rewrites the JSON).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np


def leaf(distance: float, semantic: int = 0) -> int:
    bits = int(np.asarray([distance], dtype=np.float16).view(np.uint16)[0])
    return (1 << 63) | ((semantic & 0xFFFF) << 16) | bits


def internal(mask: int, child_base: int) -> int:
    return ((mask & 0xFF) << 55) | (child_base & 0xFFFFFFFF)


def octant_path_centre(octants, lo, hi):
    lo, hi = list(lo), list(hi)
    for o in octants:
        for a in range(3):
            mid = (lo[a] + hi[a]) * 0.5
            if o & (1 << a):
                lo[a] = mid
            else:
                hi[a] = mid
    return [(lo[a] + hi[a]) * 0.5 for a in range(3)]


def single_path(octants, distance, semantic):
    """Internal node per level with one child (pointer slot right after it), then one leaf."""
    words: list[int] = []
    slots: list[int] = []
    for depth, o in enumerate(octants):
        ptr = len(words) + 1
        words += [internal(1 << o, ptr), 0]
        slots.append(ptr)
        if depth > 0:
            words[slots[depth - 1]] = ptr - 1
    leaf_index = len(words)
    if slots:
        words[slots[-1]] = leaf_index
    words.append(leaf(distance, semantic))
    return words


def prefixed_uniform(prefix, distance, semantic):
    """Single-child path, then a full node whose 8 children are identical leaves."""
    words: list[int] = []
    slots: list[int] = []
    for depth, o in enumerate(prefix):
        ptr = len(words) + 1
        words += [internal(1 << o, ptr), 0]
        slots.append(ptr)
        if depth > 0:
            words[slots[depth - 1]] = ptr - 1
    ptr = len(words) + 1
    words.append(internal(0xFF, ptr))
    words += [0] * 8
    if slots:
        words[slots[-1]] = ptr - 1
    base = len(words)
    for k in range(8):
        words[ptr + k] = base + k
    words += [leaf(distance, semantic)] * 8
    return words


UNIT = ([0.0, 0.0, 0.0], [1.0, 1.0, 1.0])
REF = "projects/torch-sdf/tests/test_sphere_tracing.py"


def case(name, line, words, origins, dirs, max_steps, max_distance, resolution, expect, bbox=UNIT):
    return {
        "name": name,
        "reference": f"{REF}:{line}",
        "words": [f"{w:016x}" for w in words],
        "origins": origins,
        "dirs": dirs,
        "max_steps": max_steps,
        "max_distance": max_distance,
        "bbox_min": bbox[0],
        "bbox_max": bbox[1],
        "resolution": resolution,
        # per ray: {"semantic": s, "distance": d, "atol": a} or {"semantic": s, "distance_gt": x}
        "expect": expect,
    }


def build() -> list[dict]:
    cases = []
    cases.append(case("outside_domain_is_miss", "683-694", [leaf(0.005, 9)],
                      [[2.0, 0.5, 0.5]], [[1.0, 0.0, 0.0]], 8, 2.0, 1,
                      [{"semantic": 0, "distance_gt": 2.0}]))
    cases.append(case("bounded_miss_max_steps", "697-710", [leaf(0.5, 7)],
                      [[0.5, 0.5, 0.5]], [[1.0, 0.0, 0.0]], 1, 10.0, 1,
                      [{"semantic": 0, "distance": 0.5, "atol": 1e-5}]))
    cases.append(case("accumulates_per_step", "713-726", [leaf(0.25, 4)],
                      [[0.5, 0.5, 0.5]], [[1.0, 0.0, 0.0]], 3, 10.0, 1,
                      [{"semantic": 0, "distance": 0.75, "atol": 1e-5}]))
    cases.append(case("hit_below_epsilon", "729-742", [leaf(0.005, 11)],
                      [[0.5, 0.5, 0.5]], [[0.0, 1.0, 0.0]], 4, 10.0, 1,
                      [{"semantic": 11, "distance": 0.0, "atol": 1e-6}]))
    # overwrite test (745-780): two calls on the same output buffers
    cases.append(case("overwrite_first_call", "745-765", [leaf(0.005, 3)],
                      [[0.5, 0.5, 0.5]], [[0.0, 1.0, 0.0]], 4, 10.0, 1,
                      [{"semantic": 3, "distance": 0.0, "atol": 1e-6}]))
    cases.append(case("overwrite_second_call", "767-780", [leaf(0.5, 9)],
                      [[0.5, 0.5, 0.5]], [[0.0, 1.0, 0.0]], 1, 10.0, 1,
                      [{"semantic": 0, "distance": 0.5, "atol": 1e-5}]))
    octant_words = [internal(0xFF, 1)] + list(range(9, 17)) + [leaf(0.005, s) for s in range(1, 9)]
    octant_origins = [[0.25, 0.25, 0.25], [0.75, 0.25, 0.25], [0.25, 0.75, 0.25], [0.75, 0.75, 0.25],
                      [0.25, 0.25, 0.75], [0.75, 0.25, 0.75], [0.25, 0.75, 0.75], [0.75, 0.75, 0.75]]
    cases.append(case("octant_selection", "783-823", octant_words, octant_origins,
                      [[1.0, 0.0, 0.0]] * 8, 4, 10.0, 2,
                      [{"semantic": k + 1, "distance": 0.0, "atol": 1e-6} for k in range(8)]))
    mask = (1 << 1) | (1 << 3) | (1 << 6)
    sparse_words = [internal(mask, 1), 4, 5, 6, leaf(0.005, 11), leaf(0.005, 33), leaf(0.005, 66)]
    cases.append(case("sparse_mask_popcount", "826-877", sparse_words,
                      [[0.75, 0.25, 0.25], [0.75, 0.75, 0.25], [0.25, 0.75, 0.75], [0.25, 0.25, 0.25]],
                      [[0.0, 1.0, 0.0]] * 4, 4, 10.0, 2,
                      [{"semantic": 11, "distance": 0.0, "atol": 1e-6},
                       {"semantic": 33, "distance": 0.0, "atol": 1e-6},
                       {"semantic": 66, "distance": 0.0, "atol": 1e-6},
                       {"semantic": 0, "distance_gt": 10.0}]))
    prefix = [0, 1, 1, 1]
    cases.append(case("deep_prefix_path", "880-902", prefixed_uniform(prefix, 0.015, 23),
                      [octant_path_centre(prefix + [0], *UNIT)], [[1.0, 0.0, 0.0]], 3, 1.0, 32,
                      [{"semantic": 0, "distance": 0.045, "atol": 2e-5}]))
    path = [0, 1, 1, 1, 0]
    cases.append(case("deep_leaf_reuse", "905-923", single_path(path, 0.012, 19),
                      [octant_path_centre(path, *UNIT)], [[0.0, 0.0, 1.0]], 2, 1.0, 32,
                      [{"semantic": 0, "distance": 0.024, "atol": 2e-5}]))
    cases.append(case("void_macro_cells", "926-949", [internal(1 << 7, 1), 2, leaf(0.005, 17)],
                      [[0.25, 0.25, 0.25]], [[1.0, 0.0, 0.0]], 2, 10.0, 2,
                      [{"semantic": 0, "distance": 0.75, "atol": 1e-4}]))
    return cases


if __name__ == "__main__":
    out = Path(__file__).with_name("known_answers.json")
    out.write_text(json.dumps({"cases": build()}, indent=1) + "\n")
    print(f"wrote {out}")
