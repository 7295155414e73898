"""GPU parity of the multi-scene entry points (reference-layout kernel and the
device-layout throughput kernel) against the CPU oracle.

Bar: hit/miss, semantic and step counts bit-exact, distance within
1e-4 * max_distance (distances are expected bit-exact and counted), and the
per-ray count of DAG words the reference algorithm loads bit-exact.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.test_gpu_trace import _full_octree_words

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).with_name("golden") / "known_answers.json"


def _corpus():
    from navi_amd import scenes as S

    corpus = [S.box_room(seed=1, resolution=64), S.cluttered(seed=2, resolution=128),
              S.rooms(seed=3, resolution=128), S.cluttered(seed=5, resolution=64)]
    for c in corpus:
        c.compile()
    return corpus


@pytest.fixture(scope="module")
def corpus():
    return _corpus()


def _rays(corpus, n_envs, az, el, seed):
    from navi_amd import scenes as S

    rng = np.random.default_rng(seed)
    env_scene = rng.integers(0, len(corpus), n_envs).astype(np.int32)
    origins = np.empty((n_envs, 3), np.float32)
    for s in range(len(corpus)):
        idx = np.flatnonzero(env_scene == s)
        if idx.size:
            origins[idx] = corpus[s].free_origins(rng, idx.size)
    dirs = S.world_directions(S.canonical_directions(az, el), rng.uniform(0, 2 * math.pi, n_envs))
    o = np.ascontiguousarray(np.broadcast_to(origins[:, None, :], dirs.shape))
    return env_scene, o, dirs


def _oracle_multi(corpus_words, bounds, env_scene, o, d, max_steps, max_distance, hit_epsilon=0.01):
    base = np.cumsum([0] + [w.size for w in corpus_words[:-1]]).astype(np.uint64)
    nw = np.array([w.size for w in corpus_words], np.uint64)
    return oracle.trace_multi(np.concatenate(corpus_words), base, nw, np.asarray(bounds, np.float32),
                              env_scene, o, d, max_steps, max_distance, hit_epsilon, threads=8)


def _run(res, env_scene, o, d, max_steps, max_distance, **kw):
    import torch

    dev = res.device
    t_es = torch.from_numpy(np.ascontiguousarray(env_scene, np.int32)).to(dev)
    t_o = torch.from_numpy(np.ascontiguousarray(o)).to(dev)
    t_d = torch.from_numpy(np.ascontiguousarray(d)).to(dev)
    shape = o.shape[:2]
    out_d = torch.full(shape, -7.0, device=dev)
    out_s = torch.full(shape, -7, device=dev, dtype=torch.int32)
    out_n = torch.full(shape, -7, device=dev, dtype=torch.int32)
    out_w = torch.full(shape, -7, device=dev, dtype=torch.int32) if kw.pop("count", False) else None
    res.cast_rays(t_es, t_o, t_d, out_d, out_s, max_steps, max_distance, out_steps=out_n,
                  out_words=out_w, **kw)
    torch.cuda.synchronize()
    return (out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(),
            None if out_w is None else out_w.cpu().numpy())


def _compare(got, ref, max_distance, label):
    gd, gs, gn, gw = got
    assert np.array_equal(gs != 0, ref["semantic"] != 0), f"{label}: hit mask"
    assert np.array_equal(gs, ref["semantic"]), f"{label}: semantics"
    assert np.array_equal(gn, ref["steps"]), f"{label}: steps differ on {np.sum(gn != ref['steps'])}"
    assert np.array_equal(np.isnan(gd), np.isnan(ref["distance"])), f"{label}: NaN pattern"
    both = np.isnan(gd) & np.isnan(ref["distance"])
    dd = np.where(both, 0.0, np.abs(gd.astype(np.float64) - ref["distance"]))
    assert float(dd.max(initial=0.0)) <= 1e-4 * max_distance, f"{label}: max |dd| {dd.max()}"
    exact = (gd.view(np.uint32) == ref["distance"].view(np.uint32)) | both
    assert exact.all(), f"{label}: {np.sum(~exact)} distances not bit-exact"
    if gw is not None:
        assert np.array_equal(gw.astype(np.uint64), ref["words"]), f"{label}: word counts"


@pytest.mark.parametrize("kernel,el_bins,sort", [("raw", None, False), ("relaid", None, False),
                                                 ("relaid", 16, True), ("relaid", 16, False)])
def test_multiscene_parity(gpu, corpus, kernel, el_bins, sort):
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    assert res.relaid_ok
    env_scene, o, d = _rays(corpus, 40, 32, 16, seed=9)
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene, o, d, 192, 30.0)
    got = _run(res, env_scene, o, d, 192, 30.0, kernel=kernel, elevation_bins=el_bins,
               sort_by_scene=sort, count=(kernel == "raw"))
    _compare(got, ref, 30.0, f"{kernel}/{el_bins}/{sort}")


def test_relaid_random_rays_and_short_budgets(gpu, corpus):
    """Random origins (inside and outside the cubes) and directions, several max_steps."""
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    rng = np.random.default_rng(21)
    n_env, rays = 12, 1000
    env_scene = rng.integers(0, len(corpus), n_env).astype(np.int32)
    lo = np.array([corpus[s].bbox_min_list for s in env_scene]) - 3.0
    hi = np.array([corpus[s].bbox_max for s in env_scene]) + 3.0
    o = rng.uniform(lo[:, None, :], hi[:, None, :], (n_env, rays, 3)).astype(np.float32)
    d = rng.normal(size=(n_env, rays, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    for max_steps in (1, 7, 300):
        ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                            env_scene, o, d, max_steps, 45.0)
        _compare(_run(res, env_scene, o, d, max_steps, 45.0), ref, 45.0, f"random/{max_steps}")


@pytest.mark.parametrize("max_distance", [30.0, 999.0, 1000.0, 1500.0])
def test_relaid_signed_zero_axes_and_long_ranges(gpu, corpus, max_distance):
    """The fast march samples in a frame mirrored along each axis whose direction
    component has its sign bit set, keeps only the faces ahead of a ray (its
    samples move one way along each axis) and ends a ray at its first step
    outside the domain; it runs while the range lies below the outside-domain
    distance (1000), the general march from there on. Direction components of +0
    and -0 (axis-aligned rays, rays in coordinate planes), origins inside, outside
    and exactly on the faces of the domains, ranges on both sides of 1000: against
    the oracle."""
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    rng = np.random.default_rng(int(max_distance))
    n_env, rays = 8, 640
    env_scene = (np.arange(n_env) % len(corpus)).astype(np.int32)
    lo = np.array([corpus[s].bbox_min_list for s in env_scene], np.float32)
    hi = np.array([corpus[s].bbox_max for s in env_scene], np.float32)
    span = hi - lo
    o = rng.uniform(lo[:, None, :] - 0.05 * span[:, None, :], hi[:, None, :] + 0.05 * span[:, None, :],
                    (n_env, rays, 3)).astype(np.float32)
    free = np.stack([corpus[s].free_origins(rng, 1)[0] for s in env_scene]).astype(np.float32)
    o[:, :320] = free[:, None, :]
    # origins on a face: one coordinate exactly a domain bound
    for k in range(320, 400):
        axis, side = k % 3, (k // 3) % 2
        o[:, k, axis] = (hi if side else lo)[:, axis]
    d = rng.normal(size=(n_env, rays, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    # signed zeros: one or two components +0 or -0, and axis-aligned rays
    for k in range(0, rays, 4):
        axis = (k // 4) % 3
        d[:, k, axis] = np.float32(-0.0) if (k // 12) % 2 else np.float32(0.0)
        if k % 8 == 0:
            other = (axis + 1) % 3
            d[:, k, other] = np.float32(0.0) if (k // 24) % 2 else np.float32(-0.0)
    assert np.signbit(d[d == 0]).any() and (~np.signbit(d[d == 0])).any()
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene, o, d, 200, max_distance)
    _compare(_run(res, env_scene, o, d, 200, max_distance), ref, max_distance, f"zeros/{max_distance}")
    _compare(_run(res, env_scene, o, d, 200, max_distance, elevation_bins=16), ref, max_distance,
             f"zeros/{max_distance}/tiles")


def test_relaid_non_finite_and_extreme_rays(gpu, corpus):
    """Directions with NaN, infinite, huge (beyond 2^126, where a reciprocal
    leaves the normal range), subnormal, below-1e-4 and signed-zero components,
    and origins with NaN or infinite coordinates: the record-layout tracer
    against the oracle (NaN distances compared as NaN)."""
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    rng = np.random.default_rng(77)
    specials = [np.nan, np.inf, -np.inf, 3e38, -1e38, 1e-40, -1e-42, 5e-5, -9e-5, 0.0, -0.0, 1.0, -1.0]
    n_env, rays = 4, 256
    env_scene = (np.arange(n_env) % len(corpus)).astype(np.int32)
    free = np.stack([corpus[s].free_origins(rng, 1)[0] for s in env_scene]).astype(np.float32)
    o = np.ascontiguousarray(np.broadcast_to(free[:, None, :], (n_env, rays, 3))).astype(np.float32)
    d = rng.normal(size=(n_env, rays, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    for k in range(rays - 16):
        axis = k % 3
        d[:, k, axis] = np.float32(specials[k % len(specials)])
        if k % 5 == 0:
            d[:, k, (axis + 1) % 3] = np.float32(specials[(k // 5) % len(specials)])
    for k in range(rays - 16, rays):  # non-finite origins
        o[:, k, k % 3] = np.float32([np.nan, np.inf, -np.inf, 1e30][k % 4])
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene, o, d, 128, 30.0)
    _compare(_run(res, env_scene, o, d, 128, 30.0), ref, 30.0, "extreme")
    _compare(_run(res, env_scene, o, d, 128, 30.0, elevation_bins=16), ref, 30.0, "extreme/tiles")


def test_relaid_fast_and_general_launches_interleaved(gpu, corpus):
    """Launches on one stream alternate between scene sets the fast kernel traces
    (monotone) and ones it hands to the general kernel (a scene with negative
    leaf distances), with and without step counts and at both sides of the
    outside-domain range: every launch against the oracle, so a fast kernel's
    record of whether it traced the launch is read by its own launch's general
    kernel only."""
    from navi_amd.multiscene import ResidentScenes

    mono = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus[:2]])
    bits = np.array([0x3C00, 0xBC00, 0x2E66, 0xAE66, 0x3800], np.uint32)  # 1, -1, 0.1, -0.1, 0.5
    words, _ = _full_octree_words(3, bits)
    neg = ResidentScenes([(words, [-1.0, -1.0, -1.0], [1.0, 1.0, 1.0])])
    from navi_amd import _native

    flags = neg.relaid_table.cpu().numpy().view(np.uint32)[11]
    assert not flags & _native.SCENE_NONNEG_LEAVES  # not monotone: the general march
    rng = np.random.default_rng(5)
    env_m, o_m, d_m = _rays(corpus[:2], 6, 32, 16, seed=12)
    o_n = rng.uniform(-1.2, 1.2, (3, 512, 3)).astype(np.float32)
    d_n = rng.normal(size=(3, 512, 3))
    d_n = (d_n / np.linalg.norm(d_n, axis=-1, keepdims=True)).astype(np.float32)
    env_n = np.zeros(3, np.int32)
    ref_m = _oracle_multi([c.words for c in corpus[:2]], [c.bbox_min_list + c.bbox_max for c in corpus[:2]],
                          env_m, o_m, d_m, 128, 30.0)
    ref_n = _oracle_multi([words], [[-1.0, -1.0, -1.0, 1.0, 1.0, 1.0]], env_n, o_n, d_n, 64, 30.0)
    ref_nl = _oracle_multi([words], [[-1.0, -1.0, -1.0, 1.0, 1.0, 1.0]], env_n, o_n, d_n, 64, 1500.0)
    import torch

    dev = mono.device
    t_es = torch.from_numpy(env_m).to(dev)
    t_o = torch.from_numpy(np.ascontiguousarray(o_m)).to(dev)
    t_d = torch.from_numpy(np.ascontiguousarray(d_m)).to(dev)
    out_d = torch.empty(o_m.shape[:2], device=dev)
    out_s = torch.empty(o_m.shape[:2], device=dev, dtype=torch.int32)
    for rep in range(3):
        _compare(_run(mono, env_m, o_m, d_m, 128, 30.0, elevation_bins=16), ref_m, 30.0, f"mono/{rep}")
        _compare(_run(neg, env_n, o_n, d_n, 64, 30.0), ref_n, 30.0, f"negative/{rep}")
        # without step counts: the fast kernel stages its outputs
        mono.cast_rays(t_es, t_o, t_d, out_d, out_s, 128, 30.0, elevation_bins=16)
        torch.cuda.synchronize()
        assert np.array_equal(out_d.cpu().numpy().view(np.uint32), ref_m["distance"].view(np.uint32)), f"staged/{rep}"
        assert np.array_equal(out_s.cpu().numpy(), ref_m["semantic"]), f"staged/{rep}"
        _compare(_run(neg, env_n, o_n, d_n, 64, 1500.0), ref_nl, 1500.0, f"negative-long/{rep}")
        _compare(_run(mono, env_m, o_m, d_m, 128, 30.0), ref_m, 30.0, f"mono-linear/{rep}")


def test_unknown_scene_id_reports_nan(gpu, corpus):
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus[:2]])
    env_scene, o, d = _rays(corpus[:2], 3, 8, 8, seed=2)
    env_scene = np.array([0, 7, -1], np.int32)
    for kernel in ("raw", "relaid"):
        gd, gs, gn, _ = _run(res, env_scene, o, d, 64, 30.0, kernel=kernel)
        assert np.isnan(gd[1:]).all() and (gs[1:] == 0).all() and (gn[1:] == 0).all(), kernel
        assert not np.isnan(gd[0]).any(), kernel


@pytest.mark.parametrize("case", json.loads(GOLDEN.read_text())["cases"], ids=lambda c: c["name"])
def test_known_answers_both_kernels(gpu, case):
    from navi_amd.multiscene import ResidentScenes

    words = np.array([int(w, 16) for w in case["words"]], dtype=np.uint64)
    res = ResidentScenes([(words, case["bbox_min"], case["bbox_max"])])
    o = np.array(case["origins"], np.float32)[None]
    d = np.array(case["dirs"], np.float32)[None]
    ref = oracle.trace(words, o, d, case["max_steps"], case["max_distance"], case["bbox_min"],
                       case["bbox_max"])
    for kernel in ("raw", "relaid"):
        got = _run(res, np.zeros(1, np.int32), o, d, case["max_steps"], case["max_distance"],
                   kernel=kernel, count=(kernel == "raw"))
        _compare(got, ref, case["max_distance"], f"{case['name']}/{kernel}")
        for i, e in enumerate(case["expect"]):
            assert int(got[1][0, i]) == e["semantic"]
            if "atol" in e:
                assert abs(float(got[0][0, i]) - e["distance"]) <= e["atol"]
            else:
                assert float(got[0][0, i]) > e["distance_gt"]


def test_relaid_malformed_dags(gpu):
    """Out-of-range child table and a self-cycle: the device layout keeps the
    reference-layout kernel's fault (NaN) and depth-exhaustion (stale) results."""
    from navi_amd.multiscene import ResidentScenes

    oob = np.array([(0xFF << 55) | 1] + [50] * 8, dtype=np.uint64)
    cyc = np.array([(0xFF << 55) | 1] + [0] * 8, dtype=np.uint64)
    table_past_end = np.array([(0xFF << 55) | 5, 1, 2], dtype=np.uint64)
    scenes = [(w, [0, 0, 0], [1, 1, 1]) for w in (oob, cyc, table_past_end)]
    res = ResidentScenes(scenes)
    rng = np.random.default_rng(4)
    o = rng.uniform(-0.2, 1.2, (3, 64, 3)).astype(np.float32)
    d = rng.normal(size=(3, 64, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    env_scene = np.arange(3, dtype=np.int32)
    ref = _oracle_multi([s[0] for s in scenes], [[0, 0, 0, 1, 1, 1]] * 3, env_scene, o, d, 9, 10.0)
    for kernel in ("raw", "relaid"):
        _compare(_run(res, env_scene, o, d, 9, 10.0, kernel=kernel, count=(kernel == "raw")), ref, 10.0,
                 f"malformed/{kernel}")


def test_relaid_exhaustive_fp16_inline_leaves(gpu):
    from navi_amd.multiscene import ResidentScenes

    bits = np.arange(65536, dtype=np.uint32)
    words, _ = _full_octree_words(6, bits)
    res = ResidentScenes([(words, [0, 0, 0], [1, 1, 1])])
    cells = np.arange(65536)
    ix = np.zeros(65536, np.int64)
    iy = np.zeros(65536, np.int64)
    iz = np.zeros(65536, np.int64)
    for lvl in range(6):
        digit = (cells // (8 ** (5 - lvl))) % 8
        ix, iy, iz = ix * 2 + (digit & 1), iy * 2 + ((digit >> 1) & 1), iz * 2 + ((digit >> 2) & 1)
    o = ((np.stack([ix, iy, iz], -1) + 0.5) / 64).astype(np.float32)[None]
    d = np.tile(np.array([1.0, 0.0, 0.0], np.float32), (1, 65536, 1))
    gd, gs, gn, _ = _run(res, np.zeros(1, np.int32), o, d, 1, 3e38, kernel="relaid")
    want = oracle.half_to_float(bits.astype(np.uint16)) + np.float32(0.0)
    same = (gd[0].view(np.uint32) == want.view(np.uint32)) | (np.isnan(gd[0]) & np.isnan(want))
    assert same.all()


def test_relayout_wide_semantics_need_a_leaf_table(gpu):
    """A semantic beyond the inline slot's 15 bits: navi_relayout refuses it,
    navi_relayout_leaves puts it in the leaf table (traced in test_gpu_work_queues)."""
    from navi_amd import _native

    words = np.array([(1 << 63) | (0x9000 << 16) | 0x3C00], dtype=np.uint64)
    with pytest.raises(RuntimeError, match="leaf table"):
        _native.relayout(words)
    rec, root, _, leaves = _native.relayout_leaves(words)
    assert rec.shape[0] == 0 and root == 0xFFFF0000 and leaves.tolist() == [(0x9000 << 16) | 0x3C00]


def test_relaid_huge_domains(gpu, corpus):
    """Scene boxes with coordinates of 2^126 and more, where split planes can
    overflow to infinity and boxes stop nesting: the tracer's leaf-run shortcut
    must fall back to the full cache tests (same batch as an ordinary scene)."""
    from navi_amd.multiscene import ResidentScenes

    words = corpus[0].words
    bounds = [corpus[0].bbox_min_list + list(corpus[0].bbox_max),
              [-3e38, -3e38, -3e38, 3e38, 3e38, 3e38],
              [1.5e38, 1.5e38, 1.5e38, 3.4e38, 3.4e38, 3.4e38]]
    res = ResidentScenes([(words, b[:3], b[3:]) for b in bounds])
    rng = np.random.default_rng(17)
    n_env, rays = 6, 800
    env_scene = np.array([0, 1, 2, 1, 2, 0], np.int32)
    b = np.array(bounds, np.float64)[env_scene]
    o = rng.uniform(b[:, None, :3], b[:, None, 3:], (n_env, rays, 3)).astype(np.float32)
    o = np.where(np.isfinite(o), o, 0.0).astype(np.float32)
    d = rng.normal(size=(n_env, rays, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    for max_steps, max_distance in ((40, 3e38), (200, 30.0)):
        ref = _oracle_multi([words] * 3, bounds, env_scene, o, d, max_steps, max_distance)
        _compare(_run(res, env_scene, o, d, max_steps, max_distance), ref, max_distance,
                 f"huge/{max_steps}")


def test_relaid_descent_limit_chains(gpu, corpus):
    """Chains of 31 and 33 nested nodes toward the (1, 1, 1) corner: the first
    keeps every slot above depth 32, the second reaches the 32-level limit
    (stale results). Batched alone and together, so both descent loops run."""
    from navi_amd.multiscene import ResidentScenes
    from tests.test_host_layout import _chain_words

    chains = [_chain_words(31), _chain_words(33)]
    rng = np.random.default_rng(5)
    rays = 256
    one = np.float32(1.0)
    near = one - np.arange(4, dtype=np.float32) * np.float32(2.0 ** -24)
    o = rng.choice(near, size=(2, rays, 3)).astype(np.float32)
    o[:, rays // 2:] = rng.uniform(0.0, 1.0, (2, rays // 2, 3)).astype(np.float32)
    d = rng.normal(size=(2, rays, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    for picks in ([0], [1], [0, 1]):
        scenes = [(chains[i], [0, 0, 0], [1, 1, 1]) for i in picks]
        res = ResidentScenes(scenes)
        env_scene = np.array([0, len(picks) - 1], np.int32)
        ref = _oracle_multi([s[0] for s in scenes], [[0, 0, 0, 1, 1, 1]] * len(picks), env_scene, o, d, 12, 4.0)
        _compare(_run(res, env_scene, o, d, 12, 4.0), ref, 4.0, f"chains/{picks}")


def test_relaid_many_scenes_and_narrow_domains(gpu, corpus):
    """120 resident scenes (more than the launch keeps split planes for in LDS),
    and domains too narrow for their magnitude (float split planes collapse),
    both located by in-register splits instead of the plane lookup."""
    from navi_amd.multiscene import ResidentScenes, plane_depth

    many = [(corpus[i % 4].words, corpus[i % 4].bbox_min_list, corpus[i % 4].bbox_max) for i in range(120)]
    res = ResidentScenes(many)
    assert res.table_depth == 6 and plane_depth(120, 6) == 0
    env_scene, o, d = _rays(corpus, 24, 16, 16, seed=31)
    env_scene = (env_scene + 4 * np.arange(24, dtype=np.int32)) % 120
    ref = _oracle_multi([s[0] for s in many], [list(s[1]) + list(s[2]) for s in many], env_scene, o, d, 128, 30.0)
    _compare(_run(res, env_scene, o, d, 128, 30.0, elevation_bins=16), ref, 30.0, "many")

    words = corpus[0].words
    narrow = [[1000.0, -2.0, 5.0, 1000.00048828125, 2.0, 5.0000019073486328],
              [-1.0, -1.0, -1.0, 1.0, 1.0, 1.0]]
    res = ResidentScenes([(words, b[:3], b[3:]) for b in narrow])
    rng = np.random.default_rng(8)
    env_scene = np.array([0, 1, 0], np.int32)
    b = np.array(narrow, np.float64)[env_scene]
    o = rng.uniform(b[:, None, :3], b[:, None, 3:], (3, 500, 3)).astype(np.float32)
    d = rng.normal(size=(3, 500, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    ref = _oracle_multi([words] * 2, narrow, env_scene, o, d, 64, 5.0)
    _compare(_run(res, env_scene, o, d, 64, 5.0), ref, 5.0, "narrow")


@pytest.mark.parametrize("depth", [4, 5, 6, 7])
def test_relaid_every_table_depth(gpu, corpus, depth):
    """Descents start at the cell table's depth (4 to 7): the cell from the LDS
    split planes, and for domains too narrow for their planes from splits in
    registers. Canonical and random rays, inside and outside the domains,
    against the oracle."""
    from navi_amd.multiscene import ResidentScenes

    scenes = [(c.words, c.bbox_min_list, c.bbox_max) for c in corpus]
    bounds = [c.bbox_min_list + c.bbox_max for c in corpus]
    res = ResidentScenes(scenes, table_depth=depth)
    assert res.table_depth == depth
    env_scene, o, d = _rays(corpus, 16, 32, 16, seed=40 + depth)
    ref = _oracle_multi([c.words for c in corpus], bounds, env_scene, o, d, 256, 30.0)
    _compare(_run(res, env_scene, o, d, 256, 30.0, elevation_bins=16), ref, 30.0, f"depth{depth}")
    rng = np.random.default_rng(depth)
    lo = np.array([bounds[s][:3] for s in env_scene]) - 2.0
    hi = np.array([bounds[s][3:] for s in env_scene]) + 2.0
    o = rng.uniform(lo[:, None, :], hi[:, None, :], (16, 512, 3)).astype(np.float32)
    d = rng.normal(size=(16, 512, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    ref = _oracle_multi([c.words for c in corpus], bounds, env_scene, o, d, 300, 45.0)
    _compare(_run(res, env_scene, o, d, 300, 45.0), ref, 45.0, f"depth{depth}/random")

    words = corpus[0].words
    narrow = [[1000.0, -2.0, 5.0, 1000.00048828125, 2.0, 5.0000019073486328], [-1.0, -1.0, -1.0, 1.0, 1.0, 1.0]]
    res = ResidentScenes([(words, b[:3], b[3:]) for b in narrow], table_depth=depth)
    env_scene = np.array([0, 1, 0], np.int32)
    b = np.array(narrow, np.float64)[env_scene]
    o = rng.uniform(b[:, None, :3], b[:, None, 3:], (3, 400, 3)).astype(np.float32)
    d = rng.normal(size=(3, 400, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    ref = _oracle_multi([words] * 2, narrow, env_scene, o, d, 64, 5.0)
    _compare(_run(res, env_scene, o, d, 64, 5.0), ref, 5.0, f"depth{depth}/narrow")


@pytest.mark.parametrize("n,depth,planes", [(16, 4, 6), (16, 5, 7), (16, 6, 8), (16, 7, 8), (30, 6, 7),
                                            (60, 5, 6), (100, 4, 5), (64, 6, 6), (128, 6, 5), (200, 6, 4),
                                            (100, 5, 5), (200, 5, 4), (200, 4, 4), (40, 7, 7)])
def test_relaid_wide_workgroups(gpu, corpus, n, depth, planes):
    """The 1024-thread fast kernel (forced for these small batches with
    navi_set_wide_min_rays): split planes one or two levels below the cell tables,
    whose levels between take their octants from the plane index, or at or above
    them for launches with many scenes. Every instance, canonical rays with step
    counts and random rays from in and around the domains (faces of cells and of
    the cached prefix cell crossed often), against the oracle."""
    from navi_amd import _native
    from navi_amd.multiscene import ResidentScenes, wide_plane_depth

    assert wide_plane_depth(n, depth) == planes
    many = [(corpus[i % 4].words, corpus[i % 4].bbox_min_list, corpus[i % 4].bbox_max) for i in range(n)]
    words = [s[0] for s in many]
    bounds = [list(s[1]) + list(s[2]) for s in many]
    prev = _native.set_wide_min_rays(0)
    try:
        res = ResidentScenes(many, table_depth=depth)
        env_scene, o, d = _rays(corpus, 20, 16, 16, seed=70 + depth)
        env_scene = (env_scene + 4 * np.arange(20, dtype=np.int32)) % n
        ref = _oracle_multi(words, bounds, env_scene, o, d, 200, 30.0)
        _compare(_run(res, env_scene, o, d, 200, 30.0, elevation_bins=16), ref, 30.0, f"wide{planes}/depth{depth}")
        rng = np.random.default_rng(n * 7 + depth)
        lo = np.array([bounds[s][:3] for s in env_scene]) - 2.0
        hi = np.array([bounds[s][3:] for s in env_scene]) + 2.0
        o = rng.uniform(lo[:, None, :], hi[:, None, :], (20, 400, 3)).astype(np.float32)
        d = rng.normal(size=(20, 400, 3))
        d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
        ref = _oracle_multi(words, bounds, env_scene, o, d, 300, 29.0)
        _compare(_run(res, env_scene, o, d, 300, 29.0), ref, 29.0, f"wide{planes}/depth{depth}/random")
    finally:
        _native.set_wide_min_rays(prev)


def test_fast_kernel_256_thread_shape(gpu, corpus):
    """The 256-thread fast kernel: launches of at least 2^19 rays below a raised
    wide threshold (navi_set_wide_min_rays). 64 envs x 128x64 rays (524,288) over
    the four scenes, staged (no step counts) and with step counts, against the
    oracle; smaller launches take the combined kernel alone and the GPU suite's
    other tests cover it."""
    import torch

    from navi_amd import _native
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    env_scene, o, d = _rays(corpus, 64, 128, 64, seed=91)
    assert o.shape[0] * o.shape[1] == 1 << 19
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene, o, d, 256, 30.0)
    prev = _native.set_wide_min_rays(1 << 30)
    try:
        _compare(_run(res, env_scene, o, d, 256, 30.0, elevation_bins=64), ref, 30.0, "wg256/steps")
        dev = res.device
        out_d = torch.full(o.shape[:2], -7.0, device=dev)
        out_s = torch.full(o.shape[:2], -7, device=dev, dtype=torch.int32)
        res.cast_rays(torch.from_numpy(env_scene).to(dev), torch.from_numpy(np.ascontiguousarray(o)).to(dev),
                      torch.from_numpy(np.ascontiguousarray(d)).to(dev), out_d, out_s, 256, 30.0, elevation_bins=64)
        torch.cuda.synchronize()
        gd, gs = out_d.cpu().numpy(), out_s.cpu().numpy()
        assert np.array_equal(gs, ref["semantic"]), "wg256/staged: semantics"
        assert np.array_equal(gd.view(np.uint32), ref["distance"].view(np.uint32)), "wg256/staged: distance bits"
    finally:
        _native.set_wide_min_rays(prev)


@pytest.mark.parametrize("n,depth,planes", [(27, 7, 5), (30, 6, 5), (60, 5, 4), (60, 6, 4), (100, 6, 4),
                                            (120, 5, 0)])
def test_relaid_tables_below_the_planes(gpu, corpus, n, depth, planes):
    """Many resident scenes: the launch stages split planes of fewer levels than
    the cell tables have (one or two levels below them come from splits in
    registers), or none at all (every cell from splits)."""
    from navi_amd.multiscene import ResidentScenes, plane_depth

    many = [(corpus[i % 4].words, corpus[i % 4].bbox_min_list, corpus[i % 4].bbox_max) for i in range(n)]
    assert plane_depth(n, depth) == planes
    res = ResidentScenes(many, table_depth=depth)
    env_scene, o, d = _rays(corpus, 20, 16, 16, seed=50 + depth)
    env_scene = (env_scene + 4 * np.arange(20, dtype=np.int32)) % n
    words = [s[0] for s in many]
    bounds = [list(s[1]) + list(s[2]) for s in many]
    ref = _oracle_multi(words, bounds, env_scene, o, d, 200, 30.0)
    _compare(_run(res, env_scene, o, d, 200, 30.0, elevation_bins=16), ref, 30.0, f"planes{planes}/depth{depth}")
    # random rays from inside and around the domains, random directions (faces of
    # void cells and of the cached prefix cell are crossed often)
    rng = np.random.default_rng(n + depth)
    lo = np.array([bounds[s][:3] for s in env_scene]) - 2.0
    hi = np.array([bounds[s][3:] for s in env_scene]) + 2.0
    o = rng.uniform(lo[:, None, :], hi[:, None, :], (20, 400, 3)).astype(np.float32)
    d = rng.normal(size=(20, 400, 3))
    d[:, :40, 0] = 0.0  # some rays parallel to the x planes
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    ref = _oracle_multi(words, bounds, env_scene, o, d, 300, 45.0)
    _compare(_run(res, env_scene, o, d, 300, 45.0), ref, 45.0, f"planes{planes}/depth{depth}/random")


@pytest.mark.parametrize("n", [31, 32])
def test_bad_child_index_at_the_descent_limit(gpu, n):
    """A child index past the array faults only when the descent examines the
    child: at depth 31 (chain of 31 nodes) the ray reports NaN, at depth 32
    (chain of 32) the 32-level limit comes first and the result is stale."""
    from navi_amd.multiscene import ResidentScenes
    from tests.test_host_layout import _chain_words

    words = _chain_words(n)
    words[2 * n - 1] = words.size + 5  # the last node's child index
    res = ResidentScenes([(words, [0, 0, 0], [1, 1, 1])])
    o = np.array([[[1, 1, 1], [1, 1, 1], [0.2, 0.9, 0.4]]], np.float32)
    d = np.array([[[-1, 0, 0], [0, 0, -1], [0, 1, 0]]], np.float32)
    ref = oracle.trace(words, o, d, 6, 4.0, [0, 0, 0], [1, 1, 1])
    assert np.isnan(ref["distance"][0, 0]) == (n == 31)
    for kernel in ("raw", "relaid"):
        _compare(_run(res, np.zeros(1, np.int32), o, d, 6, 4.0, kernel=kernel), ref, 4.0, f"badchild{n}/{kernel}")


def test_relaid_large_batch(gpu, corpus):
    """A batch large enough for 256-ray work units (small batches use 64-ray
    units): 1024 envs x 96x128 rays; every 31st env checked against the oracle."""
    import torch

    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    env_scene, o, d = _rays(corpus, 1024, 96, 128, seed=44)
    dev = res.device
    t_es = torch.from_numpy(env_scene).to(dev)
    t_o, t_d = torch.from_numpy(o).to(dev), torch.from_numpy(d).to(dev)
    out_d = torch.full(o.shape[:2], -7.0, device=dev)
    out_s = torch.full(o.shape[:2], -7, device=dev, dtype=torch.int32)
    out_n = torch.full(o.shape[:2], -7, device=dev, dtype=torch.int32)
    res.cast_rays(t_es, t_o, t_d, out_d, out_s, 96, 30.0, out_steps=out_n, elevation_bins=128)
    torch.cuda.synchronize()
    assert int((out_n == -7).sum().item()) == 0
    pick = np.arange(0, 1024, 31)
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene[pick], o[pick], d[pick], 96, 30.0)
    got = (out_d.cpu().numpy()[pick], out_s.cpu().numpy()[pick], out_n.cpu().numpy()[pick], None)
    _compare(got, ref, 30.0, "large")


def test_relaid_env_order_entries_out_of_range_are_skipped(gpu, corpus):
    """A caller-built env_order with entries outside [0, n_envs): those work items
    are skipped (their rays keep the sentinel), every named env is traced."""
    import torch

    from navi_amd import _native
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    env_scene, o, d = _rays(corpus, 6, 16, 8, seed=3)
    dev = res.device
    order = torch.tensor([5, 4, 99, 1, -3, 0], dtype=torch.int32, device=dev)  # envs 2 and 3 unnamed
    t_es = torch.from_numpy(env_scene).to(dev)
    t_o, t_d = torch.from_numpy(o).to(dev), torch.from_numpy(d).to(dev)
    out_d = torch.full(o.shape[:2], -7.0, device=dev)
    out_s = torch.full(o.shape[:2], -7, device=dev, dtype=torch.int32)
    code = _native.lib().navi_trace_relaid(
        res.records.data_ptr(), res.n_records, res.relaid_table.data_ptr(), res.n_scenes,
        res.cell_tables.data_ptr(), res.table_depth, t_es.data_ptr(), order.data_ptr(), 6, 16 * 8, 8, t_o.data_ptr(),
        t_d.data_ptr(), out_d.data_ptr(), out_s.data_ptr(), 64, 30.0, 0.01, None,
        torch.cuda.current_stream().cuda_stream)
    _native.check(code)
    torch.cuda.synchronize()
    gd = out_d.cpu().numpy()
    assert (gd[[2, 3]] == -7.0).all()
    named = [0, 1, 4, 5]
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene[named], o[named], d[named], 64, 30.0)
    assert np.array_equal(gd[named].view(np.uint32), ref["distance"].view(np.uint32))
    assert np.array_equal(out_s.cpu().numpy()[named], ref["semantic"])


@pytest.mark.parametrize("seed", range(6))
def test_relaid_randomized_sweep(gpu, seed):
    """Seeded random scenes (box room / cluttered / rooms at 32..256), shifted and
    scaled domains, random hit epsilons and step budgets, rays from inside and
    outside the domains in random directions: the record-layout tracer against
    the oracle."""
    import torch

    from navi_amd import scenes as S
    from navi_amd.multiscene import ResidentScenes

    rng = np.random.default_rng(1000 + seed)
    makers = [lambda s, r: S.box_room(seed=s, resolution=r), lambda s, r: S.cluttered(seed=s, resolution=r),
              lambda s, r: S.rooms(seed=s, resolution=r, grid=3)]
    scenes = []
    for k in range(3):
        sc = makers[int(rng.integers(0, 3))](int(rng.integers(0, 10_000)), int(rng.choice([32, 64, 128, 256])))
        words = sc.compile()
        # the same DAG over another domain: shift and scale the cube
        scale = float(rng.choice([1.0, 0.37, 3.3]))
        shift = rng.uniform(-50, 50, 3)
        lo = [float(np.float32(v * scale + sh)) for v, sh in zip(sc.bbox_min_list, shift)]
        hi = [float(np.float32(v * scale + sh)) for v, sh in zip(sc.bbox_max, shift)]
        scenes.append((words, lo, hi))
    res = ResidentScenes(scenes)
    n_env, rays = 9, 700
    env_scene = rng.integers(0, 3, n_env).astype(np.int32)
    lo = np.array([scenes[s][1] for s in env_scene], np.float64)
    hi = np.array([scenes[s][2] for s in env_scene], np.float64)
    span = hi - lo
    o = rng.uniform(lo[:, None, :] - 0.1 * span[:, None, :], hi[:, None, :] + 0.1 * span[:, None, :],
                    (n_env, rays, 3)).astype(np.float32)
    d = rng.normal(size=(n_env, rays, 3))
    d[:, :50, 1] = 0.0  # some rays in the horizontal plane
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    max_steps = int(rng.integers(1, 300))
    max_distance = float(np.float32(rng.uniform(1.0, 60.0)))
    eps = float(np.float32(rng.choice([0.01, 1e-3, 0.05])))
    ref = _oracle_multi([s[0] for s in scenes], [s[1] + s[2] for s in scenes], env_scene, o, d, max_steps,
                        max_distance, hit_epsilon=eps)
    _compare(_run(res, env_scene, o, d, max_steps, max_distance, hit_epsilon=eps), ref, max_distance,
             f"sweep{seed}")


def test_scene_order_follows_measured_cost(gpu, corpus):
    """The first sorted launch counts steps per ray (also when the caller asks for
    none) and reduces them per scene on the device; a later launch adopts the
    costs and hands out the costliest scenes' envs first, unknown scene ids last.
    Results are the oracle's in either order."""
    import torch

    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    env_scene, o, d = _rays(corpus, 24, 16, 8, seed=17)
    env_scene[[3, 11]] = [-1, len(corpus)]
    n = len(corpus)
    known = (env_scene >= 0) & (env_scene < n)
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene[known], o[known], d[known], 160, 30.0)
    dev = res.device
    t_es = torch.from_numpy(env_scene).to(dev)
    t_o = torch.from_numpy(np.ascontiguousarray(o)).to(dev)
    t_d = torch.from_numpy(np.ascontiguousarray(d)).to(dev)
    out_d = torch.full(o.shape[:2], -7.0, device=dev)
    out_s = torch.full(o.shape[:2], -7, device=dev, dtype=torch.int32)
    out_n = torch.full(o.shape[:2], -7, device=dev, dtype=torch.int32)
    res.cast_rays(t_es, t_o, t_d, out_d, out_s, 160, 30.0, elevation_bins=8)  # measures
    torch.cuda.synchronize()
    assert res.scene_cost is None  # adopted by the next launch
    first = (out_d.cpu().numpy(), out_s.cpu().numpy())
    res.cast_rays(t_es, t_o, t_d, out_d, out_s, 160, 30.0, out_steps=out_n, elevation_bins=8)
    torch.cuda.synchronize()
    assert res.scene_cost is not None
    got = (out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(), None)
    _compare(tuple(g[known] for g in got[:3]) + (None,), ref, 30.0, "cost-ordered")
    assert np.isnan(got[0][~known]).all() and (got[1][~known] == 0).all() and (got[2][~known] == 0).all()
    assert np.array_equal(first[0].view(np.uint32), got[0].view(np.uint32))
    assert np.array_equal(first[1], got[1])
    for s in range(n):
        m = env_scene[known] == s
        if m.any():
            assert res.scene_cost[s] == pytest.approx(float(ref["steps"][m].mean()), rel=1e-12, abs=0)
    pos = np.empty(n, np.int64)
    pos[np.argsort(-res.scene_cost, kind="stable")] = np.arange(n)
    key = np.where(known, pos[np.clip(env_scene, 0, n - 1)], n)
    assert np.array_equal(res.env_order(t_es).cpu().numpy(), np.argsort(key, kind="stable"))


@pytest.mark.parametrize("seed", range(8))
def test_relaid_random_scene_counts_and_depths(gpu, seed):
    """Random scenes replicated to 3, 27, 60, 100 or 120 resident scenes at a random table
    depth (so every split-plane depth the launch picks, none included), random rays
    from inside and around the domains, and rays generated from poses: against the
    oracle."""
    import torch

    from navi_amd import scenes as S
    from navi_amd.multiscene import ResidentScenes

    rng = np.random.default_rng(5000 + seed)
    makers = [lambda s, r: S.box_room(seed=s, resolution=r), lambda s, r: S.cluttered(seed=s, resolution=r),
              lambda s, r: S.rooms(seed=s, resolution=r, grid=3)]
    base = []
    for _ in range(3):
        sc = makers[int(rng.integers(0, 3))](int(rng.integers(0, 10_000)), int(rng.choice([32, 64, 128])))
        words = sc.compile()
        scale = float(rng.choice([1.0, 0.37, 3.3]))
        shift = rng.uniform(-50, 50, 3)
        lo = [float(np.float32(v * scale + sh)) for v, sh in zip(sc.bbox_min_list, shift)]
        hi = [float(np.float32(v * scale + sh)) for v, sh in zip(sc.bbox_max, shift)]
        base.append((words, lo, hi))
    n = int(rng.choice([3, 27, 60, 100, 120]))
    scenes = [base[i % 3] for i in range(n)]
    res = ResidentScenes(scenes, table_depth=int(rng.integers(4, 8)))
    words = [s[0] for s in scenes]
    bounds = [s[1] + s[2] for s in scenes]
    n_env = 12
    env_scene = rng.integers(0, n, n_env).astype(np.int32)
    lo = np.array([scenes[s][1] for s in env_scene], np.float64)
    hi = np.array([scenes[s][2] for s in env_scene], np.float64)
    span = hi - lo
    o = rng.uniform(lo[:, None, :] - 0.1 * span[:, None, :], hi[:, None, :] + 0.1 * span[:, None, :],
                    (n_env, 256, 3)).astype(np.float32)
    d = rng.normal(size=(n_env, 256, 3))
    d[:, :20, 2] = 0.0  # some rays parallel to the z planes
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    max_steps = int(rng.integers(1, 300))
    max_distance = float(np.float32(rng.uniform(1.0, 60.0)))
    label = f"n{n}/depth{res.table_depth}"
    ref = _oracle_multi(words, bounds, env_scene, o, d, max_steps, max_distance)
    _compare(_run(res, env_scene, o, d, max_steps, max_distance), ref, max_distance, label)

    # rays from poses: each env's first origin, a yawed 16 x 8 canonical table
    pos = np.ascontiguousarray(o[:, 0, :])
    yaw = rng.uniform(0, 2 * math.pi, n_env).astype(np.float32)
    rot = np.stack([np.cos(yaw), np.sin(yaw)], 1).astype(np.float32)
    local = oracle.ray_directions(16, 8)
    c, s = rot[:, None, 0:1], rot[:, None, 1:2]
    x, y, z = local[None, :, 0:1], local[None, :, 1:2], local[None, :, 2:3]
    dirs = np.ascontiguousarray(np.concatenate(
        [x * c + z * s, np.broadcast_to(y, (n_env,) + y.shape[1:]), (-x) * s + z * c], -1), np.float32)
    origins = np.ascontiguousarray(np.broadcast_to(pos[:, None, :], dirs.shape))
    ref = _oracle_multi(words, bounds, env_scene, origins, dirs, max_steps, max_distance)
    dev = res.device
    out_d = torch.full((n_env, 128), -7.0, device=dev)
    out_s = torch.full((n_env, 128), -7, device=dev, dtype=torch.int32)
    out_n = torch.full((n_env, 128), -7, device=dev, dtype=torch.int32)
    res.cast_rays_poses(torch.from_numpy(env_scene).to(dev), torch.from_numpy(local).to(dev),
                        torch.from_numpy(pos).to(dev), torch.from_numpy(rot).to(dev), out_d, out_s, max_steps,
                        max_distance, out_steps=out_n, elevation_bins=8)
    torch.cuda.synchronize()
    _compare((out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(), None), ref, max_distance,
             label + "/poses")
