"""GPU parity of the observation-step entry points against the CPU oracle:
rays generated from poses in the tracer (navi_trace_relaid_poses), point-SDF
queries (navi_point_query) and the fused post-pass (navi_observe).

Bars: traced rays as in test_gpu_multiscene (bit-exact); point queries
bit-exact (distance bits, semantic, kind); post-pass min distance and
collision exact, ratios within 1e-6, fp16 depth within one binary16 ulp,
float32 depth within DEPTH_RTOL of the oracle's. A launch that writes no
float32 depth computes the fp16 depth with a binary16-accuracy log1p
(depth16_log1p in navi_amd/csrc/observation.hip): within one binary16 ulp of
the exact value for every float input in [0, max_distance], checked here
exhaustively for max_distance 30.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from tests.test_gpu_multiscene import _compare, _corpus, _oracle_multi, _run

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    import sys

    print(f"[test_gpu_observation] {msg}", file=sys.stderr, flush=True)

# The float32 depth q = log1p(c) / log1p(max) against the oracle's: the
# device's is within 2.31e-7 relative of the exact value (its log1p within
# 0.92 ulp, checked on the host for every float in [0, 32] by
# tests/native/log1p_check.c; then RN(1 / log1p(max)) and the product round
# once each), the oracle's (torch CPU log1p within one ulp, one division)
# within 1.8e-7: 4.2e-7 between them. q <= 1, so the same bound is absolute
# for the delta of two frames that start from the same previous depth.
DEPTH_RTOL = 4.2e-7


@pytest.fixture(scope="module")
def corpus():
    return _corpus()


def _resident(corpus):
    from navi_amd.multiscene import ResidentScenes

    return ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])


def _poses(corpus, n_envs, seed):
    rng = np.random.default_rng(seed)
    env_scene = rng.integers(0, len(corpus), n_envs).astype(np.int32)
    pos = np.empty((n_envs, 3), np.float32)
    for s in range(len(corpus)):
        idx = np.flatnonzero(env_scene == s)
        if idx.size:
            pos[idx] = corpus[s].free_origins(rng, idx.size)
    yaw = rng.uniform(-math.pi, 3 * math.pi, n_envs).astype(np.float32)
    rot = np.stack([np.cos(yaw), np.sin(yaw)], axis=1).astype(np.float32)
    return env_scene, pos, rot


def _rotate(local, rot):
    """x' = x c + z s, y' = y, z' = (-x) s + z c with float32 rounding after each
    operation (sdfdag_backend.py:1300-1310 in eager tensor code)."""
    c = rot[:, None, 0:1]
    s = rot[:, None, 1:2]
    x, y, z = local[None, :, 0:1], local[None, :, 1:2], local[None, :, 2:3]
    d = np.concatenate([x * c + z * s, np.broadcast_to(y, (rot.shape[0],) + y.shape[1:]), (-x) * s + z * c], -1)
    return np.ascontiguousarray(d, np.float32)


@pytest.mark.parametrize("az,el,depth", [(32, 16, None), (24, 5, None), (16, 8, 4), (16, 8, 5), (16, 8, 6)])
def test_pose_rays_equal_explicit_rays(gpu, corpus, az, el, depth):
    """Rays generated in the tracer from poses against the oracle and against the same
    rays passed explicitly; at the default cell-table depth and at depths 4 to 6."""
    import torch

    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus], table_depth=depth)
    env_scene, pos, rot = _poses(corpus, 20, seed=az)
    local = oracle.ray_directions(az, el)
    dirs = _rotate(local, rot)
    origins = np.ascontiguousarray(np.broadcast_to(pos[:, None, :], dirs.shape))
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene, origins, dirs, 160, 30.0)
    dev = res.device
    t = {k: torch.from_numpy(v).to(dev) for k, v in
         (("es", env_scene), ("local", local), ("pos", pos), ("rot", rot))}
    out_d = torch.full((20, az * el), -7.0, device=dev)
    out_s = torch.full((20, az * el), -7, device=dev, dtype=torch.int32)
    out_n = torch.full((20, az * el), -7, device=dev, dtype=torch.int32)
    res.cast_rays_poses(t["es"], t["local"], t["pos"], t["rot"], out_d, out_s, 160, 30.0, out_steps=out_n,
                        elevation_bins=el)
    torch.cuda.synchronize()
    got = (out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(), None)
    _compare(got, ref, 30.0, f"poses/{az}x{el}")
    explicit = _run(res, env_scene, origins, dirs, 160, 30.0, elevation_bins=el)
    assert np.array_equal(explicit[0].view(np.uint32), got[0].view(np.uint32))


@pytest.mark.parametrize("n,depth,planes", [(27, 7, 5), (60, 6, 4), (100, 6, 4), (120, 5, 0)])
def test_pose_rays_with_planes_above_the_tables(gpu, corpus, n, depth, planes):
    """Rays from poses over many resident scenes, where the launch stages split planes
    one or two levels above the cell tables, or none: against the oracle."""
    import torch

    from navi_amd.multiscene import ResidentScenes, plane_depth

    many = [corpus[i % len(corpus)] for i in range(n)]
    assert plane_depth(n, depth) == planes
    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in many], table_depth=depth)
    env_scene, pos, rot = _poses(corpus, 20, seed=n)
    env_scene = ((env_scene + len(corpus) * np.arange(20)) % n).astype(np.int32)
    local = oracle.ray_directions(16, 8)
    dirs = _rotate(local, rot)
    origins = np.ascontiguousarray(np.broadcast_to(pos[:, None, :], dirs.shape))
    ref = _oracle_multi([c.words for c in many], [c.bbox_min_list + c.bbox_max for c in many],
                        env_scene, origins, dirs, 160, 30.0)
    dev = res.device
    t = {k: torch.from_numpy(v).to(dev) for k, v in
         (("es", env_scene), ("local", local), ("pos", pos), ("rot", rot))}
    out_d = torch.full((20, 128), -7.0, device=dev)
    out_s = torch.full((20, 128), -7, device=dev, dtype=torch.int32)
    out_n = torch.full((20, 128), -7, device=dev, dtype=torch.int32)
    res.cast_rays_poses(t["es"], t["local"], t["pos"], t["rot"], out_d, out_s, 160, 30.0, out_steps=out_n,
                        elevation_bins=8)
    torch.cuda.synchronize()
    got = (out_d.cpu().numpy(), out_s.cpu().numpy(), out_n.cpu().numpy(), None)
    _compare(got, ref, 30.0, f"poses/{n}/{depth}")


def _point_cases(corpus, n, seed):
    rng = np.random.default_rng(seed)
    scene = rng.integers(0, len(corpus), n).astype(np.int32)
    lo = np.array([corpus[s].bbox_min_list for s in scene], np.float64)
    hi = np.array([corpus[s].bbox_max for s in scene], np.float64)
    pts = rng.uniform(lo - 0.5, hi + 0.5, (n, 3)).astype(np.float32)
    pts[: n // 8] = lo[: n // 8].astype(np.float32)  # on the lower domain faces
    pts[n // 8: n // 4] = hi[n // 8: n // 4].astype(np.float32)  # on the upper faces (inclusive)
    return scene, pts


def _point_oracle(words_by_scene, bounds, scene, pts):
    d = np.empty(len(pts), np.float32)
    s = np.empty(len(pts), np.int32)
    k = np.empty(len(pts), np.int32)
    for sc in np.unique(scene):
        idx = np.flatnonzero(scene == sc)
        r = oracle.point_query(words_by_scene[sc], pts[idx], bounds[sc][:3], bounds[sc][3:])
        d[idx], s[idx], k[idx] = r["distance"], r["semantic"], r["kind"]
    return d, s, k


def _same_bits(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or np.array_equal(
        np.where(np.isnan(a), np.float32(np.nan), a).view(np.uint32),
        np.where(np.isnan(b), np.float32(np.nan), b).view(np.uint32))


@pytest.mark.parametrize("depth", [None, 4, 7])
def test_point_queries(gpu, corpus, depth):
    import torch

    from tests.test_host_layout import _chain_words

    chain = _chain_words(33)
    bad = _chain_words(32)
    bad[63] = bad.size + 5
    leaf = np.array([(1 << 63) | (7 << 16) | 0x3C00], np.uint64)
    scenes = [(c.words, c.bbox_min_list, c.bbox_max) for c in corpus]
    scenes += [(chain, [0, 0, 0], [1, 1, 1]), (bad, [0, 0, 0], [1, 1, 1]), (leaf, [-1, -1, -1], [1, 1, 1])]
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes(scenes, table_depth=depth)
    bounds = [list(s[1]) + list(s[2]) for s in scenes]
    scene, pts = _point_cases(corpus, 3000, seed=12)
    extra = np.array([[1, 1, 1], [0.999, 0.999, 0.999], [0.3, 0.2, 0.9]], np.float32)
    for sc in (4, 5, 6):
        scene = np.concatenate([scene, np.full(3, sc, np.int32)])
        pts = np.concatenate([pts, extra])
    want = _point_oracle([s[0] for s in scenes], bounds, scene, pts)
    assert {0, 1, 2, 3}.issubset(set(want[2].tolist()))
    dev = res.device
    tp = torch.from_numpy(pts).to(dev)
    ts = torch.from_numpy(scene).to(dev)
    out_d = torch.full((len(pts),), -7.0, device=dev)
    out_s = torch.full((len(pts),), -7, device=dev, dtype=torch.int32)
    out_k = torch.full((len(pts),), -7, device=dev, dtype=torch.int32)
    res.point_query(tp, out_d, out_s, point_scene=ts, out_kind=out_k)
    torch.cuda.synchronize()
    assert np.array_equal(out_k.cpu().numpy(), want[2])
    assert np.array_equal(out_s.cpu().numpy(), want[1])
    assert _same_bits(out_d.cpu().numpy(), want[0])
    # unknown scene ids: NaN, kind 4
    ts_bad = torch.tensor([-1, 99], dtype=torch.int32, device=dev)
    tp2 = torch.zeros((2, 3), device=dev)
    d2, s2, k2 = (torch.zeros(2, device=dev), torch.zeros(2, device=dev, dtype=torch.int32),
                  torch.zeros(2, device=dev, dtype=torch.int32))
    res.point_query(tp2, d2, s2, point_scene=ts_bad, out_kind=k2)
    torch.cuda.synchronize()
    assert torch.isnan(d2).all() and k2.tolist() == [4, 4] and s2.tolist() == [0, 0]


def _observe_oracle_check(got, want):
    d16, stats, coll = got
    assert np.array_equal(coll, want["collision"])
    assert _same_bits(stats[:, 0].copy(), want["stats"][:, 0].copy())
    np.testing.assert_allclose(stats[:, 1:], want["stats"][:, 1:], atol=1e-6, rtol=0)
    a = d16.astype(np.float32)
    b = want["depth16"].astype(np.float32)
    assert np.array_equal(np.isnan(a), np.isnan(b))
    ulp = np.spacing(np.abs(np.nan_to_num(b)).astype(np.float16)).astype(np.float32)
    assert (np.abs(np.nan_to_num(a) - np.nan_to_num(b)) <= ulp).all()


@pytest.mark.parametrize("az,el,band", [(256, 48, (1.5, 30.0)), (12, 3, (1.5, 8.0)), (7, 5, (3.0, 3.0)),
                                         (256, 128, (1.5, 30.0)), (10, 1000, (1.5, 30.0)), (2, 4, (0.5, 20.0))])
def test_observe_matches_oracle(gpu, corpus, az, el, band):
    """(256, 48), (12, 3), (10, 1000) and (2, 4) stage the fp16 tile in LDS (odd
    row pitch 49, 3, 1001, 5; 10,000 and 8 elements end in a partial batch); (7, 5)
    (odd Az) and (256, 128) (a 66 KB tile) write it directly."""
    import torch

    res = _resident(corpus)
    rng = np.random.default_rng(az + el)
    e = 9
    d = rng.uniform(-1.0, 40.0, (e, az * el)).astype(np.float32)
    d[0, :5] = [np.inf, -np.inf, 0.0, 30.0, 29.999]
    d[1, 7] = np.nan
    d[2] = rng.uniform(0.0, 0.3, az * el)  # a collision
    sem = rng.integers(0, 40, (e, az * el)).astype(np.int32)
    prev = rng.uniform(0.0, 1.0, (e, az, el)).astype(np.float32)
    prev[3] = 0.0  # first frame for env 3
    want = oracle.observe(d, az, el, 30.0, band[0], band[1], 2.0, 0.15, semantics=sem, prev_depth=prev)
    dev = res.device
    td = torch.from_numpy(d).to(dev)
    ts = torch.from_numpy(sem).to(dev)
    tprev = torch.from_numpy(prev).to(dev)
    d16 = torch.empty((e, 1, el, az), dtype=torch.float16, device=dev)
    st = torch.empty((e, 5), device=dev)
    co = torch.empty((e,), dtype=torch.int32, device=dev)
    obs = torch.empty((e, 3, az, el), device=dev)
    delta = torch.empty((e, az, el), device=dev)
    res.observe(td, az, el, 30.0, structure_band_min=band[0], structure_band_max=band[1], out_depth_f16=d16,
                out_stats=st, out_collision=co, semantics=ts, out_obs=obs, prev_depth=tprev, out_delta=delta)
    torch.cuda.synchronize()
    _observe_oracle_check((d16.cpu().numpy(), st.cpu().numpy(), co.cpu().numpy()), want)
    # the same with only the fp16 depth and the statistics (the observation step's outputs):
    # a kernel compiled without the float32 outputs, its depth from the binary16-accuracy
    # log1p; statistics and collision identical, the fp16 depth to the same bar
    d16b = torch.empty_like(d16)
    stb = torch.empty_like(st)
    cob = torch.empty_like(co)
    res.observe(td, az, el, 30.0, structure_band_min=band[0], structure_band_max=band[1], out_depth_f16=d16b,
                out_stats=stb, out_collision=cob)
    torch.cuda.synchronize()
    assert torch.equal(stb.view(torch.int32), st.view(torch.int32)) and torch.equal(cob, co)
    _observe_oracle_check((d16b.cpu().numpy(), stb.cpu().numpy(), cob.cpu().numpy()), want)
    assert int((d16b.view(torch.int16).int() - d16.view(torch.int16).int()).abs().max()) <= 1
    # float32 outputs: depth within DEPTH_RTOL, semantic / valid exact
    go = obs.cpu().numpy()
    np.testing.assert_array_equal(go[:, 1:], want["obs"][:, 1:])
    wd = want["obs"][:, 0]
    assert np.array_equal(np.isnan(go[:, 0]), np.isnan(wd))
    np.testing.assert_allclose(np.nan_to_num(go[:, 0]), np.nan_to_num(wd), rtol=DEPTH_RTOL, atol=1e-7)
    gdel = delta.cpu().numpy()
    assert (gdel[3] == 0).all()
    assert np.array_equal(np.isnan(gdel), np.isnan(want["delta"]))
    np.testing.assert_allclose(np.nan_to_num(gdel), np.nan_to_num(want["delta"]), rtol=0, atol=DEPTH_RTOL)
    # prev_depth now holds the depth
    assert np.array_equal(tprev.cpu().numpy().view(np.uint32), go[:, 0].view(np.uint32))


def test_observe_depth_against_exact_log1p(gpu, corpus):
    """The normalised depth over every 531st binary32 in [0, 30] (every binade,
    subnormals included) against log1p(c) / log1p(30) in float64: float32 within
    2.31e-7 relative (the bound in DEPTH_RTOL's comment) plus half the smallest
    subnormal, fp16 within one binary16 ulp of the exact value rounded to
    binary16. Pins the device log1p and reciprocal on the hardware itself."""
    import torch

    az, el = 64, 16
    top = int(np.float32(30.0).view(np.uint32))
    bits = np.arange(0, top + 1, 531, dtype=np.uint32)
    special = np.array([0.0, 30.0, 2.0 ** -24, np.nextafter(np.float32(2.0 ** -24), 1), 1.0, 29.999998],
                       np.float32).view(np.uint32)
    bits = np.concatenate([bits, special])
    n_envs = -(-bits.size // (az * el))
    c = np.ones(n_envs * az * el, np.float32)
    c[: bits.size] = bits.view(np.float32)
    c = c.reshape(n_envs, az * el)
    res = _resident(corpus)
    dev = res.device
    td = torch.from_numpy(c).to(dev)
    sem = torch.zeros((n_envs, az * el), dtype=torch.int32, device=dev)
    obs = torch.empty((n_envs, 3, az, el), device=dev)
    d16 = torch.empty((n_envs, 1, el, az), dtype=torch.float16, device=dev)
    res.observe(td, az, el, 30.0, semantics=sem, out_obs=obs, out_depth_f16=d16)
    torch.cuda.synchronize()
    q = obs[:, 0].cpu().numpy().reshape(-1).astype(np.float64)
    exact = np.log1p(c.reshape(-1).astype(np.float64)) / math.log1p(30.0)
    err = np.abs(q - exact)
    bound = 2.31e-7 * exact + 2.0 ** -150
    worst = int(np.argmax(err / bound))
    assert (err <= bound).all(), f"c={c.reshape(-1)[worst]!r}: {q[worst]!r} vs {exact[worst]!r}"
    h = d16.cpu().numpy().transpose(0, 1, 3, 2).reshape(-1).astype(np.float64)
    h_exact = exact.astype(np.float16)
    ulp = np.spacing(h_exact).astype(np.float64)
    assert (np.abs(h - h_exact.astype(np.float64)) <= ulp).all()


def _rn16(torch, exact):
    """float64 -> the nearest binary16 (one rounding): the float32 cast's result or a
    neighbour of it, whichever is nearest to the exact value."""
    h = exact.float().half().view(torch.int16).int()
    best, pick = None, None
    for dlt in (-1, 0, 1):
        cand = (h + dlt).clamp(0, 0x7BFF).short().view(torch.float16)
        err = (cand.double() - exact).abs()
        if best is None:
            best, pick = err, cand
        else:
            better = err < best
            best, pick = torch.where(better, err, best), torch.where(better, cand, pick)
    return pick


@pytest.mark.parametrize("max_distance", [30.0, 1.0, 100.0])
def test_fp16_depth_every_float(gpu, corpus, max_distance):
    """The fp16-only launch (no float32 depth asked for: the observation step's) over
    every binary32 c in [0, max_distance] (1.1e9 inputs for 30 m) as 256 x 48 envs: the
    fp16 depth within one binary16 ulp of RN16(log1p(c) / log1p(max_distance)), the
    quotient in float64 (device log1p). 1 m keeps every 1 + c below 2 (the rounding-error
    term of depth16_log1p always on), 100 m takes 1 + c to 101. At 30 m, the same envs
    through the general pass (the distances at an address that is not 16-byte aligned)
    and through the two-half copy-out (an fp16 output that is not 8-byte aligned): the
    same fp16 depth and statistics, bit for bit."""
    import torch

    az, el = 256, 48
    n = az * el
    res = _resident(corpus)
    dev = res.device
    top = int(np.float32(max_distance).view(np.uint32))
    chunk = (1 << 28) // n * n
    not_rn, worst = 0, 0
    for lo in range(0, top + 1, chunk):
        e = -(-min(chunk, top + 1 - lo) // n)
        bits = torch.arange(lo, lo + e * n, device=dev, dtype=torch.int64).clamp_(max=top).to(torch.int32)
        c = bits.view(torch.float32).view(e, n)
        d16 = torch.empty((e, 1, el, az), dtype=torch.float16, device=dev)
        res.observe(c, az, el, max_distance, out_depth_f16=d16)
        want = _rn16(torch, torch.log1p(c.double()) / math.log1p(max_distance))
        got = d16.view(e, el, az).transpose(1, 2).reshape(e, n)
        diff = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs()
        not_rn += int((diff != 0).sum())
        worst = max(worst, int(diff.max()))
        del bits, want, diff
    _say(f"max_distance {max_distance}: {not_rn} inputs not RN16(exact), worst {worst} ulp")
    assert worst <= 1, f"fp16 depth {worst} binary16 ulps from the exact value"
    assert not_rn < 100_000  # about 1.3e-5 of the inputs at 30 m differ from RN16(exact), by one ulp
    if max_distance != 30.0:
        return
    # general pass against the 16-byte pass, with NaN, infinities and statistics
    rng = np.random.default_rng(11)
    e = 64
    d = rng.uniform(-1.0, 40.0, (e, n)).astype(np.float32)
    d[0, :6] = [np.inf, -np.inf, np.nan, 0.0, 30.0, 29.999]
    d[5, 100] = np.nan
    d[7] = rng.uniform(0.0, 0.3, n)
    aligned = torch.from_numpy(d).to(dev)
    store = torch.empty(e * n + 1, device=dev)
    shifted = store[1:].view(e, n)
    shifted.copy_(aligned)
    assert aligned.data_ptr() % 16 == 0 and shifted.data_ptr() % 16 == 4
    outs = []
    for src in (aligned, shifted):
        d16 = torch.empty((e, 1, el, az), dtype=torch.float16, device=dev)
        st = torch.empty((e, 5), device=dev)
        co = torch.empty((e,), dtype=torch.int32, device=dev)
        res.observe(src, az, el, 30.0, out_depth_f16=d16, out_stats=st, out_collision=co)
        outs.append((d16, st, co))
    torch.cuda.synchronize()
    (a16, ast, aco), (b16, bst, bco) = outs
    assert torch.equal(a16.view(torch.int16), b16.view(torch.int16))
    assert torch.equal(ast.view(torch.int32), bst.view(torch.int32)) and torch.equal(aco, bco)
    # an fp16 output 4 bytes off an 8-byte boundary: copied out two halves per lane
    # instead of four, same bits
    store16 = torch.empty(e * n + 2, dtype=torch.float16, device=dev)
    c16 = store16[2:].view(e, 1, el, az)
    assert c16.data_ptr() % 8 == 4
    res.observe(aligned, az, el, 30.0, out_depth_f16=c16)
    torch.cuda.synchronize()
    assert torch.equal(c16.view(torch.int16), a16.view(torch.int16))
    want = oracle.observe(d, az, el, 30.0, 1.5, 30.0, 2.0, 0.15)
    _observe_oracle_check((a16.cpu().numpy(), ast.cpu().numpy(), aco.cpu().numpy()), want)


def test_observation_step_end_to_end(gpu, corpus):
    """Poses -> traced rays -> fused post-pass with point queries, against the oracle
    pipeline on the same inputs."""
    import torch

    res = _resident(corpus)
    az, el, e = 64, 16, 12
    env_scene, pos, rot = _poses(corpus, e, seed=77)
    local = oracle.ray_directions(az, el)
    dirs = _rotate(local, rot)
    origins = np.ascontiguousarray(np.broadcast_to(pos[:, None, :], dirs.shape))
    ref = _oracle_multi([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus],
                        env_scene, origins, dirs, 128, 30.0)
    want = oracle.observe(ref["distance"], az, el, 30.0)
    rng = np.random.default_rng(3)
    pts = (np.repeat(pos, 4, axis=0) + rng.uniform(-0.3, 0.3, (4 * e, 3))).astype(np.float32)
    pscene = np.repeat(env_scene, 4).astype(np.int32)
    pwant = _point_oracle([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus], pscene, pts)
    dev = res.device
    t = {k: torch.from_numpy(v).to(dev) for k, v in
         (("es", env_scene), ("local", local), ("pos", pos), ("rot", rot), ("pts", pts), ("ps", pscene))}
    out_d = torch.empty((e, az * el), device=dev)
    out_s = torch.empty((e, az * el), device=dev, dtype=torch.int32)
    res.cast_rays_poses(t["es"], t["local"], t["pos"], t["rot"], out_d, out_s, 128, 30.0, elevation_bins=el)
    d16 = torch.empty((e, 1, el, az), dtype=torch.float16, device=dev)
    st = torch.empty((e, 5), device=dev)
    co = torch.empty((e,), dtype=torch.int32, device=dev)
    pd = torch.empty((4 * e,), device=dev)
    ps = torch.empty((4 * e,), device=dev, dtype=torch.int32)
    pk = torch.empty((4 * e,), device=dev, dtype=torch.int32)
    res.observe(out_d, az, el, 30.0, out_depth_f16=d16, out_stats=st, out_collision=co, points=t["pts"],
                point_scene=t["ps"], point_distances=pd, point_semantics=ps, point_kind=pk)
    torch.cuda.synchronize()
    assert np.array_equal(out_d.cpu().numpy().view(np.uint32), ref["distance"].view(np.uint32))
    _observe_oracle_check((d16.cpu().numpy(), st.cpu().numpy(), co.cpu().numpy()), want)
    assert np.array_equal(pk.cpu().numpy(), pwant[2]) and np.array_equal(ps.cpu().numpy(), pwant[1])
    assert _same_bits(pd.cpu().numpy(), pwant[0])
    # 64 points per env (the most that ride in the env workgroups), 65 (workgroups of
    # their own) and 3 for 12 envs (some env workgroups take none): the same answers
    for per_env in (64, 65):
        m = per_env * e
        mp = (np.repeat(pos, per_env, axis=0) + rng.uniform(-0.3, 0.3, (m, 3))).astype(np.float32)
        msc = np.repeat(env_scene, per_env).astype(np.int32)
        mw = _point_oracle([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus], msc, mp)
        md, ms, mk = (torch.empty((m,), device=dev), torch.empty((m,), device=dev, dtype=torch.int32),
                      torch.empty((m,), device=dev, dtype=torch.int32))
        res.observe(out_d, az, el, 30.0, out_depth_f16=d16, points=torch.from_numpy(mp).to(dev),
                    point_scene=torch.from_numpy(msc).to(dev), point_distances=md, point_semantics=ms,
                    point_kind=mk)
        torch.cuda.synchronize()
        assert np.array_equal(mk.cpu().numpy(), mw[2]) and np.array_equal(ms.cpu().numpy(), mw[1])
        assert _same_bits(md.cpu().numpy(), mw[0])
    few = (pos[:3] + 0.01).astype(np.float32)
    fsc = env_scene[:3].astype(np.int32)
    fw = _point_oracle([c.words for c in corpus], [c.bbox_min_list + c.bbox_max for c in corpus], fsc, few)
    fd, fs = torch.empty((3,), device=dev), torch.empty((3,), device=dev, dtype=torch.int32)
    res.observe(out_d, az, el, 30.0, out_depth_f16=d16, points=torch.from_numpy(few).to(dev),
                point_scene=torch.from_numpy(fsc).to(dev), point_distances=fd, point_semantics=fs)
    torch.cuda.synchronize()
    assert np.array_equal(fs.cpu().numpy(), fw[1]) and _same_bits(fd.cpu().numpy(), fw[0])


def test_bench_sdfdag_harness(gpu, tmp_path, capsys):
    """The bench-sdfdag harness on two .gmdag files resident together: the command
    runs and reports the reference's summary keys, and one harness step's rays,
    observation, delta and statistics match the oracle pipeline on the poses that
    step traced, each actor in its own scene."""
    import json as _json

    import torch

    from navi_amd import bench_sdfdag, gmdag
    from navi_amd import scenes as S

    paths = []
    for name, scene in (("room", S.box_room(seed=4, resolution=64)), ("clutter", S.cluttered(seed=2, resolution=64))):
        paths.append(tmp_path / f"{name}.gmdag")
        gmdag.write_gmdag(paths[-1], scene.compile(), scene.resolution, scene.bbox_min_list, scene.voxel_size)
    assert bench_sdfdag.main(["--gmdag-file", str(paths[0]), str(paths[1]), "--actors", "6", "--steps", "3",
                              "--warmup-steps", "1", "--azimuth-bins", "32", "--elevation-bins", "8", "--json"]) == 0
    summary = _json.loads(capsys.readouterr().out)
    for key in ("measured_sps", "avg_batch_ms", "avg_actor_ms", "total_batches", "total_actor_steps"):
        assert key in summary
    assert summary["total_actor_steps"] == 6 * 4 and summary["scenes"] == 2

    assets = [gmdag.load_gmdag_asset(p) for p in paths]
    h = bench_sdfdag.ObservationHarness([(a.nodes, a.bbox_min, a.bbox_max) for a in assets], 5, 32, 8, 30.0, 128)
    assert h.env_scene.cpu().tolist() == [0, 1, 0, 1, 0]
    seen = {}
    real = h.res.cast_rays_poses

    def spy(env_scene, local, pos, rot, *a, **k):
        seen["pos"], seen["rot"] = pos.cpu().numpy().copy(), rot.cpu().numpy().copy()
        return real(env_scene, local, pos, rot, *a, **k)

    h.res.cast_rays_poses = spy
    h.step()
    prev0 = h.prev_depth.cpu().numpy().copy()  # the first step's depth
    h.step()
    torch.cuda.synchronize()
    dirs = _rotate(oracle.ray_directions(32, 8), seen["rot"])
    origins = np.ascontiguousarray(np.broadcast_to(seen["pos"][:, None, :], dirs.shape))
    dist = np.empty(dirs.shape[:2], np.float32)
    sem = np.empty(dirs.shape[:2], np.int32)
    for s_id, a in enumerate(assets):
        rows = np.arange(5)[np.arange(5) % 2 == s_id]
        r = oracle.trace(a.nodes, origins[rows], dirs[rows], 128, 30.0, list(a.bbox_min), list(a.bbox_max))
        dist[rows], sem[rows] = r["distance"], r["semantic"]
    want = oracle.observe(dist, 32, 8, 30.0, semantics=sem, prev_depth=prev0)
    assert np.array_equal(h.out_d.cpu().numpy().view(np.uint32), dist.view(np.uint32))
    assert np.array_equal(h.out_s.cpu().numpy(), sem)
    go = h.obs.cpu().numpy()
    np.testing.assert_array_equal(go[:, 1:], want["obs"][:, 1:])
    np.testing.assert_allclose(go[:, 0], want["obs"][:, 0], rtol=DEPTH_RTOL, atol=1e-7)
    np.testing.assert_allclose(h.delta.cpu().numpy(), want["delta"], rtol=0, atol=DEPTH_RTOL)
    np.testing.assert_allclose(h.stats.cpu().numpy()[:, 1:], want["stats"][:, 1:], atol=1e-6)
    assert np.array_equal(h.stats.cpu().numpy()[:, 0], want["stats"][:, 0])


def test_bench_sdfdag_kinematics_closed_forms(gpu):
    """The harness's kinematics against values worked out by hand from
    sdfdag_backend.py:560-617 and config.py:94-109: full speed when the previous
    frame's forward depth is far (log-normalised 1.0: 30 m), the 0.05 floor when it
    is 0, velocity smoothing 0.85 / 0.15 across two steps, yaw integrated over 0.02
    s, and the clamp to the scene box."""
    import torch

    from navi_amd import bench_sdfdag
    from navi_amd import scenes as S

    sc = S.box_room(seed=4, resolution=64)
    h = bench_sdfdag.ObservationHarness([(sc.compile(), sc.bbox_min_list, sc.bbox_max)], 3, 32, 8, 30.0, 64)
    lo = np.asarray(sc.bbox_min_list, np.float64)
    mid = (lo + np.asarray(sc.bbox_max)) / 2
    start = np.array([mid, mid, [mid[0], mid[1], lo[2] + 0.01]], np.float32)
    h.pos.copy_(torch.from_numpy(start))
    h.yaw.copy_(torch.tensor([0.0, math.pi / 2, 0.0]))
    h.prev_depth.fill_(1.0)
    h.prev_depth[1].zero_()
    yaw0 = h.yaw.cpu().numpy().astype(np.float64)
    h.kinematics()
    pos1, yaw1 = h.pos.cpu().numpy().astype(np.float64), h.yaw.cpu().numpy().astype(np.float64)
    # actor 0: factor 1, forward 1.5 * 5 = 7.5, smoothed 0.85 * 7.5 = 6.375 along -z
    np.testing.assert_allclose(pos1[0], mid + [0.0, 0.0, -6.375 * 0.02], atol=2e-6)
    assert abs(yaw1[0] - 0.85 * 0.15 * 3.0 * 0.02) < 1e-6
    # actor 1: factor 0.05 (depth 0), facing -x at yaw pi/2, yaw rate -0.15 * 3
    np.testing.assert_allclose(pos1[1], mid + [-0.85 * 7.5 * 0.05 * 0.02, 0.0, 0.0], atol=2e-6)
    assert abs(yaw1[1] - (yaw0[1] - 0.85 * 0.15 * 3.0 * 0.02)) < 1e-6
    # actor 2 starts 1 cm inside the -z face and moves 12.75 cm towards it: clamped to the face
    assert pos1[2][2] == np.float32(lo[2])
    # second step: smoothed 0.85 * 7.5 + 0.15 * 6.375 = 7.33125 along the new heading
    h.kinematics()
    pos2 = h.pos.cpu().numpy().astype(np.float64)
    v = 0.85 * 7.5 + 0.15 * 6.375
    np.testing.assert_allclose(pos2[0] - pos1[0], [-v * math.sin(yaw1[0]) * 0.02, 0.0, -v * math.cos(yaw1[0]) * 0.02],
                               atol=2e-6)
    np.testing.assert_allclose(h.prev_linear.cpu().numpy()[0], [v, 0.0, 0.0], rtol=1e-6)
