"""Caller-side restatements, no GPU: canonical ray directions and yaw rotation
(projects/environment/src/navi_environment/backends/sdfdag_backend.py:205-221,1300-1310),
checked with the assertions of projects/environment/tests/unit/test_ray_direction_oracle.py
and test_yaw_rotation_oracle.py; the depth post-pass (sdfdag_backend.py:408-452) with the
known values of test_postprocessing_oracle.py. The product's generator
(navi_amd.scenes.canonical_directions / world_directions) must equal the oracle's.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from navi_amd import scenes as S


def _dir(d, az, el, el_bins):
    return d[az * el_bins + el]


def test_cardinal_directions():
    d = oracle.ray_directions(256, 48)
    np.testing.assert_allclose(_dir(d, 0, 24, 48), [0, 0, -1], atol=0.07)
    np.testing.assert_allclose(_dir(d, 64, 24, 48), [1, 0, 0], atol=0.07)
    np.testing.assert_allclose(_dir(d, 128, 24, 48), [0, 0, 1], atol=0.07)
    np.testing.assert_allclose(_dir(d, 192, 24, 48), [-1, 0, 0], atol=0.07)
    np.testing.assert_allclose(_dir(d, 0, 0, 48), [0, 1, 0], atol=1e-5)
    np.testing.assert_allclose(_dir(d, 0, 47, 48), [0, -1, 0], atol=1e-5)


@pytest.mark.parametrize("az,el", [(8, 3), (64, 16), (256, 48)])
def test_unit_norms(az, el):
    np.testing.assert_allclose(np.linalg.norm(oracle.ray_directions(az, el), axis=-1), 1.0, atol=1e-6)


def test_poles_and_index_map():
    d = oracle.ray_directions(256, 48)
    top = np.array([_dir(d, a, 0, 48) for a in range(256)])
    bot = np.array([_dir(d, a, 47, 48) for a in range(256)])
    assert np.all(np.ptp(top, axis=0) < 1e-5) and np.all(np.ptp(bot, axis=0) < 1e-5)
    small = oracle.ray_directions(16, 5)
    grid = small.reshape(16, 5, 3)
    for a in range(16):
        for e in range(5):
            assert np.array_equal(grid[a, e], small[a * 5 + e])


def test_yaw_rotation():
    local = oracle.ray_directions(32, 8)
    rot = oracle.yaw_rotate(local, [math.pi / 2])[0]
    # forward (0,0,-1) rotated by +90 degrees about y: x' = z sin = -1
    f = _dir(local, 0, 4, 8)
    want = np.array([f[0] * 0 + f[2] * 1, f[1], -f[0] * 1 + f[2] * 0])
    np.testing.assert_allclose(_dir(rot, 0, 4, 8), want, atol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(rot, axis=-1), 1.0, atol=1e-6)


def test_product_ray_generator_equals_oracle():
    assert np.array_equal(S.canonical_directions(256, 48), oracle.ray_directions(256, 48))
    yaw = np.array([0.0, 1.0, 4.0])
    assert np.array_equal(S.world_directions(S.canonical_directions(64, 16), yaw),
                          oracle.yaw_rotate(oracle.ray_directions(64, 16), yaw))


def test_postpass_known_values():
    raw = np.array([[0.5, 1.0, 5.0, 100.0, np.inf, np.nan]], np.float32)
    sem = np.array([[1, 1, 1, 1, 0, 0]], np.int32)
    depth, s, valid, min_d, clamped = oracle.postprocess(raw, sem, 6, 1, 100.0)
    ld = math.log1p(100.0)
    want = [math.log1p(0.5) / ld, math.log1p(1.0) / ld, math.log1p(5.0) / ld, 1.0, 1.0]
    np.testing.assert_allclose(depth.reshape(-1)[:5].numpy(), want, atol=1e-6)
    # the backend marks every finite reading valid (sdfdag_backend.py:432-440)
    assert valid.reshape(-1).tolist() == [True, True, True, True, False, False]
    # torch's amin propagates NaN, as in the reference's post-pass
    assert math.isnan(float(min_d[0]))
    _, _, _, min_d, _ = oracle.postprocess(raw[:, :5], sem[:, :5], 5, 1, 100.0)
    assert float(min_d[0]) == 0.5


def test_fp16_observation_layout():
    rng = np.random.default_rng(0)
    d = rng.uniform(0, 40, (2, 8 * 4)).astype(np.float32)
    obs = oracle.fp16_depth_obs(d, 8, 4, 30.0)
    assert obs.shape == (2, 1, 4, 8) and obs.dtype == np.float16
    ref = (torch.log1p(torch.from_numpy(d).clamp(0, 30)) / math.log1p(30.0)).reshape(2, 8, 4)
    np.testing.assert_allclose(obs[:, 0].astype(np.float32), ref.permute(0, 2, 1).numpy(), atol=1e-3)


def test_postpass_horizon_cases():
    """projects/environment/tests/unit/test_sdfdag_conventions.py:604-730: readings past
    the horizon clamp to depth 1 and stay valid, the horizon itself is depth 1, negative
    (inside-solid) readings clamp to depth 0."""
    depth, _, valid, _, _ = oracle.postprocess(np.array([[5.0, 25.0]], np.float32), np.array([[1, 2]], np.int32),
                                               2, 1, 10.0)
    np.testing.assert_allclose(depth.reshape(-1).numpy(), [math.log1p(5.0) / math.log1p(10.0), 1.0], rtol=1e-6)
    assert valid.reshape(-1).tolist() == [True, True]
    depth, *_ = oracle.postprocess(np.array([[10.0]], np.float32), np.array([[3]], np.int32), 1, 1, 10.0)
    assert float(depth.reshape(-1)[0]) == 1.0
    depth, *_ = oracle.postprocess(np.array([[-0.25]], np.float32), np.array([[9]], np.int32), 1, 1, 10.0)
    assert float(depth.reshape(-1)[0]) == 0.0


def test_observation_ratios_known_answer():
    """test_sdfdag_conventions.py:123-142: one of four pixels each starved (30 >= 20 - 1e-3),
    near (0.6 <= 1.0) and in the structure band [1.5, 10] (3.0), forward sector = both bins."""
    metric = np.array([[30.0, 0.6], [3.0, 15.0]], np.float32)[None]
    clamped = np.clip(metric, 0.0, 20.0)
    r = oracle.observation_ratios(clamped, np.ones_like(metric, bool), 20.0, 1.5, 10.0, 1.0)
    np.testing.assert_allclose(r[0], [0.25, 0.25, 0.25, 0.25])
    obs = oracle.observe(metric.reshape(1, 4), 2, 2, 20.0, band_min=1.5, band_max=10.0, proximity=1.0,
                         clearance=0.7)
    np.testing.assert_allclose(obs["stats"][0], [0.6, 0.25, 0.25, 0.25, 0.25])
    assert obs["collision"].tolist() == [1]


def test_observation_ratios_by_hand():
    """Counts written out cell by cell: 12 azimuth bins x 3 elevations, max 10; the forward
    sector is azimuth bins {0, 1, 10, 11} (12 // 6 = 2 on each side)."""
    az, el = 12, 3
    m = np.full((az, el), 5.0, np.float32)  # in band [1.5, 8], not near, not starved
    m[0, 0] = 0.2                            # near (<= 0.5), not in band
    m[11, 2] = 9.9995                        # starved (>= 9.999) and out of band
    m[5, 1] = np.inf                         # starved after clamping, invalid
    m[6, 1] = np.nan                         # invalid, nothing
    obs = oracle.observe(m.reshape(1, -1), az, el, 10.0, band_min=1.5, band_max=8.0, proximity=0.5, clearance=0.15)
    band = az * el - 4
    fwd_band = 4 * el - 2
    want = [np.nan, 2 / 36, 1 / 36, band / 36, fwd_band / (4 * el)]
    np.testing.assert_allclose(obs["stats"][0, 1:], want[1:], rtol=1e-6)
    assert np.isnan(obs["stats"][0, 0]) and obs["collision"].tolist() == [0]
    m[6, 1] = 3.0
    obs = oracle.observe(m.reshape(1, -1), az, el, 10.0, band_min=1.5, band_max=8.0, proximity=0.5, clearance=0.25)
    assert float(obs["stats"][0, 0]) == np.float32(0.2) and obs["collision"].tolist() == [1]
    # one azimuth bin: the first and last sixth are the same bin, counted twice (torch.cat)
    one = oracle.observe(np.array([[2.0, 20.0]], np.float32), 1, 2, 30.0, band_min=1.5, band_max=8.0)
    assert float(one["stats"][0, 4]) == 0.5
    assert one["depth16"].shape == (1, 1, 2, 1)


def test_observation_stack_and_delta():
    """_consume_observation_batch (sdfdag_backend.py:1501-1526) with the known values of
    test_postprocessing_oracle.py::TestDeltaDepthComputation: delta = current - previous,
    zero on the first frame (previous all zero); obs stacks depth, semantic, valid."""
    az, el = 2, 2
    d = np.array([[0.5, 1.0, np.inf, 3.0], [2.0, 2.0, 2.0, 2.0]], np.float32)
    s = np.array([[1, 2, 0, 4], [5, 5, 5, 5]], np.int32)
    prev = np.zeros((2, az, el), np.float32)
    prev[0] = [[0.2, 0.3], [0.4, 0.5]]
    out = oracle.observe(d, az, el, 10.0, semantics=s, prev_depth=prev)
    ld = math.log1p(10.0)
    want0 = np.array([[math.log1p(0.5), math.log1p(1.0)], [ld, math.log1p(3.0)]]) / ld
    np.testing.assert_allclose(out["depth"][0], want0, atol=1e-6)
    np.testing.assert_allclose(out["delta"][0], want0 - prev[0], atol=1e-6)
    assert (out["delta"][1] == 0).all()  # previous frame was all zeros
    assert out["obs"].shape == (2, 3, az, el)
    assert out["obs"][0, 1].tolist() == [[1.0, 2.0], [0.0, 4.0]]
    assert out["obs"][0, 2].tolist() == [[1.0, 1.0], [0.0, 1.0]]
