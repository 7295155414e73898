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
