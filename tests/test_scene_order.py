"""Host logic of the cost-ordered work queue (navi_amd/multiscene.py): the
measured per-scene step sums become scene costs, and envs are handed to the
tracer grouped by scene, costliest first, unknown scene ids last. The GPU test
test_scene_order_follows_measured_cost runs the measurement end to end."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.test_host_layout import _chain_words


class _Done:
    def query(self) -> bool:
        return True


class _Pending:
    def query(self) -> bool:
        return False


def _scenes(n):
    words = _chain_words(3)
    return [(words, [0.0, 0.0, 0.0], [1.0 + i, 1.0, 1.0]) for i in range(n)]


def _expected_order(env_scene, cost):
    n = cost.size
    pos = np.empty(n, np.int64)
    pos[np.argsort(-cost, kind="stable")] = np.arange(n)
    known = (env_scene >= 0) & (env_scene < n)
    key = np.where(known, pos[np.clip(env_scene, 0, n - 1)], n)
    return np.argsort(key, kind="stable")


def test_costs_become_the_env_order():
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes(_scenes(4), "cpu")
    assert res.order_by_cost and res.scene_cost is None
    env_scene = torch.tensor([2, 0, 3, -1, 1, 2, 4, 0, 3, 1], dtype=torch.int32)
    # before any measurement: by scene id, unknown ids where they sort
    assert np.array_equal(res.env_order(env_scene).numpy(), np.argsort(env_scene.numpy(), kind="stable"))
    # step sums and ray counts per scene (the last column collects unknown ids);
    # scene 3 has the most steps per ray, scene 1 none measured (gets the mean)
    host = torch.tensor([[300, 0, 500, 2000, 77], [100, 0, 100, 400, 9]], dtype=torch.int64)
    res._cost_host.copy_(host)
    res._cost_pending, res._cost_event = True, _Pending()
    res._poll_cost()
    assert res.scene_cost is None  # the copy has not completed: nothing changes
    res._cost_event = _Done()
    res._poll_cost()
    want = np.array([3.0, (3.0 + 5.0 + 5.0) / 3, 5.0, 5.0])
    assert np.allclose(res.scene_cost, want, rtol=0, atol=1e-12)
    got = res.env_order(env_scene).numpy()
    assert np.array_equal(got, _expected_order(env_scene.numpy(), res.scene_cost))
    # scenes 2 and 3 tie at 5 steps per ray and keep their id order; then 1, then 0
    assert env_scene.numpy()[got].tolist() == [2, 2, 3, 3, 1, 1, 0, 0, -1, 4]
    # a changed env_scene is re-sorted with the adopted costs
    env_scene[0] = 0
    got = res.env_order(env_scene).numpy()
    assert np.array_equal(got, _expected_order(env_scene.numpy(), res.scene_cost))


@pytest.mark.parametrize("order_by_cost,n_scenes", [(False, 3), (True, 1)])
def test_no_measurement_when_off_or_single_scene(order_by_cost, n_scenes):
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes(_scenes(n_scenes), "cpu", order_by_cost=order_by_cost)
    assert not res.order_by_cost
    steps, measure = res._cost_steps(None, 2, 8, True)
    assert steps is None and not measure


def test_measurement_uses_the_callers_steps_once():
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes(_scenes(2), "cpu")
    mine = torch.zeros((2, 8), dtype=torch.int32)
    steps, measure = res._cost_steps(mine, 2, 8, True)
    assert steps is mine and measure
    steps, measure = res._cost_steps(None, 2, 8, False)  # unsorted launches never measure
    assert steps is None and not measure
    res._cost_pending, res._cost_event = True, _Pending()
    steps, measure = res._cost_steps(None, 2, 8, True)  # one measurement at a time
    assert steps is None and not measure


def test_empty_measurements_are_retried():
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes(_scenes(2), "cpu")
    assert res._cost_steps(None, 0, 8, True) == (None, False)  # empty batches measure nothing
    # only unknown scene ids (last column) were traced: nothing adopted, measured again later
    res._cost_host.copy_(torch.tensor([[0, 0, 50], [0, 0, 10]], dtype=torch.int64))
    res._cost_pending, res._cost_event = True, _Done()
    res._poll_cost()
    assert res.scene_cost is None and not res._cost_pending
    steps, measure = res._cost_steps(None, 2, 8, True)
    assert measure and tuple(steps.shape) == (2, 8)


def test_host_resident_scenes_refuse_to_trace():
    """Scenes kept on the CPU (host logic only) never hand host pointers to the kernels."""
    from navi_amd.multiscene import ResidentScenes

    res = ResidentScenes(_scenes(2), "cpu")
    es = torch.zeros(1, dtype=torch.int32)
    o = torch.zeros((1, 4, 3))
    with pytest.raises(RuntimeError, match="GPU device"):
        res.cast_rays(es, o, o, torch.zeros(1, 4), torch.zeros(1, 4, dtype=torch.int32), 8, 1.0)
    with pytest.raises(RuntimeError, match="GPU device"):
        res.cast_rays_poses(es, torch.zeros(4, 3), torch.zeros(1, 3), torch.zeros(1, 2), torch.zeros(1, 4),
                            torch.zeros(1, 4, dtype=torch.int32), 8, 1.0)
    with pytest.raises(RuntimeError, match="GPU device"):
        res.point_query(torch.zeros(2, 3), torch.zeros(2), torch.zeros(2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU device"):
        res.observe(torch.zeros(1, 4), 2, 2, 1.0)
