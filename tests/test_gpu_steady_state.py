"""The boundary's steady state on the GPU: once scenes are loaded (ResidentScenes, or
``torch_sdf.prepare`` for the drop-in), every entry point allocates nothing and never
waits for the device, as the reference's binding on its fast path
(``projects/torch-sdf/cpp_src/bindings.cpp:91-109``, scratch slots preallocated by
its caller, ``sdfdag_backend.py:750-769``). Also: a launch captured into a HIP graph
and replayed on other streams, concurrently with eager launches on the capture
stream, gives the eager results on every replay.
"""

from __future__ import annotations

import sys
import time

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SPIN_CYCLES = 200_000_000  # torch.cuda._sleep: holds the stream for ~0.1 s (2 s at a 100 MHz clock)


def _say(msg: str) -> None:
    print(f"[test_gpu_steady_state] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def scenes():
    from navi_amd import scenes as S

    out = [S.rooms(seed=3, resolution=128), S.cluttered(seed=2, resolution=128)]
    for sc in out:
        sc.compile()
    return out


@pytest.fixture(scope="module")
def setup(gpu, scenes):
    import torch

    from navi_amd import scenes as S
    from navi_amd.multiscene import ResidentScenes

    dev = torch.device("cuda:0")
    res = ResidentScenes([(sc.words, sc.bbox_min_list, sc.bbox_max) for sc in scenes], dev)
    rng = np.random.default_rng(11)
    E, az, el = 6, 64, 16
    env_scene = np.array([0, 1, 1, 0, 1, 0], np.int32)
    origins_env = np.concatenate([scenes[s].free_origins(rng, 1) for s in env_scene])
    yaw = rng.uniform(0, 2 * np.pi, E)
    local = S.canonical_directions(az, el)
    dirs = S.world_directions(local, yaw)
    origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))
    t = {
        "res": res, "E": E, "R": az * el, "az": az, "el": el, "env_scene_np": env_scene,
        "origins_np": origins, "dirs_np": dirs,
        "es": torch.from_numpy(env_scene).to(dev), "o": torch.from_numpy(origins).to(dev),
        "d": torch.from_numpy(dirs).to(dev), "local": torch.from_numpy(local).to(dev),
        "pos": torch.from_numpy(origins_env).to(dev),
        "rot": torch.from_numpy(np.stack([np.cos(yaw), np.sin(yaw)], 1).astype(np.float32)).to(dev),
    }
    return t


def _steady(fn, calls: int = 20) -> None:
    """Warm ``fn`` up, then check that ``calls`` more calls allocate nothing (the caching
    allocator's cumulative allocation count stays put) and that none waits for the
    device: with the stream held by a long spin kernel, every call returns while the
    spin still runs."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    fn()  # a launch that adopts what the first ones measured (scene costs)
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    torch.cuda._sleep(SPIN_CYCLES)
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    host_s = time.perf_counter() - t0
    done = torch.cuda.Event()
    done.record()
    pending = not done.query()
    torch.cuda.synchronize()
    after = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    assert after == before, f"{after - before} allocations in {calls} calls"
    assert pending, f"the calls waited for the device ({host_s:.3f} s of host time)"


def test_resident_scenes_entry_points_steady_state(setup):
    import torch

    t = setup
    res, E, R = t["res"], t["E"], t["R"]
    dev = res.device
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    _say("ResidentScenes.cast_rays")
    _steady(lambda: res.cast_rays(t["es"], t["o"], t["d"], out_d, out_s, 128, 30.0, elevation_bins=t["el"]))
    assert res.scene_cost is not None  # the cost order was measured and adopted during warm-up
    _say("ResidentScenes.cast_rays_poses")
    _steady(lambda: res.cast_rays_poses(t["es"], t["local"], t["pos"], t["rot"], out_d, out_s, 128, 30.0,
                                        elevation_bins=t["el"]))
    pts = t["pos"] + 0.1
    pd = torch.empty(E, device=dev)
    ps = torch.empty(E, device=dev, dtype=torch.int32)
    _say("ResidentScenes.point_query")
    _steady(lambda: res.point_query(pts, pd, ps, point_scene=t["es"]))
    d16 = torch.empty((E, 1, t["el"], t["az"]), device=dev, dtype=torch.float16)
    stats = torch.empty((E, 5), device=dev)
    coll = torch.empty(E, device=dev, dtype=torch.int32)
    _say("ResidentScenes.observe")
    _steady(lambda: res.observe(out_d, t["az"], t["el"], 30.0, out_depth_f16=d16, out_stats=stats,
                                out_collision=coll, points=pts, point_scene=t["es"], point_distances=pd,
                                point_semantics=ps))
    # and the results are still right
    res.cast_rays(t["es"], t["o"], t["d"], out_d, out_s, 128, 30.0, elevation_bins=t["el"])
    torch.cuda.synchronize()
    for e in range(E):
        sc = t["env_scene_np"][e]
        ref = oracle.trace(_words(res, sc), t["origins_np"][e], t["dirs_np"][e], 128, 30.0,
                           *_bounds(res, sc))
        assert np.array_equal(out_d[e].cpu().numpy().view(np.uint32), ref["distance"].view(np.uint32))
        assert np.array_equal(out_s[e].cpu().numpy(), ref["semantic"])


def _words(res, s):
    off = int(res.host_table[s]["word_offset"])
    return res.pool.cpu().numpy().view(np.uint64)[off:off + int(res.host_table[s]["n_words"])]


def _bounds(res, s):
    return [float(v) for v in res.host_table[s]["bbox_min"]], [float(v) for v in res.host_table[s]["bbox_max"]]


def test_dropin_steady_state_after_prepare(setup, scenes):
    """torch_sdf.cast_rays with skip_direction_validation=True, after torch_sdf.prepare at
    scene load: no copy, allocation or wait per call; the record layout is kept until the
    tensor changes (an in-place write bumps its version) or invalidate() drops it."""
    import torch

    from navi_amd import torch_sdf
    from navi_amd import torch_sdf_backend as tsb

    sc = scenes[0]
    dev = setup["res"].device
    dag = torch.from_numpy(sc.words.view(np.int64)).to(dev)
    assert torch_sdf.prepare(dag, sc.bbox_min_list, sc.bbox_max)
    o, d = setup["o"][:2].contiguous(), setup["d"][:2].contiguous()
    out_d = torch.empty(o.shape[:2], device=dev)
    out_s = torch.empty(o.shape[:2], device=dev, dtype=torch.int32)
    _say("torch_sdf.cast_rays")
    _steady(lambda: torch_sdf.cast_rays(dag, o, d, out_d, out_s, 128, 30.0, sc.bbox_min_list, sc.bbox_max, 128,
                                        True, elevation_bins=setup["el"]))
    layout = tsb._layouts[id(dag)]
    torch_sdf.cast_rays(dag, o, d, out_d, out_s, 128, 30.0, sc.bbox_min_list, sc.bbox_max, 128, True)
    assert tsb._layouts[id(dag)] is layout  # no reconversion
    torch_sdf.invalidate(dag)
    assert id(dag) not in tsb._layouts
    torch_sdf.cast_rays(dag, o, d, out_d, out_s, 128, 30.0, sc.bbox_min_list, sc.bbox_max, 128, True)
    torch.cuda.synchronize()
    ref = oracle.trace(sc.words, setup["origins_np"][:2], setup["dirs_np"][:2], 128, 30.0, sc.bbox_min_list,
                       sc.bbox_max)
    assert np.array_equal(out_d.cpu().numpy().view(np.uint32), ref["distance"].view(np.uint32))
    assert np.array_equal(out_s.cpu().numpy(), ref["semantic"])


def test_graph_replay_on_other_streams(setup):
    """A record-layout launch captured into a graph on stream S, replayed on other streams
    while eager launches run on S: each replay and each eager launch gives the eager
    result (each captured launch has a work-queue counter pair of its own)."""
    import torch

    t = setup
    res, E, R = t["res"], t["E"], t["R"]
    dev = res.device
    ref_d = torch.empty((E, R), device=dev)
    ref_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    res.cast_rays(t["es"], t["o"], t["d"], ref_d, ref_s, 128, 30.0, elevation_bins=t["el"])
    torch.cuda.synchronize()
    res.cast_rays(t["es"], t["o"], t["d"], ref_d, ref_s, 128, 30.0, elevation_bins=t["el"])
    torch.cuda.synchronize()  # cost order adopted before the capture: its sort stays out of the graph
    g_d = torch.empty((E, R), device=dev)
    g_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    e_d = torch.empty((E, R), device=dev)
    e_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    _say("capturing one launch")
    with torch.cuda.graph(graph, stream=cap):
        res.cast_rays(t["es"], t["o"], t["d"], g_d, g_s, 128, 30.0, elevation_bins=t["el"])
    torch.cuda.synchronize()
    others = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(4):
        g_d.fill_(float("nan"))
        g_s.fill_(-7)
        e_d.fill_(float("nan"))
        e_s.fill_(-7)
        torch.cuda.synchronize()
        with torch.cuda.stream(cap):
            torch.cuda._sleep(1_000_000)
            res.cast_rays(t["es"], t["o"], t["d"], e_d, e_s, 128, 30.0, elevation_bins=t["el"])
        with torch.cuda.stream(others[rep % 2]):
            graph.replay()
        torch.cuda.synchronize()
        for name, dd, ss in (("replay", g_d, g_s), ("eager", e_d, e_s)):
            assert torch.equal(dd.view(torch.int32), ref_d.view(torch.int32)), f"{name} {rep}: distances"
            assert torch.equal(ss, ref_s), f"{name} {rep}: semantics"
