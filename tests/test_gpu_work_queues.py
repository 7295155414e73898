"""Work-queue pairs, launch info and 16-bit semantics on the record layout, on the GPU,
each against the oracle or an eager launch bit for bit:

* the 1024-thread fast kernel (the benchmark's shape, forced for a small batch)
  captured into a graph and replayed on other streams beside eager launches;
* capture pairs given back when their graphs are destroyed: the fast kernel still
  runs after more captures than the table holds;
* reserve pairs leased per launch once every table pair is taken (one raw HIP
  stream per launch);
* leaves of semantic 0x7fff and above traced on the record layout (fast and general
  march, rays from poses, point queries, the drop-in).
"""

from __future__ import annotations

import contextlib
import ctypes
import gc
import os
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[test_gpu_work_queues] {msg}", file=sys.stderr, flush=True)


def _threads() -> int:
    return min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1)


@contextlib.contextmanager
def wide_for_every_launch():
    """Every launch whose planes fit takes the 1024-thread fast kernel (restored after)."""
    from navi_amd import _native

    old = _native.set_wide_min_rays(0)
    try:
        yield
    finally:
        _native.set_wide_min_rays(old)


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
    rng = np.random.default_rng(23)
    E, az, el = 6, 64, 16
    env_scene = np.array([0, 1, 1, 0, 1, 0], np.int32)
    origins_env = np.concatenate([scenes[s].free_origins(rng, 1) for s in env_scene])
    dirs = S.world_directions(S.canonical_directions(az, el), rng.uniform(0, 2 * np.pi, E))
    origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))
    pool = np.concatenate([sc.words for sc in scenes])
    base = np.cumsum([0] + [sc.words.size for sc in scenes[:-1]]).astype(np.uint64)
    nw = np.array([sc.words.size for sc in scenes], np.uint64)
    bounds = np.array([sc.bbox_min_list + sc.bbox_max for sc in scenes], np.float32)
    ref = oracle.trace_multi(pool, base, nw, bounds, env_scene, origins, dirs, 128, 30.0, threads=_threads())
    return {"res": res, "E": E, "R": az * el, "el": el, "env_scene": env_scene, "origins": origins, "dirs": dirs,
            "es": torch.from_numpy(env_scene).to(dev), "o": torch.from_numpy(origins).to(dev),
            "d": torch.from_numpy(dirs).to(dev), "ref": ref}


def _check(out_d, out_s, ref, what):
    gd, gs = out_d.cpu().numpy(), out_s.cpu().numpy()
    assert np.array_equal(gs, ref["semantic"]), f"{what}: semantics"
    assert np.array_equal(gd.view(np.uint32), ref["distance"].view(np.uint32)), f"{what}: distances"


def test_wide_fast_kernel_graph_replay_on_other_streams(setup):
    """The benchmark's launch shape (trace_fast_kernel in 1024-thread workgroups, then
    trace_relaid_kernel reading whether the first traced the launch) captured on stream S
    and replayed on other streams while eager launches run on S: every replay and every
    eager launch gives the oracle's results."""
    import torch

    from navi_amd import _native

    t = setup
    res, E, R = t["res"], t["E"], t["R"]
    dev = res.device
    out = [torch.empty((E, R), device=dev), torch.empty((E, R), device=dev, dtype=torch.int32)]
    with wide_for_every_launch():
        for _ in range(2):  # the first launch measures the scenes' costs, the second adopts the order
            res.cast_rays(t["es"], t["o"], t["d"], out[0], out[1], 128, 30.0, elevation_bins=t["el"])
            torch.cuda.synchronize()
        info = _native.last_launch()
        assert info["fast"] and info["fast_wide"] and info["combined"] and info["queue"] == "stream", info
        _check(out[0], out[1], t["ref"], "eager")
        g_d, e_d = torch.empty((E, R), device=dev), torch.empty((E, R), device=dev)
        g_s = torch.empty((E, R), device=dev, dtype=torch.int32)
        e_s = torch.empty((E, R), device=dev, dtype=torch.int32)
        cap = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        _say("capturing the wide fast kernel")
        with torch.cuda.graph(graph, stream=cap):
            res.cast_rays(t["es"], t["o"], t["d"], g_d, g_s, 128, 30.0, elevation_bins=t["el"])
        info = _native.last_launch()
        assert info["fast_wide"] and info["queue"] == "capture", info
        torch.cuda.synchronize()
        others = [torch.cuda.Stream(), torch.cuda.Stream()]
        for rep in range(6):
            for x in (g_d, e_d):
                x.fill_(float("nan"))
            for x in (g_s, e_s):
                x.fill_(-7)
            torch.cuda.synchronize()
            with torch.cuda.stream(cap):
                torch.cuda._sleep(1_000_000)
                res.cast_rays(t["es"], t["o"], t["d"], e_d, e_s, 128, 30.0, elevation_bins=t["el"])
            with torch.cuda.stream(others[rep % 2]):
                graph.replay()
            torch.cuda.synchronize()
            _check(g_d, g_s, t["ref"], f"replay {rep}")
            _check(e_d, e_s, t["ref"], f"eager {rep}")


def test_capture_pairs_are_given_back(setup):
    """A capture's pair stays its own while its executable graph lives (two live graphs
    replayed at once on two streams both give the oracle's results) and comes back when
    the graph is destroyed: 4,200 captures, more than the table's 4,032 pairs, all get a
    capture pair and enqueue the fast kernel."""
    import torch

    from navi_amd import _native

    t = setup
    res, E, R = t["res"], t["E"], t["R"]
    dev = res.device
    cap = torch.cuda.Stream()
    bufs = [(torch.empty((E, R), device=dev), torch.empty((E, R), device=dev, dtype=torch.int32)) for _ in range(2)]
    with wide_for_every_launch():
        graphs, pairs = [], []
        for k in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                res.cast_rays(t["es"], t["o"], t["d"], bufs[k][0], bufs[k][1], 128, 30.0, elevation_bins=t["el"])
            info = _native.last_launch()
            assert info["queue"] == "capture" and info["fast"], info
            graphs.append(g)
            pairs.append(info["pair"])
        assert pairs[0] != pairs[1], "a live graph's pair was handed to another capture"
        torch.cuda.synchronize()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for rep in range(3):
            for k in range(2):
                bufs[k][0].fill_(float("nan"))
                bufs[k][1].fill_(-7)
            torch.cuda.synchronize()
            for k in range(2):
                with torch.cuda.stream(streams[k]):
                    graphs[k].replay()
            torch.cuda.synchronize()
            for k in range(2):
                _check(bufs[k][0], bufs[k][1], t["ref"], f"graph {k}, replay {rep}")
        del graphs
        gc.collect()
        torch.cuda.synchronize()
        _say("4200 capture / destroy cycles")
        seen = set()
        for i in range(4200):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                res.cast_rays(t["es"], t["o"], t["d"], bufs[0][0], bufs[0][1], 128, 30.0, elevation_bins=t["el"])
            info = _native.last_launch()
            assert info["queue"] == "capture" and info["fast"] and 0 <= info["pair"] < 4032, (i, info)
            seen.add(info["pair"])
            if i == 4199:
                bufs[0][0].fill_(float("nan"))
                bufs[0][1].fill_(-7)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                _check(bufs[0][0], bufs[0][1], t["ref"], "the 4200th capture")
            del g
        _say(f"distinct capture pairs used: {len(seen)}")
        assert len(seen) < 4032


def test_leased_pairs_when_the_table_is_full(setup):
    """Launches on new streams until the table's pairs are all taken: further launches
    lease reserve pairs (index 4032 and up), traced with the fast kernel, and a lease
    is free again once its launch has completed."""
    import torch

    from navi_amd import _native

    t = setup
    res, E, R = t["res"], t["E"], t["R"]
    dev = res.device
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    order = res.env_order(t["es"])
    L = res._launch_args(t["es"].data_ptr(), order, E, R, t["el"], out_d.data_ptr(), out_s.data_ptr(), None, 128,
                         30.0, 0.01)
    L.origins, L.dirs = t["o"].data_ptr(), t["d"].data_ptr()
    torch.cuda.synchronize()
    streams = []
    leases = []
    try:
        with wide_for_every_launch():
            for i in range(4200):
                s = ctypes.c_void_p()
                assert hip.hipStreamCreate(ctypes.byref(s)) == 0
                streams.append(s)
                _native.check(_native.lib().navi_trace_relaid_ex(ctypes.byref(L), s))
                info = _native.last_launch()
                assert info["queue"] in ("stream", "lease"), (i, info)
                if info["queue"] == "lease":
                    assert info["pair"] >= 4032 and info["fast"], info
                    assert hip.hipStreamSynchronize(s) == 0
                    leases.append(info["pair"])
                    if len(leases) == 3:
                        break
            assert len(leases) == 3, "no launch leased a reserve pair"
            torch.cuda.synchronize()
            _check(out_d, out_s, t["ref"], "leased launch")
            assert len(set(leases)) >= 1
    finally:
        torch.cuda.synchronize()
        for s in streams:
            hip.hipStreamDestroy(s)


def _wide_scene_words(words, seed=5):
    """The DAG with every non-zero leaf semantic moved into [0x7ff0, 0xffff]."""
    w = np.asarray(words, np.uint64).copy()
    leaf = (w >> np.uint64(63)) == 1
    sem = (w >> np.uint64(16)) & np.uint64(0xFFFF)
    new = np.random.default_rng(seed).integers(0x7FF0, 0x10000, w.size).astype(np.uint64)
    sel = leaf & (sem != 0)
    w[sel] = (w[sel] & ~np.uint64(0xFFFF << 16)) | (new[sel] << np.uint64(16))
    return w


def test_wide_semantics_on_the_record_layout(gpu, scenes):
    """A pool of a scene with 16-bit semantics (leaf table), one without, and one with
    16-bit semantics and a negative leaf (no NAVI_SCENE_NONNEG_LEAVES: the general
    march): explicit rays, rays from poses, point queries and the drop-in, every output
    against the oracle (which reads the word layout's 16-bit field), on the record
    layout."""
    import torch

    from navi_amd import _native, torch_sdf
    from navi_amd import scenes as S
    from navi_amd.multiscene import ResidentScenes
    from navi_amd import torch_sdf_backend as tsb

    dev = torch.device("cuda:0")
    wide = _wide_scene_words(scenes[0].words)
    neg = _wide_scene_words(scenes[1].words, seed=6)
    leaf_idx = np.flatnonzero((neg >> np.uint64(63)) == 1)
    neg[leaf_idx[len(leaf_idx) // 2]] |= np.uint64(0x8000)  # one leaf distance made negative
    words = [wide, scenes[1].words, neg]
    sc_of = [scenes[0], scenes[1], scenes[1]]
    res = ResidentScenes([(w, s.bbox_min_list, s.bbox_max) for w, s in zip(words, sc_of)], dev)
    assert res.relaid_ok and res.n_leaves > 0
    flags = res.relaid_table.cpu().numpy().view(_native.RELAID_SCENE_DTYPE)["flags"]
    assert list(flags) == [1, 1, 0]
    pool = np.concatenate(words)
    base = np.cumsum([0] + [w.size for w in words[:-1]]).astype(np.uint64)
    nw = np.array([w.size for w in words], np.uint64)
    bounds = np.array([s.bbox_min_list + s.bbox_max for s in sc_of], np.float32)
    rng = np.random.default_rng(41)
    E, az, el = 12, 64, 16
    R = az * el
    for launch_scenes in ((0, 1), (0, 1, 2)):  # without and with the negative-leaf scene
        env_scene = np.array([launch_scenes[i % len(launch_scenes)] for i in range(E)], np.int32)
        origins_env = np.concatenate([sc_of[s].free_origins(rng, 1) for s in env_scene]).astype(np.float32)
        yaw = rng.uniform(0, 2 * np.pi, E)
        local = S.canonical_directions(az, el)
        dirs = S.world_directions(local, yaw)
        origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))
        ref = oracle.trace_multi(pool, base, nw, bounds, env_scene, origins, dirs, 128, 30.0, threads=_threads())
        assert (ref["semantic"] >= 0x8000).any()
        es, o, d = (torch.from_numpy(x).to(dev) for x in (env_scene, origins, dirs))
        out_d = torch.empty((E, R), device=dev)
        out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
        out_n = torch.empty((E, R), device=dev, dtype=torch.int32)
        for with_steps in (False, True):
            for wide_shape in (False, True):  # the combined kernel alone, or the 1024-thread fast kernel first
                with wide_for_every_launch() if wide_shape else contextlib.nullcontext():
                    out_d.fill_(float("nan"))
                    out_s.fill_(-7)
                    res.cast_rays(es, o, d, out_d, out_s, 128, 30.0, elevation_bins=el,
                                  out_steps=out_n if with_steps else None)
                info = _native.last_launch()
                assert not info["raw"] and info["combined"] and info["fast_wide"] == wide_shape, info
                torch.cuda.synchronize()
                _check(out_d, out_s, ref, f"scenes {launch_scenes}, steps {with_steps}, wide {wide_shape}")
                if with_steps:
                    assert np.array_equal(out_n.cpu().numpy(), ref["steps"])
        # rays from poses: the same rays, built in the kernel
        rot = torch.from_numpy(np.stack([np.cos(yaw), np.sin(yaw)], 1).astype(np.float32)).to(dev)
        c, s_ = rot[:, 0].cpu().numpy()[:, None], rot[:, 1].cpu().numpy()[:, None]
        pd = np.empty((E, R, 3), np.float32)
        pd[..., 0] = local[None, :, 0] * c + local[None, :, 2] * s_
        pd[..., 1] = local[None, :, 1]
        pd[..., 2] = (-local[None, :, 0]) * s_ + local[None, :, 2] * c
        pref = oracle.trace_multi(pool, base, nw, bounds, env_scene, origins, pd, 128, 30.0, threads=_threads())
        for wide_shape in (False, True):
            with wide_for_every_launch() if wide_shape else contextlib.nullcontext():
                res.cast_rays_poses(es, torch.from_numpy(local).to(dev), torch.from_numpy(origins_env).to(dev), rot,
                                    out_d, out_s, 128, 30.0, elevation_bins=el)
            torch.cuda.synchronize()
            _check(out_d, out_s, pref, f"poses, scenes {launch_scenes}, wide {wide_shape}")
    # point queries in every scene
    pts = np.concatenate([rng.uniform(s.bbox_min_list, s.bbox_max, (300, 3)) for s in sc_of]).astype(np.float32)
    pscene = np.repeat(np.arange(3, dtype=np.int32), 300)
    pdist = torch.empty(900, device=dev)
    psem = torch.empty(900, device=dev, dtype=torch.int32)
    pkind = torch.empty(900, device=dev, dtype=torch.int32)
    res.point_query(torch.from_numpy(pts).to(dev), pdist, psem, point_scene=torch.from_numpy(pscene).to(dev),
                    out_kind=pkind)
    torch.cuda.synchronize()
    for k in range(3):
        q = oracle.point_query(words[k], pts[pscene == k], sc_of[k].bbox_min_list, sc_of[k].bbox_max)
        sel = pscene == k
        assert np.array_equal(psem.cpu().numpy()[sel], q["semantic"]), f"point semantics, scene {k}"
        assert np.array_equal(pkind.cpu().numpy()[sel], q["kind"]), f"point kinds, scene {k}"
        assert np.array_equal(pdist.cpu().numpy()[sel].view(np.uint32), q["distance"].view(np.uint32))
    # the drop-in: prepare converts the wide DAG to the record layout
    dag = torch.from_numpy(wide.view(np.int64)).to(dev)
    sc = scenes[0]
    assert torch_sdf.prepare(dag, sc.bbox_min_list, sc.bbox_max)
    o1, d1 = torch.from_numpy(origins[:2].copy()).to(dev), torch.from_numpy(dirs[:2].copy()).to(dev)
    out_d1 = torch.empty((2, R), device=dev)
    out_s1 = torch.empty((2, R), device=dev, dtype=torch.int32)
    torch_sdf.cast_rays(dag, o1, d1, out_d1, out_s1, 128, 30.0, sc.bbox_min_list, sc.bbox_max, 128, True)
    assert not _native.last_launch()["raw"]
    torch.cuda.synchronize()
    ref1 = oracle.trace(wide, origins[:2], dirs[:2], 128, 30.0, sc.bbox_min_list, sc.bbox_max)
    _check(out_d1, out_s1, ref1, "drop-in")
    tsb.invalidate(dag)
