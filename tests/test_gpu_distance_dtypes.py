"""Distances written as bfloat16 or float16: the reference roadmap's T2 item
(docs/FUTURE_HARDWARE_ROADMAP.md:140-222: output dtype float32 or bfloat16, float16 as the
fallback, accumulation kept in float32). Every ray against the oracle's float32 distance
rounded to nearest even by torch on the CPU (NaN compared as NaN; the kernel's bfloat16
NaN is 0x7fc0), semantics and step counts exact, through each store site of the record-layout
tracer: output staging (launches without step counts), direct stores (with step counts),
the general march (ranges of 1000 m and more), unknown scene ids, rays from poses, both
shapes of the fast kernel, and the drop-in (which refuses these dtypes on the word-layout
kernel)."""

from __future__ import annotations

import contextlib
import math
import sys

import numpy as np
import pytest

import oracle
from tests.test_gpu_multiscene import _corpus, _oracle_multi, _rays

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[test_gpu_distance_dtypes] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def corpus():
    return _corpus()


@contextlib.contextmanager
def _wide(on: bool):
    from navi_amd import _native

    if not on:
        yield
        return
    old = _native.set_wide_min_rays(0)
    try:
        yield
    finally:
        _native.set_wide_min_rays(old)


def _check_bits(torch, got, ref_d, dtype, label):
    """Non-NaN distances bit-exact against torch's round-to-nearest-even conversion of the
    oracle's; NaN where the oracle has NaN (the kernel's bfloat16 NaN is 0x7fc0)."""
    g = got.cpu().view(torch.int16).numpy()
    want = torch.from_numpy(np.ascontiguousarray(ref_d)).to(dtype).view(torch.int16).numpy()
    nan = np.isnan(ref_d)
    bad = int(np.sum(g[~nan] != want[~nan]))
    assert bad == 0, f"{label}: {bad} {dtype} distances differ"
    assert np.isnan(got.float().cpu().numpy()[nan]).all(), f"{label}: NaN distances"
    if dtype == torch.bfloat16 and nan.any():
        assert (g[nan].view(np.uint16) == 0x7FC0).all(), f"{label}: bfloat16 NaN bits"


def _unknown_as_nan(ref, env):
    """An env of an unknown scene id gets distance NaN, semantic 0 and no steps from the
    tracers (test_gpu_multiscene.py::test_unknown_scene_id_reports_nan); the oracle
    restates the reference, which has no scene table."""
    ref = {k: v.copy() for k, v in ref.items()}
    ref["distance"][env] = np.nan
    ref["semantic"][env] = 0
    ref["steps"][env] = 0
    return ref


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_reduced_distances_every_store_site(gpu, corpus, dtype_name):
    import torch

    from navi_amd import _native
    from navi_amd.multiscene import ResidentScenes

    dtype = getattr(torch, dtype_name)
    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus])
    dev = res.device
    words = [c.words for c in corpus]
    bounds = [c.bbox_min_list + c.bbox_max for c in corpus]
    az, el, E = 32, 16, 12
    env_scene, o, d = _rays(corpus, E, az, el, seed=31)
    env_scene[3] = 77  # an unknown scene id: NaN, semantic 0, no steps
    R = az * el
    t_es = torch.from_numpy(env_scene).to(dev)
    t_o, t_d = torch.from_numpy(o).to(dev), torch.from_numpy(d).to(dev)
    for max_distance in (30.0, 1500.0):  # the fast march, the general march
        ref = _unknown_as_nan(_oracle_multi(words, bounds, env_scene, o, d, 128, max_distance), 3)
        for wide in (False, True):
            for steps in (False, True):  # staged stores, direct stores
                label = f"{dtype_name} range {max_distance} wide {wide} steps {steps}"
                _say(label)
                out_d = torch.full((E, R), -7.0, device=dev, dtype=dtype)
                out_s = torch.full((E, R), -7, device=dev, dtype=torch.int32)
                out_n = torch.full((E, R), -7, device=dev, dtype=torch.int32) if steps else None
                with _wide(wide):
                    res.cast_rays(t_es, t_o, t_d, out_d, out_s, 128, max_distance, out_steps=out_n,
                                  elevation_bins=el)
                    info = _native.last_launch()
                torch.cuda.synchronize()
                _check_bits(torch, out_d, ref["distance"], dtype, label)
                assert np.array_equal(out_s.cpu().numpy(), ref["semantic"]), f"{label}: semantics"
                if steps:
                    assert np.array_equal(out_n.cpu().numpy(), ref["steps"]), f"{label}: steps"
                if wide:  # at 30 m the fast kernel runs; at 1500 m the general march alone
                    assert info["fast"] == (max_distance < 1000.0), (label, info)
    # rays from poses
    valid = env_scene < len(corpus)
    es_p = np.where(valid, env_scene, 0).astype(np.int32)
    from navi_amd import scenes as S

    local = S.canonical_directions(az, el)
    yaw = np.random.default_rng(5).uniform(0, 2 * math.pi, E)
    rot = torch.from_numpy(np.stack([np.cos(yaw), np.sin(yaw)], 1).astype(np.float32)).to(dev)
    c, s_ = rot[:, 0].cpu().numpy()[:, None], rot[:, 1].cpu().numpy()[:, None]
    pd = np.empty((E, R, 3), np.float32)
    pd[..., 0] = local[None, :, 0] * c + local[None, :, 2] * s_
    pd[..., 1] = local[None, :, 1]
    pd[..., 2] = (-local[None, :, 0]) * s_ + local[None, :, 2] * c
    pos = np.ascontiguousarray(o[:, 0])
    ref = _oracle_multi(words, bounds, es_p, o, pd, 128, 30.0)
    out_d = torch.full((E, R), -7.0, device=dev, dtype=dtype)
    out_s = torch.full((E, R), -7, device=dev, dtype=torch.int32)
    res.cast_rays_poses(torch.from_numpy(es_p).to(dev), torch.from_numpy(local).to(dev),
                        torch.from_numpy(pos).to(dev), rot, out_d, out_s, 128, 30.0, elevation_bins=el)
    torch.cuda.synchronize()
    _check_bits(torch, out_d, ref["distance"], dtype, f"{dtype_name} poses")
    assert np.array_equal(out_s.cpu().numpy(), ref["semantic"])
    # float32 launches interleaved on the same stream are unaffected
    out_f = torch.full((E, R), -7.0, device=dev)
    res.cast_rays(t_es, t_o, t_d, out_f, out_s, 128, 30.0, elevation_bins=el)
    torch.cuda.synchronize()
    ref = _unknown_as_nan(_oracle_multi(words, bounds, env_scene, o, d, 128, 30.0), 3)
    gd = out_f.cpu().numpy()
    both = np.isnan(gd) & np.isnan(ref["distance"])
    assert ((gd.view(np.uint32) == ref["distance"].view(np.uint32)) | both).all()
    # the word-layout kernel writes float32 only: refused, not converted
    with pytest.raises(RuntimeError, match="record-layout tracer"):
        res.cast_rays(t_es, t_o, t_d, out_d, out_s, 128, 30.0, kernel="raw")


def test_dropin_reduced_distances(gpu, corpus):
    import torch

    from navi_amd import torch_sdf_backend as B

    sc = corpus[2]
    dev = torch.device("cuda:0")
    env_scene, o, d = _rays([sc], 6, 48, 8, seed=8)
    ref = oracle.trace(sc.words, o, d, 96, 30.0, sc.bbox_min_list, sc.bbox_max, threads=8)
    dag = torch.from_numpy(sc.words.view(np.int64)).to(dev)
    assert B.prepare(dag, sc.bbox_min_list, list(sc.bbox_max))
    t_o, t_d = torch.from_numpy(o).to(dev), torch.from_numpy(d).to(dev)
    for dtype in (torch.bfloat16, torch.float16):
        out_d = torch.empty(o.shape[:2], device=dev, dtype=dtype)
        out_s = torch.empty(o.shape[:2], device=dev, dtype=torch.int32)
        B.cast_rays(dag, t_o, t_d, out_d, out_s, 96, 30.0, sc.bbox_min_list, list(sc.bbox_max), sc.resolution)
        torch.cuda.synchronize()
        _check_bits(torch, out_d, ref["distance"], dtype, f"drop-in {dtype}")
        assert np.array_equal(out_s.cpu().numpy(), ref["semantic"])
        with pytest.raises(RuntimeError, match="record-layout tracer"):
            B.cast_rays(dag, t_o, t_d, out_d, out_s, 96, 30.0, sc.bbox_min_list, list(sc.bbox_max),
                        sc.resolution, kernel="raw")
