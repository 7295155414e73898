"""The largest launches. Exactly 2^30 rays through the record-layout tracer, its limit
(32-bit ray indexing: 3 x (2^30 - 1) + 2 < 2^32), and 2^30 + 16,384 rays through the
drop-in, which then takes the word-layout kernel (64-bit indexing). The rays are 4,096
distinct ones repeated, so every one of the outputs is checked against the oracle's answer
for its ray, on the device. About 36 GB of device memory."""

from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

P = 4096                    # distinct rays
R = 1 << 14                 # rays per env (4 repeats of the pattern)
E = (1 << 30) // R          # 65,536 envs: 2^30 rays
MAX_STEPS, MAX_DISTANCE = 64, 30.0


def _say(msg: str) -> None:
    print(f"[test_gpu_limits] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def case():
    from navi_amd import scenes as S

    sc = S.rooms(seed=3, resolution=128)
    sc.compile()
    rng = np.random.default_rng(30)
    o = sc.free_origins(rng, P).astype(np.float32)
    d = rng.normal(size=(P, 3))
    d = (d / np.linalg.norm(d, axis=-1, keepdims=True)).astype(np.float32)
    ref = oracle.trace(sc.words, o[None], d[None], MAX_STEPS, MAX_DISTANCE, sc.bbox_min_list, sc.bbox_max,
                       threads=8)
    assert (ref["semantic"] != 0).any() and (ref["semantic"] == 0).any()
    return sc, o, d, ref


def _check(torch, out_d, out_s, ref, label):
    """Every output against the oracle's answer for its pattern ray (distance bits, NaN
    as NaN, semantic), counted on the device."""
    dev = out_d.device
    want_d = torch.from_numpy(ref["distance"][0].view(np.int32)).to(dev)
    want_s = torch.from_numpy(ref["semantic"][0].astype(np.int32)).to(dev)
    got_d = out_d.view(-1, P)
    nan_ref = torch.from_numpy(np.isnan(ref["distance"][0])).to(dev)
    bad_d = ((got_d.view(torch.int32) != want_d[None]) & ~(torch.isnan(got_d) & nan_ref[None])).sum().item()
    bad_s = (out_s.view(-1, P) != want_s[None]).sum().item()
    _say(f"{label}: {bad_d} distances and {bad_s} semantics differ")
    assert bad_d == 0 and bad_s == 0, label


def test_largest_launches(gpu, case):
    import torch

    from navi_amd import _native
    from navi_amd import torch_sdf_backend as B
    from navi_amd.multiscene import ResidentScenes

    sc, o, d, ref = case
    dev = torch.device("cuda:0")
    reps = E * R // P
    _say(f"{E} envs x {R} rays = {E * R} rays, record-layout tracer")
    origins = torch.from_numpy(o).to(dev).repeat(reps, 1).view(E, R, 3)
    dirs = torch.from_numpy(d).to(dev).repeat(reps, 1).view(E, R, 3)
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    res = ResidentScenes([(sc.words, sc.bbox_min_list, sc.bbox_max)], dev)
    es = torch.zeros(E, dtype=torch.int32, device=dev)
    res.cast_rays(es, origins, dirs, out_d, out_s, MAX_STEPS, MAX_DISTANCE)
    info = _native.last_launch()
    torch.cuda.synchronize()
    assert info["n_rays"] == 1 << 30 and not info["raw"], info
    _check(torch, out_d, out_s, ref, "2^30 rays, record layout")
    del origins, dirs, out_d, out_s, res, es
    torch.cuda.empty_cache()

    # one env more: the drop-in takes the word-layout kernel (64-bit ray indices)
    E2 = E + 1
    _say(f"{E2} envs x {R} rays = {E2 * R} rays, drop-in (word-layout kernel)")
    origins = torch.from_numpy(o).to(dev).repeat(E2 * R // P, 1).view(E2, R, 3)
    dirs = torch.from_numpy(d).to(dev).repeat(E2 * R // P, 1).view(E2, R, 3)
    out_d = torch.empty((E2, R), device=dev)
    out_s = torch.empty((E2, R), device=dev, dtype=torch.int32)
    dag = torch.from_numpy(sc.words.view(np.int64)).to(dev)
    B.cast_rays(dag, origins, dirs, out_d, out_s, MAX_STEPS, MAX_DISTANCE, sc.bbox_min_list, list(sc.bbox_max),
                sc.resolution, skip_direction_validation=True)
    info = _native.last_launch()
    torch.cuda.synchronize()
    assert info["raw"] and info["n_rays"] == E2 * R, info
    _check(torch, out_d, out_s, ref, "2^30 + 16384 rays, word layout")
