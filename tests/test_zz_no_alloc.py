"""navi_trace_relaid_noalloc, the tracer entry point that allocates nothing (its
work-queue counters live in a static device array), called through the C ABI and
checked against navi_trace_relaid on the same inputs: distances, semantics and step
counts bit for bit, on two calls in a row, the second with a smaller batch. The scene
pool is built here without ResidentScenes, so in a fresh process the first call is
also the entry point's first call on the device (before any navi_device_init).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pool(scenes, depth):
    """Record pool, scene descriptors and cell tables of several scenes (host arrays)."""
    from navi_amd import _native

    rtable = np.zeros(len(scenes), dtype=_native.RELAID_SCENE_DTYPE)
    recs, roff = [], 0
    for i, sc in enumerate(scenes):
        rec, root, _ = _native.relayout(sc.words)
        rec = rec.copy()
        rec[rec < 0x7FFFFFFD] += np.uint32(roff)
        rtable[i]["rec_offset"], rtable[i]["n_records"] = roff, rec.shape[0]
        rtable[i]["root_slot"] = root if root & 0x80000000 else roff + root
        rtable[i]["bbox_min"], rtable[i]["bbox_max"] = sc.bbox_min_list, sc.bbox_max
        recs.append(rec)
        roff += rec.shape[0]
    allrec = np.concatenate(recs)
    for i in range(len(scenes)):
        rtable[i]["max_depth"] = _native.record_depth(allrec, int(rtable[i]["root_slot"]))
    tables = np.concatenate([_native.cell_table(allrec, int(rtable[i]["root_slot"]), depth)
                             for i in range(len(scenes))])
    return allrec, rtable, tables


def test_noalloc_matches_navi_trace_relaid(gpu):
    import torch

    from navi_amd import _native
    from navi_amd import scenes as S

    scenes = [S.rooms(seed=3, resolution=128), S.cluttered(seed=2, resolution=128)]
    for sc in scenes:
        sc.compile()
    depth = 6
    allrec, rtable, tables = _pool(scenes, depth)
    dev = torch.device("cuda:0")
    records = torch.from_numpy(allrec.view(np.int32).reshape(-1).copy()).to(dev)
    table = torch.from_numpy(rtable.view(np.uint8).copy()).to(dev)
    cells = torch.from_numpy(tables.view(np.int64)).to(dev)
    lib = _native.lib()
    rng = np.random.default_rng(17)
    for call, (E, az, el) in enumerate(((12, 64, 16), (3, 32, 8))):
        R = az * el
        env_scene = rng.integers(0, len(scenes), E).astype(np.int32)
        origins_env = np.concatenate([scenes[s].free_origins(rng, 1) for s in env_scene])
        dirs = S.world_directions(S.canonical_directions(az, el), rng.uniform(0, 2 * np.pi, E))
        origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))
        es = torch.from_numpy(env_scene).to(dev)
        o, d = torch.from_numpy(origins).to(dev), torch.from_numpy(dirs).to(dev)
        outs = {}
        for name in ("navi_trace_relaid_noalloc", "navi_trace_relaid"):
            od = torch.full((E, R), float("nan"), device=dev)
            os_ = torch.full((E, R), -7, device=dev, dtype=torch.int32)
            on = torch.full((E, R), -7, device=dev, dtype=torch.int32)
            print(f"[wip_no_alloc] call {call}: {name}, {E} envs x {R} rays", file=sys.stderr, flush=True)
            stream = torch.cuda.current_stream(dev).cuda_stream
            code = getattr(lib, name)(
                records.data_ptr(), allrec.shape[0], table.data_ptr(), len(scenes), cells.data_ptr(), depth,
                es.data_ptr(), None, E, R, el, o.data_ptr(), d.data_ptr(), od.data_ptr(), os_.data_ptr(),
                128, 30.0, 0.01, on.data_ptr(), stream)
            _native.check(code)
            torch.cuda.synchronize()
            outs[name] = (od.cpu().numpy(), os_.cpu().numpy(), on.cpu().numpy())
        got, want = outs["navi_trace_relaid_noalloc"], outs["navi_trace_relaid"]
        assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), f"call {call}: distances"
        assert np.array_equal(got[1], want[1]), f"call {call}: semantics"
        assert np.array_equal(got[2], want[2]), f"call {call}: step counts"
        assert (want[2] > 0).all() and not np.isnan(want[0]).any()  # every ray traced and written
