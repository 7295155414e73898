"""Throughput of the batched .gmdag sphere tracer on one MI355X.

Headline workload: 16 seeded procedural scenes compiled at 1024^3 and all
resident on the GPU (8 cluttered volumes, 8 room grids; seeds 100..115), 1024
envs each assigned a scene id by seed, 256 x 48 rays per env (12,582,912 rays
per step), max 256 steps, max distance 30 m, hit epsilon 0.01. A "step" is one
trace of every ray of the batch, inputs already in HBM.

Prints one JSON line: rays/s, the dominant kernel's roofline (algorithmic bytes
per launch / HIP-event launch time vs the 8 TB/s HBM peak), the CPU oracle timed
on the host cores, and the parity of the timed kernel's outputs against it; the
same columns for each smaller workload of the benchmark definition and for the
observation step (navi_amd/workloads.py defines all of them).
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
# MI355X: 256 CUs of 4 SIMDs in 8 XCDs; a SIMD issues one wave64 VALU instruction per
# 4 cycles (16 lanes), at the 2.4 GHz peak engine clock of the published 157.3 TFLOP/s
# fp32 figure (packed FMA: 4 flops per lane and cycle).
SIMDS = 256 * 4
XCDS = 8
VALU_PEAK = SIMDS * 2.4e9 / 4  # wave64 VALU instructions per second
CPU_RUNS = 5  # timed oracle runs (after one warm-up); the median is reported
PROFILE_PATH = ROOT / "profiles" / "tracer_counters.json"
# the sources of libnavi_trace.so (a counter profile is keyed by their digest)
TRACER_SOURCES = ("navi_amd/csrc/trace_relaid.hip", "navi_amd/csrc/navi_trace.hip", "navi_amd/csrc/observation.hip",
                  "navi_amd/csrc/relayout.cpp", "navi_amd/csrc/errors.cpp", "navi_amd/csrc/trace_common.hpp",
                  "navi_amd/csrc/log1p_nonneg.h",
                  "navi_amd/csrc/Makefile", "include/navi_trace.h")
# one rocprofv3 run per counter group and workload, each followed by the copy
# calibration (cd /tmp && export TMPDIR=/tmp first; W = a --profile-workload name)
PROFILE_COMMANDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof/W/kt -o run -- "
    "python -u bench.py --profile-workload W --copy-calibration-mb 1024",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/prof/W/fetch -o run -- "
    "python -u bench.py --profile-workload W --copy-calibration-mb 1024",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/prof/W/write -o run -- "
    "python -u bench.py --profile-workload W --copy-calibration-mb 1024",
    "rocprofv3 --pmc SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR SQ_INSTS_LDS SQ_INSTS_BRANCH "
    "SQ_WAVES GRBM_GUI_ACTIVE --output-format csv -d gpurun_out/prof/W/sq -o run -- "
    "python -u bench.py --profile-workload W --copy-calibration-mb 1024",
    "python bench.py --summarize-profiles gpurun_out/prof profiles/tracer_counters.json",
]
PROFILE: dict = {}  # the counter profile's workloads (main loads it)
PROFILE_CURRENT = False  # whether it was taken on this run's sources
PROFILE_WORKLOADS = ("headline", "box_room_64@0.01", "box_room_64@0.001", "cluttered_128@0.01", "rooms_512@0.01",
                     "observation")


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(fn, launches: int, warmup: int):
    """HIP events on the current stream around each of ``launches`` calls of ``fn`` (after
    ``warmup`` untimed calls): per-launch times in ms."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(launches + 1)]
    evs[0].record(stream)
    for k in range(launches):
        fn()
        evs[k + 1].record(stream)
    torch.cuda.synchronize()
    return np.array([evs[k].elapsed_time(evs[k + 1]) for k in range(launches)])


def time_graph(fn, calls: int, replays: int):
    """``calls`` calls of ``fn`` captured into one HIP graph (launched back to back, no host
    in between), the graph replayed ``replays`` times between HIP events on the current
    stream: per-call times in ms, one per replay. For kernels shorter than a host launch,
    where events around single launches also time the dispatch."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on the capture's stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    out = []
    for _ in range(replays):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) / calls)
    del graph
    return np.array(out)


def time_cpu(fn):
    """One warm-up, then the median of CPU_RUNS timed calls (s); returns (median, last result)."""
    out = fn()
    times = []
    for _ in range(CPU_RUNS):
        t = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times)), out


def parity(gd, gs, gn, ref, gw=None) -> dict:
    """Mismatch counts of GPU outputs against the oracle's (distances compared bit for bit;
    both NaN counts as equal)."""
    both_nan = np.isnan(gd) & np.isnan(ref["distance"])
    dd = np.where(both_nan, 0.0, np.abs(gd.astype(np.float64) - ref["distance"]))
    out = {
        "rays": int(gd.size),
        "hit_mismatch": int(np.sum((gs != 0) != (ref["semantic"] != 0))),
        "semantic_mismatch": int(np.sum(gs != ref["semantic"])),
        "steps_mismatch": int(np.sum(gn != ref["steps"])),
        "max_abs_dd": float(np.nanmax(dd)) if dd.size else 0.0,
        "bit_exact_distance": int(np.sum((gd.view(np.uint32) == ref["distance"].view(np.uint32)) | both_nan)),
    }
    if gw is not None:
        out["words_mismatch"] = int(np.sum(gw.astype(np.uint64) != ref["words"]))
    return out


def source_digest() -> str:
    """First 16 hex digits of the SHA-256 over the tracer library's sources: a counter
    profile applies to the launches of this run only when it was taken on these."""
    h = hashlib.sha256()
    for rel in TRACER_SOURCES:
        h.update(rel.encode())
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def load_profile(path: Path) -> tuple[dict, bool]:
    """The committed counter profile's per-workload entries and whether it was taken on
    this run's sources ({}, False when there is none)."""
    if not path.exists():
        return {}, False
    prof = json.loads(path.read_text())
    return prof.get("workloads", {}), prof.get("source_sha16") == source_digest()


def roofline(kernel: str, ms: float, alg_bytes: int, counters: dict | None = None, current: bool = False) -> dict:
    """The dominant kernel against the resource that bounds it, at this run's launch time
    ``ms``. With a counter profile of the same sources and workload (``counters``):
    ``bound`` "valu" when VALU issue fills more of the SIMDs' cycles than the measured HBM
    bytes fill of the HBM peak, else "hbm"; ``achieved`` is VALU wave-instructions (or
    measured HBM bytes) per launch over ``ms``; the other resource's fraction is given
    beside it. Without one, ``bound`` is "hbm" and the fractions are null. Either way
    ``hbm_equivalent`` prices the reference algorithm's DAG-word loads, ray inputs and
    outputs (``alg_bytes``) at ``ms``: what the reference kernel would move, not a bound
    of this one (it exceeds the HBM peak where the cell tables, LDS split planes and leaf
    runs serve those loads on chip)."""
    s = ms / 1e3
    eq = alg_bytes / s / 1e9
    out = {"bound": "hbm", "achieved": None, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": None,
           "traffic": None, "kernel": kernel,
           "hbm_equivalent": {"achieved": round(eq, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(eq / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": int(alg_bytes)},
           "counters": None}
    if not counters:
        return out
    traffic = counters.get("hbm_bytes_per_launch")
    valu = counters.get("valu_per_launch")
    out["counters"] = {"instance": counters.get("instance"), "source_current": current,
                       "profile_median_ms": counters.get("median_ms"), "valu_per_launch": valu,
                       "hbm_bytes_per_launch": traffic}
    if not current:  # taken on other sources: reported, not used
        return out
    hbm = None
    if traffic:
        hbm = {"achieved": round(traffic / s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
               "frac": round(traffic / s / 1e9 / HBM_PEAK_GBS, 4)}
        out["traffic"] = int(traffic)
    valu_frac = valu / s / VALU_PEAK if valu else None
    if valu_frac is not None and (hbm is None or valu_frac >= hbm["frac"]):
        out.update({"bound": "valu", "achieved": round(valu / s / 1e9, 2), "peak": round(VALU_PEAK / 1e9, 1),
                    "unit": "G VALU wave64-instructions/s", "frac": round(valu_frac, 4), "hbm": hbm})
    elif hbm is not None:
        out.update(achieved=hbm["achieved"], frac=hbm["frac"])
        if valu_frac is not None:
            out["valu"] = {"achieved": round(valu / s / 1e9, 2), "peak": round(VALU_PEAK / 1e9, 1),
                           "unit": "G VALU wave64-instructions/s", "frac": round(valu_frac, 4)}
    return out


def summarize_profiles(root: Path, out_path: Path) -> None:
    """Writes the counter profile from rocprofv3 CSV output under ``root``: one folder per
    workload (named as bench.py's --profile-workload), each with the sub-folders ``kt``
    (--kernel-trace), ``fetch`` (--pmc FETCH_SIZE), ``write`` (--pmc WRITE_SIZE) and
    ``sq`` (--pmc SQ_INSTS_VALU ... GRBM_GUI_ACTIVE). Per workload: the tracer kernel with
    the most time (and the observation kernel where present), medians over its
    dispatches; FETCH_SIZE and WRITE_SIZE scaled by what they read for the run's
    calibration copy (bench.py --copy-calibration-mb)."""
    import csv
    import statistics

    def rows(d: Path, suffix: str):
        files = sorted(d.glob(f"**/*{suffix}"))
        return list(csv.DictReader(open(files[0]))) if files else []

    def per_dispatch(d: Path):
        acc: dict = {}
        for r in rows(d, "counter_collection.csv"):
            key = (r["Dispatch_Id"], r["Kernel_Name"])
            acc.setdefault(key, {}).setdefault(r["Counter_Name"], 0.0)
            acc[key][r["Counter_Name"]] += float(r["Counter_Value"])
        return acc

    def short(name: str) -> str:
        # the name without its trailing parameter list (the parenthesis matching the last)
        depth, cut = 0, len(name)
        for i in range(len(name) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(name[i], 0)
            if depth == 0 and name[i] == "(":
                cut = i
                break
        return name[:cut].replace("void ", "").replace("(anonymous namespace)::", "").replace("navi::", "")

    workloads = {}
    cal_mib = None
    for wdir in sorted(p for p in root.iterdir() if p.is_dir()):
        kt = rows(wdir / "kt", "kernel_trace.csv")
        if not kt:
            continue
        times: dict = {}
        for r in kt:
            times.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6)
        tracers = [k for k in times if ("trace_fast_kernel" in k or "trace_relaid_kernel" in k)]
        kernels = [max(tracers, key=lambda k: sum(times[k]))] if tracers else []
        kernels += [k for k in times if "observation_kernel" in k]
        fetch, write, sq = per_dispatch(wdir / "fetch"), per_dispatch(wdir / "write"), per_dispatch(wdir / "sq")

        def scale(acc, counter):
            cal = [v[counter] for (d, k), v in acc.items() if "copyBuffer" in k and counter in v]
            return max(cal) if cal else None

        log = (wdir / "cal_mib.txt")
        mib = int(log.read_text()) if log.exists() else 1024
        cal_mib = mib
        f_cal, w_cal = scale(fetch, "FETCH_SIZE"), scale(write, "WRITE_SIZE")
        f_scale = mib * 1024 / f_cal if f_cal else None
        w_scale = mib * 1024 / w_cal if w_cal else None
        for k in kernels:
            def med(acc, counter):
                v = [c[counter] for (d, name), c in acc.items() if name == k and counter in c]
                return statistics.median(v) if v else None

            entry = {"instance": short(k), "dispatches": len(times[k]),
                     "median_ms": round(statistics.median(times[k]), 5),
                     "mean_ms": round(statistics.fmean(times[k]), 5)}
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR", "SQ_INSTS_LDS",
                      "SQ_INSTS_BRANCH", "SQ_WAVES", "GRBM_GUI_ACTIVE"):
                v = med(sq, c)
                if v is not None:
                    entry[c] = v
            fk, wk = med(fetch, "FETCH_SIZE"), med(write, "WRITE_SIZE")
            if fk is not None and wk is not None and f_scale and w_scale:
                entry["fetch_kib"], entry["write_kib"] = fk, wk
                entry["fetch_scale"], entry["write_scale"] = round(f_scale, 5), round(w_scale, 5)
                entry["hbm_bytes_per_launch"] = int(round((fk * f_scale + wk * w_scale) * 1024))
            if "SQ_INSTS_VALU" in entry:
                entry["valu_per_launch"] = entry["SQ_INSTS_VALU"]
                if "GRBM_GUI_ACTIVE" in entry:
                    # VALU issue cycles (4 per wave64 instruction) over the SIMDs' cycles
                    # (GRBM_GUI_ACTIVE sums the dispatch's cycles over the 8 XCDs)
                    entry["valu_issue_frac"] = round(entry["SQ_INSTS_VALU"] * 4 / SIMDS
                                                     / (entry["GRBM_GUI_ACTIVE"] / XCDS), 4)
            name = wdir.name if "observation_kernel" not in k else wdir.name + ":observation_kernel"
            workloads[name] = entry
    out = {"source_sha16": source_digest(), "calibration_copy_mib": cal_mib,
           "valu_peak_per_s": VALU_PEAK, "workloads": workloads,
           "commands": PROFILE_COMMANDS}
    out_path.write_text(json.dumps(out, indent=1) + "\n")


def single_scene_config(cfg, dev, threads, profile_eps=None):
    """One smaller workload: the record-layout tracer timed per launch, the word-layout
    counting launch for the algorithmic bytes, the oracle timed on the whole ray set, and
    the parity of the timed kernel's outputs (one entry per hit epsilon). With
    ``profile_eps`` only that epsilon's timed launches run (a profiler's workload)."""
    import torch

    import oracle
    from navi_amd import workloads as W
    from navi_amd.multiscene import ResidentScenes

    sc = cfg.scene()
    sc.compile(threads=threads)
    res = ResidentScenes([(sc.words, sc.bbox_min_list, sc.bbox_max)], dev)
    o_np, d_np = W.single_scene_rays(cfg, sc)
    o = torch.from_numpy(o_np).to(dev)
    d = torch.from_numpy(d_np).to(dev)
    E, R = d_np.shape[:2]
    es = torch.zeros(E, dtype=torch.int32, device=dev)
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    out_n = torch.empty((E, R), device=dev, dtype=torch.int32)
    out_w = torch.empty((E, R), device=dev, dtype=torch.int32)
    out = []
    for eps in cfg.hit_epsilons:
        def launch():
            res.cast_rays(es, o, d, out_d, out_s, cfg.max_steps, W.MAX_DISTANCE, hit_epsilon=eps,
                          elevation_bins=cfg.el)

        if profile_eps is not None:
            if eps == profile_eps:
                time_launches(launch, 50, 10)
            continue
        res.cast_rays(es, o, d, out_d, out_s, cfg.max_steps, W.MAX_DISTANCE, hit_epsilon=eps, out_words=out_w,
                      kernel="raw")
        torch.cuda.synchronize()
        words = int(out_w.to(torch.int64).sum().item())
        launches = time_launches(launch, 50, 10)
        ms = float(np.median(launches))
        # the last timed launch's outputs, then the step counts of one more launch
        timed_d, timed_s = out_d.cpu().numpy(), out_s.cpu().numpy()
        res.cast_rays(es, o, d, out_d, out_s, cfg.max_steps, W.MAX_DISTANCE, hit_epsilon=eps, out_steps=out_n,
                      elevation_bins=cfg.el)
        torch.cuda.synchronize()
        t_cpu, ref = time_cpu(lambda: oracle.trace(sc.words, o_np, d_np, cfg.max_steps, W.MAX_DISTANCE,
                                                   sc.bbox_min_list, sc.bbox_max, hit_epsilon=eps,
                                                   threads=threads))
        alg = E * R * (24 + 8) + 8 * words
        out.append({
            "workload": cfg.describe() + f", hit epsilon {eps:g}",
            "rays": E * R,
            "ms": round(ms, 4),
            "launch_ms": {"median": round(ms, 4), "p10": round(float(np.percentile(launches, 10)), 4),
                          "p90": round(float(np.percentile(launches, 90)), 4), "launches": int(launches.size)},
            "rays_per_s": round(E * R / (ms / 1e3), 1),
            "dag_words_per_ray": round(words / (E * R), 3),
            "roofline": roofline("record-layout tracer", ms, alg, PROFILE.get(f"{cfg.name}@{eps:g}"), PROFILE_CURRENT),
            "cpu_baseline": {"value": round(E * R / t_cpu, 1), "unit": "rays/s", "cores": threads, "kind": "port",
                             "sample": f"the whole ray set ({E * R} rays), median of {CPU_RUNS} runs "
                                       f"after 1 warm-up"},
            "parity": parity(timed_d, timed_s, out_n.cpu().numpy(), ref, out_w.cpu().numpy()),
        })
        _log(f"{out[-1]['workload']}: {ms:.4f} ms, parity {out[-1]['parity']}")
    return out


def observation_walk(res, corpus, env_scene, origins_env, yaw, args, threads, cpu_envs):
    """The observation step, 128 seeded random-walk steps (navi_amd.workloads.ObservationWalk),
    timed with HIP events; then the last step's trace, fp16 depth, statistics and point
    queries against the oracle, and its algorithmic bytes from a counting launch."""
    import torch

    import oracle
    from navi_amd import workloads as W

    E, R = len(env_scene), W.AZ * W.EL
    walk = W.ObservationWalk(res, env_scene, origins_env, yaw, args.obs_steps, max_steps=args.max_steps,
                             max_distance=args.max_distance)
    walk.step(0)  # warm-up (the poses then start from step 1's state)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for k in range(args.obs_steps):
        walk.step(k)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.obs_steps
    moved = float((walk.pd.view(E, W.POINTS_PER_ENV)[:, 0] >= W.CLEARANCE).float().mean().item())
    observe_ms = float(np.median(time_launches(walk.observe, 20, 3)))
    # the post-pass kernel alone: 32 launches back to back in a graph (events around one
    # launch of ~20 us also time its dispatch)
    observe_kernel_ms = float(np.median(time_graph(walk.observe, 32, 5)))
    trace_ms = float(np.median(time_launches(walk.trace, 20, 3)))

    # the final poses: trace and observe once more, then check against the oracle
    walk.trace()
    walk.observe()
    torch.cuda.synchronize()
    o_np, d_np = walk.explicit_rays()
    t_o = torch.from_numpy(o_np).to(res.device)
    t_d = torch.from_numpy(d_np).to(res.device)
    t_es = walk.env_scene
    out_w = torch.empty((E, R), device=res.device, dtype=torch.int32)
    out_n = torch.empty((E, R), device=res.device, dtype=torch.int32)
    cd = torch.empty((E, R), device=res.device)
    cs = torch.empty((E, R), device=res.device, dtype=torch.int32)
    res.cast_rays(t_es, t_o, t_d, cd, cs, args.max_steps, args.max_distance, out_words=out_w, kernel="raw")
    res.cast_rays_poses(t_es, walk.local, walk.pos, walk.rot, cd, cs, args.max_steps, args.max_distance,
                        out_steps=out_n, elevation_bins=W.EL)
    torch.cuda.synchronize()
    words = int(out_w.to(torch.int64).sum().item())
    del t_o, t_d, cd, cs

    pool, base, nw, bounds = W.corpus_oracle_inputs(corpus)
    sample = _env_sample(env_scene, len(corpus), cpu_envs)
    es_np = np.asarray(env_scene)[sample]
    t_cpu, ref = time_cpu(lambda: oracle.trace_multi(pool, base, nw, bounds, es_np, o_np[sample], d_np[sample],
                                                     args.max_steps, args.max_distance, threads=threads))
    gd = walk.out_d.cpu().numpy()[sample]
    trace_parity = parity(gd, walk.out_s.cpu().numpy()[sample], out_n.cpu().numpy()[sample], ref)
    want = oracle.observe(ref["distance"], W.AZ, W.EL, args.max_distance)
    got16 = walk.depth16.cpu().numpy()[sample]
    stats = walk.stats.cpu().numpy()[sample]
    pts = walk.pts.view(-1, 3).cpu().numpy()
    pscene = walk.pscene.cpu().numpy()
    pw_total, pq_mismatch = 0, 0
    gpd, gps, gpk = walk.pd.cpu().numpy(), walk.ps.cpu().numpy(), walk.pk.cpu().numpy()
    for s, c in enumerate(corpus):
        idx = np.flatnonzero(pscene == s)
        if idx.size == 0:
            continue
        q = oracle.point_query(c.words, pts[idx], c.bbox_min_list, c.bbox_max)
        pw_total += int(q["words"].sum())
        pq_mismatch += int(np.sum((gpd[idx].view(np.uint32) != q["distance"].view(np.uint32))
                                  & ~(np.isnan(gpd[idx]) & np.isnan(q["distance"]))))
        pq_mismatch += int(np.sum(gps[idx] != q["semantic"]) + np.sum(gpk[idx] != q["kind"]))
    # depths lie in [0, 1]: the difference of their binary16 bit patterns counts ulps
    depth_ulps = np.abs(got16.view(np.uint16).astype(np.int32) - want["depth16"].view(np.uint16).astype(np.int32))
    n_pts = int(pts.shape[0])
    alg = E * R * (24 + 8) + 8 * words + 2 * E * R + n_pts * (12 + 8) + 8 * pw_total
    obs_alg = E * R * (4 + 2) + E * 5 * 4 + E * 4 + n_pts * (12 + 8) + 8 * pw_total
    trace_alg = E * R * (24 + 8) + 8 * words
    return {
        "workload": f"{E} envs x {W.AZ}x{W.EL} rays from poses, {args.obs_steps} seeded random-walk steps "
                    f"(dpos ~ N(0, 0.05 m), dyaw ~ N(0, 0.1 rad), move kept if its point SDF >= 0.15 m), "
                    f"fp16 (env, 1, {W.EL}, {W.AZ}) depth + per-env stats + {n_pts} point queries per step",
        "rays_per_s": round(E * R / (ms / 1e3), 1),
        "ms_per_step": round(ms, 4),
        "observe_launch_ms": round(observe_ms, 4),
        "observe_kernel_ms": round(observe_kernel_ms, 4),
        "entry_points": ["navi_trace_relaid_poses", "navi_observe"],
        "last_step_moves_kept": round(moved, 4),
        "mean_min_distance": round(float(walk.stats[:, 0].mean().item()), 4),
        "trace_launch_ms": round(trace_ms, 4),
        "roofline": roofline("trace_fast_kernel (rays from poses)", trace_ms, trace_alg,
                             PROFILE.get("observation"), PROFILE_CURRENT),
        "observation_kernel_roofline": roofline("observation_kernel", observe_kernel_ms, obs_alg,
                                                PROFILE.get("observation:observation_kernel"), PROFILE_CURRENT),
        "step_hbm_equivalent": {"achieved": round(alg / (ms / 1e3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(alg / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                                "algorithmic_bytes_per_step": int(alg)},
        "cpu_baseline": {"value": round(sample.size * R / t_cpu, 1), "unit": "rays/s", "cores": threads,
                         "kind": "port",
                         "sample": f"the last step's rays of {sample.size} envs (the first "
                                   f"{max(1, cpu_envs // len(corpus))} of each scene), tracing only, median of "
                                   f"{CPU_RUNS} runs after 1 warm-up"},
        "parity": dict(trace_parity,
                       depth16_max_ulp=int(depth_ulps.max()) if depth_ulps.size else 0,
                       min_distance_mismatch=int(np.sum(stats[:, 0].view(np.uint32)
                                                        != want["stats"][:, 0].view(np.uint32))),
                       ratio_max_abs_diff=float(np.abs(stats[:, 1:] - want["stats"][:, 1:]).max()),
                       point_queries=n_pts, point_query_mismatch=pq_mismatch),
    }


def _env_sample(env_scene, n_scenes, cpu_envs):
    """The first cpu_envs // n_scenes envs of each scene (all envs when cpu_envs >= E)."""
    E = len(env_scene)
    if cpu_envs >= E:
        return np.arange(E)
    per = max(1, cpu_envs // n_scenes)
    sample = []
    for s in range(n_scenes):
        sample.extend(np.flatnonzero(np.asarray(env_scene) == s)[:per].tolist())
    return np.array(sorted(sample))


def dropin_timing(corpus, env_scene, t_o, t_d, args):
    """The drop-in torch_sdf.cast_rays on one resident DAG (scene 0) for the envs that use
    it: record-layout tracer (prepared once per DAG tensor) versus the word-layout kernel."""
    import torch

    from navi_amd import torch_sdf
    from navi_amd import workloads as W

    idx = torch.from_numpy(np.flatnonzero(env_scene == 0)).to(t_o.device)
    o = t_o.index_select(0, idx).contiguous()
    d = t_d.index_select(0, idx).contiguous()
    sc = corpus[0]
    dag = torch.from_numpy(sc.words.view(np.int64)).to(t_o.device)
    out_d = torch.empty(o.shape[:2], device=t_o.device)
    out_s = torch.empty(o.shape[:2], device=t_o.device, dtype=torch.int32)
    result = {"envs": int(idx.numel()), "rays": int(o.shape[0] * o.shape[1]), "scene": sc.name}
    t0 = time.perf_counter()
    torch_sdf.prepare(dag, sc.bbox_min_list, list(sc.bbox_max))
    result["prepare_s"] = round(time.perf_counter() - t0, 3)
    for kernel, reps in (("auto", 10), ("raw", 2)):
        def call():
            torch_sdf.cast_rays(dag, o, d, out_d, out_s, args.max_steps, args.max_distance, sc.bbox_min_list,
                                list(sc.bbox_max), args.resolution, True, elevation_bins=W.EL, kernel=kernel)
        ms = float(np.mean(time_launches(call, reps, 1)))
        # host wall time per call with a synchronize after each (Python checks included)
        t0 = time.perf_counter()
        for _ in range(reps):
            call()
            torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) / reps * 1e3
        result[kernel] = {"rays_per_s": round(result["rays"] / (ms / 1e3), 1), "ms": round(ms, 3),
                          "wall_ms": round(wall_ms, 3)}
    return result


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--envs", type=int, default=1024)
    ap.add_argument("--resolution", type=int, default=1024)
    ap.add_argument("--scenes", type=int, default=16)
    ap.add_argument("--max-steps", type=int, default=256)
    ap.add_argument("--max-distance", type=float, default=30.0)
    ap.add_argument("--cpu-envs", type=int, default=1024,
                    help="envs in the CPU-baseline sample (taken evenly over the scenes; all by default)")
    ap.add_argument("--obs-cpu-envs", type=int, default=128,
                    help="envs of the observation step's last step traced by the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-raw", action="store_true", help="skip timing the reference-layout kernel")
    ap.add_argument("--headline-only", action="store_true",
                    help="time the headline workload only (no smaller workloads, observation step or drop-in)")
    ap.add_argument("--obs-steps", type=int, default=128,
                    help="observation-step workload: steps of seeded random-walk poses (0 to skip)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="first run one device copy of this many MiB (known HBM bytes) so a "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE run can scale the tracer's counters")
    ap.add_argument("--profile", default=str(PROFILE_PATH),
                    help="counter profile of the tracer's launches (bench.py --summarize-profiles writes it)")
    ap.add_argument("--profile-workload", choices=PROFILE_WORKLOADS,
                    help="run only this workload's timed launches and print nothing (for rocprofv3)")
    ap.add_argument("--summarize-profiles", nargs=2, metavar=("PROF_DIR", "OUT_JSON"),
                    help="write the counter profile from rocprofv3 output (see PROFILE_COMMANDS) and exit")
    args = ap.parse_args()

    global PROFILE, PROFILE_CURRENT
    if args.summarize_profiles:
        summarize_profiles(Path(args.summarize_profiles[0]), Path(args.summarize_profiles[1]))
        return 0
    PROFILE, PROFILE_CURRENT = load_profile(Path(args.profile))

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(rays shard by env with no exchange; see DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    import oracle
    from navi_amd import scenes as S
    from navi_amd import workloads as W
    from navi_amd.multiscene import ResidentScenes

    n_cpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    dev = torch.device("cuda:0")
    if args.copy_calibration_mb > 0:
        n_cal = args.copy_calibration_mb * (1 << 20) // 4
        src = torch.ones(n_cal, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # reads and writes exactly copy_calibration_mb MiB each
        torch.cuda.synchronize()
        del src, dst
    if args.profile_workload and "@" in args.profile_workload:
        name, eps = args.profile_workload.split("@")
        cfg = next(c for c in W.SMALL_CONFIGS if c.name == name)
        single_scene_config(cfg, dev, n_cpu, profile_eps=float(eps))
        torch.cuda.synchronize()
        return 0
    t0 = time.time()
    seeds = list(range(100, 100 + args.scenes))
    corpus = W.build_corpus(seeds, args.resolution, n_cpu, W.scene_cache_dir(ROOT))
    t_compile = time.time() - t0
    _log(f"compiled {len(corpus)} scenes @{args.resolution}^3 in {t_compile:.1f}s, "
         f"{sum(c.words.size for c in corpus) * 8 / 1e6:.1f} MB of words")

    env_scene, origins_env, yaw, local = W.corpus_rays(corpus, args.envs)
    dirs = S.world_directions(local, yaw)
    origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))

    res = ResidentScenes([(c.words, c.bbox_min_list, c.bbox_max) for c in corpus], dev)
    t_es = torch.from_numpy(env_scene).to(dev)
    t_o = torch.from_numpy(origins).to(dev)
    t_d = torch.from_numpy(dirs).to(dev)
    E, R = dirs.shape[:2]
    n_rays = E * R
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    out_n = torch.empty((E, R), device=dev, dtype=torch.int32)
    out_w = torch.empty((E, R), device=dev, dtype=torch.int32)

    def step(kernel="relaid"):
        res.cast_rays(t_es, t_o, t_d, out_d, out_s, args.max_steps, args.max_distance, kernel=kernel,
                      elevation_bins=W.EL)

    def timed(kernel, steps, warmup):
        for _ in range(warmup):
            step(kernel)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(dev)
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(steps):
            step(kernel)
        ev1.record(stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / steps

    if args.profile_workload is None:
        # untimed: counts of words the reference algorithm loads (word-layout counting kernel)
        res.cast_rays(t_es, t_o, t_d, out_d, out_s, args.max_steps, args.max_distance, out_words=out_w,
                      kernel="raw")
        torch.cuda.synchronize()
        total_words = int(out_w.to(torch.int64).sum().item())

    # untimed set-up, whatever --warmup says: the first record-layout launch measures the
    # scenes' costs and a later one adopts the cost order (then cached)
    for _ in range(4):
        step()
        torch.cuda.synchronize()
        if res.scene_cost is not None:
            break
    step()
    torch.cuda.synchronize()
    if args.profile_workload == "headline":
        timed("relaid", 12, 3)
        return 0
    if args.profile_workload == "observation":
        walk = W.ObservationWalk(res, env_scene, origins_env, yaw, 16, max_steps=args.max_steps,
                                 max_distance=args.max_distance)
        for k in range(16):
            walk.step(k)
        torch.cuda.synchronize()
        return 0
    ms_raw = timed("raw", max(1, args.steps // 4), 1) if not args.no_raw else None
    ms = timed("relaid", args.steps, args.warmup)
    rays_per_s = n_rays / (ms / 1e3)
    launches = time_launches(step, args.steps, 0)
    launch_ms = {"median": round(float(np.median(launches)), 4), "p10": round(float(np.percentile(launches, 10)), 4),
                 "p90": round(float(np.percentile(launches, 90)), 4), "launches": int(launches.size)}
    # the last timed launch's distances and semantics, then one more launch with its
    # own step counts (a launch asked for step counts stores each ray's outputs itself)
    timed_d, timed_s = out_d.cpu().numpy(), out_s.cpu().numpy()
    res.cast_rays(t_es, t_o, t_d, out_d, out_s, args.max_steps, args.max_distance, out_steps=out_n,
                  elevation_bins=W.EL)
    torch.cuda.synchronize()
    mean_steps = float(out_n.float().mean().item())
    hit_rate = float((out_s != 0).float().mean().item())
    alg_bytes = n_rays * (24 + 8) + 8 * total_words
    _log(f"headline: {ms:.4f} ms per step, {rays_per_s / 1e9:.3f} G rays/s")

    cpu = None
    par = None
    if not args.no_cpu:
        sample = _env_sample(env_scene, len(corpus), args.cpu_envs)
        if sample.size == E:
            sample_text = f"the whole batch: {E} envs x {R} rays = {E * R} rays"
        else:
            sample_text = (f"{sample.size} envs x {R} rays = {sample.size * R} rays (the first "
                           f"{max(1, args.cpu_envs // len(corpus))} envs of each of the {len(corpus)} scenes)")
        pool, base, nw, bounds = W.corpus_oracle_inputs(corpus)
        o_s, d_s, es_s = origins[sample], dirs[sample], env_scene[sample]
        t_cpu, ref = time_cpu(lambda: oracle.trace_multi(pool, base, nw, bounds, es_s, o_s, d_s, args.max_steps,
                                                         args.max_distance, threads=n_cpu))
        cpu = {"value": round(sample.size * R / t_cpu, 1), "unit": "rays/s", "cores": n_cpu,
               "kind": "port", "cpu_model": _cpu_model(),
               "sample": f"{sample_text}, median of {CPU_RUNS} timed runs after 1 warm-up"}
        # distances and semantics of the last timed launch, step counts of the launch that returns them
        par = parity(timed_d[sample], timed_s[sample], out_n.cpu().numpy()[sample], ref, out_w.cpu().numpy()[sample])
        par["timed_vs_step_launch_mismatch"] = int(np.sum(
            (timed_d.view(np.uint32) != out_d.cpu().numpy().view(np.uint32)) | (timed_s != out_s.cpu().numpy())))
        _log(f"headline parity {par}")

    # the same launches writing bfloat16 distances (the reference roadmap's T2 output):
    # timed alike, and every distance against the float32 launch's rounded to bfloat16
    out_bf = torch.empty((E, R), device=dev, dtype=torch.bfloat16)
    res.cast_rays(t_es, t_o, t_d, out_bf, out_s, args.max_steps, args.max_distance, elevation_bins=W.EL)
    bf_launches = time_launches(
        lambda: res.cast_rays(t_es, t_o, t_d, out_bf, out_s, args.max_steps, args.max_distance,
                              elevation_bins=W.EL), 20, 3)
    want_bf = torch.from_numpy(timed_d).to(dev).to(torch.bfloat16)
    nan_bf = torch.isnan(want_bf)
    bf16 = {"ms": round(float(np.median(bf_launches)), 4),
            "rays_per_s": round(n_rays / (float(np.median(bf_launches)) / 1e3), 1),
            "mismatch_vs_float32_rounded": int(((out_bf.view(torch.int16) != want_bf.view(torch.int16)) & ~nan_bf)
                                               .sum().item() + (torch.isnan(out_bf) != nan_bf).sum().item()),
            "output_bytes": n_rays * 2}
    del out_bf, want_bf, nan_bf

    small = obs = dropin = None
    if not args.headline_only:
        small = []
        for cfg in W.SMALL_CONFIGS:
            small.extend(single_scene_config(cfg, dev, n_cpu))
        if args.obs_steps > 0:
            obs = observation_walk(res, corpus, env_scene, origins_env, yaw, args, n_cpu, args.obs_cpu_envs)
            _log(f"observation step: {obs['ms_per_step']} ms, parity {obs['parity']}")
        dropin = dropin_timing(corpus, env_scene, t_o, t_d, args)

    default_workload = (len(corpus), args.resolution, E, R, args.max_steps) == (16, 1024, 1024, 12288, 256)
    line = {
        "metric": "rays/sec on 1 MI355X (256x48 rays/env)",
        "value": round(rays_per_s, 1),
        "unit": "rays/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "launch_ms": launch_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded procedural scenes and poses)",
        "config": {
            "workload": f"{len(corpus)} resident scenes @{args.resolution}^3 (seeds {seeds[0]}..{seeds[-1]}), "
                        f"{E} envs x {W.AZ}x{W.EL} rays, max {args.max_steps} steps, max {args.max_distance} m",
            "envs": E, "rays_per_env": R, "rays_per_step": n_rays, "scenes": len(corpus),
            "resolution": args.resolution, "max_steps": args.max_steps,
            "max_distance": args.max_distance, "hit_epsilon": 0.01,
            "entry_point": "navi_trace_relaid", "dag_bytes": res.pool_bytes,
            "record_bytes": res.record_bytes,
            "raw_layout_kernel_rays_per_s": None if ms_raw is None else round(n_rays / (ms_raw / 1e3), 1),
            "mean_steps_per_ray": round(mean_steps, 3), "hit_rate": round(hit_rate, 4),
            "dag_words_per_ray": round(total_words / n_rays, 3),
        },
        "roofline": roofline("trace_fast_kernel", ms, alg_bytes, PROFILE.get("headline") if default_workload else None,
                             PROFILE_CURRENT),
        "cpu_baseline": cpu,
        "parity": par,
        "small_configs": small,
        "observation_step": obs,
        "dropin_cast_rays": dropin,
        "bf16_distances": bf16,
        "scene_compile_s": round(t_compile, 2),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
