"""Throughput of the batched .gmdag sphere tracer on one MI355X.

Workload (default): 16 seeded procedural scenes compiled at 1024^3 and all
resident on the GPU (8 cluttered volumes, 8 room grids; seeds 100..115),
1024 envs each assigned a scene id by seed, 256 x 48 rays per env
(12,582,912 rays per step), max 256 steps, max distance 30 m, hit epsilon 0.01.
A "step" is one trace of every ray of the batch, inputs already in HBM.

Prints one JSON line: rays/s, the dominant kernel's roofline (algorithmic bytes
per launch / HIP-event launch time vs the 8 TB/s HBM peak), the CPU oracle
timed on a bounded sample on the host cores, and the parity of that sample.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
AZ, EL = 256, 48


def _cache_dir() -> Path | None:
    d = os.environ.get("NAVI_SCENE_CACHE", str(ROOT / ".scene_cache"))
    if d in ("", "0", "off"):
        return None
    p = Path(d)
    p.mkdir(parents=True, exist_ok=True)
    return p


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def build_corpus(seeds, resolution, threads_total):
    from navi_amd import scenes as S

    cache = _cache_dir()
    corpus = [S.corpus_scene(int(s), resolution) for s in seeds]
    per = max(1, threads_total // 4)

    def work(sc_seed):
        sc, seed = sc_seed
        path = cache / f"{sc.name}_{seed}_{resolution}.npy" if cache else None
        if path is not None and path.exists():
            sc.words = np.load(path)
        else:
            sc.compile(threads=per)
            if path is not None:
                np.save(path, sc.words)
        return sc

    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        corpus = list(ex.map(work, zip(corpus, seeds)))
    return corpus


def make_rays(corpus, n_envs, seed=4):
    from navi_amd import scenes as S

    rng = np.random.default_rng(seed)
    env_scene = rng.integers(0, len(corpus), n_envs).astype(np.int32)
    yaw = rng.uniform(0.0, 2.0 * math.pi, n_envs)
    origins = np.empty((n_envs, 3), np.float32)
    for s in range(len(corpus)):
        idx = np.flatnonzero(env_scene == s)
        if idx.size:
            origins[idx] = corpus[s].free_origins(rng, idx.size)
    local = S.canonical_directions(AZ, EL)
    return env_scene, origins, yaw, local


def observation_steps(res, t_es, origins_env, yaw_env, E, args):
    """The full observation step, repeated for seeded random-walk poses: trace rays
    generated in the kernel from each env's pose, then one launch that packs the fp16
    (env, 1, El, Az) depth, reduces per-env clearance / ratios / collision and answers 4
    point-SDF queries per env (the proposed move and three probes jittered +-0.3 m). A
    move is kept when the proposed point clears 0.15 m. Returns rays/s over the steps."""
    import torch

    from navi_amd import scenes as S

    dev = res.device
    steps = args.obs_steps
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    pos = torch.from_numpy(np.ascontiguousarray(origins_env, np.float32)).to(dev)
    yaw = torch.from_numpy(np.asarray(yaw_env, np.float32)).to(dev)
    local = torch.from_numpy(S.canonical_directions(AZ, EL)).to(dev)
    dpos = torch.randn((steps, E, 3), generator=gen, device=dev) * 0.05
    dyaw = torch.randn((steps, E), generator=gen, device=dev) * 0.1
    jitter = torch.rand((steps, E, 3, 3), generator=gen, device=dev) * 0.6 - 0.3
    pscene = t_es.repeat_interleave(4)
    rot = torch.empty((E, 2), device=dev)
    pts = torch.empty((E, 4, 3), device=dev)
    R = AZ * EL
    out_d = torch.empty((E, R), device=dev)
    out_s = torch.empty((E, R), device=dev, dtype=torch.int32)
    d16 = torch.empty((E, 1, EL, AZ), device=dev, dtype=torch.float16)
    stats = torch.empty((E, 5), device=dev)
    coll = torch.empty((E,), device=dev, dtype=torch.int32)
    pd = torch.empty((4 * E,), device=dev)
    ps = torch.empty((4 * E,), device=dev, dtype=torch.int32)
    pk = torch.empty((4 * E,), device=dev, dtype=torch.int32)

    def observe():
        res.observe(out_d, AZ, EL, args.max_distance, out_depth_f16=d16, out_stats=stats, out_collision=coll,
                    points=pts.view(-1, 3), point_scene=pscene, point_distances=pd, point_semantics=ps,
                    point_kind=pk)

    def one(k):
        torch.stack((torch.cos(yaw), torch.sin(yaw)), 1, out=rot)
        res.cast_rays_poses(t_es, local, pos, rot, out_d, out_s, args.max_steps, args.max_distance,
                            elevation_bins=EL)
        pts[:, 0] = pos + dpos[k]
        pts[:, 1:] = pos[:, None, :] + jitter[k]
        observe()
        keep = pd.view(E, 4)[:, 0] >= 0.15
        pos.copy_(torch.where(keep[:, None], pts[:, 0], pos))
        yaw.add_(dyaw[k])

    one(0)  # warm-up (the poses then start from step 1's state)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for k in range(steps):
        one(k)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    moved = float((pd.view(E, 4)[:, 0] >= 0.15).float().mean().item())
    ev0.record(stream)
    for _ in range(20):
        observe()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_observe = ev0.elapsed_time(ev1) / 20
    return {
        "workload": f"{E} envs x {AZ}x{EL} rays from poses, {steps} seeded random-walk steps "
                    f"(dpos ~ N(0, 0.05 m), dyaw ~ N(0, 0.1 rad), move kept if its point SDF >= 0.15 m), "
                    f"fp16 (env, 1, {EL}, {AZ}) depth + per-env stats + {4 * E} point queries per step",
        "rays_per_s": round(E * R / (ms / 1e3), 1),
        "ms_per_step": round(ms, 4),
        "observe_launch_ms": round(ms_observe, 4),
        "entry_points": ["navi_trace_relaid_poses", "navi_observe"],
        "last_step_moves_kept": round(moved, 4),
        "mean_min_distance": round(float(stats[:, 0].mean().item()), 4),
    }


def dropin_timing(corpus, env_scene, t_o, t_d, args):
    """The drop-in torch_sdf.cast_rays on one resident DAG (scene 0) for the envs that use
    it: record-layout tracer (converted once per DAG tensor) versus the word-layout kernel."""
    import torch

    from navi_amd import torch_sdf

    idx = torch.from_numpy(np.flatnonzero(env_scene == 0)).to(t_o.device)
    o = t_o.index_select(0, idx).contiguous()
    d = t_d.index_select(0, idx).contiguous()
    sc = corpus[0]
    dag = torch.from_numpy(sc.words.view(np.int64)).to(t_o.device)
    out_d = torch.empty(o.shape[:2], device=t_o.device)
    out_s = torch.empty(o.shape[:2], device=t_o.device, dtype=torch.int32)
    result = {"envs": int(idx.numel()), "rays": int(o.shape[0] * o.shape[1]), "scene": sc.name}
    for kernel, reps in (("auto", 10), ("raw", 2)):
        def call():
            torch_sdf.cast_rays(dag, o, d, out_d, out_s, args.max_steps, args.max_distance, sc.bbox_min_list,
                                list(sc.bbox_max), args.resolution, True, elevation_bins=EL, kernel=kernel)
        t0 = time.perf_counter()
        call()  # auto: converts the DAG once
        torch.cuda.synchronize()
        first = time.perf_counter() - t0
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(reps):
            call()
        ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / reps
        # host wall time per call with a synchronize after each (Python checks included)
        t0 = time.perf_counter()
        for _ in range(reps):
            call()
            torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) / reps * 1e3
        result[kernel] = {"rays_per_s": round(result["rays"] / (ms / 1e3), 1), "ms": round(ms, 3),
                          "wall_ms": round(wall_ms, 3), "first_call_s": round(first, 3)}
    return result


def small_configs(dev):
    """The smaller workloads of the benchmark definition, on the record-layout tracer:
    they are latency-bound (too few rays to fill the chip), reported as ms per launch."""
    import torch

    from navi_amd import scenes as S
    from navi_amd.multiscene import ResidentScenes

    cases = [("1 env x 64x16 rays, box room @64^3, max 64 steps", S.box_room(seed=1, resolution=64), 1, 64, 16, 64),
             ("4 envs x 256x48 rays, cluttered @128^3, max 128 steps", S.cluttered(seed=2, resolution=128), 4, 256,
              48, 128),
             ("64 envs x 256x48 rays, rooms @512^3, max 256 steps", S.rooms(seed=3, resolution=512), 64, 256, 48,
              256)]
    out = []
    for name, sc, envs, az, el, max_steps in cases:
        sc.compile()
        res = ResidentScenes([(sc.words, sc.bbox_min_list, sc.bbox_max)], dev, keep_words=False)
        rng = np.random.default_rng(envs)
        origins = sc.free_origins(rng, envs)
        dirs = S.world_directions(S.canonical_directions(az, el), rng.uniform(0, 2 * math.pi, envs))
        o = torch.from_numpy(np.ascontiguousarray(np.broadcast_to(origins[:, None, :], dirs.shape))).to(dev)
        d = torch.from_numpy(np.ascontiguousarray(dirs)).to(dev)
        es = torch.zeros(envs, dtype=torch.int32, device=dev)
        out_d = torch.empty(o.shape[:2], device=dev)
        out_s = torch.empty(o.shape[:2], device=dev, dtype=torch.int32)
        for _ in range(3):
            res.cast_rays(es, o, d, out_d, out_s, max_steps, 30.0, elevation_bins=el)
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(20):
            res.cast_rays(es, o, d, out_d, out_s, max_steps, 30.0, elevation_bins=el)
        ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / 20
        out.append({"workload": name, "ms": round(ms, 4), "rays_per_s": round(envs * az * el / (ms / 1e3), 1)})
    return out


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
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-raw", action="store_true", help="skip timing the reference-layout kernel")
    ap.add_argument("--obs-steps", type=int, default=128,
                    help="observation-step workload: steps of seeded random-walk poses (0 to skip)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="first run one device copy of this many MiB (known HBM bytes) so a "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE run can scale the tracer's counters")
    ap.add_argument("--traffic-profile", default=str(ROOT / "profiles" / "trace_relaid_kernel_traffic.json"),
                    help="measured HBM bytes per launch (written from rocprofv3 --pmc runs)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(rays shard by env with no exchange; see DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    import oracle
    from navi_amd.multiscene import ResidentScenes

    n_cpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    t0 = time.time()
    seeds = list(range(100, 100 + args.scenes))
    corpus = build_corpus(seeds, args.resolution, n_cpu)
    t_compile = time.time() - t0
    print(f"[bench] compiled {len(corpus)} scenes @{args.resolution}^3 in {t_compile:.1f}s, "
          f"{sum(c.words.size for c in corpus) * 8 / 1e6:.1f} MB of words", file=sys.stderr, flush=True)

    env_scene, origins_env, yaw, local = make_rays(corpus, args.envs)
    from navi_amd import scenes as S

    dirs = S.world_directions(local, yaw)
    origins = np.ascontiguousarray(np.broadcast_to(origins_env[:, None, :], dirs.shape))

    dev = torch.device("cuda:0")
    if args.copy_calibration_mb > 0:
        n_cal = args.copy_calibration_mb * (1 << 20) // 4
        src = torch.ones(n_cal, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # reads and writes exactly copy_calibration_mb MiB each
        torch.cuda.synchronize()
        del src, dst
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
                      elevation_bins=EL)

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

    # untimed: counts of words the reference algorithm loads, and step counts
    res.cast_rays(t_es, t_o, t_d, out_d, out_s, args.max_steps, args.max_distance, out_steps=out_n,
                  out_words=out_w)
    torch.cuda.synchronize()
    total_words = int(out_w.to(torch.int64).sum().item())
    mean_steps = float(out_n.float().mean().item())
    hit_rate = float((out_s != 0).float().mean().item())

    def per_launch(steps):
        """Each launch between its own events (after the bracketed run): the spread."""
        stream = torch.cuda.current_stream(dev)
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        evs[0].record(stream)
        for k in range(steps):
            step("relaid")
            evs[k + 1].record(stream)
        torch.cuda.synchronize()
        return np.array([evs[k].elapsed_time(evs[k + 1]) for k in range(steps)])

    ms_raw = timed("raw", max(1, args.steps // 4), 1) if not args.no_raw else None
    ms = timed("relaid", args.steps, args.warmup)
    rays_per_s = n_rays / (ms / 1e3)
    launches = per_launch(args.steps)
    launch_ms = {"median": round(float(np.median(launches)), 4), "p10": round(float(np.percentile(launches, 10)), 4),
                 "p90": round(float(np.percentile(launches, 90)), 4), "launches": int(launches.size)}

    alg_bytes = n_rays * (24 + 8) + 8 * total_words
    achieved_gbs = alg_bytes / (ms / 1e3) / 1e9

    # CPU baseline + parity on a bounded sample: the first env of each scene
    cpu = None
    parity = None
    if not args.no_cpu:
        if args.cpu_envs >= E:
            sample = np.arange(E)
            sample_text = f"the whole batch: {E} envs x {R} rays = {E * R} rays"
        else:
            per = max(1, args.cpu_envs // len(corpus))
            sample = []
            for s in range(len(corpus)):
                sample.extend(np.flatnonzero(env_scene == s)[:per].tolist())
            sample = np.array(sorted(sample)[: max(args.cpu_envs, len(corpus))])
            sample_text = (f"{sample.size} envs x {R} rays = {sample.size * R} rays (the first {per} envs "
                           f"of each of the {len(corpus)} scenes)")
        pool = np.concatenate([c.words for c in corpus])
        base = np.cumsum([0] + [c.words.size for c in corpus[:-1]]).astype(np.uint64)
        nw = np.array([c.words.size for c in corpus], np.uint64)
        bounds = np.array([c.bbox_min_list + c.bbox_max for c in corpus], np.float32)
        o_s, d_s, es_s = origins[sample], dirs[sample], env_scene[sample]
        threads = n_cpu

        def run_cpu():
            return oracle.trace_multi(pool, base, nw, bounds, es_s, o_s, d_s, args.max_steps,
                                      args.max_distance, threads=threads)

        ref = run_cpu()  # warm-up
        times = []
        for _ in range(2):
            t = time.perf_counter()
            run_cpu()
            times.append(time.perf_counter() - t)
        t_cpu = float(np.median(times))
        cpu = {"value": round(sample.size * R / t_cpu, 1), "unit": "rays/s", "cores": threads,
               "kind": "port", "cpu_model": _cpu_model(),
               "sample": f"{sample_text}, median of 2 timed runs after 1 warm-up"}
        gd = out_d.cpu().numpy()[sample]
        gs = out_s.cpu().numpy()[sample]
        gn = out_n.cpu().numpy()[sample]
        gw = out_w.cpu().numpy()[sample]
        both_nan = np.isnan(gd) & np.isnan(ref["distance"])
        dd = np.where(both_nan, 0.0, np.abs(gd.astype(np.float64) - ref["distance"]))
        parity = {
            "rays": int(gd.size),
            "hit_mismatch": int(np.sum((gs != 0) != (ref["semantic"] != 0))),
            "semantic_mismatch": int(np.sum(gs != ref["semantic"])),
            "steps_mismatch": int(np.sum(gn != ref["steps"])),
            "words_mismatch": int(np.sum(gw.astype(np.uint64) != ref["words"])),
            "max_abs_dd": float(np.nanmax(dd)),
            "bit_exact_distance": int(np.sum((gd.view(np.uint32) == ref["distance"].view(np.uint32)) | both_nan)),
        }

    obs = observation_steps(res, t_es, origins_env, yaw, E, args) if args.obs_steps > 0 else None
    dropin = dropin_timing(corpus, env_scene, t_o, t_d, args) if args.obs_steps > 0 else None
    small = small_configs(dev) if args.obs_steps > 0 else None

    traffic = None
    tp = Path(args.traffic_profile)
    if tp.exists():
        prof = json.loads(tp.read_text())
        if prof.get("workload") == f"{len(corpus)}x{args.resolution}^3/{E}x{R}/{args.max_steps}":
            traffic = int(prof["hbm_bytes_per_launch"])

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
                        f"{E} envs x {AZ}x{EL} rays, max {args.max_steps} steps, max {args.max_distance} m",
            "envs": E, "rays_per_env": R, "rays_per_step": n_rays, "scenes": len(corpus),
            "resolution": args.resolution, "max_steps": args.max_steps,
            "max_distance": args.max_distance, "hit_epsilon": 0.01,
            "entry_point": "navi_trace_relaid", "dag_bytes": res.pool_bytes,
            "record_bytes": res.record_bytes,
            "raw_layout_kernel_rays_per_s": None if ms_raw is None else round(n_rays / (ms_raw / 1e3), 1),
            "mean_steps_per_ray": round(mean_steps, 3), "hit_rate": round(hit_rate, 4),
            "dag_words_per_ray": round(total_words / n_rays, 3),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "trace_relaid_kernel",
            "algorithmic_bytes_per_launch": alg_bytes,
        },
        "cpu_baseline": cpu,
        "parity": parity,
        "observation_step": obs,
        "dropin_cast_rays": dropin,
        "small_configs": small,
        "scene_compile_s": round(t_compile, 2),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
