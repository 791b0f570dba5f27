#!/usr/bin/env python3
"""Benchmark of the temporal random walk hot path on one MI355X.

Workload (the headline config): directed power-law
graph, 1,000,000 node ids, 20,000,000 edges, src/dst Zipf(s=1.8) mapped through
one shared random permutation, self-loops redrawn, timestamps uniform in
[0, 1e8) quantised to 100,000 values (numpy PCG64, seed 44).  One step =
ingest the whole batch (index build) + sample 10,000,000 walks with
max_walk_len=80, walk_bias=ExponentialIndex, initial_edge_bias=Uniform,
forward in time.  Inputs are resident in HBM before the timed region; the
walks stay in HBM (device-resident boundary).

Prints ONE JSON line.  `value` = walk steps/s (sum of walk lengths, the
reference's definition, test_run/walk_sampling_speed_test.cpp:39-50) over the
wall time of the sampling calls; index-build edges/s is reported beside it.
`roofline` is the walk kernel's compulsory HBM bytes per launch over its
launch time (HIP events), against the 8 TB/s peak; `traffic` is the HBM
traffic one launch measured with rocprofv3 counters, read from
profiles/walk_kernel_cfg2_pmc.json only while the kernel sources still hash to
what that profile measured.  `host_boundary` times the reference's own
boundary once (numpy in, numpy out), and `cpu_baseline` the oracle on the
host cores, in a child process.

`--summarize-pmc` turns rocprofv3 counter runs into the profiles/*_pmc.json
summaries this line reads (see its help).
"""
from __future__ import annotations

import argparse
import glob
import hashlib
import json
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "temporal-random-walk_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "sampled walk steps/s + index-build edges/s, 20M-edge power-law graph, 1 GPU"
HBM_PEAK_GBS = 8000.0
PMC_FILE = os.path.join(ROOT, "profiles", "walk_kernel_cfg2_pmc.json")
CSRC = os.path.join(PKG, "csrc")
# the sources each profiled kernel family is compiled from: a counter profile
# describes the code only while these hash to what it measured
KERNEL_SOURCES = {
    "walk": ["walk.hip", "trw_device.h", "index_layout.h"],
    "build": ["build.hip", "primitives.hip", "primitives.h", "index_layout.h"],
}


# kernels of the walk path; every other kernel belongs to the index build
WALK_PATH_KERNELS = ("walk_kernel", "walk_rows_kernel", "walk_start_kernel", "layout_",
                     "walk_stats",
                     "node_group_init", "node_group_segment", "gather_walk_features")


def sources_sha256(family):
    h = hashlib.sha256()
    for name in KERNEL_SOURCES[family]:
        with open(os.path.join(CSRC, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read() + b"\0")
    return h.hexdigest()


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def make_cfg2(n_nodes, n_edges, n_ts, seed=44):
    from tests import graphs
    return graphs.powerlaw(n_nodes, n_edges, s=1.8, n_ts=n_ts, ts_hi=100_000_000, seed=seed)


def index_algorithmic_bytes(E, Vc, T, g_o, g_i):
    """Compulsory bytes of one ingest of E edges into an empty store
    (directed): read batch 16E, write store 16E, node_ts_sorted 8E out + 8E in,
    node-timestamp groups 8(g_o+g_i), four per-node size_t arrays 32 Vc,
    active flags 4(Vc-1), timestamp groups 16T + 8."""
    return 16 * E + 16 * E + 8 * E + 8 * E + 8 * (g_o + g_i) + 32 * Vc + 4 * (Vc - 1) + 16 * T + 8


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline_child(args):
    """Runs in a child process started by cpu_baseline() (no GPU is touched):
    the oracle -- the C restatement of the reference CPU path -- on the host
    cores with OpenMP, on the cfg2 graph.  One untimed warm-up, then the
    median of `reps` timed rounds of each leg: the full ingest of all 20M
    edges, and a bounded sample of walks (draw generation included, as in the
    reference's CPU sampler, core/temporal_random_walk.cu:568-569).  Prints one
    JSON object."""
    import numpy as np
    from oracle import pyoracle as po

    src, dst, ts = make_cfg2(args.nodes, args.edges, args.timestamps)
    threads = args.cpu_threads
    L, n_walks = args.walk_len, args.cpu_walks
    builds, walks = [], []
    og = None
    for r in range(1 + args.cpu_reps):
        og = po.OracleGraph(True)
        t0 = time.perf_counter()
        og.add_edges(src, dst, ts, num_threads=threads)
        tb = time.perf_counter() - t0
        t0 = time.perf_counter()
        draws = np.random.default_rng(1 + r).random(n_walks * (1 + 2 * L))
        starts = -np.ones(n_walks, dtype=np.int32)
        w = og.walks(L, "ExponentialIndex", "Uniform", True, starts, draws, num_threads=threads)
        tw = time.perf_counter() - t0
        steps = int(w.lens.sum())
        del w, draws
        if r:  # round 0 warms up
            builds.append(tb)
            walks.append(steps / tw)
        print(f"[bench cpu] round {r}: build {tb:.2f} s, {steps} walk steps in {tw:.2f} s",
              file=sys.stderr, flush=True)
    print(json.dumps({"walk_steps_per_s": statistics.median(walks),
                      "build_s": statistics.median(builds),
                      "walk_steps_per_s_all": walks, "build_s_all": builds,
                      "edges": int(len(src))}))


def cpu_baseline(args):
    """The oracle on the host cores, timed in a child process whose OpenMP
    runtime starts with OMP_PROC_BIND=spread and OMP_PLACES=cores (this
    process has already loaded torch's).  Threads: OMP_NUM_THREADS when set
    (the GPU box sets it to its CPU share per GPU), else every core."""
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="spread",
               OMP_PLACES="cores")
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-baseline-child",
           "--cpu-threads", str(threads), "--cpu-walks", str(args.cpu_walks),
           "--cpu-reps", str(args.cpu_reps), "--edges", str(args.edges),
           "--nodes", str(args.nodes), "--timestamps", str(args.timestamps),
           "--walk-len", str(args.walk_len)]
    log(f"cpu baseline: {threads} threads, {args.cpu_walks} walks, median of {args.cpu_reps}")
    r = subprocess.run(cmd, env=env, stdout=subprocess.PIPE, text=True, check=True)
    res = json.loads(r.stdout.strip().splitlines()[-1])
    return {
        "value": res["walk_steps_per_s"],
        "unit": "walk steps/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/trw_oracle.c on the GPU box's host: {args.cpu_walks} walks "
                   f"(L={args.walk_len}, ExponentialIndex/Uniform, fwd) on the full cfg2 graph, "
                   f"draw generation included, and the ingest of all {res['edges']} edges; "
                   f"{threads} OpenMP threads (OMP_PROC_BIND=spread, OMP_PLACES=cores), "
                   f"median of {args.cpu_reps} rounds after a warm-up"),
        "index_build_edges_per_s": res["edges"] / res["build_s"],
        "index_build_cores": threads,
        "walk_steps_per_s_rounds": res["walk_steps_per_s_all"],
        "build_s_rounds": res["build_s_all"],
        "nproc": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
        "cpu_model": cpu_model(),
    }


def summarize_pmc(args):
    """Summarises rocprofv3 counter runs of one kernel into a JSON profile.

    Each --pmc-dir holds one `rocprofv3 --pmc ... -f csv -d DIR -o pmc -- python3
    bench.py ...` run.  Counter values are summed over a dispatch's rows
    (instances), then averaged over the dispatches whose kernel name contains
    --kernel.  FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what
    the same counter read for the plain device copy of --copy-calibration-mib
    MiB that the run made first (the largest __amd_rocclr_copyBuffer
    dispatch), so bytes = KiB * (copy bytes / copy KiB).  The profile is
    stamped with the sha256 of the kernel family's sources."""
    import csv

    def selected(kname, in_build):
        if args.kernel == "@build":  # every dispatch of an ingest
            return in_build
        return any(k in kname for k in args.kernel.split("|"))

    per = {}  # counter -> list of per-dispatch values of the selected kernels
    copy = {}
    for d in args.pmc_dir:
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit(f"no counter_collection.csv under {d}")
        rows = {}
        for fn in files:
            with open(fn) as f:
                for r in csv.DictReader(f):
                    key = (fn, r["Dispatch_Id"], r["Kernel_Name"], r["Counter_Name"])
                    rows[key] = rows.get(key, 0.0) + float(r["Counter_Value"])
        # the calibration copy: the largest copyBuffer dispatch of the run
        cal = {}
        for (fn, disp, kname, cname), v in rows.items():
            if "copyBuffer" in kname and v > cal.get(cname, (None, -1.0))[1]:
                cal[cname] = (disp, v)
        for cname, (disp, v) in cal.items():
            copy[cname] = max(copy.get(cname, 0.0), v)
        # the dispatches of an ingest: from its first kernel (the batch's
        # min/max reduction) to the first kernel of the next sample
        in_build, build_of = False, {}
        for fn, disp, kname in sorted({(k[0], k[1], k[2]) for k in rows},
                                      key=lambda x: (x[0], int(x[1]))):
            if "minmax_partial_kernel" in kname:
                in_build = True
            elif any(k in kname for k in WALK_PATH_KERNELS):
                in_build = False
            build_of[(fn, disp)] = in_build
        for (fn, disp, kname, cname), v in rows.items():
            if cname in cal and cal[cname][0] == disp and "copyBuffer" in kname:
                continue  # not part of the measured work
            if selected(kname, build_of[(fn, disp)]):
                per.setdefault(cname, []).append(v)
    if not per:
        raise SystemExit(f"no dispatch of a kernel named like {args.kernel!r}")
    # per launch: the mean over the selected dispatches, or their sum over
    # --per launches (a kernel set: one ingest is many dispatches)
    avg = {c: (sum(v) / args.per if args.per else sum(v) / len(v)) for c, v in per.items()}
    out = {"kernel": args.kernel, "workload": args.workload, "command": args.command,
           "dispatches": max(len(v) for v in per.values()), "per": args.per or None,
           "sources_sha256": sources_sha256(args.family), "source_family": args.family,
           "counters": avg}
    cal = args.copy_calibration_mib * (1 << 20)
    for c, key in (("FETCH_SIZE", "hbm_read_bytes_per_launch"),
                   ("WRITE_SIZE", "hbm_write_bytes_per_launch")):
        if c in avg and copy.get(c):
            scale = cal / (copy[c] * 1024)
            out[c.lower() + "_scale"] = scale
            out[key] = avg[c] * 1024 * scale
    if "hbm_read_bytes_per_launch" in out and "hbm_write_bytes_per_launch" in out:
        out["hbm_bytes_per_launch"] = out["hbm_read_bytes_per_launch"] + out["hbm_write_bytes_per_launch"]
    if "TCC_HIT_sum" in avg and "TCC_MISS_sum" in avg:
        out["l2_hit_rate"] = avg["TCC_HIT_sum"] / (avg["TCC_HIT_sum"] + avg["TCC_MISS_sum"])
    if os.path.exists(args.summarize_pmc):
        with open(args.summarize_pmc) as f:
            old = json.load(f)
        if old.get("sources_sha256") == out["sources_sha256"] and old.get("kernel") == args.kernel:
            # a profile built up over several counter runs of the same sources
            merged = dict(old)
            merged.update({k: v for k, v in out.items() if k != "counters"})
            merged["counters"] = dict(old.get("counters", {}), **avg)
            for k in ("hbm_read_bytes_per_launch", "hbm_write_bytes_per_launch"):
                if k not in out and k in old:
                    merged[k] = old[k]
            if "hbm_read_bytes_per_launch" in merged and "hbm_write_bytes_per_launch" in merged:
                merged["hbm_bytes_per_launch"] = (merged["hbm_read_bytes_per_launch"] +
                                                  merged["hbm_write_bytes_per_launch"])
            out = merged
    with open(args.summarize_pmc, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


def copy_calibration(dev, mib):
    """One plain device copy of `mib` MiB (torch copy_, dispatched as
    __amd_rocclr_copyBuffer): the reference that scales the HBM byte counters
    of a --pmc profile (--summarize-pmc)."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    log(f"copy calibration: {mib} MiB read + written")
    del a, b


def pmc_profile(path, family):
    """(profile, current): current is False when the kernel sources no longer
    hash to what the profile measured."""
    if not os.path.exists(path):
        return None, False
    with open(path) as f:
        prof = json.load(f)
    return prof, prof.get("sources_sha256") == sources_sha256(family)


def other_roofline(k, compulsory, kernel_ms, kernel):
    """The walk kernel's compulsory bytes per launch over its mean launch
    time, with the measured traffic and L2 hit rate of the config's counter
    profile while it is current."""
    path = os.path.join(ROOT, "profiles", f"walk_kernel_cfg{k}_pmc.json")
    pmc, current = pmc_profile(path, "walk")
    achieved = compulsory / (kernel_ms * 1e-3) / 1e9
    traffic = pmc.get("hbm_bytes_per_launch") if pmc and current else None
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "kernel": kernel,
            "algorithmic_bytes_per_launch": compulsory,
            "traffic_GB_per_s": (traffic / (kernel_ms * 1e-3) / 1e9) if traffic else None,
            "l2_hit_rate": pmc.get("l2_hit_rate") if pmc and current else None,
            "pmc_profile": os.path.relpath(path, ROOT) if pmc else None, "pmc_current": current}


GATHER_TABLES = (("l2_2MiB", 2 << 20), ("mall_128MiB", 128 << 20), ("hbm_4GiB", 4 << 30))


def gather_ceiling(pmc, pmc_current, walk_kernel_ms):
    """Random 8-byte gather rates of this GPU (the probe library, libtrw_probe.so: 512K lanes x
    256 gathers per launch, mean of 5 launches after a warm-up) from tables
    that fit L2, the Infinity Cache and neither, as independent loads and as
    dependent chains; beside them the walk kernel's L1 -> L2 read rate from
    its counter profile (every one of its per-lane record, panel and header
    loads that misses L1 is one such read)."""
    import probe  # temporal-random-walk_amd/probe: the probe library's wrapper

    out = {"unit": "gathers/s", "independent": {}, "chained": {}}
    for name, size in GATHER_TABLES:
        for mode in ("independent", "chained"):
            r = probe.gather(size, lanes=256 * 2048, rounds=256, chained=(mode == "chained"),
                             reps=5)
            out[mode][name] = r["gathers_per_s"]
    c = (pmc or {}).get("counters", {}) if pmc_current else {}
    reads = c.get("TCP_TCC_READ_REQ_sum")
    out["walk_l1_l2_reads_per_s"] = None
    out["walk_read_l2_hit_rate"] = None
    out["walk_mixed_ceiling"] = None
    out["walk_frac_of_mixed_ceiling"] = None
    if reads:
        rate = reads / (walk_kernel_ms * 1e-3)
        out["walk_l1_l2_reads_per_s"] = rate
        hit, miss = c.get("TCC_HIT_sum"), c.get("TCC_MISS_sum")
        if hit is not None and miss:
            # the L2 hit rate of the walk's reads lies between the hit rate
            # of all its L2 requests (writes included, nearly all misses) and
            # the one with every hit counted as a read; its misses are served
            # by the Infinity Cache or by HBM
            h = (hit / (hit + miss), min(1.0, hit / reads))
            l2 = out["independent"]["l2_2MiB"]
            out["walk_read_l2_hit_rate"] = list(h)
            out["walk_mixed_ceiling"] = {}
            out["walk_frac_of_mixed_ceiling"] = {}
            for name, far in (("misses_in_infinity_cache", out["independent"]["mall_128MiB"]),
                              ("misses_in_hbm", out["independent"]["hbm_4GiB"])):
                ceil = [1.0 / (x / l2 + (1.0 - x) / far) for x in h]
                out["walk_mixed_ceiling"][name] = ceil
                out["walk_frac_of_mixed_ceiling"][name] = [rate / x for x in ceil]
    out["note"] = ("probe: 512K lanes gather 8-byte words at random places of a table of the "
                   "named size, one L1 miss each; chained = each address follows from the "
                   "previous load's value (one load in flight per lane, as in a walk). "
                   "walk_l1_l2_reads_per_s = TCP_TCC_READ_REQ of one walk-kernel launch "
                   "(profile) / its time here; walk_mixed_ceiling = the independent L2 rate "
                   "mixed with the Infinity-Cache or the HBM rate at the walk's read hit rate "
                   "(both bounds of it).")
    return out


def run_other_config(k, args):
    """One of BASELINE.json's other workloads (configs[k-1]), timed on the
    device (HIP events of the engine): index build and sampling.  These are
    parity-test configs; the bench line proper is cfg2."""
    import numpy as np
    import torch
    from temporal_random_walk import capi
    from tests import configs

    dev = torch.device("cuda:0")

    def resident(*arrs):
        out = [torch.from_numpy(a).to(dev) for a in arrs]
        torch.cuda.synchronize()
        return out

    res = {"config": f"cfg{k}", "unit": "walk steps/s"}
    if k == 5 and args.late_frac > 0:
        res["late_frac"] = args.late_frac
    if args.copy_calibration_mib > 0:
        copy_calibration(dev, args.copy_calibration_mib)
    log(f"generating cfg{k} inputs")
    if k in (1, 3, 4):
        if k == 1:
            src, dst, ts = configs.cfg1()
            feats = None
            eng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False)
            call = ("all_nodes", 20, "Uniform", 10, "Uniform", "Forward_In_Time")
        elif k == 3:
            src, dst, ts, feats = configs.cfg3()
            eng = capi.Engine(is_directed=False, global_seed=42, shuffle_walk_order=False)
            call = ("all_nodes", 40, "Linear", 5, "Linear", "Backward_In_Time")
        else:
            src, dst, ts = configs.cfg4()
            feats = None
            eng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False,
                              enable_weight_computation=True, timescale_bound=50.0)
            call = ("total", 80, "ExponentialWeight", 20_000_000, "ExponentialWeight",
                    "Forward_In_Time")
        arrs = resident(src, dst, ts) + ([] if feats is None else resident(feats))
        E = len(src)
        dim = 0 if feats is None else feats.shape[1]
        builds, samples, kernels = [], [], []
        for i in range(1 + args.steps):
            eng.clear()
            eng.add_edges_device(arrs[0].data_ptr(), arrs[1].data_ptr(), arrs[2].data_ptr(), E,
                                 arrs[3].data_ptr() if feats is not None else None, dim)
            tb = eng.timings()["build_ms"]
            mode, L, bias, n, start, direction = call
            eng.sample_device(mode, L, bias, n, initial_edge_bias=start, direction=direction,
                              walk_order=args.walk_order,
                              walk_layout=args.walk_layout)
            tm = eng.timings()
            if i:  # the first round warms up
                builds.append(tb)
                samples.append(tm["sample_ms"])
                kernels.append(tm["walk_kernel_ms"])
            log(f"round {i}: build {tb:.2f} ms, sample {tm['sample_ms']:.2f} ms, "
                f"walk kernel {tm['walk_kernel_ms']:.2f} ms")
        st = eng.walk_stats()
        res.update(edges=E, walks=int(st["nonempty_walks"]), walk_steps=int(st["total_len"]),
                   build_ms=sum(builds) / len(builds), sample_ms=sum(samples) / len(samples),
                   walk_kernel_ms=sum(kernels) / len(kernels))
        res["index_build_edges_per_s"] = E / (res["build_ms"] * 1e-3)
        res["value"] = st["total_len"] / (res["sample_ms"] * 1e-3)
        kname = "walk_rows_kernel" if st["rows_by_walk_kernel"] else "walk_kernel"
        res["roofline"] = other_roofline(
            k, st["compulsory_read_bytes"] + st["compulsory_write_bytes"], res["walk_kernel_ms"],
            kname)
        eng.close()
        if not args.no_gather_ceiling:
            pmc, current = pmc_profile(os.path.join(ROOT, "profiles", f"walk_kernel_cfg{k}_pmc.json"),
                                       "walk")
            res["gather_ceiling"] = gather_ceiling(pmc, current, res["walk_kernel_ms"])
    elif k == 5:
        eng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False,
                          max_time_capacity=3_000_000, enable_temporal_node2vec=True,
                          node2vec_p=0.5, node2vec_q=2.0)
        # the stream's batches, resident in HBM before the timed region
        late_rng = np.random.default_rng(48)
        stream = []
        for b, (src, dst, ts) in enumerate(configs.cfg5_batches()):
            if args.late_frac > 0 and b > 0:
                # late arrivals: a share of the batch carries timestamps of the
                # previous batch's range, so the batch reaches back into the
                # store (the merge path instead of the append path)
                late = late_rng.random(len(ts)) < args.late_frac
                ts = ts.copy()
                ts[late] = late_rng.integers((b - 1) * 1_000_000, b * 1_000_000, int(late.sum()))
            stream.append(resident(src, dst, ts))
        # as the other configs: warm-up rounds of the whole stream, then the
        # timed rounds, each from an empty store (clear() keeps the buffers)
        for rnd in range(max(1, args.warmup) + 1):
            timed = rnd >= max(1, args.warmup)
            eng.clear()
            builds, samples, kernels, steps, edges, comp = [], [], [], 0, 0, 0
            for b, arrs in enumerate(stream):
                eng.add_edges_device(arrs[0].data_ptr(), arrs[1].data_ptr(), arrs[2].data_ptr(),
                                     arrs[0].numel())
                tb = eng.timings()["build_ms"]
                eng.sample_device("total", 40, "TemporalNode2Vec", 5_000_000,
                                  initial_edge_bias="Uniform", direction="Forward_In_Time",
                                  walk_order=args.walk_order,
                                  walk_layout=args.walk_layout)
                tm = eng.timings()
                builds.append(tb)
                samples.append(tm["sample_ms"])
                kernels.append(tm["walk_kernel_ms"])
                st = eng.walk_stats()
                steps += int(st["total_len"])
                comp += st["compulsory_read_bytes"] + st["compulsory_write_bytes"]
                kname = "walk_rows_kernel" if st["rows_by_walk_kernel"] else "walk_kernel"
                edges += arrs[0].numel()
                log(f"{'timed' if timed else 'warm-up'} batch {b}: store {eng.edge_count()} "
                    f"edges, build {tb:.2f} ms, sample {tm['sample_ms']:.2f} ms, walk kernel "
                    f"{tm['walk_kernel_ms']:.2f} ms")
        res.update(batches=len(builds), batch_edges=edges // len(builds),
                   build_ms=sum(builds) / len(builds), sample_ms=sum(samples) / len(samples),
                   walk_kernel_ms=sum(kernels) / len(kernels))
        res["index_build_edges_per_s"] = edges / (sum(builds) * 1e-3)
        res["value"] = steps / (sum(samples) * 1e-3)
        res["roofline"] = other_roofline(5, comp / len(builds), res["walk_kernel_ms"], kname)
        eng.close()
        if not args.no_gather_ceiling:
            pmc, current = pmc_profile(os.path.join(ROOT, "profiles", "walk_kernel_cfg5_pmc.json"),
                                       "walk")
            res["gather_ceiling"] = gather_ceiling(pmc, current, res["walk_kernel_ms"])
        if args.host_ingest:
            res["host_ingest"] = cfg5_host_ingest(capi, configs)
    else:
        raise SystemExit("--config takes 1, 3, 4 or 5 (2 is the default bench line)")
    print(json.dumps(res))


def cfg5_host_ingest(capi, configs):
    """cfg5's streaming loop from host arrays, wall clock per batch: each batch
    ingested with trw_add_edges before its sample (the reference's order), or
    the next batch prefetched (trw_prefetch_edges) while the current batch is
    sampled.  Walks stay on the device; the first batch is a warm-up."""
    batches = list(configs.cfg5_batches())
    out = {}
    for mode in ("sequential", "prefetched"):
        eng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False,
                          max_time_capacity=3_000_000, enable_temporal_node2vec=True,
                          node2vec_p=0.5, node2vec_q=2.0)
        times = []
        if mode == "prefetched":
            eng.prefetch_edges(*batches[0])
        for b in range(len(batches)):
            t0 = time.perf_counter()
            if mode == "sequential":
                eng.add_edges(*batches[b])
            else:
                eng.add_prefetched_edges()
                if b + 1 < len(batches):
                    eng.prefetch_edges(*batches[b + 1])
            eng.sample_device("total", 40, "TemporalNode2Vec", 5_000_000,
                              initial_edge_bias="Uniform", direction="Forward_In_Time")
            times.append((time.perf_counter() - t0) * 1e3)
        eng.close()
        out[mode + "_ms_per_batch"] = sum(times[1:]) / (len(times) - 1)
        log(f"host ingest, {mode}: {out[mode + '_ms_per_batch']:.2f} ms per batch")
    out["batch_bytes"] = int(sum(x.nbytes for x in batches[0]))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--edges", type=int, default=20_000_000)
    ap.add_argument("--nodes", type=int, default=1_000_000)
    ap.add_argument("--timestamps", type=int, default=100_000)
    ap.add_argument("--walks", type=int, default=10_000_000)
    ap.add_argument("--walk-len", type=int, default=80)
    ap.add_argument("--walk-order", default="auto",
                    choices=["auto", "walk_id", "start_time", "node_grouped"],
                    help="order the walks run in on the device (the output is the same)")
    ap.add_argument("--walk-layout", default="auto", choices=["auto", "scratch"],
                    help="auto: forward walks that pack are written as output rows by the walk "
                         "kernel; scratch: always walk scratch and the layout pass (the output "
                         "is the same)")
    ap.add_argument("--config", type=int, default=2,
                    help="2 (default): the cfg2 bench line; 1, 3, 4 or 5: time that BASELINE "
                         "workload instead (device timings, one JSON line)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-walks", type=int, default=1_500_000,
                    help="walks of the bounded CPU-baseline sample (about 5 s per round on "
                         "16 threads)")
    ap.add_argument("--cpu-reps", type=int, default=3,
                    help="timed CPU-baseline rounds (the median is reported)")
    ap.add_argument("--cpu-threads", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--cpu-baseline-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-host-boundary", action="store_true",
                    help="skip timing the reference's host boundary (numpy edges in through "
                         "the drop-in Python class, host->device copy included, and numpy "
                         "walks out, device->host copy included)")
    ap.add_argument("--summarize-pmc", metavar="OUT_JSON", default=None,
                    help="summarise rocprofv3 counter runs (--pmc-dir) of one kernel "
                         "(--kernel) into OUT_JSON, then exit; touches no GPU")
    ap.add_argument("--pmc-dir", action="append", default=[])
    ap.add_argument("--kernel", default="walk_rows_kernel<|walk_kernel<",
                    help="kernel name substrings joined by |, or @build for every "
                         "dispatch of an ingest (from its first kernel to the next sample's)")
    ap.add_argument("--per", type=int, default=0,
                    help="sum the selected dispatches over this many launches (0: mean "
                         "per dispatch)")
    ap.add_argument("--family", default="walk", choices=sorted(KERNEL_SOURCES))
    ap.add_argument("--workload", default="")
    ap.add_argument("--command", default="")
    ap.add_argument("--host-ingest", action="store_true",
                    help="with --config 5: also time the streaming loop from host arrays, "
                         "ingesting each batch before its sample or prefetching the next "
                         "batch while the current one is sampled")
    ap.add_argument("--late-frac", type=float, default=0.0,
                    help="--config 5: this share of every batch after the first gets "
                         "timestamps of the previous batch's range (late arrivals)")
    ap.add_argument("--no-gather-ceiling", action="store_true",
                    help="skip the random-gather rate probe (libtrw_probe.so)")
    ap.add_argument("--gather-ceiling-only", action="store_true",
                    help="run only the random-gather probe and print its rates")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB (torch copy_ "
                         "kernel): the reference point that scales the HBM byte counters of "
                         "a --pmc profile")
    args = ap.parse_args()

    if args.summarize_pmc:
        summarize_pmc(args)
        return
    if args.cpu_baseline_child:
        cpu_baseline_child(args)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only (no multi-GPU path); "
                                   "run with --gpus 1"}))
        sys.exit(2)

    if args.config != 2:
        run_other_config(args.config, args)
        return
    if args.gather_ceiling_only:
        from temporal_random_walk import capi
        print(json.dumps(gather_ceiling(None, False, 1.0)))
        return

    import numpy as np
    import torch

    from temporal_random_walk import capi

    log("generating cfg2 inputs")
    t0 = time.perf_counter()
    src, dst, ts = make_cfg2(args.nodes, args.edges, args.timestamps)
    log(f"generated {len(src)} edges in {time.perf_counter() - t0:.1f}s")

    dev = torch.device("cuda:0")
    if args.copy_calibration_mib > 0:
        copy_calibration(dev, args.copy_calibration_mib)
    d_src = torch.from_numpy(src).to(dev)
    d_dst = torch.from_numpy(dst).to(dev)
    d_ts = torch.from_numpy(ts).to(dev)
    torch.cuda.synchronize()

    eng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False)
    E = len(src)

    def step():
        eng.clear()
        t0 = time.perf_counter()
        eng.add_edges_device(d_src.data_ptr(), d_dst.data_ptr(), d_ts.data_ptr(), E)
        t1 = time.perf_counter()
        eng.sample_device("total", args.walk_len, "ExponentialIndex", args.walks,
                          initial_edge_bias="Uniform", direction="Forward_In_Time",
                          walk_order=args.walk_order,
                              walk_layout=args.walk_layout)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, eng.timings()

    for i in range(args.warmup):
        b, s, _ = step()
        log(f"warmup {i}: build {b * 1e3:.1f} ms, sample {s * 1e3:.1f} ms")

    torch.cuda.synchronize()
    T0 = time.perf_counter()
    builds, samples, tims = [], [], []
    for i in range(args.steps):
        b, s, tm = step()
        builds.append(b)
        samples.append(s)
        tims.append(tm)
        log(f"step {i}: build {b * 1e3:.1f} ms, sample {s * 1e3:.1f} ms, "
            f"walk kernel {tm['walk_kernel_ms']:.1f} ms")
    torch.cuda.synchronize()
    T1 = time.perf_counter()

    stats = eng.walk_stats()  # identical every step (fixed seed), computed untimed
    steps_per_call = stats["total_len"]
    value = steps_per_call * args.steps / sum(samples)
    build_eps = E * args.steps / sum(builds)
    walk_kernel_ms = sum(t["walk_kernel_ms"] for t in tims) / len(tims)
    build_dev_ms = sum(t["build_ms"] for t in tims) / len(tims)
    # roofline: the walk kernel's compulsory bytes -- inputs and the sampled
    # direction's index read once, the output rows it writes (or its scratch
    # slots) and lengths written once
    # (trw_get_walk_stats) -- over its launch time (HIP events on the engine's
    # stream).  The per-hop demand bytes (every walk's reads, 72 + 8*probes B
    # with the reference's types) are reported beside it: walks running side
    # by side share most of those lines in L1/L2.
    wk_s = walk_kernel_ms * 1e-3
    compulsory = stats["compulsory_read_bytes"] + stats["compulsory_write_bytes"]
    achieved = compulsory / wk_s / 1e9

    g_o = len(eng.array("node_ts_group_outbound_offsets"))
    g_i = len(eng.array("node_ts_group_inbound_offsets"))
    Vc = len(eng.array("node_group_outbound_offsets"))
    T = len(eng.array("unique_timestamps"))
    idx_bytes = index_algorithmic_bytes(E, Vc, T, g_o, g_i)

    pmc, pmc_current = pmc_profile(PMC_FILE, "walk")
    traffic = pmc.get("hbm_bytes_per_launch") if pmc and pmc_current else None
    l2_hit = pmc.get("l2_hit_rate") if pmc and pmc_current else None

    result = {
        "metric": METRIC,
        "value": value,
        "unit": "walk steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": (T1 - T0) * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic (seeded numpy PCG64, BASELINE configs[1] shape)",
        "config": {
            "workload": "cfg2: directed Zipf(1.8) 1M ids / 20M edges, 1e5 distinct ts; "
                        "10M walks L=80 ExponentialIndex/Uniform forward",
            "edges": E,
            "num_walks": args.walks,
            "max_walk_len": args.walk_len,
            "parallelism": "1 GPU",
            "walk_order": args.walk_order,
            "walk_layout": args.walk_layout,
        },
        "index_build_edges_per_s": build_eps,
        "index_build_ms": sum(builds) * 1e3 / args.steps,
        "index_build_device_ms": build_dev_ms,
        "index_roofline": {"bound": "hbm", "achieved": idx_bytes / (build_dev_ms * 1e-3) / 1e9,
                           "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": idx_bytes / (build_dev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                           "algorithmic_bytes": idx_bytes},
        "walk_steps_per_call": steps_per_call,
        "mean_walk_len": steps_per_call / args.walks,
        "sample_ms": sum(samples) * 1e3 / args.steps,
        "walk_kernel_ms": walk_kernel_ms,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": ("walk_rows_kernel<true,true,0,16>" if stats["rows_by_walk_kernel"]
                       else "walk_kernel<true,true,0>"),
            "algorithmic_bytes_per_launch": compulsory,
            "compulsory_read_bytes": stats["compulsory_read_bytes"],
            "compulsory_write_bytes": stats["compulsory_write_bytes"],
            "demand_bytes_per_launch": stats["reference_bytes"],
            "demand_engine_types_bytes_per_launch": stats["algorithmic_bytes"],
            "demand_GB_per_s": stats["reference_bytes"] / wk_s / 1e9,
            "traffic_GB_per_s": (traffic / wk_s / 1e9) if traffic else None,
            "traffic_frac": (traffic / wk_s / 1e9 / HBM_PEAK_GBS) if traffic else None,
            "l2_hit_rate": l2_hit,
            "pmc_profile": os.path.relpath(PMC_FILE, ROOT) if pmc else None,
            "pmc_current": pmc_current,
            "note": "algorithmic bytes = compulsory bytes of one launch (start states, "
                    "processing order and the sampled direction's index arrays read once; "
                    "the output rows -- or packed scratch, when a layout pass writes the rows -- "
                    "and walk lengths written once). demand bytes count every "
                    "walk's per-hop reads (72 + 8*ceil(log2(G+1)) B in the reference's types) "
                    "and exceed the HBM rate because walks in start-time order share lines "
                    "in L1/L2. traffic = FETCH_SIZE + WRITE_SIZE of one launch from the "
                    "rocprofv3 profile, null when the walk sources changed since it was "
                    "measured.",
        },
    }
    bpmc, bpmc_current = pmc_profile(os.path.join(ROOT, "profiles", "index_build_cfg2_pmc.json"),
                                     "build")
    if bpmc and bpmc_current:
        result["index_roofline"]["traffic"] = bpmc.get("hbm_bytes_per_launch")
        result["index_roofline"]["l2_hit_rate"] = bpmc.get("l2_hit_rate")
        result["index_roofline"]["pmc_profile"] = "profiles/index_build_cfg2_pmc.json"

    eng.close()
    if not args.no_gather_ceiling:
        log("random-gather probe")
        result["gather_ceiling"] = gather_ceiling(pmc, pmc_current, walk_kernel_ms)
    if not args.no_host_boundary:
        from temporal_random_walk import TemporalRandomWalk

        log("host boundary (PCIe-inclusive) run")
        trw = TemporalRandomWalk(is_directed=True, use_gpu=True, global_seed=42,
                                 shuffle_walk_order=False)
        trw.add_multiple_edges(src, dst, ts)  # warm-up: sizes the device buffers
        trw.clear()
        t0 = time.perf_counter()
        trw.add_multiple_edges(src, dst, ts)
        t1 = time.perf_counter()
        nodes, times, lens, _ = trw.get_random_walks_and_times(
            max_walk_len=args.walk_len, walk_bias="ExponentialIndex",
            num_walks_total=args.walks, initial_edge_bias="Uniform")
        t2 = time.perf_counter()
        steps = float(lens.sum())
        del nodes, times, lens, trw
        # the same call through the C ABI, for the handoff's own timing
        heng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False)
        heng.add_edges(src, dst, ts)  # first call sizes the buffers
        heng.clear()
        t5 = time.perf_counter()
        heng.add_edges(src, dst, ts)
        t6 = time.perf_counter()
        ingest_build_ms = heng.timings()["build_ms"]
        t3 = time.perf_counter()
        hw = heng.sample("total", args.walk_len, "ExponentialIndex", args.walks,
                         initial_edge_bias="Uniform", direction="Forward_In_Time")
        t4 = time.perf_counter()
        ht = heng.timings()
        del hw
        heng.close()
        result["host_boundary"] = {
            "walk_steps_per_s": steps / (t2 - t1),
            "index_build_edges_per_s": E / (t1 - t0),
            "sample_s": t2 - t1,
            "ingest_s": t1 - t0,
            "capi_sample_s": t4 - t3,
            "capi_ingest_s": t6 - t5,
            "capi_ingest_edges_per_s": E / (t6 - t5),
            "ingest_copy_GB_per_s": 16 * E / ((t6 - t5) - ingest_build_ms * 1e-3) / 1e9,
            "handoff_ms": ht["handoff_ms"],
            "handoff_bytes": ht["handoff_bytes"],
            "handoff_GB_per_s": ht["handoff_bytes"] / (ht["handoff_ms"] * 1e6),
            "note": "numpy in / numpy out through the pybind11 class after one warm-up "
                    "ingest; includes H2D of the batch and D2H of all walk arrays into "
                    "caller-owned host memory; handoff_* is trw_sample's device->host "
                    "delivery alone, ingest_copy_* trw_add_edges' host->device staging",
        }

    if not args.no_cpu_baseline:
        del d_src, d_dst, d_ts
        result["cpu_baseline"] = cpu_baseline(args)
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result))


if __name__ == "__main__":
    main()
