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
"""
from __future__ import annotations

import argparse
import json
import os
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


def cpu_baseline(src, dst, ts, n_walks, L, threads):
    """The oracle (C restatement of the reference CPU path) on the host cores:
    full ingest of the graph (single-threaded, as written) and a bounded
    sample of walks (OpenMP over walks), draw generation included as in the
    reference's CPU sampler."""
    import numpy as np
    from oracle import pyoracle as po

    og = po.OracleGraph(True)
    t0 = time.perf_counter()
    og.add_edges(src, dst, ts)
    t_build = time.perf_counter() - t0
    t0 = time.perf_counter()
    draws = np.random.default_rng(1).random(n_walks * (1 + 2 * L))
    starts = -np.ones(n_walks, dtype=np.int32)
    w = og.walks(L, "ExponentialIndex", "Uniform", True, starts, draws, num_threads=threads)
    t_walk = time.perf_counter() - t0
    steps = int(w.lens.sum())
    return {
        "value": steps / t_walk,
        "unit": "walk steps/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/trw_oracle.c: {n_walks} walks (L={L}, ExponentialIndex/Uniform, fwd) "
                   f"on the full cfg2 graph with {threads} OpenMP threads, draw generation "
                   f"included; index build of all {len(src)} edges single-threaded"),
        "index_build_edges_per_s": len(src) / t_build,
        "index_build_cores": 1,
        "walk_s": t_walk,
        "build_s": t_build,
    }


def run_other_config(k, args):
    """One of BASELINE.json's other workloads (configs[k-1]), timed on the
    device (HIP events of the engine): index build and sampling.  These are
    parity-test configs; the bench line proper is cfg2."""
    import torch
    from temporal_random_walk import capi
    from tests import configs

    dev = torch.device("cuda:0")

    def resident(*arrs):
        out = [torch.from_numpy(a).to(dev) for a in arrs]
        torch.cuda.synchronize()
        return out

    res = {"config": f"cfg{k}", "unit": "walk steps/s"}
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
                              walk_order=args.walk_order)
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
        eng.close()
    elif k == 5:
        eng = capi.Engine(is_directed=True, global_seed=42, shuffle_walk_order=False,
                          max_time_capacity=3_000_000, enable_temporal_node2vec=True,
                          node2vec_p=0.5, node2vec_q=2.0)
        builds, samples, kernels, steps, edges = [], [], [], 0, 0
        for b, (src, dst, ts) in enumerate(configs.cfg5_batches()):
            arrs = resident(src, dst, ts)
            eng.add_edges_device(arrs[0].data_ptr(), arrs[1].data_ptr(), arrs[2].data_ptr(),
                                 len(src))
            tb = eng.timings()["build_ms"]
            eng.sample_device("total", 40, "TemporalNode2Vec", 5_000_000,
                              initial_edge_bias="Uniform", direction="Forward_In_Time",
                              walk_order=args.walk_order)
            tm = eng.timings()
            builds.append(tb)
            samples.append(tm["sample_ms"])
            kernels.append(tm["walk_kernel_ms"])
            steps += int(eng.walk_stats()["total_len"])
            edges += len(src)
            log(f"batch {b}: store {eng.edge_count()} edges, build {tb:.2f} ms, sample "
                f"{tm['sample_ms']:.2f} ms, walk kernel {tm['walk_kernel_ms']:.2f} ms")
        res.update(batches=len(builds), batch_edges=edges // len(builds),
                   build_ms=sum(builds) / len(builds), sample_ms=sum(samples) / len(samples),
                   walk_kernel_ms=sum(kernels) / len(kernels))
        res["index_build_edges_per_s"] = edges / (sum(builds) * 1e-3)
        res["value"] = steps / (sum(samples) * 1e-3)
        eng.close()
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
    ap.add_argument("--walk-order", default="auto", choices=["auto", "walk_id", "start_time"],
                    help="order the walks run in on the device (the output is the same)")
    ap.add_argument("--config", type=int, default=2,
                    help="2 (default): the cfg2 bench line; 1, 3, 4 or 5: time that BASELINE "
                         "workload instead (device timings, one JSON line)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-walks", type=int, default=2_500_000,
                    help="walks of the bounded CPU-baseline sample (about 10 s on 16 threads)")
    ap.add_argument("--host-boundary", action="store_true",
                    help="also time the reference's host boundary once through the drop-in "
                         "Python class: numpy edges in (host->device copy included) and "
                         "numpy walks out (device->host copy included)")
    ap.add_argument("--host-ingest", action="store_true",
                    help="with --config 5: also time the streaming loop from host arrays, "
                         "ingesting each batch before its sample or prefetching the next "
                         "batch while the current one is sampled")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB (torch copy_ "
                         "kernel): the reference point that scales the HBM byte counters of "
                         "a --pmc profile")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only (no multi-GPU path); "
                                   "run with --gpus 1"}))
        sys.exit(2)

    if args.config != 2:
        run_other_config(args.config, args)
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
        n = args.copy_calibration_mib * (1 << 20) // 4
        a = torch.ones(n, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        log(f"copy calibration: {args.copy_calibration_mib} MiB read + written")
        del a, b
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
                          walk_order=args.walk_order)
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
    # roofline.achieved: the per-unit algorithmic bytes with the reference's
    # element types (per hop 72 + 8*ceil(log2(G_u+1)) B, per walk 8 B + the start
    # + the first two slots' output), summed over this launch's walks on the
    # device; the same sum restated for this engine's 4-byte positions and ranks
    # is reported beside it.
    achieved = stats["reference_bytes"] / (walk_kernel_ms * 1e-3) / 1e9
    achieved_engine = stats["algorithmic_bytes"] / (walk_kernel_ms * 1e-3) / 1e9

    g_o = len(eng.array("node_ts_group_outbound_offsets"))
    g_i = len(eng.array("node_ts_group_inbound_offsets"))
    Vc = len(eng.array("node_group_outbound_offsets"))
    T = len(eng.array("unique_timestamps"))
    idx_bytes = index_algorithmic_bytes(E, Vc, T, g_o, g_i)

    traffic = l2_hit = None
    if os.path.exists(PMC_FILE):
        with open(PMC_FILE) as f:
            pmc = json.load(f)
        traffic = pmc.get("hbm_bytes_per_launch")
        l2_hit = pmc.get("l2_hit_rate")

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
            "kernel": "walk_kernel<true,true,0>",
            "algorithmic_bytes_per_launch": stats["reference_bytes"],
            "engine_types_bytes_per_launch": stats["algorithmic_bytes"],
            "engine_types_achieved": achieved_engine,
            "traffic_GB_per_s": (traffic / (walk_kernel_ms * 1e-3) / 1e9) if traffic else None,
            "l2_hit_rate": l2_hit,
            "note": "algorithmic bytes count every walk's per-hop index reads (72 + 8*probes B "
                    "with the reference's types); walks run in start-time order share those "
                    "lines, so most are L2 hits and frac can exceed 1. traffic (PMC, L2 <-> "
                    "fabric bytes of one launch) over the launch time is the HBM-side rate.",
        },
    }

    eng.close()
    if args.host_boundary:
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
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
        log(f"cpu baseline ({threads} threads)")
        result["cpu_baseline"] = cpu_baseline(src, dst, ts, args.cpu_walks, args.walk_len,
                                              threads)
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result))


if __name__ == "__main__":
    main()
