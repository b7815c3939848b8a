"""Fused-block latency on one MI355X, with its roofline fraction and the CPU path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]
                    [--blocks | --no-blocks]

A step is one launch of the fused block over one batch of synthetic
(seeded) inputs that are already resident in HBM.  W untimed steps, then K
timed steps back to back on the launch stream, bracketed by a device
synchronize on both sides; HIP events recorded on that same stream give the
average device time per step.  The JSON line's ``value`` is that latency in
microseconds (lower is better).

``roofline`` relates the algorithmic work of one launch (compulsory HBM
bytes, or MFMA FLOPs, of the fused block) to the measured launch duration and
the MI355X published peak.  ``graph_us`` is the same step's device time with
the host's per-launch cost removed (20 steps captured in one HIP graph,
replayed); ``cost_model`` compares it with the MI355X launch model's
prediction from the launch plans the entry points record.  ``cpu_baseline`` times the CPU restatement of the
reference's execution path (the oracle: unfused scalar loop nests, one
thread) on a bounded sample of the same workload on this host.  ``blocks``
repeats the GPU measurement for every other configuration.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "npu-dialect_amd"))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--blocks", dest="blocks", action="store_true", default=True)
    ap.add_argument("--no-blocks", dest="blocks", action="store_false")
    ap.add_argument("--dump-plans", default=None,
                    help="write every configuration's launch plans and graph time to this JSON file")
    return ap.parse_args()


def time_gpu(w, steps, warmup):
    """Returns (avg seconds per launch from HIP events, wall seconds, outputs)."""
    import torch

    from npu_amd import configs
    d = configs.to_device(w.make_inputs())
    o = w.make_outputs(d)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        w.run(d, o, stream)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        w.run(d, o, stream)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) * 1e-3 / steps, wall, o


def time_graph(w, steps, reps=10):
    """Device time per step with host launch overhead removed: `steps` steps
    captured in one HIP graph, replayed `reps` times between HIP events.
    Also checks that the graph's outputs equal an eager run's, bit for bit.
    Returns (seconds per step, outputs match)."""
    import torch

    from npu_amd import configs
    d = configs.to_device(w.make_inputs())
    o = w.make_outputs(d)
    w.run(d, o, torch.cuda.current_stream())  # eager run: initialises lazy launch state
    torch.cuda.synchronize()
    eager = [t.clone() for t in o.values()]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream()
        for _ in range(steps):
            w.run(d, o, cs)
    stream = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    same = all(torch.equal(a, b) for a, b in zip(eager, o.values()))
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / (reps * steps), same


def model_prediction(w):
    """Launch-model prediction for one step: the launch plans the entry points
    record, through the MI355X model of libnpu_host.so."""
    import torch

    from npu_amd import configs, groups, host
    d = configs.to_device(w.make_inputs())
    o = w.make_outputs(d)
    with groups.collect_plans() as cp:
        w.run(d, o, torch.cuda.current_stream())
    torch.cuda.synchronize()
    total, parts = host.predict_block(cp.plans)
    plans = [{f: (getattr(pl, f).decode() if f == "kernel" else getattr(pl, f))
              for f, _ in pl._fields_} for pl in cp.plans]
    return total, [{"kernel": k, "us": round(c.time_us, 3), "bound": host.BOUNDS[c.bound]}
                   for k, c in parts], plans


def cpu_sample(w, budget_s=30.0):
    """Times the oracle on a bounded sample; returns the cpu_baseline object.

    Batched workloads time one image first; if the whole batch is estimated
    to fit the budget it is timed in full, otherwise as many images as fit,
    scaled to the batch (images are independent)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import refs

    inp = w.make_inputs()
    n = w.units
    if w.unit_name == "images" and n > 1:
        t0 = time.perf_counter()
        refs.run_oracle(w.name, inp, images=[0])
        one = time.perf_counter() - t0
        k = max(1, min(n, int(budget_s / max(one, 1e-6))))
        imgs = list(range(k))
    else:
        k, imgs = n, None
    t0 = time.perf_counter()
    refs.run_oracle(w.name, inp, images=imgs)
    dt = time.perf_counter() - t0
    if imgs is not None and k < n:
        sample = f"{k} of {n} images (images are independent), scaled x{n / k:g}"
        dt *= n / k
    else:
        sample = "the full workload"
    return {"value": dt * 1e6, "unit": "us", "cores": 1, "kind": "port",
            "sample": sample + "; unfused scalar loop nests, -O2 -ffp-contract=off, 1 thread",
            "host": host_cpu()}


def measured_traffic(workload_name):
    """HBM bytes per launch from the committed counter summary, if there is one."""
    path = os.path.join(ROOT, "profiles", f"{workload_name}_hbm_traffic.txt")
    try:
        for line in open(path):
            if line.strip().startswith("#   traffic_bytes_per_launch"):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def host_cpu():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return f"{line.split(':', 1)[1].strip()} ({os.cpu_count()} logical CPUs visible)"
    except OSError:
        pass
    return f"{os.cpu_count()} logical CPUs"


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the fused blocks are single-GPU kernels and "
              "this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    from npu_amd import configs
    import npu_amd
    npu_amd.lib()  # fail loudly if the HIP library is missing
    torch.cuda.set_device(0)

    name = args.workload or configs.HEADLINE
    w = configs.by_name(name)
    sec, wall, _ = time_gpu(w, args.steps, args.warmup)
    gsec, gsame = time_graph(w, 20)
    pred, parts, plans = model_prediction(w)
    dumped = [{"workload": w.name, "graph_us": gsec * 1e6, "plans": plans}]
    line = {
        "metric": "fused-block latency",
        "value": round(sec * 1e6, 3),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic: SplitMix64-seeded inputs, distributions of the configuration",
        "config": {"workload": w.name, "desc": w.desc, "batch": w.units,
                   "parallelism": "single GPU"},
        "throughput": {"value": w.units / sec, "unit": f"{w.unit_name}/s"},
        "wall_s_timed_region": wall,
        "roofline": dict(w.roofline(sec), traffic=measured_traffic(w.name),
                         flops=w.flops, mfma_flops=w.mfma_flops, bytes=w.bytes,
                         floor_us=w.floor_s() * 1e6),
        "graph_us": round(gsec * 1e6, 3),
        "graph_matches_eager": gsame,
        "cost_model": {"predicted_us": round(pred, 3), "measured_us": round(gsec * 1e6, 3),
                       "error": round(pred / (gsec * 1e6) - 1, 3), "kernels": parts},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_sample(w)
    if args.blocks:
        blocks = []
        for other in configs.all_workloads():
            if other.name == w.name:
                continue
            s, _, _ = time_gpu(other, max(20, args.steps // 2), max(5, args.warmup // 2))
            gs, same = time_graph(other, 20)
            p, pk, opl = model_prediction(other)
            dumped.append({"workload": other.name, "graph_us": gs * 1e6, "plans": opl})
            rl = other.roofline(s)
            blocks.append({"workload": other.name, "latency_us": round(s * 1e6, 3),
                           "traffic": measured_traffic(other.name),
                           "graph_us": round(gs * 1e6, 3), "graph_matches_eager": same,
                           "bound": rl["bound"], "frac": round(rl["frac"], 4),
                           "graph_frac": round(other.roofline(gs)["frac"], 4),
                           "floor_us": round(other.floor_s() * 1e6, 3),
                           "model_us": round(p, 3), "model_error": round(p / (gs * 1e6) - 1, 3),
                           "model_kernels": pk})
        line["blocks"] = blocks
        errs = [abs(line["cost_model"]["error"])] + [abs(b["model_error"]) for b in blocks]
        line["cost_model"]["within_25pct"] = f"{sum(e <= 0.25 for e in errs)}/{len(errs)}"
    if args.dump_plans:
        with open(args.dump_plans, "w") as f:
            json.dump(dumped, f, indent=1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
