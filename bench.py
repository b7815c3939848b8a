"""Fused-block latency on one MI355X, with its roofline fraction and the CPU path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]
                    [--blocks | --no-blocks]

A step is one launch of the fused block over one batch of synthetic
(seeded) inputs that are already resident in HBM.  W untimed steps, then K
timed steps back to back on the launch stream, bracketed by a device
synchronize on both sides; HIP events recorded on that same stream give the
average device time per step.  The JSON line's ``value`` is that latency in
microseconds (lower is better).

Per configuration (the headline and every entry of ``blocks``):
* ``latency_us``: the K-launch average as for ``value`` (the roofline's time);
  ``median_us`` / ``p10_us`` / ``p90_us``: over 100 event pairs, each around
  10 back-to-back launches (an event pair adds about 2 us to what it
  brackets); ``event_pair_median_us``: single launches between event pairs;
  ``cold_event_pair_median_us``: the same with L2 and MALL flushed before
  every launch (a 2 x 256 MiB device copy), and ``cold_median_us`` that less
  the pair's own cost.  Every timed launch is queued behind a spin kernel, so
  the events time device work only, not the host's launch calls;
* ``graph_us``: device time per step with the host's per-launch cost removed
  (20 steps captured in one HIP graph, replayed 10 times), outputs checked
  equal to an eager run's;
* ``roofline``: the algorithmic work of one launch (compulsory HBM bytes, or
  MFMA FLOPs, of the fused block) over the median launch time, against the
  MI355X published peak, with the measured HBM ``traffic`` per launch
  (rocprofv3 counters, profiles/<workload>_hbm_traffic.txt);
* ``cost_model``: the MI355X launch model's prediction from the launch plans
  the entry points record, against ``graph_us``; the headline's
  ``cost_model.holdout`` does the same on shapes outside the nine
  configurations (configs.holdout_workloads), which no work term of the
  model was written against;
* ``reference_cost_model``: the reference's own cost model
  (CostModel.cpp, restated in libnpu_host.so) on the block's linalg form
  through the reference's pipeline, at the MI355X target
  (npu_hw_target_mi355x): ``one_core_us`` is the sum of its outlined
  functions' ``time_sec``, which prices the whole op on one core, and
  ``per_core_share_us`` that divided by the target's 256 cores;
* ``cpu_baseline``: the CPU restatement of the reference's execution path
  (the oracle: unfused scalar loop nests) on this host, one thread, on the
  full workload when that fits about 30 s (else as many images as fit,
  scaled); ``cpu_all_cores``: the OpenMP build of the same loops (outer
  parallel loops split over the threads, same results) on every thread given.
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
    ap.add_argument("--quick", action="store_true",
                    help="time only the K back-to-back launches of each configuration (for "
                         "counter and trace runs: every launch is then the workload itself)")
    ap.add_argument("--model-check", action="store_true",
                    help="only the launch model against graph times: the nine configurations "
                         "and the held-out shapes, one JSON line")
    ap.add_argument("--dump-plans", default=None,
                    help="write every configuration's launch plans and graph time to this JSON file")
    return ap.parse_args()


_SPIN_CYCLES_PER_US = None


def _spin_cycles_per_us():
    """Clock rate of torch's spin kernel (torch.cuda._sleep), measured once."""
    global _SPIN_CYCLES_PER_US
    if _SPIN_CYCLES_PER_US is None:
        import torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        a.record()
        torch.cuda._sleep(2_000_000)
        b.record()
        torch.cuda.synchronize()
        _SPIN_CYCLES_PER_US = 2_000_000 / max(a.elapsed_time(b) * 1e3, 1.0)
    return _SPIN_CYCLES_PER_US


def hold_stream(host_us):
    """Queues a spin kernel long enough for the host to enqueue `host_us` of
    launch calls behind it, so the timed launches then run back to back on
    the device and the events time device work only (not the host's launch
    cost).  The spin precedes the first timed event."""
    import torch
    torch.cuda._sleep(int((2.0 * host_us + 2000.0) * _spin_cycles_per_us()))


def _enqueue_us(w, d, o, stream, n=20):
    """Host microseconds per launch call of the block."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        w.run(d, o, stream)
    t = (time.perf_counter() - t0) / n * 1e6
    torch.cuda.synchronize()
    return t


def time_gpu(w, steps, warmup):
    """Returns (avg seconds per launch from HIP events, wall seconds, outputs):
    `steps` launches back to back behind a stream hold, between two events."""
    import torch

    from npu_amd import configs
    d = configs.to_device(w.make_inputs())
    o = w.make_outputs(d)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        w.run(d, o, stream)
    host = _enqueue_us(w, d, o, stream)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hold_stream(host * steps)
    start.record(stream)
    for _ in range(steps):
        w.run(d, o, stream)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) * 1e-3 / steps, wall, o


def time_per_launch(w, reps=100, warmup=10, cold=False, batch=1):
    """Device times per launch (seconds, sorted): an event pair around each of
    `reps` batches of `batch` back-to-back launches, queued behind a stream
    hold, divided by `batch`.  An event pair adds about 2 us to what it
    brackets, so batches of 10 give the per-launch time; single launches
    between event pairs carry the pair's cost.  cold: before every batch, a
    device copy between two 256 MiB buffers pushes the block's data out of L2
    and MALL."""
    import torch

    from npu_amd import configs
    d = configs.to_device(w.make_inputs())
    o = w.make_outputs(d)
    stream = torch.cuda.current_stream()
    flush = None
    if cold:
        flush = (torch.empty(64 << 20, dtype=torch.float32, device="cuda"),
                 torch.empty(64 << 20, dtype=torch.float32, device="cuda"))
        flush[0].zero_()
    for _ in range(warmup):
        w.run(d, o, stream)
    host = _enqueue_us(w, d, o, stream) * batch + (30.0 if cold else 10.0)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    torch.cuda.synchronize()
    hold_stream(host * reps)
    for a, b in ev:
        if flush is not None:
            flush[1].copy_(flush[0])
        a.record(stream)
        for _ in range(batch):
            w.run(d, o, stream)
        b.record(stream)
    torch.cuda.synchronize()
    return sorted(a.elapsed_time(b) * 1e-3 / batch for a, b in ev)


def _pct(xs, q):
    return xs[min(len(xs) - 1, int(round(q * (len(xs) - 1))))]


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


def reference_model(w):
    """The reference's cost model on the workload's linalg form at the MI355X
    target, next to the measured time (see the module docstring)."""
    from npu_amd import configs, host, mlir, pipeline
    bits = {"f32": 32, "bf16": 16, "i8": 8}[w.dtype]
    t = host.mi355x_target(bits)
    rep = pipeline.run(mlir.parse_functions(configs.linalg_text(w))[0], t)
    one = sum(f["cost"].time_sec for f in rep["functions"]) * 1e6
    return {"target": f"npu_hw_target_mi355x({bits})", "functions": len(rep["functions"]),
            "one_core_us": round(one, 2), "cores": t.num_cores,
            "per_core_share_us": round(one / t.num_cores, 3)}


def holdouts():
    """Launch-model prediction against the graph time on shapes outside the
    nine configurations."""
    from npu_amd import configs
    out = []
    for w in configs.holdout_workloads():
        gsec, _ = time_graph(w, 20)
        pred, parts, _ = model_prediction(w)
        out.append({"workload": w.name, "desc": w.desc, "graph_us": round(gsec * 1e6, 3),
                    "model_us": round(pred, 3), "model_error": round(pred / (gsec * 1e6) - 1, 3),
                    "model_kernels": parts, "reference_cost_model": reference_model(w)})
        print(f"# holdout {w.name}: graph {gsec * 1e6:.2f} us, model {pred:.2f} us",
              file=sys.stderr, flush=True)
    return out


def cpu_threads():
    """Threads the all-cores baseline uses: OMP_NUM_THREADS when set (the GPU
    box sets it to its CPU share), else every logical CPU visible."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "")))
    except ValueError:
        return os.cpu_count() or 1


def cpu_sample(w, budget_s=30.0, threaded=False):
    """Times the oracle on a bounded sample; returns the baseline object.

    Batched workloads time one image first; if the whole batch is estimated
    to fit the budget it is timed in full, otherwise as many images as fit,
    scaled to the batch (images are independent).  threaded: the OpenMP
    build of the oracle on cpu_threads() threads."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import contextlib

    import oracle
    import refs

    ctx = oracle.threaded if threaded else contextlib.nullcontext
    inp = w.make_inputs()
    n = w.units
    with ctx():
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
    cores = cpu_threads() if threaded else 1
    how = (f"OpenMP build, outer parallel loops over {cores} threads" if threaded
           else "1 thread")
    return {"value": round(dt * 1e6, 1), "unit": "us", "cores": cores, "kind": "port",
            "sample": sample + f"; unfused scalar loop nests, -O2 -ffp-contract=off, {how}",
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
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return (f"{line.split(':', 1)[1].strip()} (nproc {nproc}, "
                        f"{os.cpu_count()} logical CPUs visible)")
    except OSError:
        pass
    return f"nproc {nproc}, {os.cpu_count()} logical CPUs"


def measure(w, steps, warmup, cpu=True, quick=False):
    """Every figure of one configuration (see the module docstring)."""
    import functools
    w.make_inputs = functools.lru_cache(maxsize=1)(w.make_inputs)  # seeded: same arrays
    sec, wall, _ = time_gpu(w, steps, warmup)
    if quick:
        rl = dict(w.roofline(sec), traffic=measured_traffic(w.name), bytes=w.bytes)
        rl["timed_on"] = "latency_us"
        return {"workload": w.name, "latency_us": round(sec * 1e6, 3), "wall_s": wall,
                "median_us": None, "p10_us": None, "p90_us": None, "reps": steps,
                "cold_median_us": None, "graph_us": None, "graph_matches_eager": None,
                "roofline": rl, "model_us": None, "model_error": 0.0, "model_kernels": [],
                "plans": []}
    warm = time_per_launch(w, 100, max(10, warmup), batch=10)
    pair = time_per_launch(w, 100, max(10, warmup))
    cold = time_per_launch(w, 100, max(10, warmup), cold=True)
    gsec, gsame = time_graph(w, 20)
    pred, parts, plans = model_prediction(w)
    med = _pct(warm, 0.5)
    # cold: the single-launch event-pair time with caches flushed, less the
    # pair's own cost (warm single launches minus the warm median)
    cold_us = _pct(cold, 0.5) - (_pct(pair, 0.5) - med)
    rl = dict(w.roofline(sec), traffic=measured_traffic(w.name), flops=w.flops,
              mfma_flops=w.mfma_flops, bytes=w.bytes, floor_us=round(w.floor_s() * 1e6, 3))
    rl["timed_on"] = "latency_us"
    if rl["traffic"]:
        rl["traffic_over_algorithmic"] = round(rl["traffic"] / w.bytes, 3)
    m = {"workload": w.name, "latency_us": round(sec * 1e6, 3), "wall_s": wall,
         "median_us": round(med * 1e6, 3), "p10_us": round(_pct(warm, 0.1) * 1e6, 3),
         "p90_us": round(_pct(warm, 0.9) * 1e6, 3), "reps": f"{len(warm)} x 10 launches",
         "event_pair_median_us": round(_pct(pair, 0.5) * 1e6, 3),
         "cold_event_pair_median_us": round(_pct(cold, 0.5) * 1e6, 3),
         "cold_median_us": round(cold_us * 1e6, 3),
         "graph_us": round(gsec * 1e6, 3), "graph_matches_eager": gsame,
         "roofline": rl, "median_frac": round(w.roofline(med)["frac"], 4),
         "cold_frac": round(w.roofline(cold_us)["frac"], 4),
         "model_us": round(pred, 3), "model_error": round(pred / (gsec * 1e6) - 1, 3),
         "model_kernels": parts, "plans": plans, "reference_cost_model": reference_model(w)}
    if cpu:
        m["cpu_baseline"] = cpu_sample(w)
        m["cpu_all_cores"] = cpu_sample(w, budget_s=15.0, threaded=True)
    return m


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

    if args.model_check:
        rows = []
        for w in configs.all_workloads():
            gsec, _ = time_graph(w, 20)
            pred, parts, _ = model_prediction(w)
            rows.append({"workload": w.name, "graph_us": round(gsec * 1e6, 3),
                         "model_us": round(pred, 3), "model_error": round(pred / (gsec * 1e6) - 1, 3),
                         "model_kernels": parts})
            print(f"# {w.name}: graph {gsec * 1e6:.2f} us, model {pred:.2f} us", file=sys.stderr,
                  flush=True)
        print(json.dumps({"configs": rows, "holdout": holdouts()}), flush=True)
        return

    name = args.workload or configs.HEADLINE
    w = configs.by_name(name)
    head = measure(w, args.steps, args.warmup, cpu=not args.no_cpu, quick=args.quick)
    sec = head["latency_us"] * 1e-6
    dumped = [{"workload": w.name, "graph_us": head["graph_us"], "plans": head.pop("plans")}]
    line = {
        "metric": "fused-block latency",
        "value": head["latency_us"],
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
        "wall_s_timed_region": head.pop("wall_s"),
        "median_us": head["median_us"], "p10_us": head["p10_us"], "p90_us": head["p90_us"],
        "reps": head["reps"], "cold_median_us": head["cold_median_us"],
        "event_pair_median_us": head.get("event_pair_median_us"),
        "cold_event_pair_median_us": head.get("cold_event_pair_median_us"),
        "roofline": head["roofline"],
        "graph_us": head["graph_us"],
        "graph_matches_eager": head["graph_matches_eager"],
        "cost_model": {"predicted_us": head["model_us"], "measured_us": head["graph_us"],
                       "error": head["model_error"], "kernels": head["model_kernels"]},
        "reference_cost_model": head.get("reference_cost_model"),
    }
    if "cpu_baseline" in head:
        line["cpu_baseline"] = head["cpu_baseline"]
        line["cpu_all_cores"] = head["cpu_all_cores"]
    if args.blocks:
        blocks = []
        for other in configs.all_workloads():
            if other.name == w.name:
                continue
            b = measure(other, args.steps if args.quick else max(100, args.steps // 2),
                        args.warmup if args.quick else max(10, args.warmup // 2),
                        cpu=not args.no_cpu, quick=args.quick)
            dumped.append({"workload": other.name, "graph_us": b["graph_us"],
                           "plans": b.pop("plans")})
            b.pop("wall_s")
            blocks.append(b)
            print(f"# {other.name}: {b['latency_us']} us avg, median {b['median_us']} us, frac "
                  f"{b['roofline']['frac']:.3f}", file=sys.stderr, flush=True)
        line["blocks"] = blocks
        errs = [abs(line["cost_model"]["error"])] + [abs(b["model_error"]) for b in blocks]
        line["cost_model"]["within_25pct"] = f"{sum(e <= 0.25 for e in errs)}/{len(errs)}"
        if not args.quick:
            hold = holdouts()
            herrs = [abs(h["model_error"]) for h in hold]
            line["cost_model"]["holdout"] = hold
            line["cost_model"]["holdout_within_25pct"] = f"{sum(e <= 0.25 for e in herrs)}/{len(herrs)}"
            line["cost_model"]["holdout_mean_abs_error"] = round(sum(herrs) / len(herrs), 3)
    if args.dump_plans:
        with open(args.dump_plans, "w") as f:
            json.dump(dumped, f, indent=1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
