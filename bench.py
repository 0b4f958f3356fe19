"""Benchmark of the MI355X sampler on the north-star workload.

One step = one batched sampling step (``axs_sample_batch``) over B=256 rows of
V=262,144 bf16 logits already resident in HBM (config C3: repetition 1.05,
presence 0.5, frequency 0.3, T 1.0, top_k 64, top_p 0.95, min_p 0.02,
2,048-token histories, Philox draws).  Four input sets (4 x 136 MB, more than
the 256 MB MALL) rotate so repeated steps do not read from the Infinity Cache.

Prints one JSON line:
  value      rows/s of the whole step (all kernels), timed over K steps
  roofline   the single HBM pass (k_stream, which also decides the rows):
             algorithmic bytes per launch / its average duration from
             hipEvents on its launch stream
  cpu_baseline  the CPU restatement of the reference sampler (oracle/, the
             reference's own Rust cannot be built here) on a bounded sample
             of the same rows, timed on this host
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ax-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def measured_traffic():
    """HBM bytes per k_stream launch on this workload, from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (copy-calibrated); None if absent."""
    path = os.path.join(ROOT, "profiles", "k_stream_c3.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch"):
                    return int(line.split("=")[1])
    except OSError:
        pass
    return None


def cpu_baseline(w, seconds=12.0, max_threads=16):
    """Times the CPU restatement of sample_categorical_into on f32 copies of the
    workload's rows (the reference samples host f32 logits after readback)."""
    from oracle import oracle

    oracle.lib()
    rows = min(w.B, 64)
    lf = w.logits_f32()[:rows].copy()
    hoff = w.hist_off[: rows + 1].copy()
    us = np.linspace(0.01, 0.99, rows).astype(np.float32)
    res = {}
    for threads in (1, min(max_threads, os.cpu_count() or 1)):
        n, t0 = 0, time.perf_counter()
        while True:
            oracle.sample_batch(lf, 0, rows, w.V, w.V, w.params[:rows], w.hist, hoff, uniforms=us,
                                nthreads=threads, explain=False)
            n += rows
            el = time.perf_counter() - t0
            if el >= seconds / 2 or n >= 64 * rows:
                break
        res[threads] = (n / el, n, el)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sets", type=int, default=4)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device-to-device copy (known HBM bytes) a few "
                         "times: the reference reading for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this sampler benchmark runs on one GPU only (--gpus {args.gpus} "
              "requested); rows are independent, multi-GPU would shard rows with no exchange.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel(), "launches": 5}), flush=True)
        return

    from ax_sampler import HipSampler, _abi
    from ax_sampler.synth import make_c3

    t0 = time.perf_counter()
    w = make_c3(3)
    log(f"workload generated in {time.perf_counter() - t0:.1f}s")
    dev = torch.device("cuda", 0)
    base = torch.from_numpy(w.logits.view(np.int16)).view(torch.bfloat16).to(dev)
    sets = [base] + [torch.roll(base, shifts=7919 * k, dims=1).contiguous() for k in range(1, args.sets)]
    hist = torch.from_numpy(w.hist.view(np.int32)).to(dev)
    hoff = torch.from_numpy(w.hist_off).to(dev)
    s = HipSampler(0, max_batch=w.B, max_vocab=w.V)
    params = torch.from_numpy(w.params.view(np.uint8)).to(dev)
    stream = torch.cuda.current_stream(dev)

    def step(i):
        return s.sample(sets[i % len(sets)], params, history=(hist, hoff))

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # timed region: exactly K steps, synchronized on both sides
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    rows_per_s = w.B * args.steps / (ev0.elapsed_time(ev1) / 1e3)

    # per-kernel durations over a second timed pass (events on the launch stream)
    s.timing(True)
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    kern = {}
    for k, name in enumerate(_abi.KERNEL_NAMES):
        ms, n = s.timing_read(k)
        if n:
            kern[name] = {"avg_us": 1e3 * ms / n, "launches": n}
    s.timing(False)
    chunk_us = kern["k_stream"]["avg_us"]
    alg = w.algorithmic_bytes()
    achieved = alg / (chunk_us * 1e-6) / 1e9
    step_gbs = alg / (ms_step * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        cb = cpu_baseline(w)
        one = cb[1]
        allc = max(cb.items())
        cpu = {
            "value": round(allc[1][0], 1),
            "unit": "rows/s",
            "cores": allc[0],
            "kind": "port",
            "sample": (f"first 64 C3 rows as host f32, repeated; {allc[1][1]} rows in "
                       f"{allc[1][2]:.1f}s on {allc[0]} threads; 1 thread: {one[0]:.1f} rows/s "
                       f"({one[1]} rows in {one[2]:.1f}s)"),
            "value_1thread": round(one[0], 1),
        }

    line = {
        "metric": "rows/s sampled at B=256,V=262144 bf16; achieved HBM GB/s (% of 8 TB/s peak)",
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded C3 workload, 4 rotating 136 MB input sets)",
        "config": {
            "workload": "C3: B=256 V=262144 bf16, rep 1.05 + presence 0.5 + freq 0.3, T 1.0, "
                        "top_k 64, top_p 0.95, min_p 0.02, 2048-token histories, Philox draws",
            "global_batch": w.B,
            "vocab": w.V,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "k_stream",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "profiles/k_stream_c3.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                              "scaled by a 256 MiB copy's readings)",
            "algorithmic_bytes": alg,
            "kernel_avg_us": round(chunk_us, 3),
            "step_GBps": round(step_gbs, 1),
        },
        "kernels": {k: {"avg_us": round(v["avg_us"], 3), "launches": v["launches"]} for k, v in kern.items()},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    s.close()


if __name__ == "__main__":
    main()
