"""Benchmark of the MI355X sampler on the benchmark configs (C3 by default).

One step = one batched sampling step (``axs_sample_batch``; for C5 one MTP
verify step, ``axs_mtp_verify``) over synthetic inputs already resident in
HBM.  Input sets rotate so that their total exceeds 512 MB and the 256 MB
MALL cannot serve repeats.

Default workload, C3 (the north star): B=256 rows of V=262,144 bf16 logits,
repetition 1.05, presence 0.5, frequency 0.3, T 1.0, top_k 64, top_p 0.95,
min_p 0.02, 2,048-token histories, Philox draws.  ``--config C1|C2|C4|C5``
measures the other configs the same way.

Prints one JSON line:
  value         rows/s of the whole step (all kernels, hipEvents on the
                launch stream, K timed steps)
  roofline      the dominant kernel: its algorithmic bytes per launch / its
                average duration.  When the step is that one kernel (C2,
                C3, C4: k_row decides every row in place), the duration is
                the step time of back-to-back launches (hipEvents on the
                launch stream around K steps) if that is below the
                hipEvent-bracketed time of single launches; otherwise the
                latter (``kernel_timing`` says which).  ``traffic`` = HBM
                bytes per launch of that kernel measured by rocprofv3
                (FETCH_SIZE + WRITE_SIZE, copy-calibrated) and
                ``rocprof_avg_us`` its kernel-trace average, both from the
                committed profile summary of this config
  cpu_baseline  the CPU restatement of the reference sampler (oracle/, the
                reference's own Rust cannot be built here) on a bounded sample
                of the same rows, timed on this host
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ax-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "rows/s sampled at B=256,V=262144 bf16; achieved HBM GB/s (% of 8 TB/s peak)"
ROTATE_BYTES = 600e6  # input sets rotate over more than the 256 MB MALL, twice

WORKLOADS = {
    "C1": "C1: B=1 V=151936 f32, rep 1.1, T 0.7, top_k 40, top_p 0.95, 256-token history",
    "C2": "C2: B=64 V=151936 bf16, T U[0.3,1.2], top_k {0,20,50}, top_p U[0.8,1], min_p 0.05, "
          "presence 0.5, freq 0.3, 1024-token histories",
    "C3": "C3: B=256 V=262144 bf16, rep 1.05 + presence 0.5 + freq 0.3, T 1.0, top_k 64, "
          "top_p 0.95, min_p 0.02, 2048-token histories, Philox draws",
    "C4": "C4: B=128 V=151936 f32, allowed-token bitmask 5-60%, 32 bias entries/row, T 1.0, top_p 0.9",
    "C5": "C5: MTP verify B=32 depth 3 V=151936 bf16, target [B,4,V] + draft [B,3,V], T 0.6, top_p 0.95",
    "F1": "F1: LM head + greedy argmax (producer fusion) B=1 H=4096 V=151936, bf16 hidden and weight, "
          "token id only (logits not written)",
    "F2": "F2: LM head + greedy argmax (producer fusion) B=64 H=4096 V=151936, bf16 hidden and weight, "
          "f32 logits written",
}
LM_HEAD_SHAPES = {"F1": (1, 4096, 151936), "F2": (64, 4096, 151936)}  # batch rows, hidden size, vocabulary


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def profile_figures(cfg):
    """Figures of the committed rocprofv3 summary for this config
    (profiles/*_<cfg>.md): `traffic_bytes_per_launch=` (copy-calibrated
    FETCH_SIZE + WRITE_SIZE of the dominant kernel) and `rocprof_avg_us=`
    (its kernel-trace average).  Missing figures are None."""
    import glob

    out = {"traffic": None, "rocprof_avg_us": None, "file": None}
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", f"*_{cfg.lower()}.md"))):
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch="):
                    out["traffic"] = int(line.split("=")[1])
                    out["file"] = os.path.relpath(path, ROOT)
                elif line.startswith("rocprof_avg_us="):
                    out["rocprof_avg_us"] = float(line.split("=")[1])
    return out


def cpu_rows_per_s(fn, rows_per_call, seconds=12.0, max_threads=16, max_calls=64):
    """Times fn(nthreads) on 1 thread and on the host's cores (at most 16):
    each for seconds / 2 or max_calls calls, whichever ends first."""
    res = {}
    for threads in (1, min(max_threads, os.cpu_count() or 1)):
        n, t0 = 0, time.perf_counter()
        while True:
            fn(threads)
            n += rows_per_call
            el = time.perf_counter() - t0
            if el >= seconds / 2 or n >= max_calls * rows_per_call:
                break
        res[threads] = (n / el, n, el)
    return res


def cpu_baseline_sample(w):
    """The CPU restatement of sample_categorical_into on host f32 copies of
    (at most) 64 of the workload's rows (the reference samples host f32
    logits after a readback)."""
    from oracle import oracle

    oracle.lib()
    rows = min(w.B, 64)
    lf = np.ascontiguousarray(w.logits_f32()[:rows])
    hoff = w.hist_off[: rows + 1].copy() if w.hist is not None else None
    boff = w.bias_off[: rows + 1].copy() if w.bias_ids is not None else None
    mask = w.mask[:rows] if w.mask is not None else None
    ms = w.mask.shape[1] if w.mask is not None else 0
    us = np.linspace(0.01, 0.99, rows).astype(np.float32)

    def fn(threads):
        oracle.sample_batch(lf, 0, rows, w.V, w.V, w.params[:rows], w.hist, hoff, mask, ms, w.bias_ids,
                            w.bias_vals, boff, uniforms=us, nthreads=threads, explain=False)

    return cpu_rows_per_s(fn, rows), f"first {rows} rows as host f32"


def cpu_baseline_mtp(t, d, tp, dp, dids):
    from oracle import oracle
    from ax_sampler.synth import DTYPE_BF16

    oracle.lib()
    B, D1, V = t.shape
    us = np.linspace(0.01, 0.99, B * D1).astype(np.float32).reshape(B, D1)

    def fn(threads):
        oracle.mtp_verify_batch(t, d, DTYPE_BF16, B, D1 - 1, V, V, dids, tp, dp, uniforms=us, nthreads=threads)

    return cpu_rows_per_s(fn, B), f"all {B} sequences, bf16 target/draft widened on the host"


def cpu_baseline_lm_head(torch, hidden, weight):
    """A CPU statement of the LM-head step (f32 product of bf16 values,
    bf16 rounding, argmax) over a slice of the weight rows, scaled to the
    whole vocabulary; torch's CPU matmul on the host's cores."""
    B, H = hidden.shape
    V = weight.shape[0]
    part = 8192
    h = hidden.float().cpu()
    w = weight[:part].float().cpu()

    def fn(threads):
        torch.set_num_threads(threads)
        y = (h @ w.T).to(torch.bfloat16).float()
        y.argmax(dim=1)

    res = cpu_rows_per_s(fn, B, max_calls=1 << 20)  # time-bounded: 6 s per thread count
    scale = part / V  # rows/s over the slice -> over the full vocabulary
    res = {k: (v[0] * scale, v[1], v[2]) for k, v in res.items()}
    return res, (f"all {B} batch rows against {part} of the {V} weight rows (f32 matmul of the bf16 values, "
                 "bf16 rounding, argmax), rate scaled to the full vocabulary")


def rotating_sets(base, nbytes, torch):
    n = int(max(4, min(1024, math.ceil(ROTATE_BYTES / max(nbytes, 1)))))
    flat = base.reshape(-1)
    sets = [base] + [torch.roll(flat, shifts=7919 * k).reshape(base.shape).contiguous() for k in range(1, n)]
    return sets


def timed_steps(step, steps, warmup, stream, torch):
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return ev0.elapsed_time(ev1) / steps, wall


def kernel_times(s, step, steps, torch, _abi):
    """Per-kernel average durations over a second pass (events on the launch
    stream around each launch)."""
    s.timing(True)
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    kern = {}
    for k, name in enumerate(_abi.KERNEL_NAMES):
        ms, n = s.timing_read(k)
        if n:
            kern[name] = {"avg_us": 1e3 * ms / n, "launches": n}
    s.timing(False)
    return kern


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
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
    from ax_sampler import synth

    cfg = args.config
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    s = HipSampler(0, max_batch=256, max_vocab=262144)
    t0 = time.perf_counter()
    if cfg in LM_HEAD_SHAPES:
        B, H, V = LM_HEAD_SHAPES[cfg]
        gen = torch.Generator(device=dev).manual_seed(2)
        weight = (torch.randn(V, H, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        hidden = torch.randn(B, H, device=dev, generator=gen).to(torch.bfloat16)
        # F1 is a greedy decode step: only the token id leaves the kernel
        logits = torch.empty((B, V), dtype=torch.float32, device=dev) if cfg == "F2" else None
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        log(f"workload generated in {time.perf_counter() - t0:.1f}s")
        sptr = s._stream(stream)

        class _Res:
            token_ids = ids

        def step(i):
            _abi.check(s.L.axs_lm_head(s.ctx, hidden.data_ptr(), H, weight.data_ptr(), H, B, H, V, 1.0, 0.0,
                                       logits.data_ptr() if logits is not None else None,
                                       V if logits is not None else 0, ids.data_ptr(), sptr))
            return _Res

        rows_per_step = B
        # the weight (1.24 GB, larger than the MALL) is read once per step
        alg = V * H * 2 + B * H * 2 + (B * V * 4 if logits is not None else 0) + B * 4
        unit_rows = "rows/s"
    elif cfg == "C5":
        from oracle import oracle

        t, d, tp, dp = synth.make_c5(5)
        B, D1, V = t.shape
        D = D1 - 1
        rows = d.reshape(B * D, V)
        ur = np.random.default_rng(55).random(B * D).astype(np.float32)
        dids, _, _ = oracle.sample_batch(rows, synth.DTYPE_BF16, B * D, V, V, np.repeat(dp, D), uniforms=ur,
                                         nthreads=8, explain=False)
        dids = dids.reshape(B, D).astype(np.uint32)
        log(f"workload generated in {time.perf_counter() - t0:.1f}s")
        tt = torch.from_numpy(t.view(np.int16)).view(torch.bfloat16).to(dev)
        dd = torch.from_numpy(d.view(np.int16)).view(torch.bfloat16).to(dev)
        tsets = rotating_sets(tt, tt.numel() * 2 + dd.numel() * 2, torch)
        dsets = [torch.roll(dd.reshape(-1), shifts=104729 * k).reshape(dd.shape).contiguous()
                 for k in range(len(tsets))]
        di = torch.from_numpy(dids.view(np.int32)).to(dev)
        tpd = torch.from_numpy(tp.view(np.uint8)).to(dev)
        dpd = torch.from_numpy(dp.view(np.uint8)).to(dev)

        def step(i):
            return s.mtp_verify(tsets[i % len(tsets)], dsets[i % len(dsets)], di, tpd, dpd)

        rows_per_step = B
        alg = (t.size + d.size) * 2 + B * D * 4 + B * 2 * 64 + B * (D1 + 1) * 4
        unit_rows = "sequences/s"
    else:
        w = {"C1": lambda: synth.make_c1(1), "C2": lambda: synth.make_c2(2), "C3": lambda: synth.make_c3(3),
             "C4": lambda: synth.make_c4(4)}[cfg]()
        log(f"workload generated in {time.perf_counter() - t0:.1f}s")
        if w.dtype == synth.DTYPE_BF16:
            base = torch.from_numpy(w.logits.view(np.int16)).view(torch.bfloat16).to(dev)
        else:
            base = torch.from_numpy(w.logits).to(dev)
        sets = rotating_sets(base, base.numel() * base.element_size(), torch)
        hist = (torch.from_numpy(w.hist.view(np.int32)).to(dev), torch.from_numpy(w.hist_off).to(dev)) \
            if w.hist is not None else None
        mask = torch.from_numpy(w.mask.view(np.int32)).to(dev) if w.mask is not None else None
        bias = (torch.from_numpy(w.bias_ids.view(np.int32)).to(dev), torch.from_numpy(w.bias_vals).to(dev),
                torch.from_numpy(w.bias_off).to(dev)) if w.bias_ids is not None else None
        params = torch.from_numpy(w.params.view(np.uint8)).to(dev)

        # one prepared descriptor per input set: a step is one C-ABI call
        preps = [s.prepare_sample(x, params, history=hist, mask_words=mask, bias=bias) for x in sets]
        sptr = s._stream(stream)

        def step(i):
            p = preps[i % len(preps)]
            _abi.check(s.L.axs_sample_batch(s.ctx, p._dp, p._op, sptr))
            return p.result

        rows_per_step = w.B
        alg = w.algorithmic_bytes()
        unit_rows = "rows/s"

    ms_step, wall = timed_steps(step, args.steps, args.warmup, stream, torch)
    value = rows_per_step / (ms_step * 1e-3)
    kern = kernel_times(s, step, args.steps, torch, _abi)
    res = step(0)
    torch.cuda.synchronize()
    # the dominant kernel and its algorithmic bytes per launch
    pipeline_rows = rows_per_step * 7 if cfg == "C5" else rows_per_step  # C5: 4 target + 3 draft rows each
    name0 = "k_row" if pipeline_rows >= 64 else "k_stream"
    kern = {(name0 if k == "k_stream" else k): v for k, v in kern.items()}
    dom = max(kern.items(), key=lambda kv: kv[1]["avg_us"])
    dom_name, dom_us = dom[0], dom[1]["avg_us"]
    # One launch per step: the step time of K back-to-back launches is the
    # kernel's own time plus the gap between launches, and never more than
    # the event-bracketed time of a single launch (which adds the events'
    # latency); the roofline uses the smaller.  Several kernels per step:
    # the dominant one's event-bracketed average.
    single = len(kern) == 1 and dom[1]["launches"] == args.steps
    timing_src = "hipEvents around each launch"
    if single and ms_step * 1e3 < dom_us:
        dom_us = ms_step * 1e3
        timing_src = "step time (one launch per step, back to back)"
    prof = profile_figures(cfg)
    if dom_name in ("k_row", "k_stream", "k_lm_head"):
        dom_alg = alg
    elif dom_name == "k_exact_mat":
        # the second pass re-reads the listed rows (and their mask words)
        fl = res.flags.cpu().numpy().view(np.uint32) if cfg not in ("C5", "F1", "F2") else None
        n_ex = int(np.count_nonzero(fl & np.uint32(_abi.FLAG_EXACT_PATH))) if fl is not None else rows_per_step
        dom_alg = int(alg * n_ex / max(rows_per_step, 1))
    else:
        dom_alg = None
    achieved = dom_alg / (dom_us * 1e-6) / 1e9 if dom_alg else None

    cpu = None
    if not args.no_cpu_baseline:
        if cfg in LM_HEAD_SHAPES:
            cb, sample = cpu_baseline_lm_head(torch, hidden, weight)
        elif cfg == "C5":
            cb, sample = cpu_baseline_mtp(t, d, tp, dp, dids)
        else:
            cb, sample = cpu_baseline_sample(w)
        one, allc = cb[1], max(cb.items())
        cpu = {
            "value": round(allc[1][0], 1),
            "unit": unit_rows,
            "cores": allc[0],
            "kind": "port",
            "sample": (f"{sample}, repeated; {allc[1][1]} rows in {allc[1][2]:.1f}s on {allc[0]} threads; "
                       f"1 thread: {one[0]:.1f} {unit_rows} ({one[1]} rows in {one[2]:.1f}s)"),
            "value_1thread": round(one[0], 1),
        }

    line = {
        "metric": METRIC if cfg == "C3" else f"{unit_rows} on {cfg}; achieved HBM GB/s (% of 8 TB/s peak)",
        "value": round(value, 1),
        "unit": unit_rows,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if cfg in ("C1", "C4") else "bf16",
        "data": ("synthetic (seeded; the 1.24 GB weight exceeds the 256 MB MALL)" if cfg in LM_HEAD_SHAPES
                 else "synthetic (seeded, rotating input sets over more than 512 MB)"),
        "config": {"workload": WORKLOADS[cfg], "global_batch": rows_per_step},
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(achieved, 1) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": prof["traffic"],
            "traffic_source": (f"{prof['file']} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE of {dom_name}; "
                               "scaled by a 256 MiB copy's readings)") if prof["file"] else None,
            "algorithmic_bytes": dom_alg,
            "kernel_avg_us": round(dom_us, 3),
            "kernel_timing": timing_src,
            "rocprof_avg_us": prof["rocprof_avg_us"],
            "step_GBps": round(alg / (ms_step * 1e-3) / 1e9, 1),
        },
        "kernels": {k: {"avg_us": round(v["avg_us"], 3), "launches": v["launches"]} for k, v in kern.items()},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    s.close()


if __name__ == "__main__":
    main()
