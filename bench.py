#!/usr/bin/env python3
"""Benchmark of the token-sampling hot path on one MI355X.

Headline: the fused sampler on the full-penalty workload -- B=256 rows,
V=128256 fp32 logits, 2048-id Zipf(1.1) histories, repetition 1.1 /
presence 0.5 / frequency 0.3, T 0.7, top-k 40, top-p 0.9 -- with every input
already resident in HBM.  A step is one cx_sample_f32 call over the batch.

  value        sampled rows/s over exactly `--steps` timed steps; each step
               reads the next of several copies of the logits (together
               beyond the 256 MB Infinity Cache), so the logits come from
               HBM; the same timing on one re-read buffer is "hot_cache"
  roofline     algorithmic bytes of one launch / the fused kernel's mean
               duration (start / stop events the dispatch itself records,
               on the kernel's stream), against 8 TB/s; traffic from the
               FETCH_SIZE / WRITE_SIZE summary in profiles/
  cpu_baseline the NumPy oracle on the host, one core, on a bounded sample
               of the same rows (reported beside, not a target); also a
               process pool of up to 16 workers (cpu_baseline_pool)

The other workloads (nucleus, typical-p, speculative verify, heterogeneous bf16) are
timed the same way and reported under "other_workloads"; "host_calls" times
the drop-in Sampler on numpy rows as the reference's engine calls it
(copies to and from the device included).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBPS = 8000.0
METRIC = "sampled rows/sec + achieved HBM GB/s, B=256 V=128256 penalties+top-k+top-p"


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def copy_probe(dev) -> None:
    """Five 512 MiB device-to-device copies (torch copy_): a kernel whose HBM
    traffic is known exactly, to scale FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    _say("[bench] copy probe: 5 x 512 MiB device copy")
    src = torch.ones(128 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


# Inputs are rotated over enough copies to exceed twice MI355X's 256 MB
# Infinity Cache, so a timed step reads its logits from HBM, not from the
# cache the previous step filled.
ROTATE_BYTES = 768 << 20


def _copies(nbytes: int, rotate: bool) -> int:
    return max(1, -(-ROTATE_BYTES // max(nbytes, 1))) if rotate else 1


class DeviceSample:
    """A SampleWorkload uploaded to the GPU, ready for repeated calls; with
    ``rotate`` each call reads the next of several copies of the logits."""

    def __init__(self, w, dev, rotate: bool = True):
        import torch
        from chenxing_amd.params import pack_rows
        self.w = w
        if w.dtype == "bf16":
            x = torch.from_numpy(w.logits.view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            x = torch.from_numpy(w.logits).to(dev)
        n = _copies(x.numel() * x.element_size(), rotate)
        self.xs = [x] + [x.clone() for _ in range(n - 1)]
        self.i = 0
        self.prm = torch.from_numpy(pack_rows(w.params).view(np.uint8)).to(dev)
        self.u = torch.from_numpy(w.u).to(dev)
        self.h = torch.from_numpy(w.hist).to(dev) if w.hist.size else None
        self.hl = torch.from_numpy(w.hist_len).to(dev) if w.hist.size else None
        self.ids = torch.empty(w.B, dtype=torch.int32, device=dev)
        self.st = torch.empty(w.B, dtype=torch.int32, device=dev)

    def __call__(self):
        from chenxing_amd import _lib
        x = self.xs[self.i]
        self.i = (self.i + 1) % len(self.xs)
        _lib.sample_device(x, self.prm, self.u, self.h, self.hl, self.ids, self.st)


class DeviceVerify:
    def __init__(self, w, dev, rotate: bool = True):
        import torch
        self.w = w
        t = torch.from_numpy(w.target).to(dev)
        d = torch.from_numpy(w.draft).to(dev)
        n = _copies(t.numel() * 4 + d.numel() * 4, rotate)
        self.ts = [t] + [t.clone() for _ in range(n - 1)]
        self.ds = [d] + [d.clone() for _ in range(n - 1)]
        self.i = 0
        self.ids = torch.from_numpy(w.draft_ids).to(dev)
        self.u = torch.from_numpy(w.u).to(dev)
        self.T = torch.from_numpy(w.temperature).to(dev)
        B = w.target.shape[0]
        self.out = [torch.empty(B, dtype=torch.int32, device=dev) for _ in range(4)]

    def __call__(self):
        from chenxing_amd import _lib
        # a batch with every temperature 0 needs no draft logits (greedy verify
        # compares target argmaxes with the proposals); without them the
        # stochastic stages are not launched, as in the host variant
        t, d = self.ts[self.i], self.ds[self.i]
        self.i = (self.i + 1) % len(self.ts)
        draft = None if not np.any(self.w.temperature) else d
        _lib.spec_verify_device(t, draft, self.ids, self.u, self.T, *self.out)


# The LM head with the greedy draw fused: a Llama-3-8B-sized head (hidden
# size 4096, 128256 tokens) at a decode batch of 16 rows, bf16.
HEAD_B, HEAD_D, HEAD_V = 16, 4096, 128256


class DeviceHead:
    """Random bf16 hidden states and head weights on the GPU (the weights,
    1 GB, exceed the Infinity Cache: every step streams them from HBM)."""

    def __init__(self, dev, B=HEAD_B, D=HEAD_D, V=HEAD_V):
        import torch
        g = torch.Generator(device=dev)
        g.manual_seed(7)
        self.w = (torch.randn(V, D, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        self.h = torch.randn(B, D, generator=g, device=dev).to(torch.bfloat16)
        self.ids = torch.empty(B, dtype=torch.int32, device=dev)
        self.mx = torch.empty(B, dtype=torch.float32, device=dev)

    def __call__(self):
        from chenxing_amd import _lib
        _lib.lmhead_argmax_device(self.h, self.w, self.ids, self.mx)

    def unfused(self):
        """The same through torch: F.linear (a library GEMM, hipBLASLt) writes
        the bf16 logits, then torch.argmax reads them."""
        import torch
        return torch.argmax(torch.nn.functional.linear(self.h, self.w), dim=1)


def time_steps(fn, steps: int, warmup: int, kernel: int):
    """(ms per step over exactly `steps` calls, mean fused-kernel ms)."""
    import torch
    from chenxing_amd import _lib
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    step_ms = a.elapsed_time(b) / steps
    # a second pass with the library's per-launch events for the kernel itself
    _lib.timing_read(kernel)
    _lib.timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    kms, n = _lib.timing_read(kernel)
    for k in range(_lib.KERNEL_KINDS):
        _lib.timing_read(k)
    return step_ms, kms / max(n, 1)


def cpu_baseline(w, seconds: float) -> dict:
    """The oracle (``oracle.sampler_ref.sample_row``, numpy, one core) on as many
    rows of the workload as fit in about `seconds`."""
    from oracle import sampler_ref as R
    hl = R.hist_rows_to_lists(w.hist, w.hist_len) if w.hist.size else None
    n = 0
    t0 = time.perf_counter()
    while True:
        b = n % w.B
        R.sample_row(w.logits[b], w.params[b], None if hl is None else hl[b], float(w.u[b]))
        n += 1
        if time.perf_counter() - t0 >= seconds and n >= 8:
            break
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 2), "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"{n} rows of the B={w.B} V={w.V} workload ({dt:.1f} s, numpy "
                      f"{np.__version__}, single thread, {_cpu_model()})"}


_POOL_W = None


def _pool_init(w):
    global _POOL_W
    _POOL_W = w


def _pool_rows(args):
    """Rows [lo, hi) of the pool workload through the oracle; returns the count."""
    from oracle import sampler_ref as R
    lo, hi = args
    w = _POOL_W
    hl = R.hist_rows_to_lists(w.hist, w.hist_len) if w.hist.size else None
    for i in range(lo, hi):
        b = i % w.B
        R.sample_row(w.logits[b], w.params[b], None if hl is None else hl[b], float(w.u[b]))
    return hi - lo


def cpu_baseline_pool(w, rows_per_worker: int, workers: int) -> dict:
    """The same oracle in a process pool, `workers` processes (one core each),
    `rows_per_worker` rows each: the multi-core CPU figure."""
    import multiprocessing as mp
    ctx = mp.get_context("fork")
    with ctx.Pool(workers, initializer=_pool_init, initargs=(w,)) as pool:
        pool.map(_pool_rows, [(0, 1)] * workers)            # warm the workers
        t0 = time.perf_counter()
        n = sum(pool.map(_pool_rows, [(k * rows_per_worker, (k + 1) * rows_per_worker)
                                      for k in range(workers)]))
        dt = time.perf_counter() - t0
    return {"value": round(n / dt, 2), "unit": "rows/s", "cores": workers, "kind": "port",
            "sample": f"{n} rows of the B={w.B} V={w.V} workload in a {workers}-process pool "
                      f"({dt:.1f} s, numpy {np.__version__}, {_cpu_model()})"}


OTHER = {  # name: (workload factory, kernel whose launches are timed)
    "nucleus": ("nucleus", {}, 0),
    "nucleus_greedy": ("nucleus", {"greedy": True}, 0),
    "typical": ("typical", {}, 0),
    "hetero_bf16": ("hetero_bf16", {}, 0),
    "spec_verify": ("spec_verify", {}, 2),
    "spec_verify_greedy": ("spec_verify", {"greedy": True}, 2),
    "lmhead_greedy": ("lmhead", {}, 7),
}



def time_other(name: str, dev, steps: int, warmup: int) -> dict:
    import torch
    from chenxing_amd import _lib, workloads as W
    fac, kw, kernel = OTHER[name]
    if name == "lmhead_greedy":
        return time_head(dev, steps, warmup)
    wk = getattr(W, fac)(**kw)
    if name.startswith("spec"):
        fn = DeviceVerify(wk, dev)
        nb = W.verify_algorithmic_bytes(wk)
        rows = wk.target.shape[0]
    else:
        fn = DeviceSample(wk, dev)
        nb = W.algorithmic_bytes(wk)
        rows = wk.B
    sm, km = time_steps(fn, steps, warmup, kernel)
    entry = {"rows_per_s": round(rows / (sm / 1e3), 1), "ms_per_step": round(sm, 5),
             "algorithmic_bytes": nb, "step_GBps": round(nb / (sm / 1e3) / 1e9, 1),
             "main_kernel_ms": round(km, 5)}
    if not name.startswith("spec"):
        entry["slow_path_rows"] = int(np.sum((fn.st.cpu().numpy() & 0x100) != 0))
    del fn
    torch.cuda.empty_cache()
    return entry


def time_head(dev, steps: int, warmup: int) -> dict:
    """The fused LM head + greedy argmax, beside the unfused library path."""
    import torch
    from chenxing_amd import _lib
    fn = DeviceHead(dev)
    sm, km = time_steps(fn, steps, warmup, _lib.KERNEL_LMHEAD)
    for _ in range(warmup):
        fn.unfused()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn.unfused()
    b.record()
    torch.cuda.synchronize()
    um = a.elapsed_time(b) / steps
    nb = HEAD_V * HEAD_D * 2 + HEAD_B * HEAD_D * 2 + HEAD_B * 8
    ach = nb / (km / 1e3) / 1e9
    entry = {"rows_per_s": round(HEAD_B / (sm / 1e3), 1), "ms_per_step": round(sm, 5),
             "algorithmic_bytes": nb, "step_GBps": round(nb / (sm / 1e3) / 1e9, 1),
             "main_kernel_ms": round(km, 5),
             "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                          "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                          "mfma_TFLOPs": round(2 * HEAD_B * HEAD_D * HEAD_V / (km / 1e3) / 1e12,
                                               1)},
             "unfused_ms_per_step": round(um, 5),
             "config": {"B": HEAD_B, "D": HEAD_D, "V": HEAD_V, "dtype": "bf16"},
             "note": "logits = h @ W.T (bf16, fp32 accumulation) with the argmax fused; "
                     "unfused = torch F.linear writing bf16 logits, then torch.argmax"}
    del fn
    torch.cuda.empty_cache()
    return entry


def time_host_calls(w, calls: int, warmup: int) -> dict:
    """The drop-in ``Sampler`` as the reference's callers use it: ``sample`` on
    one numpy row per call (engine.py:165), and ``sample_batch`` on the whole
    numpy batch.  Each call copies its rows and histories to the device, runs
    both launches and copies the ids back (PCIe-inclusive, host timer)."""
    from dataclasses import asdict
    from chenxing_amd import Sampler, SamplingParams
    n = min(w.B, 16)
    s = Sampler(w.V)
    rows = [np.ascontiguousarray(w.logits[b]) for b in range(n)]
    ps = [SamplingParams(**asdict(w.params[b])) for b in range(n)]
    hl = [[int(i) for i in w.hist[b, :w.hist_len[b]]] for b in range(n)]
    for i in range(warmup):
        s.sample(rows[i % n], ps[i % n], hl[i % n])
    ts = []
    for i in range(calls):
        t0 = time.perf_counter()
        s.sample(rows[i % n], ps[i % n], hl[i % n])
        ts.append(time.perf_counter() - t0)
    ts.sort()
    one = {"median_us": round(1e6 * ts[len(ts) // 2], 1),
           "p90_us": round(1e6 * ts[(9 * len(ts)) // 10], 1), "calls": calls,
           "note": f"Sampler.sample on one numpy fp32 row (V={w.V}, {w.hist.shape[1]}-id "
                   "history, all three penalties), copies and both launches included"}
    bp = [SamplingParams(**asdict(p)) for p in w.params]
    bh = [[int(i) for i in w.hist[b, :w.hist_len[b]]] for b in range(w.B)]
    s.sample_batch(w.logits, bp, bh)
    tb = []
    for _ in range(5):
        t0 = time.perf_counter()
        s.sample_batch(w.logits, bp, bh)
        tb.append(time.perf_counter() - t0)
    tb.sort()
    batch = {"median_ms": round(1e3 * tb[2], 3), "rows_per_s": round(w.B / tb[2], 1),
             "note": f"Sampler.sample_batch on the numpy [{w.B}, {w.V}] batch: the "
                     "PCIe-inclusive rate of the host-memory entry point"}
    return {"sample": one, "sample_batch": batch}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--only", choices=list(OTHER),
                    help="time one of the other workloads alone and print its entry "
                         "(for profiling that workload)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 512 MiB device copy (torch copy_) 5 times: the "
                         "reference kernel for scaling FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the sampled rows are independent, so N GPUs "
              "would each run their own B/N slice with no exchange; run with --gpus 1",
              file=sys.stderr)
        return 2

    from chenxing_amd import workloads as W
    if args.only:
        import torch
        from chenxing_amd import _lib
        _lib.load()
        _say(f"[bench] {args.only}")
        entry = time_other(args.only, torch.device("cuda:0"), args.steps, args.warmup)
        if args.copy_probe:
            copy_probe(torch.device("cuda:0"))
        print(json.dumps({"workload": args.only, "steps": args.steps, **entry}), flush=True)
        return 0
    _say("[bench] generating full_penalty workload")
    w = W.full_penalty()

    # The CPU figures come first: the process pool forks before this process
    # touches the GPU.
    cpu = cpu_pool = None
    if args.cpu_seconds > 0:
        _say("[bench] CPU baseline (oracle)")
        cpu = cpu_baseline(w, args.cpu_seconds)
        # the pool: as many rows per worker as one core did in about half
        # the single-core time, on at most 16 workers
        workers = max(1, min(16, os.cpu_count() or 1))
        per = max(4, int(cpu["value"] * args.cpu_seconds / 2))
        _say(f"[bench] CPU baseline, {workers}-process pool")
        cpu_pool = cpu_baseline_pool(w, per, workers)

    import torch
    from chenxing_amd import _lib
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    _lib.load()
    dev = torch.device("cuda:0")
    ds = DeviceSample(w, dev)
    _say(f"[bench] timing full_penalty over {len(ds.xs)} rotating copies of the logits")
    step_ms, kern_ms = time_steps(ds, args.steps, args.warmup, _lib.KERNEL_SAMPLE)
    st = ds.st.cpu().numpy()
    del ds
    torch.cuda.empty_cache()
    nbytes = W.algorithmic_bytes(w)
    # the same with one logits buffer re-read every step (Infinity Cache warm)
    _say("[bench] timing full_penalty, one buffer")
    hot = DeviceSample(w, dev, rotate=False)
    hot_step_ms, hot_kern_ms = time_steps(hot, args.steps, args.warmup, _lib.KERNEL_SAMPLE)
    del hot
    rows_per_s = w.B / (step_ms / 1e3)
    achieved = nbytes / (kern_ms / 1e3) / 1e9
    outcomes = {"ok": int(np.sum((st & 0xFF) == _lib.ROW_OK)),
                "slow_path": int(np.sum((st & 0x100) != 0)),
                "other": int(np.sum((st & 0xFF) != _lib.ROW_OK))}

    host = None
    if not args.quick:
        _say("[bench] drop-in Sampler calls on numpy rows")
        host = time_host_calls(w, 200, 20)

    other = {}
    if not args.quick:
        for name in OTHER:
            _say(f"[bench] {name}")
            other[name] = time_other(name, dev, max(20, args.steps // 5),
                                     max(5, args.warmup // 5))

    if args.copy_probe:
        copy_probe(dev)

    out = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "full_penalty", "B": w.B, "V": w.V, "history": 2048,
                   "temperature": 0.7, "top_k": 40, "top_p": 0.9, "repetition_penalty": 1.1,
                   "presence_penalty": 0.5, "frequency_penalty": 0.3, "parallelism": "none"},
        "hbm_GBps": round(nbytes / (step_ms / 1e3) / 1e9, 1),
        "inputs": "rotated over copies totalling >= 768 MiB, beyond the 256 MB Infinity "
                  "Cache: every step reads its logits from HBM",
        "hot_cache": {"ms_per_step": round(hot_step_ms, 5), "kernel_ms": round(hot_kern_ms, 5),
                      "rows_per_s": round(w.B / (hot_step_ms / 1e3), 1),
                      "kernel_GBps": round(nbytes / (hot_kern_ms / 1e3) / 1e9, 1),
                      "note": "one logits buffer re-read every step (cache-assisted)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": None, "kernel": "cx::sample_kernel<false>",
                     "kernel_ms": round(kern_ms, 5), "algorithmic_bytes": nbytes},
        "cpu_baseline": cpu,
        "cpu_baseline_pool": cpu_pool,
        "row_outcomes": outcomes,
        "host_calls": host,
        "other_workloads": other,
    }
    prof = os.path.join(HERE, "profiles", "sample_kernel_full_penalty_traffic.json")
    if os.path.exists(prof):
        with open(prof) as f:
            out["roofline"]["traffic"] = json.load(f).get("traffic_bytes_per_launch")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
