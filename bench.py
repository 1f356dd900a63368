"""Benchmark of the gfx950 token sampler on its headline workload.

A step is one spx_sample_rows call over one batch: 256 rows x 151936 fp32 logits with a Zipf-shaped profile, a 1024-id
history per row under repetition 1.1 and presence 0.5, temperature 0.7, top-k off, top-p 0.9, one uniform per row
(the Haru-4B-style text-sampling workload). Inputs are synthetic, seeded, and resident in HBM before timing starts.

Prints one JSON line: rows/s over the timed steps (whole job), the roofline of the sampling kernel (algorithmic
bytes per launch over its average launch time, from HIP events recorded on the launch stream), and the CPU baseline:
the oracle (a C++ restatement of the reference's sampler) timed on a bounded sample of the same rows on this host.

usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--workload haru] [--cpu-rows 48] [--no-cpu]
       python bench.py --lds-peak                   the LDS read bandwidth of the device (the peak the rows small
                                                   enough for LDS are rated against)
       python bench.py --copy-mb 512 [--steps 20]   a plain device-to-device copy of known size (calibrates the
                                                   FETCH_SIZE / WRITE_SIZE counters)
       python bench.py --pmc-summary counter_collection.csv   per-kernel dispatch averages of a rocprofv3 --pmc run
"""

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
WORKLOAD_LABELS = {
    "haru": "Haru-4B-style text sampling: 256 x 151936 fp32, hist 1024, rep 1.1 + presence 0.5, T 0.7, top-p 0.9 (transformers rules, which take the penalties)",
    "haru-flavor": "Haru's own rules at its defaults: 256 x 151936 fp32, T 0.7, top-k 25, top-p 1, float32 softmax",
    "asr": "Qwen3-ASR-style greedy: 64 x 151936 fp32, 300 banned ids, argmax (spx_argmax_rows)",
    "mixed": "heterogeneous mixed batch: 2048 x 151936 bf16, per-row T/top-k/top-p, hist U[0,2048], 1% greedy",
    "predictor": "Qwen3-TTS code-predictor batch: 480 x 2048 fp32, hist 64, rep 1.05, T 0.9, top-k 50",
    "talker": "Qwen3-TTS talker step: 1 x 3072 fp32, hist 128, rep 1.05, T 0.9, top-k 50",
    "head": "LM-head pick fused with its product: 64 hidden rows x 2048 fp32, RMS norm, bf16 head 151936 x 2048, argmax",
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="haru", choices=sorted(WORKLOAD_LABELS))
    ap.add_argument("--cpu-rows", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--copy-mb", type=int, default=0)
    ap.add_argument("--pmc-summary", default=None)
    ap.add_argument("--lds-peak", action="store_true")
    return ap.parse_args()


def head_bench(args):
    """The fused LM-head pick (spx_head_argmax_rows) on 64 hidden rows of 2048 against a 151936 x 2048 bf16 head
    (several copies cycled, past the last-level cache), and the unfused path beside it: torch's bf16 product written as
    logits, then torch.argmax."""
    import torch
    import workloads
    spx = workloads.spx_module()
    rows, d, vocab = 64, 2048, 151936
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    hidden = torch.randn(rows, d, device="cuda", generator=g)
    w = torch.rand(d, device="cuda", generator=g) + 0.5
    heads = [(torch.randn(vocab, d, device="cuda", generator=g) * 0.05).to(torch.bfloat16) for _ in range(2)]
    s = spx.Sampler(max_rows=rows, max_vocab=16, max_hist=0, max_out=0)
    ids = torch.empty(rows, dtype=torch.int32, device="cuda")
    mx = torch.empty(rows, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    calls = [0]

    def fused():
        s.head_argmax(hidden, w, 1e-6, heads[calls[0] % 2], out_ids=ids, out_max=mx, stream=stream.cuda_stream)
        calls[0] += 1

    def unfused():
        hn = torch.nn.functional.rms_norm(hidden, (d,), w, 1e-6).to(torch.bfloat16)
        torch.argmax(hn @ heads[calls[0] % 2].t(), dim=1)
        calls[0] += 1

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        st = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
        en = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i in range(args.steps):
            st[i].record(stream)
            fn()
            en[i].record(stream)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, statistics.mean(a.elapsed_time(b) for a, b in zip(st, en))

    elapsed, launch_ms = timed(fused)
    _, unfused_ms = timed(unfused)
    algo = vocab * d * 2 + rows * d * 4 + d * 4 + rows * 8
    achieved = algo / (launch_ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "fused LM-head pick: hidden rows/sec + achieved HBM GB/s on the head, 1 MI355X", "value":
        rows * args.steps / elapsed, "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (random hidden states and head)",
        "config": {"workload": WORKLOAD_LABELS["head"], "rows": rows, "d": d, "vocab": vocab},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes_per_launch": algo,
                     "launch_ms": launch_ms},
        "unfused_torch_ms": unfused_ms}))


def lds_peak():
    """The device's LDS read bandwidth in GB/s, measured by speech.cpp_amd/lib/libspx_ldspeak.so: 512 work-groups of
    1024 lanes reading conflict-free 16-byte words of a 64 KiB LDS array (median of 7 launches)."""
    import ctypes
    import torch  # noqa: F401  (the library binds to the HIP runtime torch loaded)
    path = os.path.join(ROOT, "speech.cpp_amd", "lib", "libspx_ldspeak.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (make -C speech.cpp_amd)")
    lib = ctypes.CDLL(path)
    lib.spx_lds_peak.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    lib.spx_lds_peak.restype = ctypes.c_int
    gbs = ctypes.c_double()
    if lib.spx_lds_peak(512, 4096, 7, ctypes.byref(gbs)) != 0:
        raise RuntimeError("the LDS bandwidth kernel failed")
    return gbs.value


def copy_calibration(mb, steps, warmup):
    """`steps` copies of `mb` MiB from one HBM buffer to another: a kernel whose traffic is known exactly (mb MiB
    read, mb MiB written per dispatch), which scales what FETCH_SIZE and WRITE_SIZE report for the sampler."""
    import torch
    n = (mb << 20) // 4
    src = torch.arange(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_mib": mb, "bytes_read_per_dispatch": mb << 20, "bytes_written_per_dispatch": mb << 20,
                      "steps": steps}))


def pmc_summary(path):
    """Average of every counter column of a rocprofv3 counter_collection.csv, per kernel name."""
    import csv
    acc = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r.get("Kernel_Name", "?")
            key = (name, r.get("Counter_Name", "?"))
            v = float(r.get("Counter_Value", "nan"))
            a = acc.setdefault(key, [0.0, 0])
            a[0] += v
            a[1] += 1
    for (name, ctr), (tot, n) in sorted(acc.items()):
        print(json.dumps({"kernel": name, "counter": ctr, "dispatches": n, "mean_per_dispatch": tot / n}))


def cpu_baseline(w, rows, threads_list):
    """The oracle on the first `rows` rows, median of 5 timed runs after one warm-up, per thread count."""
    import oracle_lib
    sub = dict(w)
    sub["logits"] = w["logits"][:rows]
    sub["params"] = w["params"][:rows]
    sub["u"] = w["u"][:rows]
    if w["hist"] is not None:
        sub["hist_off"] = w["hist_off"][:rows + 1]
        sub["hist"] = w["hist"][:int(w["hist_off"][rows])]
    sub = type(w)(sub)
    out = {}
    for t in threads_list:
        oracle_lib.sample_rows(sub, threads=t)
        times = []
        for _ in range(5):
            t0 = time.perf_counter()
            oracle_lib.sample_rows(sub, threads=t)
            times.append(time.perf_counter() - t0)
        out[t] = rows / statistics.median(times)
    return out


def host_cores():
    n = os.cpu_count() or 1
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    share = int(os.environ.get("OMP_NUM_THREADS", n))
    return max(1, min(n, share))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "rows shard across GPUs with no exchange, so the N-GPU rate is N times the one-GPU rate.",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_mb:
        copy_calibration(args.copy_mb, args.steps, args.warmup)
        return
    if args.lds_peak:
        print(json.dumps({"lds_read_peak_gbs": lds_peak()}))
        return
    if args.workload == "head":
        head_bench(args)
        return
    import torch
    import gpu_harness
    import workloads

    spx = workloads.spx_module()
    w = workloads.make(args.workload, seed=args.seed)
    rows, vocab = w.rows, w.vocab
    max_hist = int(np.max(np.diff(w["hist_off"]))) if w["hist"] is not None else 0
    d = gpu_harness.to_device(w)
    # The logits of a large batch are cycled through several copies in HBM, together well over the 256 MB of the
    # MI355X's last-level cache (MALL), so that every step reads them from HBM as a freshly computed batch would be.
    batch_bytes = d["logits"].numel() * d["logits"].element_size()
    copies = 1 if batch_bytes < (16 << 20) else max(2, min(8, -(-(512 << 20) // batch_bytes)))
    logit_copies = [d["logits"]] + [d["logits"].clone() for _ in range(copies - 1)]
    sampler = spx.Sampler(max_rows=rows, max_vocab=vocab, max_hist=max_hist, max_out=0)
    ids = torch.empty(rows, dtype=torch.int32, device="cuda")
    status = torch.empty(rows, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    calls = [0]

    greedy_only = args.workload == "asr"  # Qwen3-ASR's pick is an argmax (src/families/qwen3-asr/decoder.cpp:108-112)

    def step():
        logits = logit_copies[calls[0] % copies]
        calls[0] += 1
        if greedy_only:
            sampler.argmax_rows(logits, banned=d["banned"], banned_stride=w["banned_stride"], out_ids=ids,
                                stream=stream.cuda_stream)
            return
        sampler.sample_rows(logits, d["params"], d["u"], hist=d["hist"], hist_off=d["hist_off"],
                            banned=d["banned"], banned_stride=w["banned_stride"], out_ids=ids, out_status=status,
                            stream=stream.cuda_stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    fb_before = sampler.last_stats().rows_fallback

    # The timed region: K steps bracketed by synchronizations; an event pair around every launch, on its stream.
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    launch_ms = statistics.mean(s.elapsed_time(e) for s, e in zip(starts, ends))
    fb_rows = (sampler.last_stats().rows_fallback - fb_before) / max(args.steps, 1)
    bad = 0 if greedy_only else int((status.cpu().numpy() != 0).sum())

    algo_bytes = workloads.algorithmic_bytes(w)
    achieved = algo_bytes / (launch_ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        t = json.load(open(tpath)).get(args.workload)
        if t:
            traffic = t.get("hbm_bytes_per_launch")

    value = rows * args.steps / elapsed
    line = {
        "metric": "sampled rows/sec + achieved HBM GB/s at 256x151936 fp32 top-p, 1 MI355X",
        "value": value,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w["dtype"] == "f32" else "bf16",
        "data": "synthetic (seeded Zipf-profile logits, random histories, MT19937-64 uniforms)",
        "config": {"workload": WORKLOAD_LABELS[args.workload], "rows": rows, "vocab": vocab,
                   "logit_copies_cycled": copies, "rows_multi_pass_per_step": fb_rows, "rows_refused": bad},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": algo_bytes, "launch_ms": launch_ms},
    }
    if batch_bytes <= 64 * 1024 * rows:
        # rows small enough for LDS (a 3072-token fp32 row is 12 KiB): the same bytes against the measured LDS peak
        peak = lds_peak()
        line["lds_bound"] = {"achieved": achieved, "peak": peak, "unit": "GB/s", "frac": achieved / peak,
                             "us_per_call_events": launch_ms * 1e3, "us_per_call_wall": elapsed * 1e6 / args.steps}
    if not args.no_cpu:
        cores = host_cores()
        n = min(args.cpu_rows, rows)
        rates = cpu_baseline(w, n, sorted({1, cores}))
        line["cpu_baseline"] = {"value": rates[cores], "unit": "rows/s", "cores": cores, "kind": "port",
                                "sample": f"the first {n} rows of the same batch, oracle restatement of the reference "
                                          f"sampler, median of 5 runs, std::thread over {cores} threads "
                                          f"({cpu_model()})",
                                "value_1core": rates[1]}
        line["vs_cpu"] = value / rates[cores]
    print(json.dumps(line))


if __name__ == "__main__":
    main()
