#!/usr/bin/env python3
"""WKV7 recurrence benchmark on one MI355X (BASELINE.json metric: decode GB/s at B=64, H=64; prefill tok/s at
T=4096).  Prints ONE JSON line.

Headline step ("value"): one decode token for B = 64 sequences drawn from a 128-slot fp32 pool, H = 64, through 32
layer slices (one kernel launch per layer, as the model's decode loop does; 32 x 128 x 64 x 16 KB = 4.3 GB of
pools, so the 256 MB Infinity Cache cannot hold the state), the 32 launches captured in one HIP graph.
value = algorithmic bytes / time: 33 664 B per (slot, head) per layer (16 KB state read + 16 KB written +
768 B operands + 128 B output).

Secondary (same line): chunked prefill B = 1, T = 4096, H = 64 (tok/s and fraction of its roofline), the
speculative verify with snapshots (config 4) and the CPU baseline (the oracle's fp32 loop on the host cores).

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--skip-cpu] [--only decode|prefill|verify]
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "rwkv-infer-next_amd"))

METRIC = "WKV7 decode GB/s (%HBM peak) @B=64,H=64; prefill tok/s (%roofline) @T=4096"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
DECODE_BYTES_PER_PAIR = 16384 + 16384 + 6 * 64 * 2 + 64 * 2       # 33 664
PREFILL_BYTES_PER_HEAD_TOKEN = 6 * 64 * 2 + 64 * 2                 # 896 (+ 32 KB state per (sequence, head))
COPY_CALIB_BYTES = 1 << 30
C = 64
PREFILL_FLOPS_PER_HEAD_TOKEN = 18 * C * 64 + 8 * 64 * 64 + (2 * C * C) // 3   # chunked form at C = 64


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def decode_bench(torch, kernels, synth, dev, steps, warmup):
    L, S, B, H = 32, 128, 64, 64
    g = torch.Generator(device=dev).manual_seed(1001)
    pools = [(0.1 * torch.randn(S, H, 64, 64, device=dev, generator=g)) for _ in range(L)]
    ins = []
    for layer in range(L):
        ops = synth.operands_torch((B, 1, H, 64), seed=2000 + layer, device=dev)
        ins.append([ops[n].reshape(B, 1, H * 64).contiguous() for n in synth.OPERAND_NAMES])
    slots = torch.randperm(S, device=dev, generator=g)[:B].contiguous()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for layer in range(L):  # warm-up outside capture
            kernels.wkv7_pool_(*ins[layer], pools[layer], slots, H, 64)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [kernels.wkv7_pool_(*ins[layer], pools[layer], slots, H, 64) for layer in range(L)]
    torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / steps
    bytes_launch = DECODE_BYTES_PER_PAIR * B * H
    us_launch = ms_step * 1e3 / L
    gbs = bytes_launch * L / (ms_step * 1e-3) / 1e9
    del outs
    return {"ms_per_step": ms_step, "GBps": gbs, "us_per_launch": us_launch, "bytes_per_launch": bytes_launch,
            "launches_per_step": L, "pairs_per_launch": B * H}


def prefill_bench(torch, kernels, synth, dev, steps, warmup):
    T, H = 4096, 64
    ops = synth.operands_torch((1, T, H, 64), seed=1002, device=dev)
    x = [ops[n].reshape(1, T, H * 64).contiguous() for n in synth.OPERAND_NAMES]
    for _ in range(warmup):
        kernels.wkv7(*x, None, H, 64)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        kernels.wkv7(*x, None, H, 64)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    bytes_ = PREFILL_BYTES_PER_HEAD_TOKEN * T * H + 2 * 16384 * H
    flops = PREFILL_FLOPS_PER_HEAD_TOKEN * T * H
    t_hbm = bytes_ / (HBM_PEAK_GBS * 1e9)
    t_fp32 = flops / (FP32_PEAK_TFLOPS * 1e12)   # every contraction currently runs on fp32 MFMA
    t_roof = max(t_hbm, t_fp32)
    return {"ms": ms, "tok_s": T / (ms * 1e-3), "roofline_bound": "mfma_fp32" if t_fp32 >= t_hbm else "hbm",
            "t_roof_us": t_roof * 1e6, "frac": t_roof / (ms * 1e-3), "flops_chunked": flops,
            "recurrence_equiv_TFLOPs": 9 * 64 * 64 * T * H / (ms * 1e-3) / 1e12}


def verify_bench(torch, kernels, synth, dev, steps, warmup):
    B, T, H = 64, 5, 64
    ops = synth.operands_torch((B, T, H, 64), seed=1004, device=dev)
    x = [ops[n].reshape(B, T, H * 64).contiguous() for n in synth.OPERAND_NAMES]
    pool = 0.1 * torch.randn(B, H, 64, 64, device=dev)
    slots = torch.arange(B, device=dev)
    snaps = torch.empty(B, T, H, 64, 64, device=dev)
    for _ in range(warmup):
        kernels.wkv7_pool_(*x, pool, slots, H, 64, final=False, snapshots=snaps)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        kernels.wkv7_pool_(*x, pool, slots, H, 64, final=False, snapshots=snaps)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    bytes_ = (16384 + T * 16384 + T * 896) * B * H
    return {"ms": ms, "GBps": bytes_ / (ms * 1e-3) / 1e9, "bytes": bytes_}


def cpu_baseline(synth):
    """The oracle's fp32 loop (a restatement of rwkv_next/kernels/wkv7.py:65-77) on the host cores, on a bounded
    sample of the decode workload: B = 64 sequences of a 128-slot pool, H = 64, T = 1, one pool, repeated for
    about 10 s."""
    import numpy as np

    import oracle
    threads = min(16, len(os.sched_getaffinity(0)))
    B, S, H = 64, 128, 64
    ops = synth.operands_np((B, 1, H, 64), seed=3001)
    ins = [ops[n] for n in synth.OPERAND_NAMES]
    pool = synth.state_np((S, H, 64, 64), seed=3002)
    slots = np.random.default_rng(3003).permutation(S)[:B].astype(np.int64)
    oracle.wkv7_ref(*ins, pool, state_idx=slots, precision="f32", threads=threads)  # warm-up
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 10.0:
        oracle.wkv7_ref(*ins, pool, state_idx=slots, precision="f32", threads=threads)
        n += 1
    dt = time.perf_counter() - t0
    gbs = DECODE_BYTES_PER_PAIR * B * H * n / dt / 1e9
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"decode B=64 of a 128-slot pool, H=64, T=1, one layer slice, {n} steps in {dt:.1f} s "
                      f"(oracle fp32 loop, OpenMP); CPU: {model}"}


def decode_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE, each
    scaled by what the same counter reads for a 1 GiB device copy), or None if absent."""
    path = os.path.join(REPO, "profiles", "wkv7_recurrent_decode_B64_H64.json")
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill", "verify"], default=None)
    ap.add_argument("--copy-calib", action="store_true",
                    help="first run a plain device copy of 1 GiB (reference dispatch for rocprofv3 --pmc scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the WKV7 recurrence has no cross-GPU exchange (heads and slots shard "
              "independently), and this build runs on single-GPU boxes; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import rwkv_next_amd.synth as synth
    from rwkv_next_amd import kernels

    dev = torch.device("cuda:0")
    res = {}
    if args.copy_calib:
        src = torch.ones(COPY_CALIB_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only in (None, "decode"):
        log("decode")
        res["decode"] = decode_bench(torch, kernels, synth, dev, args.steps, args.warmup)
    if args.only in (None, "prefill"):
        log("prefill")
        res["prefill"] = prefill_bench(torch, kernels, synth, dev, max(5, args.steps // 5), args.warmup)
    if args.only in (None, "verify"):
        log("verify")
        res["verify"] = verify_bench(torch, kernels, synth, dev, args.steps, args.warmup)
    cpu = None
    if not args.skip_cpu and args.only is None:
        log("cpu baseline")
        cpu = cpu_baseline(synth)

    d = res.get("decode")
    out = {
        "metric": METRIC,
        "value": d["GBps"] if d else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": d["ms_per_step"] if d else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded; BASELINE distributions), bf16 operands, fp32 state pools",
        "config": {"workload": "decode B=64 H=64 T=1 over 32 layer slices of a [128,64,64,64] fp32 pool, "
                               "one HIP graph of 32 launches per step",
                   "B": 64, "H": 64, "head_size": 64, "slots": 128, "layers": 32},
    }
    if d:
        achieved = d["bytes_per_launch"] / (d["us_per_launch"] * 1e-6) / 1e9
        out["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": achieved / HBM_PEAK_GBS, "traffic": decode_traffic(),
                           "kernel": "wkv7_recurrent_kernel", "us_per_launch": d["us_per_launch"]}
    if "prefill" in res:
        out["prefill"] = res["prefill"]
    if "verify" in res:
        out["verify"] = res["verify"]
    if cpu:
        out["cpu_baseline"] = cpu
    print(json.dumps(out))


if __name__ == "__main__":
    main()
