#!/usr/bin/env python3
"""WKV7 recurrence benchmark on one MI355X (headline metric: decode GB/s at B=64, H=64; prefill tok/s at
T=4096).  Prints ONE JSON line.

Headline step ("value"): one decode token for B = 64 sequences drawn from a 128-slot fp32 pool, H = 64, through 32
layer slices (one kernel launch per layer, as the model's decode loop does; 32 x 128 x 64 x 16 KB = 4.3 GB of
pools, so the 256 MB Infinity Cache cannot hold the state), the 32 launches captured in one HIP graph.
value = algorithmic bytes / time: 33 664 B per (slot, head) per layer (16 KB state read + 16 KB written +
768 B operands + 128 B output).

Secondary (same line): the same decode step at configuration 1's H = 40 (pool [128, 40, 64, 64] x 32 layers,
"decode_cfg1"), chunked prefill B = 1, T = 4096, H = 64 (tok/s and fraction of its roofline; AUTO runs the
segmented kernel), the drop-in varlen prefill call on a 4-row 2048-token chunk, the speculative verify with
snapshots (config 4), the mixed continuous-batching step in a HIP graph (config 3), the
fused time-mix prologue/epilogue at the prefill shape, the W6A16 weight GEMM at K = 4096, N = 16384, and the CPU
baseline (the oracle's fp32 loop on the host cores).

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--skip-cpu]
                    [--only decode|prefill|varlen|verify|mixed|timemix|int6|tp]
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
BF16_PEAK_TFLOPS = 2516.6
DECODE_BYTES_PER_PAIR = 16384 + 16384 + 6 * 64 * 2 + 64 * 2       # 33 664
PREFILL_BYTES_PER_HEAD_TOKEN = 6 * 64 * 2 + 64 * 2                 # 896 (+ 32 KB state per (sequence, head))
COPY_CALIB_BYTES = 1 << 30
C = 32
N = 64
# Chunked form at the segmented kernel's chunk C = 32, per (chunk, head): the state path (Grams alpha/beta, the
# triangular inverse, W, U0, the state update) and the output path (rho, sigma, R0 and the outputs).  Together
# 18 C N + 8 N^2 + 2/3 C^2 per head-token.
PREFILL_STATE_FLOPS_PER_CHUNK = 10 * C * C * N + 6 * C * N * N + (2 * C ** 3) // 3
PREFILL_OUTPUT_FLOPS_PER_CHUNK = 8 * C * C * N + 2 * C * N * N
PREFILL_FLOPS_PER_HEAD_TOKEN = (PREFILL_STATE_FLOPS_PER_CHUNK + PREFILL_OUTPUT_FLOPS_PER_CHUNK) / C
# The kernels run state-path products as three bf16 MFMAs on a hi/lo split of each fp32 operand and output-path
# products as one bf16 MFMA, so the compute roofline prices the state path at 3x the bf16 rate.
STATE_PATH_BF16_PASSES = 3


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def decode_bench(torch, kernels, synth, dev, steps, warmup, H=64):
    """B = 64 slots of a 128-slot pool, T = 1, 32 layer pools in one HIP graph.  H = 64 is the metric's shape;
    H = 40 is configuration 1 (RWKV-7 2.9B, pool [128, 40, 64, 64])."""
    L, S, B = 32, 128, 64
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


def head_size_bench(torch, kernels, synth, dev, steps, warmup, K):
    """Head sizes other than 64 (the generic token-serial kernel): H = 4096 / K heads, the 7.2B model's width.
    Decode: B = 64 slots of a 128-slot [128, H, K, K] pool, T = 1, 8 layer pools in one HIP graph; traffic per pair
    2 K^2 fp32 (state read and written in place) + 7 K bf16 (six operands, y).  Prefill: B = 1, T = 512 dense,
    state from zeros, eager; traffic 7 K bf16 per head-token + K^2 fp32 per head (the final state)."""
    H, L, S, B = 4096 // K, 8, 128, 64
    g = torch.Generator(device=dev).manual_seed(3001 + K)
    pools = [(0.1 * torch.randn(S, H, K, K, device=dev, generator=g)) for _ in range(L)]
    ins = []
    for layer in range(L):
        ops = synth.operands_torch((B, 1, H, K), seed=4000 + layer, device=dev)
        ins.append([ops[n].reshape(B, 1, H * K).contiguous() for n in synth.OPERAND_NAMES])
    slots = torch.randperm(S, device=dev, generator=g)[:B].contiguous()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for layer in range(L):
            kernels.wkv7_pool_(*ins[layer], pools[layer], slots, H, K)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [kernels.wkv7_pool_(*ins[layer], pools[layer], slots, H, K) for layer in range(L)]
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
    us_launch = e0.elapsed_time(e1) * 1e3 / (steps * L)
    bytes_launch = B * H * (2 * K * K * 4 + 7 * K * 2)
    del outs, graph, pools
    T = 512
    ops = synth.operands_torch((1, T, H, K), seed=4100 + K, device=dev)
    x = [ops[n].reshape(1, T, H * K).contiguous() for n in synth.OPERAND_NAMES]
    for _ in range(2):
        kernels.wkv7(*x, None, H, K)
    torch.cuda.synchronize()
    n = max(2, steps // 10)
    e0.record()
    for _ in range(n):
        kernels.wkv7(*x, None, H, K)
    e1.record()
    torch.cuda.synchronize()
    us_pf = e0.elapsed_time(e1) * 1e3 / n
    pf_bytes = T * H * 7 * K * 2 + H * K * K * 4
    return {"K": K, "H": H,
            "decode": {"us_per_launch": us_launch, "bytes_per_launch": bytes_launch,
                       "GBps": bytes_launch / (us_launch * 1e-6) / 1e9,
                       "frac_hbm": bytes_launch / (us_launch * 1e-6) / 1e9 / HBM_PEAK_GBS},
            "prefill_T512": {"us": us_pf, "tok_s": T / (us_pf * 1e-6), "bytes": pf_bytes,
                             "frac_hbm": pf_bytes / (us_pf * 1e-6) / 1e9 / HBM_PEAK_GBS}}


def cfg0_bench(torch, kernels, synth, dev, steps, warmup):
    """Configuration 0's shape on the GPU (B = 1, T = 512, H = 12; bf16 operands, fp32 state from zeros), eager
    calls, for every algorithm -- beside cpu_baseline.cfg0, the oracle's fp32 loop on the host at the same shape."""
    T, H = 512, 12
    ops = synth.operands_torch((1, T, H, 64), seed=1000, device=dev)
    x = [ops[n].reshape(1, T, H * 64).contiguous() for n in synth.OPERAND_NAMES]
    out = {"shape": "B=1 T=512 H=12, bf16 operands, fp32 state from zeros",
           "timing": "ms: HIP graph replay per call; ms_eager: eager calls (host dispatch included)"}
    for name, algo in (("auto", 0), ("recurrent", 1), ("chunked", 2)):
        fn = lambda algo=algo: kernels.wkv7(*x, None, H, 64, algo=algo)
        ms = graph_us(torch, [fn], steps, warmup) * 1e-3
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[f"ms_{name}"] = ms
        out[f"ms_eager_{name}"] = e0.elapsed_time(e1) / steps
        out[f"tok_s_{name}"] = T / (ms * 1e-3)
    return out


def prefill_bench(torch, kernels, synth, dev, steps, warmup, copies=4):
    """Config 2 (B = 1, T = 4096, H = 64, zero initial state, final state returned).  ms: one call per HIP graph
    replay, the same operands each time (201 MB, which the 256 MB Infinity Cache largely keeps between replays, as it
    keeps a layer's operands between the kernel that writes them and this one); ms_eager: those calls launched
    eagerly.  ms_layers_cold: `copies` layer calls, each on its own operands (none cached), in one graph, per call.
    (A graph replay ends with a fixed ~6-9 us on these boxes, which the one-call figure carries in full.)"""
    T, H = 4096, 64
    xs = []
    for i in range(copies):
        ops = synth.operands_torch((1, T, H, 64), seed=1002 + 17 * i, device=dev)
        xs.append([ops[n].reshape(1, T, H * 64).contiguous() for n in synth.OPERAND_NAMES])
    fns = [lambda x=x: kernels.wkv7(*x, None, H, 64) for x in xs]
    for _ in range(warmup):
        fns[0]()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fns[0]()
    e1.record()
    torch.cuda.synchronize()
    ms_eager = e0.elapsed_time(e1) / steps
    ms = graph_us(torch, fns[:1], steps, warmup) * 1e-3
    ms_cold = graph_us(torch, fns, steps, warmup) * 1e-3
    chunks = T // C
    bytes_ = PREFILL_BYTES_PER_HEAD_TOKEN * T * H + 2 * 16384 * H
    t_hbm = bytes_ / (HBM_PEAK_GBS * 1e9)
    f_state = PREFILL_STATE_FLOPS_PER_CHUNK * chunks * H
    f_out = PREFILL_OUTPUT_FLOPS_PER_CHUNK * chunks * H
    t_mfma = (STATE_PATH_BF16_PASSES * f_state + f_out) / (BF16_PEAK_TFLOPS * 1e12)
    t_roof = max(t_hbm, t_mfma)
    # The baseline's own compute roofline prices the (fp32-accurate) state path at the fp32 MFMA rate and the output
    # path at the bf16 rate (about 79 us at C = 32; 118 us at the chunked kernels' C = 64); reported beside the
    # stricter one above, which prices the state path as the three bf16 passes these kernels run.
    t_fp32_state = f_state / (FP32_PEAK_TFLOPS * 1e12) + f_out / (BF16_PEAK_TFLOPS * 1e12)
    t_roof_fp32_state = max(t_hbm, t_fp32_state)
    return {"ms": ms, "ms_eager": ms_eager, "ms_layers_cold": ms_cold, "copies": copies,
            "timing": "ms: one call per HIP graph replay; ms_eager: eager calls; ms_layers_cold: per call, `copies` "
                      "layer calls on their own operands per replay",
            "tok_s": T / (ms * 1e-3), "head_tok_s": T * H / (ms * 1e-3),
            "roofline": {"bound": "hbm" if t_hbm >= t_mfma else "mfma", "t_roof_us": t_roof * 1e6,
                         "t_hbm_us": t_hbm * 1e6, "t_mfma_us": t_mfma * 1e6, "frac": t_roof / (ms * 1e-3),
                         "t_roof_fp32_state_path_us": t_roof_fp32_state * 1e6,
                         "frac_fp32_state_path": t_roof_fp32_state / (ms * 1e-3),
                         "algorithmic_bytes": bytes_, "flops_state_path": f_state, "flops_output_path": f_out},
            "recurrence_equiv_TFLOPs": 9 * 64 * 64 * T * H / (ms * 1e-3) / 1e12}


def varlen_bench(torch, kernels, synth, dev, steps, warmup, copies=4):
    """The drop-in varlen prefill call kernels.wkv7(..., cu_seqlens=cu) (rwkv_next/kernels/wkv7.py:126-138) on one
    2048-token prefill chunk of the engine (rwkv_next/engine.py:218-228) split over 4 rows, H = 64, from zero states,
    final states returned.  AUTO runs it as one segmented dispatch (rows of at most 32 tokens, here none, would run
    token-serially in the same launch).  us: one call per HIP graph replay; us_layers_cold: `copies` layer calls,
    each on its own operands, per replay, per call."""
    H, lens = 64, [700, 512, 600, 236]
    total = sum(lens)
    cu = torch.tensor([0, 700, 1212, 1812, 2048], dtype=torch.int32, device=dev)
    xs = []
    for i in range(copies):
        ops = synth.operands_torch((1, total, H, 64), seed=1005 + 17 * i, device=dev)
        xs.append([ops[n].reshape(1, total, H * 64).contiguous() for n in synth.OPERAND_NAMES])
    fns = [lambda x=x: kernels.wkv7(*x, None, H, 64, cu_seqlens=cu) for x in xs]
    us = graph_us(torch, fns[:1], steps, warmup)
    us_cold = graph_us(torch, fns, steps, warmup)
    nbytes = PREFILL_BYTES_PER_HEAD_TOKEN * total * H + len(lens) * 16384 * H  # no initial states read
    t_roof_us = nbytes / (HBM_PEAK_GBS * 1e3)
    return {"us": us, "us_layers_cold": us_cold, "copies": copies,
            "timing": "us: one call per HIP graph replay; us_layers_cold: per call, `copies` layer calls per replay",
            "rows": lens, "tokens": total, "H": H,
            "tok_s": total / (us * 1e-6), "algorithmic_bytes": nbytes, "t_roof_us": t_roof_us,
            "frac": t_roof_us / us}


def mixed_bench(torch, kernels, synth, dev, steps, warmup, copies=4):
    """Config 3: one continuous-batching step over a 256-slot pool, H = 64: 8 prefill rows of U[1, 2048] tokens and
    120 decode rows, packed varlen, random distinct slots.  ms: the step captured in one HIP graph and replayed;
    ms_layers_cold: `copies` layers' steps (each its own pool and operands) per replay, per step."""
    import numpy as np
    H, S = 64, 256
    rng = np.random.default_rng(1003)
    lens = [int(v) for v in rng.integers(1, 2049, size=8)] + [1] * 120
    lens = [lens[i] for i in rng.permutation(len(lens))]
    total = int(sum(lens))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    slots = torch.from_numpy(rng.permutation(S)[:len(lens)].astype(np.int64)).to(dev)
    layers = []
    for i in range(copies):
        ops = synth.operands_torch((1, total, H, 64), seed=1003 + 17 * i, device=dev)
        x = [ops[n].reshape(1, total, H * 64).contiguous() for n in synth.OPERAND_NAMES]
        layers.append((x, 0.1 * torch.randn(S, H, 64, 64, device=dev)))
    fns = [lambda x=x, pool=pool: kernels.wkv7_pool_(*x, pool, slots, H, 64, cu_seqlens=cu, max_len=2048)
           for x, pool in layers]
    ms = graph_us(torch, fns[:1], steps, warmup) * 1e-3
    ms_cold = graph_us(torch, fns, steps, warmup) * 1e-3
    # HBM roofline: every (row, head) reads and writes its 16 KB state once, and every head-token moves 896 B of
    # operands and output
    nbytes = H * (len(lens) * 2 * 64 * 64 * 4 + total * 896)
    t_roof_us = nbytes / (HBM_PEAK_GBS * 1e3)
    return {"ms": ms, "ms_layers_cold": ms_cold, "copies": copies,
            "timing": "ms: one step per HIP graph replay; ms_layers_cold: per step, `copies` layers per replay",
            "tokens": total, "tok_s": total / (ms * 1e-3), "prefill_lens": sorted(v for v in lens if v > 1),
            "algorithmic_bytes": nbytes, "t_roof_us": t_roof_us, "frac": t_roof_us / (ms * 1e3)}


def graph_us(torch, fns, steps, warmup):
    """Capture the calls `fns` (one per layer copy) in one HIP graph and return the replay time per call in us."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for fn in fns:  # warm-up outside capture
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (steps * len(fns))


def verify_bench(torch, kernels, synth, dev, steps, warmup, H=64, copies=8):
    """Configuration 4's speculative verify (B = 64 rows, T = 5 draft tokens) with per-token snapshots, and the two
    rollbacks to accepted prefixes n = j + 1, j ~ U{0..4}: the snapshot restore (16 KB read + 16 KB written per
    (row, head)) and the reference's way, a replay of the first n tokens (rwkv_next/model.py:498-503).  Each is
    timed in a HIP graph over `copies` layer-sized copies of the pool and snapshot buffers (so no call finds its
    state in the Infinity Cache), per call."""
    B, T = 64, 5
    ops = synth.operands_torch((B, T, H, 64), seed=1004, device=dev)
    x = [ops[n].reshape(B, T, H * 64).contiguous() for n in synth.OPERAND_NAMES]
    pools = [0.1 * torch.randn(B, H, 64, 64, device=dev) for _ in range(copies)]
    snaps = [torch.empty(B, T, H, 64, 64, device=dev) for _ in range(copies)]
    slots = torch.arange(B, device=dev)
    n = torch.randint(1, T + 1, (B,), device=dev, generator=torch.Generator(device=dev).manual_seed(1005))
    us = graph_us(torch, [lambda i=i: kernels.wkv7_pool_(*x, pools[i], slots, H, 64, final=False, snapshots=snaps[i])
                          for i in range(copies)], steps, warmup)
    us_plain = graph_us(torch, [lambda i=i: kernels.wkv7_pool_(*x, pools[i], slots, H, 64, final=False)
                                for i in range(copies)], steps, warmup)
    us_restore = graph_us(torch, [lambda i=i: kernels.restore_snapshots_(pools[i], slots, snaps[i], n)
                                  for i in range(copies)], steps, warmup)
    us_replay = graph_us(torch, [lambda i=i: kernels.wkv7_replay(*x, pools[i], n, H, 64)
                                 for i in range(copies)], steps, warmup)
    bytes_ = (16384 + T * 16384 + T * 896) * B * H
    rbytes = 2 * 16384 * B * H
    return {"ms": us * 1e-3, "GBps": bytes_ / (us * 1e-6) / 1e9, "bytes": bytes_,
            "rollback_restore_us": us_restore, "rollback_restore_GBps": rbytes / (us_restore * 1e-6) / 1e9,
            "rollback_replay_us": us_replay, "verify_without_snapshots_us": us_plain,
            "step_snapshots_us": us + us_restore, "step_replay_us": us_plain + us_replay,
            "timing": f"HIP graph of {copies} calls on separate pool/snapshot copies, per call"}


TIMEMIX_PROLOGUE_BYTES = 11 * 2     # per (token, channel): k, v, o_v, o_w, o_a, v_first read; w, k', v', a, b written
TIMEMIX_EPILOGUE_BYTES = 6 * 2      # y, r, k', v', g read; out written


def timemix_bench(torch, kernels, dev, steps, warmup):
    """Fused time-mix prologue and epilogue (rwkv_next/model.py:142-158) at the prefill shape T = 4096, C = 4096,
    beside the same math as the reference's chain of bf16 torch ops (timed on the same GPU, for scale)."""
    F = torch.nn.functional
    T, H = 4096, 64
    Cc = H * 64
    g = torch.Generator(device="cpu").manual_seed(1005)
    rnd = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).to(dev)
    r, k, v, vf, gate, y = (rnd(T, Cc) for _ in range(6))
    o = rnd(3, T, Cc)
    b_w, b_a, b_v, kk_mul, ka_mul = (rnd(1, Cc) for _ in range(5))
    lnx_w, lnx_b, r_k = rnd(Cc), rnd(Cc), rnd(H, 64)
    eps = 1e-5 * 64

    def fused():
        ins, _ = kernels.timemix_prologue(r, k, v, o, vf, b_w, b_a, b_v, kk_mul, ka_mul, H, 64, False)
        return ins, kernels.timemix_epilogue(y, r, ins[2], ins[3], gate, lnx_w, lnx_b, r_k, H, 64, eps)

    def eager():
        w = -F.softplus(-(b_w + o[1])) - 0.5
        a = torch.sigmoid(b_a + o[2])
        vv = v + (vf - v) * torch.sigmoid(b_v + o[0])
        kk = F.normalize((k * kk_mul).view(T, H, 64), dim=-1, p=2.0).view(T, Cc)
        kp = k * (1 + (a - 1) * ka_mul)
        ins = (r, w, kp, vv, -kk, kk * a)
        x = F.group_norm(y, H, lnx_w, lnx_b, eps)
        x = x + ((r.view(T, H, 64) * kp.view(T, H, 64) * r_k).sum(-1, keepdim=True) * vv.view(T, H, 64)).view(T, Cc)
        return ins, x * gate

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms = timed(fused)
    ms_eager = timed(eager)
    bytes_ = (TIMEMIX_PROLOGUE_BYTES + TIMEMIX_EPILOGUE_BYTES) * T * Cc
    return {"ms": ms, "GBps": bytes_ / (ms * 1e-3) / 1e9, "frac_hbm": bytes_ / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "algorithmic_bytes": bytes_, "torch_eager_ms": ms_eager, "speedup_vs_eager": ms_eager / ms}


def int6_bench(torch, kernels, dev, steps, warmup):
    """W6A16 GEMM/GEMV (rwkv_next/kernels/int6_gemm.py) at the reference's quoted shape K = 4096, N = 16384
    (int6_gemm.py:224-226), group_k = 128, for decode-sized M (the W6A16 kernel, on the reference's planes and on the
    packed layout of prepack_int6) and M = 4096 (dequantise, then the library GEMM).  Eight weight sets (8 x 51 MB)
    are cycled so the 256 MB Infinity Cache cannot hold them: every call streams its weight from HBM, as a model's
    consecutive layers do.  Each M is one HIP graph of 8 calls.  Beside it: torch.matmul on the same shape with a
    bf16 weight (hipBLASLt), cycled the same way, and the W6A16 kernels again with fp16 activations at four M."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    K, N, G, SETS = 4096, 16384, 128, 8
    gen = torch.Generator(device=dev).manual_seed(1006)
    lo = [torch.randint(0, 256, (K // 2, N), device=dev, dtype=torch.uint8, generator=gen) for _ in range(SETS)]
    hi = [torch.randint(0, 256, (K // 4, N), device=dev, dtype=torch.uint8, generator=gen) for _ in range(SETS)]
    sc = [(torch.rand(K // G, N, device=dev, generator=gen) * 0.05 + 0.002).half() for _ in range(SETS)]
    wbf = [I6.dequantize_int6(lo[i], hi[i], sc[i], G, dtype=torch.bfloat16) for i in range(SETS)]
    pk = [I6.prepack_int6(lo[i], hi[i], sc[i], G) for i in range(SETS)]
    weight_bytes = K * N * 3 // 4 + (K // G) * N * 2

    def graph_time(fn, reps):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(max(1, warmup)):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        for _ in range(max(1, warmup)):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * SETS)   # us per call

    rows = []
    for M in (1, 2, 4, 16, 64, 128, 256):
        a = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        sk, ud = I6.plan_int6(M, N, K, 1, dev)
        us = graph_time(lambda: [I6.int6_matmul_op(a, lo[i], hi[i], sc[i], G, sk, ud) for i in range(SETS)], steps)
        sk_pk = I6.plan_int6_packed(M, N, K, 1, dev)
        us_pk = graph_time(lambda: [I6.int6_matmul_packed_op(a, pk[i].weight, pk[i].scales, 0, K, N, G, sk_pk)
                                    for i in range(SETS)], steps)
        us_bf = graph_time(lambda: [torch.matmul(a, wbf[i]) for i in range(SETS)], steps)
        byts = weight_bytes + M * K * 2 + M * N * 2
        path = "w6a16 kernel" if M <= I6.MAX_M else "dequantize + library GEMM"
        rows.append({"M": M, "path": path, "split_k": sk if M <= I6.MAX_M else None,
                     "packed_split_k": sk_pk if M <= I6.MAX_M else None, "us": us,
                     "GBps": byts / (us * 1e-6) / 1e9, "frac_hbm": byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                     "packed_us": us_pk, "packed_GBps": byts / (us_pk * 1e-6) / 1e9,
                     "packed_frac_hbm": byts / (us_pk * 1e-6) / 1e9 / HBM_PEAK_GBS,
                     "bf16_matmul_us": us_bf, "speedup_vs_bf16": us_bf / us, "packed_speedup_vs_bf16": us_bf / us_pk})
        log(f"int6 M={M} ({path}, split {sk}): {us:.2f} us ({rows[-1]['GBps']:.0f} GB/s), "
            f"packed (split {sk_pk}) {us_pk:.2f} us "
            f"({rows[-1]['packed_GBps']:.0f} GB/s), bf16 matmul {us_bf:.2f} us")
    # fp16 activations (the reference's kernel takes either dtype; the output has A's dtype), same weights
    f16_rows = []
    for M in (1, 16, 64, 256):
        a = torch.randn(M, K, device=dev, generator=gen).to(torch.float16)
        sk, ud = I6.plan_int6(M, N, K, 1, dev)
        us = graph_time(lambda: [I6.int6_matmul_op(a, lo[i], hi[i], sc[i], G, sk, ud) for i in range(SETS)], steps)
        sk_pk = I6.plan_int6_packed(M, N, K, 1, dev)
        us_pk = graph_time(lambda: [I6.int6_matmul_packed_op(a, pk[i].weight, pk[i].scales, 0, K, N, G, sk_pk)
                                    for i in range(SETS)], steps)
        f16_rows.append({"M": M, "us": us, "packed_us": us_pk})
        log(f"int6 fp16 activations M={M}: {us:.2f} us, packed {us_pk:.2f} us")
    # prefill-sized M: dequantise once, then the library GEMM
    M = 4096
    a = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    us = graph_time(lambda: [I6.int6_matmul(a, lo[i], hi[i], sc[i], G) for i in range(SETS)], max(2, steps // 10))
    us_bf = graph_time(lambda: [torch.matmul(a, wbf[i]) for i in range(SETS)], max(2, steps // 10))
    # the C ABI's own large-M kernel on the packed layout (dequantisation fused; not the module's default above MAX_M)
    max_m = I6.MAX_M
    I6.MAX_M = 1 << 30
    try:
        us_own = graph_time(lambda: [I6.int6_matmul(a, pk[i]) for i in range(SETS)], max(2, steps // 10))
    finally:
        I6.MAX_M = max_m
    rows.append({"M": M, "path": "dequantize + library GEMM", "us": us, "TFLOPs": 2 * M * K * N / (us * 1e-6) / 1e12,
                 "bf16_matmul_us": us_bf, "speedup_vs_bf16": us_bf / us, "own_kernel_packed_us": us_own,
                 "own_kernel_speedup_vs_bf16": us_bf / us_own})
    log(f"int6 M={M}: {us:.1f} us, bf16 matmul {us_bf:.1f} us, own large-M kernel (packed) {us_own:.1f} us")
    return {"K": K, "N": N, "group_k": G, "weight_bytes": weight_bytes, "rows": rows, "fp16_rows": f16_rows,
            "reference_quoted_ms": {"M=128": 0.24, "M=4096": 5.9}}


def cpu_baseline(synth):
    """The oracle's fp32 loop (a restatement of rwkv_next/kernels/wkv7.py:65-77) on the host cores, on a bounded
    sample of the decode workload: B = 64 sequences of a 128-slot pool, H = 64, T = 1, one pool, repeated for
    about 10 s with every usable thread (at most 16) and about 4 s with one thread.  Beside it, configuration 0 in
    full (B = 1, T = 512, H = 12, fp32, zero initial state) with all threads and with one, and configurations 2-4 at
    their full shapes (the same lengths, slots and snapshot layout as the GPU legs) with all threads, configuration 2
    also with one."""
    import numpy as np

    import oracle
    affinity = len(os.sched_getaffinity(0))
    threads = min(16, affinity)
    B, S, H = 64, 128, 64
    ops = synth.operands_np((B, 1, H, 64), seed=3001)
    ins = [ops[n] for n in synth.OPERAND_NAMES]
    pool = synth.state_np((S, H, 64, 64), seed=3002)
    slots = np.random.default_rng(3003).permutation(S)[:B].astype(np.int64)

    def decode_rate(nthreads, seconds):
        oracle.wkv7_ref(*ins, pool, state_idx=slots, precision="f32", threads=nthreads)  # warm-up
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            oracle.wkv7_ref(*ins, pool, state_idx=slots, precision="f32", threads=nthreads)
            n += 1
        dt = time.perf_counter() - t0
        return DECODE_BYTES_PER_PAIR * B * H * n / dt / 1e9, n, dt

    gbs, n, dt = decode_rate(threads, 10.0)
    gbs1, n1, dt1 = decode_rate(1, 4.0)

    c0 = synth.operands_np((1, 512, 12, 64), seed=1000)          # configuration 0: seed 1000 + config index
    c0_ins = [c0[nm] for nm in synth.OPERAND_NAMES]

    def cfg0_ms(nthreads):
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.wkv7_ref(*c0_ins, None, precision="f32", threads=nthreads)
            t = (time.perf_counter() - t0) * 1e3
            best = t if best is None else min(best, t)
        return best

    ms_all, ms_one = cfg0_ms(threads), cfg0_ms(1)

    def best_ms(fn, reps=2):
        best = None
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            t = (time.perf_counter() - t0) * 1e3
            best = t if best is None else min(best, t)
        return best

    # configuration 2: B = 1, T = 4096, H = 64, zero initial state
    c2 = synth.operands_np((1, 4096, 64, 64), seed=1002)
    c2_ins = [c2[nm] for nm in synth.OPERAND_NAMES]
    c2_all = best_ms(lambda: oracle.wkv7_ref(*c2_ins, None, precision="f32", threads=threads))
    c2_one = best_ms(lambda: oracle.wkv7_ref(*c2_ins, None, precision="f32", threads=1), reps=1)
    del c2, c2_ins
    # configuration 3: the mixed step (bench.py's mixed_bench lengths and slots), 256-slot pool
    rng = np.random.default_rng(1003)
    lens = [int(v) for v in rng.integers(1, 2049, size=8)] + [1] * 120
    lens = [lens[i] for i in rng.permutation(len(lens))]
    total3 = int(sum(lens))
    cu3 = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    slots3 = rng.permutation(256)[:len(lens)].astype(np.int64)
    c3 = synth.operands_np((1, total3, 64, 64), seed=1003)
    c3_ins = [c3[nm] for nm in synth.OPERAND_NAMES]
    pool3 = synth.state_np((256, 64, 64, 64), seed=1013)
    c3_all = best_ms(lambda: oracle.wkv7_ref(*c3_ins, pool3, cu_seqlens=cu3, state_idx=slots3, precision="f32",
                                             threads=threads))
    del c3, c3_ins, pool3
    # configuration 4: B = 64 rows of a 128-slot pool, T = 5, H = 64, per-token snapshots
    c4 = synth.operands_np((64, 5, 64, 64), seed=1004)
    c4_ins = [c4[nm] for nm in synth.OPERAND_NAMES]
    pool4 = synth.state_np((128, 64, 64, 64), seed=1014)
    slots4 = np.random.default_rng(1004).permutation(128)[:64].astype(np.int64)
    c4_all = best_ms(lambda: oracle.wkv7_ref(*c4_ins, pool4, state_idx=slots4, snapshots=True, precision="f32",
                                             threads=threads))
    del c4, c4_ins, pool4
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"decode B=64 of a 128-slot pool, H=64, T=1, one layer slice, {n} steps in {dt:.1f} s "
                      f"(oracle fp32 loop, OpenMP); CPU: {model}",
            "affinity": affinity, "value_1thread": gbs1, "sample_1thread": f"{n1} steps in {dt1:.1f} s",
            "cfg0": {"shape": "B=1 T=512 H=12 fp32, zero initial state", "ms_all_threads": ms_all,
                     "ms_1thread": ms_one, "tok_s_all_threads": 512 / (ms_all * 1e-3),
                     "tok_s_1thread": 512 / (ms_one * 1e-3)},
            "cfg2": {"shape": "B=1 T=4096 H=64, zero initial state (full)", "ms_all_threads": c2_all,
                     "ms_1thread": c2_one, "tok_s_all_threads": 4096 / (c2_all * 1e-3)},
            "cfg3": {"shape": f"mixed step: 8 prefill rows + 120 decode rows, {total3} tokens, H=64, 256-slot pool "
                              "(full)", "ms_all_threads": c3_all, "tok_s_all_threads": total3 / (c3_all * 1e-3)},
            "cfg4": {"shape": "B=64 T=5 H=64 of a 128-slot pool, per-token snapshots (full)",
                     "ms_all_threads": c4_all}}


def decode_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE, each
    scaled by what the same counter reads for a 1 GiB device copy), or None if absent."""
    path = os.path.join(REPO, "profiles", "wkv7_decode_B64_H64.json")
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
    ap.add_argument("--only", choices=["decode", "prefill", "varlen", "verify", "mixed", "timemix", "int6", "tp",
                                       "heads"], default=None)
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
        log("decode, configuration 1 (H = 40)")
        c1 = decode_bench(torch, kernels, synth, dev, args.steps, args.warmup, H=40)
        c1["frac_hbm"] = c1["GBps"] / HBM_PEAK_GBS
        res["decode_cfg1"] = c1
    if args.only in (None, "tp"):
        # one TP-8 rank's share of the 7.2B model (H = 8 per GPU): 512 pairs at B = 64, occupancy-limited
        log("TP share (H = 8)")
        tp = decode_bench(torch, kernels, synth, dev, args.steps, args.warmup, H=8)
        tp["frac_hbm"] = tp["GBps"] / HBM_PEAK_GBS
        v8 = verify_bench(torch, kernels, synth, dev, args.steps, args.warmup, H=8)
        res["tp_share_H8"] = {"decode": tp, "verify_us": v8["ms"] * 1e3, "verify_GBps": v8["GBps"],
                              "verify_frac_hbm": v8["GBps"] / HBM_PEAK_GBS,
                              "rollback_restore_us": v8["rollback_restore_us"]}
    if args.only in (None, "prefill"):
        log("prefill")
        res["prefill"] = prefill_bench(torch, kernels, synth, dev, max(5, args.steps // 5), args.warmup)
        log("configuration 0 on the GPU")
        res["cfg0_gpu"] = cfg0_bench(torch, kernels, synth, dev, max(5, args.steps // 5), args.warmup)
    if args.only in (None, "varlen"):
        log("varlen prefill chunk (drop-in wkv7 with cu_seqlens)")
        res["varlen"] = varlen_bench(torch, kernels, synth, dev, max(5, args.steps // 5), args.warmup)
    if args.only in (None, "verify"):
        log("verify")
        res["verify"] = verify_bench(torch, kernels, synth, dev, args.steps, args.warmup)
    if args.only in (None, "mixed"):
        log("mixed")
        res["mixed"] = mixed_bench(torch, kernels, synth, dev, max(5, args.steps // 5), args.warmup)
    if args.only in (None, "timemix"):
        log("timemix")
        res["timemix"] = timemix_bench(torch, kernels, dev, max(5, args.steps // 5), args.warmup)
    if args.only in (None, "heads"):
        log("head sizes 128 and 32 (generic kernel)")
        res["head_sizes"] = [head_size_bench(torch, kernels, synth, dev, args.steps, args.warmup, K) for K in (128, 32)]
    if args.only in (None, "int6"):
        log("int6")
        res["int6"] = int6_bench(torch, kernels, dev, args.steps, args.warmup)
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
        "data": "synthetic (seeded; the reference test's input distributions), bf16 operands, fp32 state pools",
        "config": {"workload": "decode B=64 H=64 T=1 over 32 layer slices of a [128,64,64,64] fp32 pool, "
                               "one HIP graph of 32 launches per step",
                   "B": 64, "H": 64, "head_size": 64, "slots": 128, "layers": 32},
    }
    if d:
        achieved = d["bytes_per_launch"] / (d["us_per_launch"] * 1e-6) / 1e9
        out["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": achieved / HBM_PEAK_GBS, "traffic": decode_traffic(),
                           "kernel": "wkv7_decode_kernel", "us_per_launch": d["us_per_launch"]}
    if "decode_cfg1" in res:
        out["decode_cfg1"] = res["decode_cfg1"]
    if "prefill" in res:
        out["prefill"] = res["prefill"]
    if "cfg0_gpu" in res:
        out["cfg0_gpu"] = res["cfg0_gpu"]
    if "tp_share_H8" in res:
        out["tp_share_H8"] = res["tp_share_H8"]
    if "varlen" in res:
        out["varlen"] = res["varlen"]
    if "head_sizes" in res:
        out["head_sizes"] = res["head_sizes"]
    if "verify" in res:
        out["verify"] = res["verify"]
    if "mixed" in res:
        out["mixed"] = res["mixed"]
    if "timemix" in res:
        out["timemix"] = res["timemix"]
    if "int6" in res:
        out["int6"] = res["int6"]
    if cpu:
        out["cpu_baseline"] = cpu
    print(json.dumps(out))


if __name__ == "__main__":
    main()
