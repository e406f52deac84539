#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

One step = causal flash-attention forward (O, LSE) + backward (delta, dK/dV,
dQ) at B=8 H=12 S=1024 D=64 bf16, on synthetic seeded
inputs already resident in HBM: q/k are RoPE'd views of a fused qkv tensor,
exactly as the attention block hands them over.  The kernels are called
through the C ABI (include/mi_attn.h) with pre-built argument lists so the
host keeps the GPU queue full.

Printed: ONE JSON line with the metric of BASELINE.json (algorithmic TFLOP/s of
fwd+bwd, causal counted as half of dense: 7*B*H*S^2*D flops per step) from a
timed pass of K steps with events only at its ends (after at least 50 ms of
untimed steps for the GPU to reach steady clocks, then W untimed steps), the per-kernel
durations from max(K, 100) back-to-back launches of each kernel alone, the roofline of
the dominant kernel, the RoPE bandwidth, the train step's fused operators and
config-5 tokens/s, and the CPU baseline (the oracle's fp32 eager attention on
the host cores).

Every measured launch loop (the per-kernel passes, the RoPE, operator and
D = 128 loops, the copy that calibrates the HBM byte counters) runs inside a
roctx profiler region, so that ``rocprofv3 --selected-regions`` records the
dispatches the printed averages come from and no others (not the clock
warm-up, the timed steps or the train step).  ``--summarize DIR`` prints the
per-kernel averages of the rocprofv3 CSV output under DIR.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
       python bench.py --summarize DIR
"""
import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "causal attn fwd+bwd TFLOP/s & % bf16 MFMA peak, B8 H12 S1024 D64"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # untimed steps after the clock warm-up (which alone takes care of the
    # steady clocks: without it, 20 warm-up steps measured 18% slower than 500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU time budget of the baseline sample")
    ap.add_argument("--no-gpt", action="store_true",
                    help="skip the config-5 GPT train-step measurement")
    ap.add_argument("--no-d128", action="store_true",
                    help="skip the measurements beside the headline (configs 1, 3 and 4, head dim 32, S = 1000)")
    ap.add_argument("--no-model-ops", action="store_true",
                    help="skip the config-5 model-operator kernel measurements")
    ap.add_argument("--summarize", metavar="DIR",
                    help="print per-kernel averages from the rocprofv3 CSV files under DIR "
                         "(kernel_stats / kernel_trace / counter_collection) and exit")
    return ap.parse_args()


from gpt_from_scratch_amd.profiler_regions import ProfilerRegions  # noqa: E402

REGIONS = ProfilerRegions()


def _progress(msg):
    """A progress line on stderr (stdout carries only the JSON line)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def attn_flops(B, H, S, D):
    unit = B * H * S * S * D  # one causal GEMM-equivalent (half of 2*B*H*S^2*D)
    return {"fwd": 2 * unit, "bwd": 5 * unit, "dkdv": 4 * unit, "dq": 1 * unit,
            "total": 7 * unit}


def read_traffic(kernel, fname="traffic_c2.txt"):
    """HBM bytes per launch for `kernel` from a committed rocprofv3 PMC summary,
    or None when it has not been measured."""
    path = os.path.join(ROOT, "profiles", fname)
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
            return float(parts[2])
    return None


def cpu_baseline(B, H, S, D, budget_s):
    """The oracle's fp32 eager attention fwd+bwd on the host, on a sample of heads."""
    import torch
    from oracle import attention_backward, attention_forward

    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(2)

    def run(nh):
        q, k, v, do = (torch.randn(1, nh, S, D, generator=g).to(torch.bfloat16).float()
                       for _ in range(4))
        t0 = time.perf_counter()
        attention_forward(q, k, v, True, dtype=torch.float32)
        attention_backward(q, k, v, do, True, dtype=torch.float32)
        return time.perf_counter() - t0

    run(1)  # warm-up
    per_head = run(1)
    nh = max(1, min(B * H, int(budget_s / 3 / max(per_head, 1e-6))))
    first = run(nh)
    reps = max(3, min(30, int(budget_s / max(first, 1e-6))))
    times = [first] + [run(nh) for _ in range(reps - 1)]
    t = statistics.median(times)
    flops = attn_flops(1, nh, S, D)["total"]
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{nh} of {B * H} (b,h) heads of B{B} H{H} S{S} D{D}: oracle fp32 eager "
                      f"fwd+bwd on the CPU, median of {reps} runs ({t:.2f} s each)"}


def _time_calls(stream, fn, args, n, what):
    """Average µs per call of `fn(*args)` over n back-to-back launches on
    `stream` (after 3 untimed ones), inside a profiler region."""
    return _time_rotating(stream, fn, [args], n, what)


def _time_rotating(stream, fn, arglist, n, what):
    """Average µs per call over n back-to-back launches cycling through arglist
    (after 3 untimed ones), inside a profiler region."""
    import torch
    torch.cuda.synchronize()
    REGIONS.resume()
    for i in range(3):
        if fn(*arglist[i % len(arglist)]) != 0:
            raise RuntimeError(f"{what}: {fn.__name__} failed")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        fn(*arglist[i % len(arglist)])
    e1.record(stream)
    torch.cuda.synchronize()
    REGIONS.pause()
    return e0.elapsed_time(e1) / n * 1e3


def model_ops_bench(dev, lib):
    """The train step's fused bandwidth-bound kernels at config 5's shapes, each
    against the HBM peak with its algorithmic bytes (every input read once,
    every output written once):
      * cross entropy over logits [S*B = 8192, V = 50257] bf16
        (core/tensor_parallel/loss.py:9-72): forward reads the logits and the
        int64 targets, writes the bf16 loss and the fp32 lse; backward reads the
        logits, targets, lse and dloss and writes the bf16 gradient;
      * RMSNorm over [8192, 768] bf16 (core/normalization.py:13-25): forward
        reads x and w, writes y and the fp32 rstd; backward reads x, dy, w and
        rstd, writes dx and dw (its [parts, 768] fp32 partials stay in cache
        and are not counted); the same with the residual add fused in front
        (core/transformer_layer.py:96, :102; the sum written as well);
      * SwiGLU over [8192, 2 x 3072] bf16 (core/mlp.py:24-28);
      * the optimizer step over the 190,460,160 parameters (core/optimizer.py:79-104)."""
    import torch
    from gpt_from_scratch_amd import _lib

    S, B, V = 1024, 8, 50257
    rows = S * B
    g = torch.Generator(device=dev).manual_seed(3)
    z = (torch.randn(S, B, V, generator=g, device=dev) * 2).to(torch.bfloat16)
    t = torch.randint(0, V, (S, B), generator=g, device=dev)
    loss = torch.empty(S, B, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(S, B, dtype=torch.float32, device=dev)
    dl = torch.full((S, B), 1.0 / rows, dtype=torch.bfloat16, device=dev)
    grad = torch.empty_like(z)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda x: ctypes.c_void_p(x.data_ptr())
    dt = _lib.dtype_code(z)
    fwd = (dt, rows, V, P(z), V, P(t), P(loss), P(lse), sp)
    bwd = (dt, rows, V, P(z), V, P(t), P(lse), P(dl), P(grad), V, sp)
    out = {}
    for name, fn, a, nbytes in (
            ("xent_fwd", lib.mi_xent_fwd, fwd, rows * V * 2 + rows * (8 + 2 + 4)),
            ("xent_bwd", lib.mi_xent_bwd, bwd, 2 * rows * V * 2 + rows * (8 + 4 + 2))):
        us = _time_calls(stream, fn, a, 30, name)
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"bound": "hbm", "avg_us": round(us, 2), "achieved": round(gbps, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "algorithmic_bytes": nbytes, "shape": f"[{rows}, {V}] bf16",
                     "traffic": read_traffic(name, "traffic_model_ops_c5.txt")}
    del z, grad
    torch.cuda.empty_cache()

    # RMSNorm over the residual stream [S, B, 768] bf16 with a bf16 weight (the
    # model's after the optimizer takes its parameters), core/normalization.py:13-25.
    # Inputs cycle through NC copies (NC * 12.6 MB > the 256 MB Infinity Cache),
    # so every launch reads HBM.
    H, NC = 768, 24
    gen = torch.Generator(device=dev).manual_seed(4)
    xs = [torch.randn(rows, H, generator=gen, device=dev).to(torch.bfloat16) for _ in range(NC)]
    dys = [torch.randn(rows, H, generator=gen, device=dev).to(torch.bfloat16) for _ in range(NC)]
    outs = [torch.empty(rows, H, dtype=torch.bfloat16, device=dev) for _ in range(NC)]
    w = (1 + 0.1 * torch.randn(H, generator=gen, device=dev)).to(torch.bfloat16)
    dw = torch.empty_like(w)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    ws = torch.empty(_lib.rmsnorm_workspace(rows, H), dtype=torch.float32, device=dev)
    fwd_args = [(dt, dt, rows, H, 1e-6, P(xs[i]), H, P(w), P(outs[i]), H, P(rstd), sp)
                for i in range(NC)]
    bwd_args = [(dt, dt, rows, H, P(xs[i]), H, P(w), P(rstd), P(dys[i]), H, P(outs[i]), H, P(dw),
                 P(ws), ws.numel(), sp) for i in range(NC)]
    for name, fn, arglist, nbytes in (
            ("rmsnorm_fwd", lib.mi_rmsnorm_fwd, fwd_args, 2 * rows * H * 2 + rows * 4 + H * 2),
            ("rmsnorm_bwd", lib.mi_rmsnorm_bwd, bwd_args,
             3 * rows * H * 2 + rows * 4 + 2 * H * 2)):
        us = _time_rotating(stream, fn, arglist, 4 * NC, name)
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"bound": "hbm", "avg_us": round(us, 2), "achieved": round(gbps, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "algorithmic_bytes": nbytes, "shape": f"[{rows}, {H}] bf16",
                     "traffic": read_traffic(name, "traffic_model_ops_c5.txt")}
    # The residual add fused in front (core/transformer_layer.py:96, :102): the
    # forward reads x and the branch output, writes the sum and y; the backward
    # reads the sum, dy and the sum's other gradient, writes dx (dw as above).
    sums = [torch.empty(rows, H, dtype=torch.bfloat16, device=dev) for _ in range(NC)]
    afwd_args = [(dt, dt, rows, H, 1e-6, P(xs[i]), H, P(dys[i]), H, P(w), P(sums[i]), H,
                  P(outs[i]), H, P(rstd), sp) for i in range(NC)]
    abwd_args = [(dt, dt, rows, H, P(xs[i]), H, P(w), P(rstd), P(dys[i]), H,
                  P(dys[(i + 1) % NC]), H, P(sums[i]), H, P(dw), P(ws), ws.numel(), sp)
                 for i in range(NC)]
    for name, fn, arglist, nbytes in (
            ("rmsnorm_add_fwd", lib.mi_rmsnorm_add_fwd, afwd_args,
             4 * rows * H * 2 + rows * 4 + H * 2),
            ("rmsnorm_add_bwd", lib.mi_rmsnorm_add_bwd, abwd_args,
             4 * rows * H * 2 + rows * 4 + 2 * H * 2)):
        us = _time_rotating(stream, fn, arglist, 4 * NC, name)
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"bound": "hbm", "avg_us": round(us, 2), "achieved": round(gbps, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "algorithmic_bytes": nbytes, "shape": f"[{rows}, {H}] bf16 + residual",
                     "traffic": read_traffic(name, "traffic_model_ops_c5.txt")}
    del xs, dys, outs, sums
    torch.cuda.empty_cache()

    # SwiGLU on the gate_up projection [8192, 2 * 3072] bf16 (core/mlp.py:24-28):
    # forward reads gate_up, writes h; backward reads gate_up and dh, writes
    # dgate_up.  4 copies (600 MB with dh) keep the inputs out of the cache.
    inter, NS = 3072, 4
    gus = [torch.randn(rows, 2 * inter, generator=gen, device=dev).to(torch.bfloat16)
           for _ in range(NS)]
    dhs = [torch.randn(rows, inter, generator=gen, device=dev).to(torch.bfloat16)
           for _ in range(NS)]
    hs = [torch.empty(rows, inter, dtype=torch.bfloat16, device=dev) for _ in range(NS)]
    dgus = [torch.empty_like(gus[0]) for _ in range(NS)]
    sfwd = [(dt, rows, inter, P(gus[i]), 2 * inter, P(hs[i]), inter, sp) for i in range(NS)]
    sbwd = [(dt, rows, inter, P(gus[i]), 2 * inter, P(dhs[i]), inter, P(dgus[i]), 2 * inter, sp)
            for i in range(NS)]
    for name, fn, arglist, nbytes in (
            ("swiglu_fwd", lib.mi_swiglu_fwd, sfwd, rows * inter * 2 * 3),
            ("swiglu_bwd", lib.mi_swiglu_bwd, sbwd, rows * inter * 2 * 5)):
        us = _time_rotating(stream, fn, arglist, 8 * NS, name)
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"bound": "hbm", "avg_us": round(us, 2), "achieved": round(gbps, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "algorithmic_bytes": nbytes, "shape": f"[{rows}, 2 x {inter}] bf16",
                     "traffic": read_traffic(name, "traffic_model_ops_c5.txt")}
    del gus, dhs, hs, dgus
    torch.cuda.empty_cache()

    # The optimizer step over config 5's 190,460,160 parameters
    # (core/optimizer.py:79-104 with AdamW): the squared-norm pass reads the
    # bf16 gradients; the step reads gradient, fp32 master, exp_avg, exp_avg_sq
    # and writes the last three and the bf16 parameters (3 GB, out of cache).
    n = 190_460_160
    grad = torch.randn(n, generator=gen, device=dev).to(torch.bfloat16)
    master = torch.randn(n, generator=gen, device=dev)
    m1 = torch.zeros(n, device=dev)
    m2 = torch.zeros(n, device=dev)
    prm = torch.empty(n, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(_lib.adamw_workspace(), dtype=torch.float32, device=dev)
    hp = (1 - 3e-4 * 0.1, 0.1, 0.95, 0.05, 3e-4 / 0.1, 0.05 ** 0.5, 1e-8, 1.0)
    sq = [(dt, n, P(grad), P(ws), ws.numel(), sp)]
    st = [(dt, dt, n, P(grad), P(master), P(m1), P(m2), P(prm)) + hp + (P(ws), sp)]
    for name, fn, arglist, nbytes in (
            ("grad_sumsq", lib.mi_grad_sumsq, sq, n * 2),
            ("adamw_step", lib.mi_adamw_step, st, n * (2 + 12 + 12 + 2))):
        us = _time_rotating(stream, fn, arglist, 10, name)
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"bound": "hbm", "avg_us": round(us, 2), "achieved": round(gbps, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "algorithmic_bytes": nbytes, "shape": f"{n} parameters",
                     "traffic": read_traffic(name, "traffic_model_ops_c5.txt")}
    del grad, master, m1, m2, prm
    torch.cuda.empty_cache()

    # What plain streaming reaches on this board, as a yardstick for the
    # fractions above: torch's device-to-device copy of 1 GiB (1 GiB read and
    # 1 GiB written, far past the cache), i.e. the mixed read/write ceiling of a
    # library kernel that does no arithmetic.
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev).normal_(generator=gen)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(5):
        dst.copy_(src)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / 5 * 1e3
    nbytes = 2 * src.numel() * 2
    gbps = nbytes / (us * 1e-6) / 1e9
    out["copy_reference"] = {"kernel": "torch Tensor.copy_ (not this build's)", "avg_us": round(us, 2),
                             "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                             "frac": round(gbps / PEAK_HBM_GBPS, 4), "bytes": nbytes}
    del src, dst
    torch.cuda.empty_cache()
    return out


def attn_config_bench(dev, lib, B, H, S, D, seed, std, steps, dtype=None):
    """Per-kernel times and the fwd+bwd step of one attention configuration in
    the model's layout (q/k RoPE'd out of a fused qkv, v a view of it), through
    the C ABI like the config-2 step: the forward, the delta preprocess and the
    gradient launch(es) each timed over `steps` back-to-back launches, and the
    whole step over `steps` steps with events only at its ends.  dtype: bf16
    (default; fractions of the bf16 matrix peak) or fp32 (the exact-fp32
    kernels; fractions of the fp32 peak)."""
    import torch
    dtype = torch.bfloat16 if dtype is None else dtype
    peak = PEAK_BF16_TFLOPS if dtype == torch.bfloat16 else PEAK_FP32_TFLOPS
    from gpt_from_scratch_amd import _lib
    from gpt_from_scratch_amd.rope import apply_rope_qk
    from gpt_from_scratch_amd.position_embeddings import RotaryEmbedding

    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(S, B, 3, H, D, generator=g) * std).to(dtype).to(dev)
    do = torch.randn(B, H, S, D, generator=g).to(dtype).to(dev)
    rot = RotaryEmbedding(D, max_position_embeddings=S, device="cpu")
    cos, sin = (t.to(dtype).to(dev) for t in (rot.cos_cached, rot.sin_cached))
    q, k, v = qkv.unbind(2)
    qr, kr = apply_rope_qk(q, k, cos, sin)
    Q, K, V = qr.permute(1, 2, 0, 3), kr.permute(1, 2, 0, 3), v.permute(1, 2, 0, 3)
    O = torch.empty(B, H, S, D, dtype=dtype, device=dev)
    LSE = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    DELTA = torch.empty((2,) + tuple(LSE.shape), dtype=torch.float32, device=dev)  # workspace
    dQ, dK, dV = (torch.empty(B, H, S, D, dtype=dtype, device=dev) for _ in range(3))
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ST = lambda t: (ctypes.c_int64 * 4)(*t.stride())
    hdr = (_lib.dtype_code(Q), B, H, S, D)
    scale = 1.0 / math.sqrt(D)
    fwd = hdr + (1, scale, P(Q), ST(Q), P(K), ST(K), P(V), ST(V), P(O), ST(O), P(LSE), sp)
    pre = hdr + (P(O), ST(O), P(do), ST(do), P(LSE), P(DELTA), sp)
    grads = hdr + (1, scale, P(Q), ST(Q), P(K), ST(K), P(V), ST(V), P(do), ST(do), P(LSE),
                   P(DELTA), P(dQ), ST(dQ), P(dK), ST(dK), P(dV), ST(dV), sp)
    calls = [("attn_fwd", lib.mi_attn_fwd, fwd), ("attn_bwd_preprocess", lib.mi_attn_bwd_preprocess, pre),
             ("attn_bwd", lib.mi_attn_bwd_grads, grads)]
    fl = attn_flops(B, H, S, D)
    per = {}
    for name, fn, a in calls:
        per[name] = _time_calls(stream, fn, a, steps, name)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        for name, fn, a in calls:
            fn(*a)
    e1.record(stream)
    torch.cuda.synchronize()
    step_us = e0.elapsed_time(e1) / steps * 1e3
    dname = "bf16" if dtype == torch.bfloat16 else "fp32"
    out = {"shape": f"B{B} H{H} S{S} D{D} {dname} causal", "step_us": round(step_us, 2),
           "tflops": round(fl["total"] / (step_us * 1e-6) / 1e12, 1),
           "frac": round(fl["total"] / (step_us * 1e-6) / 1e12 / peak, 4), "peak_tflops": peak}
    for name, work in (("attn_fwd", fl["fwd"]), ("attn_bwd_preprocess", None),
                       ("attn_bwd", fl["bwd"])):
        ent = {"avg_us": round(per[name], 2)}
        if work:
            tf = work / (per[name] * 1e-6) / 1e12
            ent.update(tflops=round(tf, 1), frac=round(tf / peak, 4))
        out[name] = ent
    return out


def gpt_train(dev, steps=20, warmup=3):
    """Config 5: GPT train step (12L / 768 / 12 heads / SwiGLU 3072 / RMSNorm /
    vocab 50257, B=8, S=1024, TP=1, DP=1) with attention and RoPE on the HIP
    kernels; tokens/s = B*S*steps / wall time (train.py:196-198), beside the
    same step with attention done by plain PyTorch matmul/softmax (fp32 math)
    and the loss, RMSNorm, SwiGLU and optimizer by the reference's eager torch
    ops.

    Loss parity (20 steps from the same seeded init and batch): the kernel run
    against the same step with only attention and RoPE swapped for the
    reference's maths in fp32 (softmax(QK^T/sqrt(D) + mask)V,
    core/myFlashAttn.py:9-23; the interleaved rotation, core/rope_triton.py:
    122-133), every other kernel identical.  Its scale is set by bf16 rounding:
    the same fp32 run against one that rounds P to bf16 before P V, as the
    reference's kernel does (core/myFlashAttn.py:717).  A kernel that rounds
    like the reference moves the loss by about as much; the bound allows three
    times that plus 1e-3.  Also reported: the kernel step with the residual
    adds as separate torch adds, and with the projections' weight gradients
    left to autograd's accumulation into the flat gradient buffer."""
    import torch
    from gpt_from_scratch_amd.harness import GPTConfig, SoftmaxCrossEntropy, train

    def eager_attention(q, k, v, round_p=False):
        S, Dh = q.shape[-2], q.shape[-1]
        s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / math.sqrt(Dh)
        mask = torch.ones(S, S, dtype=torch.bool, device=q.device).tril()
        p = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1)
        if round_p:
            p = p.to(q.dtype).float()
        return torch.matmul(p, v.float()).to(q.dtype)

    def eager_rope(q, k, cos, sin):
        def rot(x):
            S = x.shape[0]
            c = cos[:S].float()[:, None, None, :]
            sn = sin[:S].float()[:, None, None, :]
            xf = x.float()
            e, o = xf[..., 0::2], xf[..., 1::2]
            return torch.stack((e * c - o * sn, e * sn + o * c), dim=-1).flatten(-2).to(x.dtype)
        return rot(q), rot(k)

    cfg = GPTConfig()
    # Start from an empty allocator cache, as a training process does (with the
    # attention passes' blocks still cached, the first train run had measured
    # 473-517k tokens/s; the later variants were unaffected).
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    losses, tps = train(cfg, 8, 1024, steps=steps, seed=5, device=dev, warmup=warmup)
    _progress("config 5: kernel train run done")
    _, eager_tps = train(cfg, 8, 1024, steps=steps, seed=5, device=dev, warmup=warmup,
                         attention=eager_attention, loss_fn=SoftmaxCrossEntropy.apply,
                         eager_ops=True)
    _progress("config 5: eager train run done")
    _, sep_tps = train(cfg, 8, 1024, steps=steps, seed=5, device=dev, warmup=warmup,
                       fuse_add_norm=False)
    _, autograd_tps = train(cfg, 8, 1024, steps=steps, seed=5, device=dev, warmup=warmup,
                            gemm_grad_accumulate=False)
    # parity runs: 20 steps each from the initial parameters
    kern, _ = train(cfg, 8, 1024, steps=20, seed=5, device=dev)
    ref, _ = train(cfg, 8, 1024, steps=20, seed=5, device=dev, attention=eager_attention,
                   rope=eager_rope)
    _progress("config 5: parity runs 1-2 done")
    rnd, _ = train(cfg, 8, 1024, steps=20, seed=5, device=dev,
                   attention=lambda q, k, v: eager_attention(q, k, v, round_p=True),
                   rope=eager_rope)
    dl = max(abs(a - b) for a, b in zip(kern, ref))
    dr = max(abs(a - b) for a, b in zip(rnd, ref))
    bound = 3 * dr + 1e-3
    return {"workload": "config 5: 12L/768/12H SwiGLU RMSNorm vocab 50257, B8 S1024, bf16 params "
                        "+ fp32 AdamW master, TP=1 DP=1, synthetic uint16 ids",
            "steps": steps, "tokens_per_s": round(tps, 1),
            "ms_per_step": round(8 * 1024 / tps * 1e3, 3),
            "tokens_per_s_eager": round(eager_tps, 1),
            "tokens_per_s_separate_adds": round(sep_tps, 1),
            "tokens_per_s_autograd_grad_adds": round(autograd_tps, 1),
            "eager": "attention as torch matmul/softmax (fp32 math); loss, RMSNorm, SwiGLU and "
                     "the AdamW step as the reference's eager torch ops",
            "loss_first": round(losses[0], 4), "loss_last": round(losses[-1], 4),
            "loss_parity": {
                "steps": 20, "vs": "same step with attention and RoPE in fp32 eager maths",
                "max_abs_dloss": round(dl, 6),
                "bf16_p_rounding_max_abs_dloss": round(dr, 6),
                "bound": round(bound, 6), "within_bound": dl <= bound,
                "loss_kernels": [round(x, 5) for x in kern],
                "loss_reference": [round(x, 5) for x in ref]}}


def _short_kernel_name(name):
    """A kernel's demangled name without its return type, namespaces of this
    library and argument list (template arguments kept)."""
    name = name.replace("void ", "", 1) if name.startswith("void ") else name
    name = name.replace("mi::(anonymous namespace)::", "").replace("mi::", "")
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and i > 0:
            return name[:i]
    return name


def summarize(root):
    """Per-kernel averages from rocprofv3's CSV output under `root` (one or
    more runs), one line per kernel and grid size:
      * kernel_trace.csv: dispatch count, mean / min / max duration, the
        scratch (private segment) bytes per lane, and the back-to-back time per
        dispatch (over runs of consecutive dispatches of the same kernel and
        grid: first start to last end / dispatches, i.e. with the dispatch gaps,
        the way a loop of launches between two events measures it);
      * kernel_stats.csv rows when there is no trace;
      * counter_collection.csv: dispatch count and mean / min / max of each
        counter per dispatch (FETCH_SIZE / WRITE_SIZE are in KiB)."""
    import csv
    from collections import defaultdict
    traces, stats, counters = [], [], []
    for dirpath, _, files in os.walk(root):
        for f in sorted(files):
            path = os.path.join(dirpath, f)
            if f.endswith("kernel_trace.csv"):
                traces.append(path)
            elif f.endswith("kernel_stats.csv"):
                stats.append(path)
            elif f.endswith("counter_collection.csv"):
                counters.append(path)

    def key(row):
        grid = row.get("Grid_Size_X") or row.get("Grid_Size") or "?"
        return f"{_short_kernel_name(row['Kernel_Name'])} [grid {grid}]"

    if traces:
        disp = []
        for path in traces:
            for row in csv.DictReader(open(path)):
                disp.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]), key(row),
                             int(row.get("Scratch_Size") or 0)))
        disp.sort()
        dur, scratch = defaultdict(list), defaultdict(int)
        span, span_n = defaultdict(int), defaultdict(int)
        i = 0
        while i < len(disp):
            j = i
            while j + 1 < len(disp) and disp[j + 1][2] == disp[i][2]:
                j += 1
            k = disp[i][2]
            if j > i:
                span[k] += disp[j][1] - disp[i][0]
                span_n[k] += j - i + 1
            i = j + 1
        for start, end, k, scr in disp:
            dur[k].append(end - start)
            scratch[k] = max(scratch[k], scr)
        print("| kernel [grid threads] | dispatches | avg µs | min µs | max µs | back-to-back µs "
              "| scratch B/lane |")
        print("|---|---|---|---|---|---|---|")
        for k, d in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
            b2b = f"{span[k] / span_n[k] / 1e3:.3f}" if span_n[k] else "-"
            print(f"| {k} | {len(d)} | {sum(d) / len(d) / 1e3:.3f} | {min(d) / 1e3:.3f} "
                  f"| {max(d) / 1e3:.3f} | {b2b} | {scratch[k]} |")
        # each pass separately: maximal runs of one kernel and grid at a fixed
        # stride in the dispatch order (1: back-to-back launches; 3: the fwd,
        # delta, bwd steps of a timed pass), at least 5 dispatches
        runs, open_run = [], {}
        for idx, (start, end, k, _) in enumerate(disp):
            r = open_run.get(k)
            gap = idx - r["last"] if r is not None else None
            if r is not None and gap <= 3 and (r["gap"] is None or gap == r["gap"]):
                r["d"].append(end - start)
                r["last"], r["gap"] = idx, gap
            else:
                r = {"k": k, "last": idx, "gap": None, "d": [end - start]}
                open_run[k] = r
                runs.append(r)
        print("\n| pass (in trace order) | kernel [grid threads] | dispatches | avg µs | min µs | max µs |")
        print("|---|---|---|---|---|---|")
        for i, r in enumerate(runs):
            d = r["d"]
            if len(d) >= 5:
                print(f"| {i} | {r['k']} | {len(d)} | {sum(d) / len(d) / 1e3:.3f} "
                      f"| {min(d) / 1e3:.3f} | {max(d) / 1e3:.3f} |")
    elif stats:
        for path in stats:
            print("| kernel | calls | avg µs | min µs | max µs |")
            print("|---|---|---|---|---|")
            for r in csv.DictReader(open(path)):
                print(f"| {_short_kernel_name(r['Name'])} | {r['Calls']} "
                      f"| {float(r['AverageNs']) / 1e3:.3f} | {float(r['MinNs']) / 1e3:.3f} "
                      f"| {float(r['MaxNs']) / 1e3:.3f} |")
    if counters:
        val = defaultdict(lambda: defaultdict(list))
        for path in counters:
            for row in csv.DictReader(open(path)):
                val[row["Counter_Name"]][key(row)].append(float(row["Counter_Value"]))
        for counter, per in sorted(val.items()):
            print(f"\n| kernel [grid threads] | dispatches | {counter} mean | min | max |")
            print("|---|---|---|---|---|")
            for k, v in sorted(per.items(), key=lambda kv: -max(kv[1])):
                print(f"| {k} | {len(v)} | {sum(v) / len(v):.1f} | {min(v):.1f} | {max(v):.1f} |")


def main():
    args = parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported "
              "(attention has no cross-GPU exchange: heads and batches shard with no "
              "communication)", file=sys.stderr)
        sys.exit(2)

    import torch
    from gpt_from_scratch_amd import _lib
    from gpt_from_scratch_amd.rope import apply_rope_qk
    from gpt_from_scratch_amd.position_embeddings import RotaryEmbedding

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, S, D = 8, 12, 1024, 64
    flops = attn_flops(B, H, S, D)
    scale = 1.0 / math.sqrt(D)

    g = torch.Generator().manual_seed(2)
    qkv = torch.randn(S, B, 3, H, D, generator=g).to(torch.bfloat16).to(dev)
    do = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(dev)
    rot = RotaryEmbedding(D, max_position_embeddings=S, device="cpu")
    cos, sin = (t.to(torch.bfloat16).to(dev) for t in (rot.cos_cached, rot.sin_cached))
    q, k, v = qkv.unbind(2)
    qr, kr = apply_rope_qk(q, k, cos, sin)
    Q, K, V = qr.permute(1, 2, 0, 3), kr.permute(1, 2, 0, 3), v.permute(1, 2, 0, 3)
    O = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev)
    LSE = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    DELTA = torch.empty((2,) + tuple(LSE.shape), dtype=torch.float32, device=dev)  # workspace
    dQ, dK, dV = (torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev) for _ in range(3))

    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ST = lambda t: (ctypes.c_int64 * 4)(*t.stride())
    dt = _lib.dtype_code(Q)
    hdr = (dt, B, H, S, D)
    fwd_args = hdr + (1, scale, P(Q), ST(Q), P(K), ST(K), P(V), ST(V), P(O), ST(O), P(LSE), sp)
    pre_args = hdr + (P(O), ST(O), P(do), ST(do), P(LSE), P(DELTA), sp)
    grads_args = hdr + (1, scale, P(Q), ST(Q), P(K), ST(K), P(V), ST(V), P(do), ST(do), P(LSE),
                        P(DELTA), P(dQ), ST(dQ), P(dK), ST(dK), P(dV), ST(dV), sp)
    # The product path: mi_attn_fwd, then mi_attn_bwd = preprocess + grads.
    calls = [("attn_fwd", lib.mi_attn_fwd, fwd_args),
             ("attn_bwd_preprocess", lib.mi_attn_bwd_preprocess, pre_args),
             ("attn_bwd", lib.mi_attn_bwd_grads, grads_args)]

    def step():
        for name, fn, a in calls:
            st = fn(*a)
            if st != 0:
                raise RuntimeError(f"{name}: {lib.mi_last_error().decode()}")

    # Clock warm-up, untimed, before the W warm-up steps: the GPU reaches its
    # steady clocks only after tens of milliseconds of sustained load, so the
    # step runs until 50 ms of GPU time have passed whatever W is.
    clock_warmup_steps = 0
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    while True:
        for _ in range(50):
            step()
        clock_warmup_steps += 50
        c1.record(stream)
        c1.synchronize()
        if c0.elapsed_time(c1) >= 50.0 or clock_warmup_steps >= 20000:
            break
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly K steps between two events on the launch stream
    # and nothing else in the stream.
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t_start.elapsed_time(t_end) / args.steps
    _progress(f"config 2 timed pass: {ms_per_step * 1e3:.1f} us per step")

    # Per-kernel durations: each kernel of the step launched back to back on
    # its own (its inputs are unchanged, so every launch redoes the same work),
    # with events only at the ends of each run; the intervals hold the dispatch
    # gaps between launches.
    # These launches of each kernel (at least 100, so that the events' own
    # cost at the ends is spread thin) are the ones a profiler records
    # (`rocprofv3 --selected-regions`): its per-dispatch average is the
    # duration the roofline below divides by, less the dispatch gaps.
    n_kernel = max(args.steps, 100)
    per_kernel_us = {}
    for name, fn, a in calls:
        k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        REGIONS.resume()
        k0.record(stream)
        for _ in range(n_kernel):
            fn(*a)
        k1.record(stream)
        torch.cuda.synchronize()
        REGIONS.pause()
        per_kernel_us[name] = k0.elapsed_time(k1) / n_kernel * 1e3

    kflops = {"attn_fwd": flops["fwd"], "attn_bwd": flops["bwd"]}
    kernels = {}
    for name, us in per_kernel_us.items():
        ent = {"avg_us": round(us, 3)}
        if name in kflops:
            ent["tflops"] = round(kflops[name] / (us * 1e-6) / 1e12, 2)
        kernels[name] = ent
    dom = max(kflops, key=lambda n: per_kernel_us[n])
    achieved = kflops[dom] / (per_kernel_us[dom] * 1e-6) / 1e12
    roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "algorithmic_flop_per_launch": kflops[dom], "traffic": read_traffic(dom),
                "traffic_source": "profiles/traffic_c2.txt: rocprofv3 FETCH_SIZE and WRITE_SIZE "
                                  "passes of this bench command, scaled by the in-run copy kernel"}

    # The same step with its operands out of the Infinity Cache: NC buffer sets
    # (RoPE'd q/k, the qkv tensor V is a view of, dO, O, LSE, workspace, dQ,
    # dK, dV; ~113 MB each, 452 MB together against the 256 MB cache) used in
    # turn, so each step reads from HBM what the last NC - 1 steps evicted, as
    # a layer of the train step does.  Step time over that rotation, and each
    # kernel's average over back-to-back launches rotating the same way.
    NC = 4
    cold_sets = []
    for _ in range(NC):
        qkv_c = torch.randn(S, B, 3, H, D, generator=g).to(torch.bfloat16).to(dev)
        do_c = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(dev)
        qc, kc, vc = qkv_c.unbind(2)
        qrc, krc = apply_rope_qk(qc, kc, cos, sin)
        Qc, Kc, Vc = qrc.permute(1, 2, 0, 3), krc.permute(1, 2, 0, 3), vc.permute(1, 2, 0, 3)
        Oc = torch.empty_like(O)
        LSEc, WSc = torch.empty_like(LSE), torch.empty_like(DELTA)
        dQc, dKc, dVc = (torch.empty_like(dQ) for _ in range(3))
        keep = (qkv_c, do_c, qrc, krc, Oc, LSEc, WSc, dQc, dKc, dVc)
        fa = hdr + (1, scale, P(Qc), ST(Qc), P(Kc), ST(Kc), P(Vc), ST(Vc), P(Oc), ST(Oc),
                    P(LSEc), sp)
        pa = hdr + (P(Oc), ST(Oc), P(do_c), ST(do_c), P(LSEc), P(WSc), sp)
        ga = hdr + (1, scale, P(Qc), ST(Qc), P(Kc), ST(Kc), P(Vc), ST(Vc), P(do_c), ST(do_c),
                    P(LSEc), P(WSc), P(dQc), ST(dQc), P(dKc), ST(dKc), P(dVc), ST(dVc), sp)
        cold_sets.append((keep, fa, pa, ga))
    set_bytes = sum(t.numel() * t.element_size() for t in cold_sets[0][0])
    for i in range(4 * NC):
        for (name, fn, _), a in zip(calls, cold_sets[i % NC][1:]):
            if fn(*a) != 0:
                raise RuntimeError(f"{name} (HBM-cold pass): {lib.mi_last_error().decode()}")
    n_cold = max(args.steps, 10 * NC) // NC * NC
    torch.cuda.synchronize()
    REGIONS.resume()
    t_start.record(stream)
    for i in range(n_cold):
        for (name, fn, _), a in zip(calls, cold_sets[i % NC][1:]):
            fn(*a)
    t_end.record(stream)
    torch.cuda.synchronize()
    REGIONS.pause()
    cold_step_us = t_start.elapsed_time(t_end) / n_cold * 1e3
    cold_kernels = {}
    for j, (name, fn, _) in enumerate(calls):
        us = _time_rotating(stream, fn, [cs[1 + j] for cs in cold_sets], 25 * NC, name + " (cold)")
        ent = {"avg_us": round(us, 3)}
        if name in kflops:
            ent["tflops"] = round(kflops[name] / (us * 1e-6) / 1e12, 2)
        cold_kernels[name] = ent
    cold_tflops = flops["total"] / (cold_step_us * 1e-6) / 1e12
    hbm_cold = {"sets": NC, "set_bytes": set_bytes, "steps": n_cold,
                "step_us": round(cold_step_us, 2), "tflops": round(cold_tflops, 2),
                "frac": round(cold_tflops / PEAK_BF16_TFLOPS, 4), "kernels": cold_kernels}
    del cold_sets
    _progress(f"config 2 HBM-cold pass: {cold_step_us:.1f} us per step")

    # RoPE (q and k in one launch, the model's strided layout) — HBM-bound.
    # Called through the C ABI with a pre-built argument list, like the
    # attention calls, so that the timed loop is not bound by Python.
    rq, rk = torch.empty_like(qr), torch.empty_like(kr)
    ST2 = lambda t: (ctypes.c_int64 * 2)(*t.stride())
    rope_args = (_lib.dtype_code(q), _lib.dtype_code(cos), S, B, H, D, 0, P(q), ST(q), P(k),
                 ST(k), P(cos), ST2(cos), P(sin), ST2(sin), P(rq), ST(rq), P(rk), ST(rk), sp)
    for _ in range(10):
        if lib.mi_rope_qk(*rope_args) != 0:
            raise RuntimeError(f"rope_qk: {lib.mi_last_error().decode()}")
    torch.cuda.synchronize()
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_rope = 200
    r0.record(stream)
    for _ in range(n_rope):
        lib.mi_rope_qk(*rope_args)
    r1.record(stream)
    torch.cuda.synchronize()
    # (outside the profiler regions: a profiler's record of rope_qk is the
    # HBM-cold pass below, the one the printed roofline is quoted on)
    rope_us = r0.elapsed_time(r1) / n_rope * 1e3
    rope_bytes = 4 * B * S * H * D * 2 + 2 * S * (D // 2) * 2
    rope_gbps = rope_bytes / (rope_us * 1e-6) / 1e9
    # The loop above re-reads one q/k pair, which stays in the 256 MB Infinity
    # Cache (as the projection's fresh output would in the model).  The same
    # launch cycling through 12 qkv copies (453 MB) reads HBM:
    NQ = 12
    qkvs = [torch.randn(S, B, 3, H, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(NQ)]
    cold_args = []
    for t in qkvs:
        cq, ck, _ = t.unbind(2)
        cold_args.append((_lib.dtype_code(cq), _lib.dtype_code(cos), S, B, H, D, 0, P(cq), ST(cq),
                          P(ck), ST(ck), P(cos), ST2(cos), P(sin), ST2(sin), P(rq), ST(rq), P(rk),
                          ST(rk), sp))
    rope_cold_us = _time_rotating(stream, lib.mi_rope_qk, cold_args, 8 * NQ, "rope_qk")
    rope_cold_gbps = rope_bytes / (rope_cold_us * 1e-6) / 1e9
    # The streaming ceiling of that launch, in the same run: mi_copy_qk moves
    # the same q/k views into the same outputs with the same items, grid and
    # accesses, without the rotation (and the 131 KB of tables).
    copy_bytes = 4 * B * S * H * D * 2
    copy_args = [(a[0], S, B, H, D, a[7], a[8], a[9], a[10], a[15], a[16], a[17], a[18], sp)
                 for a in cold_args]
    copy_cold_us = _time_rotating(stream, lib.mi_copy_qk, copy_args, 8 * NQ, "copy_qk")
    copy_cold_gbps = copy_bytes / (copy_cold_us * 1e-6) / 1e9
    del qkvs

    _progress("config 2 per-kernel and RoPE passes done")
    # The config-5 train step before the operator and D = 128 passes: run after
    # them (with their multi-GB buffers allocated and freed), its first timed
    # run measured 463-540k tokens/s against 551-555k in a fresh process.
    gpt = None
    if not args.no_gpt:
        gpt = gpt_train(dev)
        _progress("config 5 train step done")
    model_ops = {} if args.no_model_ops else model_ops_bench(dev, lib)
    _progress("model operators done")

    # Reference point for the HBM byte counters: 64 Mi int32 elements, exactly
    # 256 MiB read and 256 MiB written by one elementwise kernel (torch's
    # bitwise_not, which nothing else in this run launches, so a profiler can
    # select it by name), in a profiler region of its own; its FETCH_SIZE /
    # WRITE_SIZE scale the other kernels'.
    src = torch.ones(64 * 1024 * 1024, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    REGIONS.resume()
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    REGIONS.pause()
    del src, dst

    tflops = flops["total"] / (ms_per_step * 1e-3) / 1e12
    out = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "clock_warmup_steps": clock_warmup_steps,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO, RoPE theta=10000 on q/k)",
        "config": {"workload": "causal flash attention fwd+bwd (O, LSE, dQ, dK, dV), config 2",
                   "B": B, "H": H, "S": S, "D": D, "causal": True, "layout": "model views"},
        "pct_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "algorithmic_gflop_per_step": flops["total"] / 1e9,
        "kernels": kernels,
        "roofline": roofline,
        "config2_hbm_cold": hbm_cold,
        # RoPE's roofline line is measured from HBM (inputs cycled through 12 qkv
        # copies, 453 MB, more than the 256 MB Infinity Cache); the
        # cache-resident rate (one q/k pair re-read) is reported beside it
        "rope": {"bound": "hbm", "avg_us": round(rope_cold_us, 3),
                 "achieved": round(rope_cold_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                 "frac": round(rope_cold_gbps / PEAK_HBM_GBPS, 4), "algorithmic_bytes": rope_bytes,
                 "traffic": read_traffic("rope_qk"), "inputs": "12 rotating qkv copies (HBM)",
                 "copy_yardstick": {"kernel": "mi_copy_qk (the same launch without the rotation)",
                                    "avg_us": round(copy_cold_us, 3),
                                    "achieved": round(copy_cold_gbps, 1),
                                    "frac": round(copy_cold_gbps / PEAK_HBM_GBPS, 4),
                                    "bytes": copy_bytes},
                 "frac_of_copy": round(rope_cold_gbps / copy_cold_gbps, 4),
                 "cache_resident": {"avg_us": round(rope_us, 3), "achieved": round(rope_gbps, 1),
                                    "frac": round(rope_gbps / PEAK_HBM_GBPS, 4),
                                    "inputs": "one q/k pair re-read (Infinity Cache)"}},
    }
    if not args.no_d128:
        # config 1 (fp32, the exact-fp32 kernels): a parity case, measured beside the headline
        out["attn_c1_fp32"] = attn_config_bench(dev, lib, 1, 12, 256, 64, 1, 1.0, args.steps,
                                                dtype=torch.float32)
        _progress("config 1 done")
        # shapes outside the benchmark configs that the matrix-core kernels also cover:
        # head dim 32 (the D = 64 layout, padded) at config 2's FLOPs, and a sequence
        # length with a partial last tile
        out["attn_other_shapes"] = {
            "d32": attn_config_bench(dev, lib, 8, 24, 1024, 32, 5, 1.0, args.steps),
            "s1000": attn_config_bench(dev, lib, 2, 12, 1000, 64, 6, 1.0, args.steps)}
        torch.cuda.empty_cache()
        _progress("head dim 32 and S = 1000 done")
        # configs 3 and 4 (D = 128): parity cases, measured beside the headline
        out["attn_d128"] = {
            "config3": attn_config_bench(dev, lib, 2, 16, 4096, 128, 3, 0.5, args.steps),
            "config4": attn_config_bench(dev, lib, 1, 32, 8192, 128, 4, 1.0, args.steps)}
        torch.cuda.empty_cache()
        _progress("configs 3 and 4 done")
    if model_ops:
        out["model_ops"] = model_ops
    if gpt is not None:
        out["gpt_train"] = gpt
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(B, H, S, D, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
