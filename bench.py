"""Benchmark of the GLoRCQ hot path on one MI355X.

Metric: 2-bit dequant-GEMV+LoRA HBM GB/s (% of peak).

Workload (config 1's 2-bit expert projection, K=2048 -> N=1408, group 128,
rank 64, M=1): a cold-cache pool of POOL distinct layers (own codes, scales,
zeros, U, SV, x, y each; 2048 x 1.26 MB = 2.58 GB, ten times the 256 MB
Infinity Cache, so no layer's data survives until the next step reads it, as
in a model's decode step).  One step = the fused op over the whole pool, i.e. one
call of the batched entry point, which is ONE launch (gemv_lane_kernel with
the x*U form): each workgroup forms a = fp16(x*U) for its layer, then streams
the packed codes, dequantizes in registers (v_dot2 against x) and adds the
low-rank term a*SV^T per row.
  value = POOL * algorithmic_bytes / step time, algorithmic bytes per layer =
  N*K*b/8 + 4*N*G + 2*r*(K+N) + 2*M*(K+N) = 1,260,288 B.

roofline: that one kernel, timed with HIP events on the launch stream, over
the same algorithmic bytes.  Beside it, the same GEMV fed a = x*U precomputed
by the library (the separate-launch form; bytes per layer N*K*b/8 + 4*N*G +
2*r*N + 2*M*(K+N) + 2*M*r = 998,272 B), whose output must agree with the
step's to the fp32 summation order of a.

Also reported: the MoE block decode step of config 2 at B = 1, 4, 16, 32
(microseconds per step and per token under hipGraph replay, achieved GB/s on
the step's algorithmic bytes), single-call latency of config 0 (one layer,
one launch; eager and per call in a hipGraph), and
the CPU baseline = the reference's CPU fallback restated in oracle/ (fp16
dequant loop + fp16 x@W.T + fp16 LoRA) on config 0, timed on the host cores;
its output doubles as the parity check of the GPU result for the same input.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --pmc-workload   (the GEMV kernel alone + a plain copy
                                         of known size, for rocprofv3 --pmc)
       python bench.py --pmc-workload-kernels   (MoE decode steps and prefill
                                                 GEMMs, for rocprofv3 --pmc)
       python bench.py --model-only [--model-layers L] [--model-batches 1,16]
       python bench.py --turbo-step-only [--turbo-batches 1]   (the TurboQuant-
                                         expert MoE step, then 5 eager steps)
       python bench.py --single-only   (config-0 single calls, eager and in a
                                        hipGraph)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "2b dequant-GEMV+LoRA HBM GB/s (% of peak); MoE-block decode µs/token"
HBM_PEAK_GBS = 8000.0
POOL = 2048
K_, N_, BITS, GROUP, RANK, M_ = 2048, 1408, 2, 128, 64, 1


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_bytes(M=M_, K=K_, N=N_, bits=BITS, group=GROUP, rank=RANK):
    from glorcq_amd import format as fmt

    return fmt.algorithmic_bytes(M, K, N, bits, group, rank)


def gemv_kernel_bytes(M=M_, K=K_, N=N_, bits=BITS, group=GROUP, rank=RANK):
    """Bytes the GEMV kernel must move when a = x*U is given: codes, scales and
    zeros, SV, x, y and a."""
    G = K // group
    return N * K * bits // 8 + 4 * N * G + 2 * rank * N + 2 * M * (K + N) + 2 * M * rank


def make_pool(dev, pool, seed=1):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    G = K_ // GROUP
    kw = K_ * BITS // 32
    codes = torch.randint(-(2**31), 2**31 - 1, (pool, N_, kw), generator=g, device=dev,
                          dtype=torch.int32)
    scales = (torch.randn(pool, N_, G, generator=g, device=dev) * 0.02).abs().half()
    zeros = torch.randint(1, 3, (pool, N_, G), generator=g, device=dev).half()
    U = (torch.randn(pool, K_, RANK, generator=g, device=dev) * 0.01).half()
    SV = (torch.randn(pool, N_, RANK, generator=g, device=dev) * 0.01).half()
    x = torch.randn(pool, M_, K_, generator=g, device=dev).half()
    return codes, scales, zeros, U, SV, x


def time_events(fn, steps, warmup):
    """Mean ms per call of `fn` over `steps` back-to-back calls, HIP events
    recorded on torch's current stream (the stream the library launches on)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def bench_single(dev, calls=200):
    """Config 0 (one layer, one token row, x U from U in the launch): mean µs
    per call over `calls` back-to-back eager calls (HIP events, host launch
    cost included), and per call of 100 calls captured in one hipGraph (the
    best of 5 replays).  Returns the figures and the call's output."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd import kernels

    p0 = fmt.make_linear(K_, N_, bits=BITS, group=GROUP, rank=RANK, M=M_, seed=0)
    d0 = [t.to(dev) for t in (p0.x, p0.codes, p0.scales, p0.zeros, p0.U, p0.SV)]
    y0 = torch.empty(M_, N_, dtype=torch.float16, device=dev)

    def single():
        kernels.packed_dequant_matmul_fused(d0[0], d0[1], d0[2], d0[3], BITS, GROUP, U=d0[4],
                                            SV=d0[5], out=y0)

    eager_ms = time_events(single, calls, 20)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(3):
            single()
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(100):
            single()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / 100)
    return {"single_call_config0_us": round(eager_ms * 1e3, 2),
            "single_call_config0_graph_us": round(best, 2)}, y0


def cpu_model_name():
    """The host CPU's model name (what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_call(fn, budget_s, max_calls=2000):
    """3 warm-ups, then timed calls until the budget (at least 20), median s."""
    for _ in range(3):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while (time.perf_counter() < t_end or len(times) < 20) and len(times) < max_calls:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(gpu_y_config0, budget_s=4.0):
    """Times the oracle's restatements of the reference's CPU fallbacks on
    config 0 (bounded samples, median of >= 20 calls after 3 warm-ups) and
    checks the GPU's config-0 output against the fp16 one.  `value` is the
    fp16 GLoRCQLinear fallback (quantized_linear.py:271-284,313-314,338-349)
    at all torch threads; `rows` adds it at 1 thread, the fp32
    _gptq_pytorch_fallback + lora_out (inference/kernels/__init__.py:149-178,
    311-315) at both thread counts, and the fp16 path at M = 16."""
    import torch

    from glorcq_amd import format as fmt
    from oracle import glorcq_oracle as O

    p = fmt.make_linear(K_, N_, bits=BITS, group=GROUP, rank=RANK, M=M_, seed=0)
    p16 = fmt.make_linear(K_, N_, bits=BITS, group=GROUP, rank=RANK, M=16, seed=0)
    threads = torch.get_num_threads()
    ref = O.linear_forward_fp16(p.x, p.q, p.scales, p.zeros, GROUP, U=p.U, SV=p.SV)

    def fp16(pp):
        return lambda: O.linear_forward_fp16(pp.x, pp.q, pp.scales, pp.zeros, GROUP, U=pp.U,
                                             SV=pp.SV)

    def fp32(pp):
        return lambda: O.linear_forward_fp32(pp.x, pp.q, pp.scales, pp.zeros, GROUP, U=pp.U,
                                             SV=pp.SV)

    rows = []
    for path, M, fn in (("fp16", 1, fp16(p)), ("fp32", 1, fp32(p)), ("fp16", 16, fp16(p16))):
        for t in ((threads, 1) if M == 1 else (threads,)):
            torch.set_num_threads(t)
            try:
                med, n = _median_call(fn, budget_s)
            finally:
                torch.set_num_threads(threads)
            rows.append({"path": path, "M": M, "threads": t, "calls": n,
                         "us_per_call": round(med * 1e6, 1),
                         "GB/s": round(layer_bytes(M=M) / med / 1e9, 4)})
    main_row = rows[0]
    parity = O.parity_ok(gpu_y_config0, ref)
    err = float((gpu_y_config0.float().cpu() - ref.float()).abs().max())
    return {
        "value": main_row["GB/s"], "unit": "GB/s", "cores": threads,
        "kind": "port", "us_per_call": main_row["us_per_call"],
        "sample": (f"{main_row['calls']} config-0 calls (K=2048,N=1408,2-bit,g128,r64,M=1) of "
                   f"the reference CPU fallback restated in oracle/ (fp16 dequant loop + fp16 "
                   f"x@W.T + fp16 LoRA), median after 3 warm-ups, torch threads={threads}, "
                   f"os.cpu_count()={os.cpu_count()}"),
        "cpu_model": cpu_model_name(),
        "rows": rows,
    }, parity, err


def read_traffic():
    """HBM bytes per fused launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE scaled by a plain copy's reading), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_lane_fused_pool2048_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def pmc_workload():
    """What the traffic profile runs: 5 launches of the fused kernel over the
    pool (the bench step), then 5 plain device copies of 512 MiB."""
    import torch

    from glorcq_amd import kernels

    dev = torch.device("cuda:0")
    codes, scales, zeros, U, SV, x = make_pool(dev, POOL)
    out = torch.empty(POOL, M_, N_, dtype=torch.float16, device=dev)
    for _ in range(5):
        kernels.packed_dequant_matmul_batched(x, codes, scales, zeros, BITS, GROUP, U=U, SV=SV,
                                              out=out)
    src = torch.empty(512 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc workload done", flush=True)


def pmc_workload_kernels():
    """What the MoE and prefill counter profiles run: 4 calls each of the
    config-4 attention projections at one token (q/k/v as one launch of 10
    items of 512 x 2048 with q's 8 sharing a U, then o, 2048 x 4096; 4-bit,
    rank 64, x U from U), 4 eager decode steps of the config-2 block (B = 1,
    16) and of the config-3 layer (B = 1, 16), then 4 prefill GEMMs with a
    precomputed a per config-1 shape at M = 512."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd import kernels
    from glorcq_amd.moe_block import GraphCompatibleMoeBlock

    dev = torch.device("cuda:0")
    ps = [fmt.make_linear(2048, 512, bits=4, group=GROUP, rank=RANK, M=1, seed=s)
          for s in range(10)]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(dev)  # noqa: E731
    U = torch.stack([ps[0].U, ps[8].U, ps[9].U]).to(dev)
    uidx = torch.tensor([0] * 8 + [1, 2], dtype=torch.int32, device=dev)
    po = fmt.make_linear(4096, 2048, bits=4, group=GROUP, rank=RANK, M=1, seed=11)
    do = {k: getattr(po, k).to(dev) for k in ("codes", "scales", "zeros", "U", "SV", "x")}
    for _ in range(4):
        kernels.packed_dequant_matmul_batched(ps[0].x.to(dev), st("codes"), st("scales"),
                                              st("zeros"), 4, GROUP, U=U, SV=st("SV"),
                                              u_index=uidx)
    for _ in range(4):
        kernels.packed_dequant_matmul_fused(do["x"], do["codes"], do["scales"], do["zeros"], 4,
                                            GROUP, U=do["U"], SV=do["SV"])
    torch.cuda.synchronize()
    print("config 4 q/k/v and o at one token", flush=True)
    for tag, p in (("config 2 B=1", fmt.make_moe(B=1, seed=6)),
                   ("config 2 B=16", fmt.make_moe(B=16, seed=6)),
                   ("config 3 B=1", fmt.make_mixtral_layer(B=1, seed=3)),
                   ("config 3 B=16", fmt.make_mixtral_layer(B=16, seed=3))):
        blk = GraphCompatibleMoeBlock.from_problem(p, dev)
        h = p.h.reshape(1, p.B, p.H).to(dev)
        for _ in range(4):
            blk(h)
        torch.cuda.synchronize()
        print(tag, flush=True)
        del blk
    for K, N, bits, name in PREFILL:
        M = 512
        p = fmt.make_linear(K, N, bits=bits, group=GROUP, rank=RANK, M=M, seed=3)
        d = {k: getattr(p, k).to(dev) for k in ("codes", "scales", "zeros", "U", "SV", "x")}
        xu = kernels.lowrank_xu(d["x"], d["U"])
        out = torch.empty(M, N, dtype=torch.float16, device=dev)
        for _ in range(4):
            kernels.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"],
                                                bits, GROUP, SV=d["SV"], precomputed_xU=xu,
                                                out=out)
        torch.cuda.synchronize()
        print(name, flush=True)


MOE_BATCHES = (1, 2, 4, 16, 32)
MFMA_FP16_PEAK_TFLOPS = 2500.0
PREFILL = ((2048, 1408, 2, "expert gate/up 2-bit"), (2048, 2048, 4, "attention q/k/v/o 4-bit"))


def graph_time_us(fn, reps=20, trials=15):
    """Median time of one call of fn, from hipGraph replays of `reps` calls
    timed with HIP events (no host launch cost in the figure)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    ts = []
    for _ in range(trials):
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / reps)
    ts.sort()
    return ts[len(ts) // 2]


def bench_prefill(dev):
    """Config 1's prefill batches (M = 128, 512) on the MFMA GEMM path
    (glq_gemm_lora): the whole op (x U launches + GEMM) and the GEMM kernel
    alone (a = x U given), as MFMA utilisation F(M) / time against the fp16
    dense peak, F(M) = 2 M (N K + r (K + N)); beside it torch's fp16 GEMM
    (hipBLASLt) of the same M x N x K on a dense fp16 W, the library ceiling
    for the shape."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd import kernels

    res = {}
    for K, N, bits, name in PREFILL:
        for M in (128, 512):
            p = fmt.make_linear(K, N, bits=bits, group=GROUP, rank=RANK, M=M, seed=M + bits)
            d = {k: getattr(p, k).to(dev) for k in ("codes", "scales", "zeros", "U", "SV", "x")}
            xu = kernels.lowrank_xu(d["x"], d["U"])
            out = torch.empty(M, N, dtype=torch.float16, device=dev)
            W = torch.randn(N, K, generator=torch.Generator().manual_seed(1)).half().to(dev)

            def op():
                kernels.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"],
                                                    bits, GROUP, U=d["U"], SV=d["SV"], out=out)

            def gemm():
                kernels.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"],
                                                    bits, GROUP, SV=d["SV"], precomputed_xU=xu,
                                                    out=out)

            def dense():
                torch.matmul(d["x"], W.t())

            t_op, t_gemm, t_dense = graph_time_us(op), graph_time_us(gemm), graph_time_us(dense)
            F = fmt.algorithmic_flops(M, K, N, RANK)
            res[f"{name} M={M}"] = {
                "K": K, "N": N, "bits": bits, "M": M, "flops": F,
                "op_us": round(t_op, 2), "gemm_kernel_us": round(t_gemm, 2),
                "gemm_tflops": round(F / t_gemm / 1e6, 1),
                "mfma_util_vs_fp16_peak": round(F / t_gemm / 1e6 / MFMA_FP16_PEAK_TFLOPS, 4),
                "torch_fp16_dense_gemm_us": round(t_dense, 2),
                "torch_fp16_dense_tflops": round(2 * M * N * K / t_dense / 1e6, 1)}
            log(f"prefill {name} M={M}: op {t_op:.2f} us, GEMM {t_gemm:.2f} us "
                f"({F / t_gemm / 1e6:.0f} TF/s), dense fp16 {t_dense:.2f} us")
    return res


def _graph_step_us(fn, reps, trials):
    """Median over `trials` replays of one hipGraph holding `reps` calls of fn
    (captured after 3 warm-up calls on a side stream), us per call."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    ts = []
    for _ in range(trials):
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / reps)
    ts.sort()
    del graph
    return ts[len(ts) // 2]


def _moe_decode_leg(dev, p, reps, trials):
    """One decode step of the block built from MoE problem p: us, bytes, GB/s."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd.moe_block import GraphCompatibleMoeBlock

    B = p.B
    blk = GraphCompatibleMoeBlock.from_problem(p, dev)
    h = p.h.reshape(1, B, p.H).to(dev)
    _, logits = blk(h)
    us = _graph_step_us(lambda: blk(h), reps, trials)
    sel = torch.topk(logits.float().cpu(), p.top_k, dim=-1).indices
    act = sorted(set(sel.flatten().tolist()))
    clusters = {proj: len({int(p.cluster_of[proj][e]) for e in act}) for proj in fmt.PROJS}
    nbytes = fmt.moe_step_bytes(p, len(act), clusters)
    gbs = nbytes / (us * 1e-6) / 1e9
    del blk
    return {"us_per_step": round(us, 2), "us_per_token": round(us / B, 3),
            "tokens_per_s": round(B / (us * 1e-6), 1),
            "active_experts": len(act), "active_clusters": clusters,
            "algorithmic_bytes": nbytes, "achieved_GBps": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def bench_moe(dev, seed=6, reps=20, trials=15):
    """Config 2 (Qwen1.5-MoE-A2.7B block): one decode step of
    the whole block per call (router, top-4 dispatch, routed 2-bit experts with
    cluster-shared LoRA, 4-bit shared expert, combine), `reps` steps captured
    in one hipGraph, replays timed with HIP events (median of `trials`).
    Bytes per step follow format.moe_step_bytes with this run's active
    experts and clusters, read off the GPU's own router logits."""
    from glorcq_amd import format as fmt

    res = {}
    for B in MOE_BATCHES:
        r = _moe_decode_leg(dev, fmt.make_moe(B=B, seed=seed), reps, trials)
        res[str(B)] = r
        log(f"moe B={B}: {r['us_per_step']:.2f} us/step, {r['us_per_token']:.3f} us/token, "
            f"{r['achieved_GBps']:.0f} GB/s")
    return res


def bench_moe_cold(dev, seed=6, copies=8, rounds=3, trials=9):
    """Config 2's decode step with cold caches: `copies` distinct copies of the
    block (each about 200 MB, 1.6 GB in all: more than twice the L2s and the
    256 MB Infinity Cache together) stepped in turn inside one hipGraph, so
    no step finds its weights left in a cache by the step before; the same
    routing and bytes as bench_moe's warm figure, which replays one block."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd.moe_block import GraphCompatibleMoeBlock

    res = {}
    for B in MOE_BATCHES:
        p = fmt.make_moe(B=B, seed=seed)
        blks = [GraphCompatibleMoeBlock.from_problem(p, dev) for _ in range(copies)]
        h = p.h.reshape(1, B, p.H).to(dev)
        _, logits = blks[0](h)

        def rotate():
            for b in blks:
                b(h)

        us = _graph_step_us(rotate, rounds, trials) / copies
        sel = torch.topk(logits.float().cpu(), p.top_k, dim=-1).indices
        act = sorted(set(sel.flatten().tolist()))
        clusters = {proj: len({int(p.cluster_of[proj][e]) for e in act}) for proj in fmt.PROJS}
        nbytes = fmt.moe_step_bytes(p, len(act), clusters)
        gbs = nbytes / (us * 1e-6) / 1e9
        res[str(B)] = {"us_per_step": round(us, 2), "us_per_token": round(us / B, 3),
                       "algorithmic_bytes": nbytes, "achieved_GBps": round(gbs, 1),
                       "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"moe cold B={B}: {us:.2f} us/step, {us / B:.3f} us/token, {gbs:.0f} GB/s")
        del blks
        torch.cuda.empty_cache()
    return res


def bench_moe_turbo(dev, seed=6, reps=10, trials=9, batches=(1, 4, 16), eager=0):
    """Config 2's block with TurboQuant routed experts (the reference's 2-bit
    expert format; format.make_turbo_moe: gate/up rotated by an RHT, down by a
    QR Pi, the 4-bit GPTQ shared expert): one decode step per call through
    GraphCompatibleMoeBlock's turbo step, hipGraph replays as bench_moe; then
    `eager` eager steps (for a kernel trace)."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd.moe_block import GraphCompatibleMoeBlock

    res = {}
    for B in batches:
        p = fmt.make_turbo_moe(B=B, seed=seed)
        blk = GraphCompatibleMoeBlock.from_problem(p, dev)
        h = p.h.reshape(1, B, p.H).to(dev)
        blk(h)
        us = _graph_step_us(lambda: blk(h), reps, trials)
        res[str(B)] = {"us_per_step": round(us, 2), "us_per_token": round(us / B, 3)}
        log(f"moe turbo experts B={B}: {us:.2f} us/step")
        for _ in range(eager):
            blk(h)
        torch.cuda.synchronize()
        del blk
    return res


def bench_mixtral(dev, seed=3, reps=20, trials=11, prefill_tokens=512):
    """Config 3 (a Mixtral-8x7B-shaped MoE layer: H 4096, ffn 14336, 8 experts,
    top-2 renormalised, 2-bit g128 experts, rank-64 LoRA over 2 clusters, no
    shared expert): decode steps at B = 1, 4, 16 (hipGraph replays, bytes as
    bench_moe), and a prefill of `prefill_tokens` tokens through the grouped
    GEMM path (glq_moe_prefill), timed the same way."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd.moe_block import GraphCompatibleMoeBlock

    res = {"decode": {}}
    for B in (1, 4, 16):
        r = _moe_decode_leg(dev, fmt.make_mixtral_layer(B=B, seed=seed), reps, trials)
        res["decode"][str(B)] = r
        log(f"mixtral decode B={B}: {r['us_per_step']:.2f} us/step, "
            f"{r['achieved_GBps']:.0f} GB/s")
    T = prefill_tokens
    p = fmt.make_mixtral_layer(B=T, seed=seed)
    blk = GraphCompatibleMoeBlock.from_problem(p, dev)
    h = p.h.reshape(1, T, p.H).to(dev)
    us = _graph_step_us(lambda: blk(h), 3, trials)
    q = p.experts["gate"]
    flops = 2 * T * p.top_k * 3 * p.H * p.inter + 2 * T * p.top_k * 3 * p.rank * (p.H + p.inter)
    res["prefill"] = {"tokens": T, "us": round(us, 1), "tokens_per_s": round(T / (us * 1e-6), 1),
                      "flops": flops, "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                      "expert_bits": q.bits}
    log(f"mixtral prefill T={T}: {us:.1f} us, {flops / (us * 1e-6) / 1e12:.1f} TF/s")
    del blk
    torch.cuda.synchronize()
    return res


def bench_model(dev, layers=48, prompt_len=512, gen=128, batches=(1, 16), seed=0,
                eager_check=8):
    """Config 4: a random-init Qwen3-30B-A3B-shaped model (48 layers, hidden
    2048, GQA 32/4 heads of 128 with 4-bit GPTQ q/k/v/o and rank-64 LoRA, 128
    experts of 768 top-8 renormalised, 2-bit experts with rank-64 LoRA whose U
    rows come from 128 clusters per projection shared by all layers, fp16
    embeddings and lm_head over 151936 tokens), greedy decode through
    GLoRCQGraphWrapper: a 512-token random prompt per sequence (prefill as an
    ordinary forward into the static KV cache), then `gen` tokens, each after
    the first one replay of the captured decode step.  tokens/s counts the
    replayed tokens of all sequences over the wall time of the replay loop
    (including the per-token argmax and id copies).  The first `eager_check`
    tokens of the timed run are compared with the same model run eagerly."""
    import torch

    from glorcq_amd.graph_wrapper import GLoRCQGraphWrapper, _static_cache
    from glorcq_amd.synthetic_model import build_qwen3_moe, qwen3_moe_config

    cfg = qwen3_moe_config(num_hidden_layers=layers, max_position_embeddings=prompt_len + gen)
    t0 = time.perf_counter()
    model, _ = build_qwen3_moe(cfg, dev, seed=seed)
    torch.cuda.synchronize()
    res = {"layers": layers, "prompt_len": prompt_len, "gen_tokens": gen,
           "build_s": round(time.perf_counter() - t0, 1),
           "device_GB_after_build": round(torch.cuda.memory_allocated(dev) / 1e9, 2)}
    log(f"model: {layers} layers built in {res['build_s']} s, "
        f"{res['device_GB_after_build']} GB on the device")
    g = torch.Generator().manual_seed(seed + 1)
    for B in batches:
        ids = torch.randint(0, cfg.vocab_size, (B, prompt_len), generator=g).to(dev)
        w = GLoRCQGraphWrapper(model, max_batch_size=B, max_seq_len=prompt_len + gen)
        w.generate(ids, max_new_tokens=4)  # capture + a warm pass
        out, secs = w.generate(ids, max_new_tokens=gen)
        tm = w.last_timing
        n = B * tm["decode_tokens"]
        tok_s = n / tm["decode_s"]
        r = {"decode_tokens_per_s": round(tok_s, 1),
             "ms_per_decode_step": round(1e3 * tm["decode_s"] / tm["decode_tokens"], 3),
             "prefill_s": round(tm["prefill_s"], 3),
             "prefill_tokens_per_s": round(B * prompt_len / tm["prefill_s"], 1)}
        if eager_check:
            cache = _static_cache(model, B, prompt_len + eager_check, dev, torch.float16)
            with torch.no_grad():
                logits = model(input_ids=ids, cache_position=torch.arange(prompt_len, device=dev),
                               past_key_values=cache, use_cache=True, return_dict=False)[0]
                toks = []
                for i in range(eager_check):
                    t = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
                    toks.append(t)
                    if i + 1 < eager_check:
                        logits = model(input_ids=t,
                                       cache_position=torch.tensor([prompt_len + i], device=dev),
                                       past_key_values=cache, use_cache=True,
                                       return_dict=False)[0]
            eager = torch.cat(toks, dim=1)
            r[f"graph_tokens_equal_eager_first{eager_check}"] = bool(
                torch.equal(out[:, prompt_len:prompt_len + eager_check], eager))
            del cache
        res[f"B{B}"] = r
        log(f"model B={B}: {tok_s:.1f} tokens/s decode ({r['ms_per_decode_step']} ms/step), "
            f"prefill {r['prefill_s']} s")
        del w
        torch.cuda.empty_cache()
    del model
    torch.cuda.empty_cache()
    return res


def bench_turbo(dev, pool_mb=1536, reps_cap=48, trials=11):
    """The reference's own 2-bit routed-expert format (TurboQuant codebook,
    joint_optim.py:715-721) on the codebook kernel, M = 1, cold cache: (a) the graph-mode MoE gate
    GEMV over every expert's rows at once (inference/moe_block.py:783-787:
    60 x 1408 rows, K 2048), (b) the grouped down GEMV, 60 experts each with
    its own input row (moe_block.py:858-865, turbo_matmul.cu:329-415).  A
    hipGraph of launches cycling through distinct weight copies (>= 1.5 GB in
    all), replays timed with HIP events; bytes = fmt.turbo_bytes."""
    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd import kernels

    res = {}
    cases = (("all-experts gate rows", 2048, 60 * 1408, 1),
             ("grouped down, 60 experts", 1408, 2048, 60))
    for name, K, N, items in cases:
        per = items * N * K // 4
        copies = max(2, min(reps_cap, (pool_mb << 20) // per))
        g = torch.Generator(device=dev).manual_seed(7)
        words = torch.randint(-2**31, 2**31 - 1, (copies, items, N, K // 16), dtype=torch.int32,
                              device=dev, generator=g)
        norms = torch.rand(items, N, device=dev, generator=g) + 0.1
        x = torch.randn(items, 1, K, device=dev, generator=g).half()
        cent = torch.tensor(fmt.LLOYD_MAX_2BIT, device=dev) / K ** 0.5
        out = torch.empty(items, 1, N, dtype=torch.float16, device=dev)
        fns = [lambda i=i: kernels.turbo_gemv(x, words[i], norms, cent, out=out)
               for i in range(copies)]
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for f in fns[:3]:
                f()
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for f in fns:
                f()
        graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        ts = []
        for _ in range(trials):
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3 / copies)
        ts.sort()
        us = ts[len(ts) // 2]
        nbytes = fmt.turbo_bytes(1, K, N, items)
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"K": K, "N": N, "items": items, "M": 1, "us_per_launch": round(us, 2),
                     "algorithmic_bytes": nbytes, "achieved_GBps": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "weight_copies": copies}
        log(f"turbo {name}: {us:.2f} us, {gbs:.0f} GB/s")
        del graph, words
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--pool", type=int, default=POOL)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--pmc-workload", action="store_true")
    ap.add_argument("--pmc-workload-kernels", action="store_true",
                    help="the MoE and prefill counter profiles' workload")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE block leg")
    ap.add_argument("--no-turbo", action="store_true", help="skip the TurboQuant codec leg")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the model-level decode leg (config 4)")
    ap.add_argument("--model-only", action="store_true",
                    help="run only the model-level decode leg and print its JSON (profiling)")
    ap.add_argument("--model-layers", type=int, default=48)
    ap.add_argument("--model-batches", default="1,16")
    ap.add_argument("--turbo-step-only", action="store_true",
                    help="run only the TurboQuant-expert MoE step leg, then 5 eager steps, "
                         "and print its JSON (profiling)")
    ap.add_argument("--turbo-batches", default="1")
    ap.add_argument("--single-only", action="store_true",
                    help="run only the config-0 single-call leg and print its JSON (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (every box here has one); "
              "multi-GPU sharding is described in DESIGN.md, not built. Use --gpus 1.",
              file=sys.stderr)
        return 2
    if args.pmc_workload_kernels:
        pmc_workload_kernels()
        return 0
    if args.pmc_workload:
        pmc_workload()
        return 0
    if args.single_only:
        import torch

        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        print(json.dumps(bench_single(dev)[0]), flush=True)
        return 0
    if args.turbo_step_only:
        import torch

        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        batches = tuple(int(b) for b in args.turbo_batches.split(","))
        print(json.dumps(bench_moe_turbo(dev, batches=batches, eager=5)), flush=True)
        return 0
    if args.model_only:
        import torch

        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        batches = tuple(int(b) for b in args.model_batches.split(","))
        print(json.dumps(bench_model(dev, layers=args.model_layers, batches=batches)),
              flush=True)
        return 0

    import torch

    from glorcq_amd import format as fmt
    from glorcq_amd import kernels

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; building pool of {args.pool} layers")
    codes, scales, zeros, U, SV, x = make_pool(dev, args.pool)
    out = torch.empty(args.pool, M_, N_, dtype=torch.float16, device=dev)

    def step():
        kernels.packed_dequant_matmul_batched(x, codes, scales, zeros, BITS, GROUP, U=U, SV=SV,
                                              out=out)

    # The step's one kernel, HIP events on the launch stream (the roofline
    # figure).  It runs first, after 60 untimed calls: the device's first
    # passes over a fresh 2.6 GB pool are slower than its steady state (about
    # 450 against 417 us a step for the first 25 steps on an MI355X), so
    # neither this figure nor the timed step loop below measures a device that
    # has only just allocated the pool.
    log("timing the fused kernel with HIP events")
    k_ms = time_events(step, args.steps, max(args.warmup, 60))
    k_bytes = layer_bytes() * args.pool
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9

    log("timing steps (one fused launch over the pool)")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    gbs = layer_bytes() * args.pool / (ms * 1e-3) / 1e9

    # the GEMV fed a precomputed a = x*U (the separate-launch form)
    xu = kernels.lowrank_xu(x, U)
    out2 = torch.empty_like(out)

    def gemv_only():
        kernels.packed_dequant_matmul_batched(x, codes, scales, zeros, BITS, GROUP, SV=SV,
                                              out=out2, precomputed_xU=xu)

    log("timing the GEMV with a precomputed a = x*U")
    g_ms = time_events(gemv_only, args.steps, args.warmup)
    g_bytes = gemv_kernel_bytes() * args.pool
    diff = (out.float() - out2.float()).abs()
    agree = bool((diff <= 1e-4 + 2e-3 * out2.float().abs()).all())

    log("timing single calls")
    single, y0 = bench_single(dev)

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u2 codes -> f16 pairs (v_dot2_f32_f16), f32 accumulate",
        "data": "synthetic (seeded random codes, scales, zeros, LoRA factors, activations)",
        "config": {
            "workload": (f"config 1 expert gate/up projection: {args.pool} distinct 2-bit "
                         f"2048->1408 g128 r64 layers at M=1, cold cache, one fused launch "
                         f"(a = x*U, dequant-GEMV, + a*SV^T) per step"),
            "K": K_, "N": N_, "bits": BITS, "group": GROUP, "rank": RANK, "M": M_,
            "layers_per_step": args.pool,
        },
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "roofline": {
            "bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
            "kernel": "glq::gemv_lane_kernel<2,false,32,1,4,1,false,true>",
            "kernel_avg_us": round(k_ms * 1e3, 2),
            "algorithmic_bytes_per_launch": k_bytes,
        },
        "gemv_with_precomputed_a": {
            "kernel": "glq::gemv_lane_kernel<2,false,32,1,4,1,false,false>",
            "kernel_avg_us": round(g_ms * 1e3, 2),
            "achieved_gbs": round(g_bytes / (g_ms * 1e-3) / 1e9, 1),
            "algorithmic_bytes_per_launch": g_bytes,
            "matches_step_output": agree,
            "max_abs_diff": float(diff.max()),
        },
        "single_call_config0_us": single["single_call_config0_us"],
        "single_call_config0_graph_us": single["single_call_config0_graph_us"],
    }
    log("prefill GEMM (config 1, M = 128 and 512)")
    result["prefill_gemm"] = bench_prefill(dev)
    if not args.no_moe:
        log("MoE block decode step (config 2), hipGraph replays")
        moe = bench_moe(dev)
        result["moe_block_decode_us_per_token"] = {b: v["us_per_token"] for b, v in moe.items()}
        result["moe_block_decode"] = {
            "workload": ("config 2: Qwen1.5-MoE-A2.7B block (H 2048, 60 experts, inter 1408, "
                         "top-4, 2-bit g128 routed experts with rank-64 LoRA, U shared over 16 "
                         "clusters, 4-bit shared expert inter 5632), seed 6, one hipGraph of 20 "
                         "steps per replay of ONE block: warm caches (its weights stay in the "
                         "256 MB Infinity Cache between steps)"),
            "by_batch": moe}
        log("MoE block decode step (config 2), cold caches: 8 block copies in turn")
        cold = bench_moe_cold(dev)
        result["moe_block_decode_cold_us_per_token"] = {b: v["us_per_token"]
                                                        for b, v in cold.items()}
        result["moe_block_decode_cold"] = {
            "workload": ("config 2 as moe_block_decode, 8 distinct copies of the block "
                         "(1.6 GB) stepped in turn inside one hipGraph: cold L2 and "
                         "Infinity Cache"),
            "by_batch": cold}
        log("Mixtral-shaped MoE layer (config 3): decode steps and a prefill")
        result["mixtral_layer"] = bench_mixtral(dev)
        log("config 2 block with TurboQuant routed experts")
        result["moe_turbo_experts_decode"] = bench_moe_turbo(dev)
    if not args.no_turbo:
        log("TurboQuant codebook GEMV (the reference's 2-bit expert format), M = 1")
        result["turbo_codec_gemv"] = bench_turbo(dev)
    if not args.no_model:
        log("model-level greedy decode (config 4), hipGraph replays")
        try:
            batches = tuple(int(b) for b in args.model_batches.split(","))
            result["model_decode"] = bench_model(dev, layers=args.model_layers, batches=batches)
        except Exception as exc:  # reported in the line; the kernel legs above stand
            result["model_decode"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu:
        log("cpu baseline (oracle restatement of the reference CPU fallback)")
        cb, parity, err = cpu_baseline(y0)
        result["cpu_baseline"] = cb
        result["config0_parity_vs_cpu_fallback"] = {"ok": parity, "max_abs_err": err,
                                                    "bar": "atol 1e-3 + rtol 1e-2"}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
