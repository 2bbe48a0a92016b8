#!/usr/bin/env python3
"""Benchmark of the quantized-GEMM / fused-MoE hot path on one MI355X.

Headline (the JSON `value`): BASELINE config 1 -- the FP8 e4m3 W8A8 linear on
Llama-3-8B MLP shapes. One step = the up projection (K=4096 -> N=14336) and
the down projection (K=14336 -> N=4096) at M=4096 tokens, each with its
per-token dynamic activation quantization; `value` is TFLOP/s over the timed
steps (inputs resident in HBM).

`sweep` (same JSON line) times every BASELINE config point on the device
(CUDA-graph replays, HIP events): configs 0-2 as GEMM TFLOP/s and GB/s with
the fraction of the bounding roofline, configs 3-4 as microseconds per MoE
layer (routing + dispatch + both grouped GEMMs + combine, plus the shared
expert for config 4) against the HBM roofline of the experts actually routed.

`cpu_baseline` times the CPU oracle (numpy fp32 dequantize-then-matmul, the
reference semantics restated in oracle/) on a bounded sample of the headline
workload.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-sweep] [--no-cpu]
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vllm-torchtpu_amd"))

HBM_PEAK = 8.0e12  # B/s
PEAK = {"fp8": 5.0e15, "int8": 5.0e15, "bf16": 2.5e15, "fp4": 10.1e15}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--m", type=int, default=4096, help="tokens of the headline step")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of sweep configs to run (0-4; 5 = NVFP4 / INT4)")
    ap.add_argument("--profile", nargs="?", const="headline", default=None,
                    choices=["headline", "decode", "moe"],
                    help="rocprofv3 targets: the headline kernel + a copy calibration (default), "
                         "the decode GEMMs (cfg 0/1/2 at M=1), or the MoE layers at T=1 (cfg 3/4)")
    return ap.parse_args()


# ------------------------------------------------------------------ timing


def graph_time_us(fn, iters=20, warm=3, target_us=2000.0, max_reps=64):
    """Device time (us) per call of fn(): `reps` back-to-back calls are
    captured in ONE HIP graph (so per-launch host cost and graph-launch
    latency are amortised away, inter-kernel gaps inside the graph are kept),
    the graph is replayed `iters` times, and the median replay time / reps is
    returned (with p10 / p90)."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    est = event_time_us(fn, iters=3, warm=0)[0]
    reps = int(max(1, min(max_reps, target_us / max(est, 1.0))))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        fn()  # allocations of the first call happen outside the capture
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(reps):
                fn()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    times = []
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(iters):
        st.record()
        g.replay()
        en.record()
        en.synchronize()
        times.append(st.elapsed_time(en) * 1e3 / reps)
    del g
    return float(np.median(times)), float(np.percentile(times, 10)), float(np.percentile(times, 90))


def event_time_us(fn, iters=20, warm=3):
    """Median device time (us) of fn() on the current stream (eager)."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(iters):
        st.record()
        fn()
        en.record()
        en.synchronize()
        times.append(st.elapsed_time(en) * 1e3)
    return float(np.median(times)), float(np.percentile(times, 10)), float(np.percentile(times, 90))


# ------------------------------------------------------------------ data


def fp8_weights(N, K, gen, tiles=False):
    """randn*0.02 weights quantized on the device: per-channel (load-time
    quantizer kernel) or per 128x128 tile (checkpoint form, torch ops)."""
    import torch

    from qmoe import ops

    w = torch.randn((N, K), device="cuda", generator=gen) * 0.02
    if not tiles:
        q, s = ops.row_quant(w, "fp8", mode="load")
        return q, s
    t = w.view(N // 128, 128, K // 128, 128)
    s = t.abs().amax(dim=(1, 3)) / 448.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    q = (t / s[:, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(N, K)
    return q, s.float().contiguous()


def mxfp4_weights(shape, gen):
    import torch

    *lead, N, K = shape
    codes = torch.randint(0, 256, (*lead, N, K // 2), device="cuda", dtype=torch.uint8, generator=gen)
    sc = (127 + torch.randint(-8, 1, (*lead, N, K // 32), device="cuda", generator=gen)).to(torch.uint8)
    return codes, sc


# ------------------------------------------------------------------ headline


def headline(args):
    import torch

    from qmoe import _capi, ops
    from qmoe.layers.linear_common import quantized_matmul

    gen = torch.Generator(device="cuda").manual_seed(0)
    M = args.m
    w_up, s_up = fp8_weights(14336, 4096, gen)
    w_dn, s_dn = fp8_weights(4096, 14336, gen)
    x1 = torch.randn((M, 4096), device="cuda", generator=gen).to(torch.bfloat16)
    x2 = torch.randn((M, 14336), device="cuda", generator=gen).to(torch.bfloat16)
    flops = 2.0 * M * 4096 * 14336 * 2

    def step():
        quantized_matmul(x1, w_up.t(), s_up)
        quantized_matmul(x2, w_dn.t(), s_dn)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps

    # dominant kernel: the tiled FP8 GEMM of the up projection
    xq, xs = ops.row_quant(x1, "fp8")
    xqu = xq.view(torch.uint8)
    wu = w_up.view(torch.uint8)
    gemm = lambda: ops.gemm(_capi.W8A8_PC, xqu, wu, a_scale=xs, w_scale=s_up)  # noqa: E731
    k_us, _, _ = event_time_us(gemm, iters=max(10, args.steps))
    k_flops = 2.0 * M * 4096 * 14336
    k_bytes = 14336 * 4096 + 14336 * 4 + M * 4096 + 4 * M + 2 * M * 14336
    return dict(dt=dt, flops=flops, k_us=k_us, k_flops=k_flops, k_bytes=k_bytes)


# ------------------------------------------------------------------ sweep


def roof(flops, nbytes, us, peak_key):
    t = us * 1e-6
    tf = flops / t / 1e12
    gbs = nbytes / t / 1e9
    t_mem = nbytes / HBM_PEAK
    t_mfma = flops / PEAK[peak_key]
    bound = "hbm" if t_mem >= t_mfma else "mfma"
    frac = (t_mem if bound == "hbm" else t_mfma) / t
    return dict(us=round(us, 2), tflops=round(tf, 2), gbs=round(gbs, 1), bound=bound,
                roofline_frac=round(frac, 3), t_roof_us=round(max(t_mem, t_mfma) * 1e6, 2))


def sweep_linear(only):
    import torch

    from qmoe.layers.linear_common import quantized_matmul, quantized_matmul_fp4
    from qmoe import ops

    gen = torch.Generator(device="cuda").manual_seed(1)
    out = []
    if not only or "0" in only:
        K, N = 2880, 5760
        codes, sc = mxfp4_weights((N, K), gen)
        for M in (1, 16, 128):
            x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
            us = graph_time_us(lambda: quantized_matmul_fp4(x, codes, sc))[0]
            nbytes = N * K // 2 + N * K // 32 + 2 * M * K + 2 * M * N
            out.append(dict(cfg=0, kind="mxfp4_w4a16", M=M, K=K, N=N,
                            **roof(2.0 * M * N * K, nbytes, us, "bf16")))
            log(out[-1])
    if not only or "1" in only:
        for qd in ("fp8", "int8"):
            for K, N in ((4096, 14336), (14336, 4096)):
                w = torch.randn((N, K), device="cuda", generator=gen) * 0.02
                q, s = ops.row_quant(w, qd, mode="load")
                del w
                for M in (1, 8, 64, 512, 4096):
                    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
                    us = graph_time_us(lambda: quantized_matmul(x, q.t(), s), iters=30)[0]
                    nbytes = N * K + 4 * N + 2 * M * K + 2 * M * N
                    out.append(dict(cfg=1, kind=f"{qd}_w8a8_pc", M=M, K=K, N=N,
                                    **roof(2.0 * M * N * K, nbytes, us, qd)))
                    log(out[-1])
    if not only or "2" in only:
        K = 7168
        for N in (18432, 24576):
            q, s = fp8_weights(N, K, gen, tiles=True)
            for M in (1, 32, 256, 2048, 8192):
                x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
                us = graph_time_us(lambda: quantized_matmul(x, q.t(), s), iters=20)[0]
                nbytes = N * K + 4 * (N // 128) * (K // 128) + 2 * M * K + 2 * M * N
                out.append(dict(cfg=2, kind="fp8_w8a8_blk128", M=M, K=K, N=N,
                                **roof(2.0 * M * N * K, nbytes, us, "fp8")))
                log(out[-1])
    return out


def moe_layer_cfg(topk, scoring, activation, bias=None, rsf=1.0, groups=None):
    """The attributes a MoE method reads from its vLLM layer (routing
    settings, activation), for `moe_forward`."""
    from types import SimpleNamespace

    return SimpleNamespace(moe_config=SimpleNamespace(experts_per_token=topk), scoring_func=scoring,
                           renormalize=True, e_score_correction_bias=bias, routed_scaling_factor=rsf,
                           use_grouped_topk=groups is not None, num_expert_group=groups[0] if groups else 1,
                           topk_group=groups[1] if groups else 1, custom_routing_function=None,
                           _qmoe_activation=activation)


def nvfp4_weights(shape, gen):
    """NVFP4 codes + fused bf16 block scales (e4m3 block scale x a float32
    global, as a ModelOpt checkpoint's load makes them)."""
    import torch

    *lead, N, K = shape
    codes = torch.randint(0, 256, (*lead, N, K // 2), device="cuda", dtype=torch.uint8, generator=gen)
    blk = torch.randint(0x20, 0x48, (*lead, N, K // 16), device="cuda", generator=gen).to(torch.uint8)
    sc = (blk.view(torch.float8_e4m3fn).float() * 0.0123456789).to(torch.bfloat16)
    return codes, sc


def int4_weights(shape, gen, group=128):
    """Packed-int4 weights (int32 carriers read as bytes) + bf16 group scales."""
    import torch

    *lead, N, K = shape
    carriers = torch.randint(0, 256, (*lead, N, K // 2), device="cuda", dtype=torch.uint8, generator=gen)
    sc = (torch.rand((*lead, N, K // group), device="cuda", generator=gen) * 0.004 + 0.001).to(torch.bfloat16)
    return carriers, sc


def sweep_nvfp4(only):
    """NVFP4 W4A16 (the reference's ModelOpt FP4 path) and packed-INT4 W4A16
    (group 128, the compressed-tensors MoE recipe) on the config-0 dense and
    config-3 MoE shapes (silu: the reference's NVFP4 MoE takes no swigluoai).
    Algorithmic scale bytes are the checkpoint's (e4m3 for NVFP4, bf16 for
    INT4)."""
    import torch

    from qmoe import ops
    from qmoe.layers.fused_moe import moe_forward
    from qmoe.layers.linear_common import quantized_matmul_fp4

    out = []
    if only and "5" not in only:
        return out
    gen = torch.Generator(device="cuda").manual_seed(5)
    K, N = 2880, 5760
    codes, sc = nvfp4_weights((N, K), gen)
    for M in (1, 16, 128, 4096):
        x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
        us = graph_time_us(lambda: quantized_matmul_fp4(x, codes, sc))[0]
        nbytes = N * K // 2 + N * K // 16 + 2 * M * K + 2 * M * N
        out.append(dict(cfg=5, kind="nvfp4_w4a16", M=M, K=K, N=N, **roof(2.0 * M * N * K, nbytes, us, "bf16")))
        log(out[-1])
    E, k, H, I = 128, 4, 2880, 2880
    w13, s13 = nvfp4_weights((E, 2 * I, H), gen)
    w2, s2 = nvfp4_weights((E, H, I), gen)
    per_expert = 3 * I * H // 2 + 3 * I * H // 16
    lcfg = moe_layer_cfg(k, "softmax", "silu")
    for T in (1, 16, 1024):
        x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
        logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)

        def layer():
            return moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "nvfp4")

        us = graph_time_us(layer, iters=20)[0]
        _, ids = ops.moe_route(logits, k, "softmax", True)
        touched = int(torch.unique(ids).numel())
        nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
        out.append(dict(cfg=5, kind="moe_nvfp4", T=T, experts_touched=touched,
                        **roof(T * k * 6.0 * H * I, nbytes, us, "bf16")))
        log(out[-1])
    del w13, s13, w2, s2
    from qmoe import _capi

    K, N = 2880, 5760
    codes, sc = int4_weights((N, K), gen, group=32 if K % 128 else 128)
    grp = K // sc.shape[-1]
    for M in (1, 16, 128, 4096):
        x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
        us = graph_time_us(lambda: ops.gemm(_capi.W4A16_I4, x, codes, w_scale=sc))[0]
        nbytes = N * K // 2 + 2 * N * K // grp + 2 * M * K + 2 * M * N
        out.append(dict(cfg=5, kind=f"int4_w4a16_g{grp}", M=M, K=K, N=N, **roof(2.0 * M * N * K, nbytes, us, "bf16")))
        log(out[-1])
    w13, s13 = int4_weights((E, 2 * I, H), gen, group=grp)
    w2, s2 = int4_weights((E, H, I), gen, group=grp)
    per_expert = 3 * I * H // 2 + 2 * 3 * I * H // grp
    for T in (1, 16, 1024):
        x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
        logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)

        def layer():
            return moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "int4")

        us = graph_time_us(layer, iters=20)[0]
        _, ids = ops.moe_route(logits, k, "softmax", True)
        touched = int(torch.unique(ids).numel())
        nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
        out.append(dict(cfg=5, kind=f"moe_int4_g{grp}", T=T, experts_touched=touched,
                        **roof(T * k * 6.0 * H * I, nbytes, us, "bf16")))
        log(out[-1])
    return out


def sweep_moe(only):
    import torch

    from qmoe import ops
    from qmoe.layers.fused_moe import moe_forward

    gen = torch.Generator(device="cuda").manual_seed(2)
    out = []
    if not only or "3" in only:
        E, k, H, I = 128, 4, 2880, 2880
        w13, s13 = mxfp4_weights((E, 2 * I, H), gen)
        w2, s2 = mxfp4_weights((E, H, I), gen)
        per_expert = 2 * I * H // 2 + 2 * I * H // 32 + H * I // 2 + H * I // 32
        lcfg = moe_layer_cfg(k, "softmax", "swigluoai")
        for T in (1, 16, 128, 1024, 8192):
            x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
            logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)

            def layer():
                return moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "mxfp4")

            us = graph_time_us(layer, iters=20)[0]
            _, ids = ops.moe_route(logits, k, "softmax", True)
            touched = int(torch.unique(ids).numel())
            nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
            out.append(dict(cfg=3, kind="moe_mxfp4_gptoss", T=T, experts_touched=touched,
                            **roof(T * k * 6.0 * H * I, nbytes, us, "bf16")))
            log(out[-1])
        del w13, s13, w2, s2
        torch.cuda.empty_cache()
    if not only or "4" in only:
        E, k, H, I = 256, 8, 7168, 2048

        def tile_q(shape):
            n, kk = shape
            q, s = fp8_weights(n, kk, gen, tiles=True)
            return q, s

        w13 = torch.empty((E, 2 * I, H), device="cuda", dtype=torch.float8_e4m3fn)
        s13 = torch.empty((E, 2 * I // 128, H // 128), device="cuda", dtype=torch.float32)
        w2 = torch.empty((E, H, I), device="cuda", dtype=torch.float8_e4m3fn)
        s2 = torch.empty((E, H // 128, I // 128), device="cuda", dtype=torch.float32)
        for e in range(E):
            w13[e], s13[e] = tile_q((2 * I, H))
            w2[e], s2[e] = tile_q((H, I))
        sh13, ss13 = tile_q((2 * I, H))
        sh2, ss2 = tile_q((H, I))
        bias = torch.randn(E, device="cuda", generator=gen) * 0.1
        lcfg = moe_layer_cfg(k, "sigmoid", "silu", bias=bias, rsf=2.5, groups=(8, 4))
        per_expert = 3 * H * I + 4 * (2 * I // 128) * (H // 128) + 4 * (H // 128) * (I // 128)
        for skew in (False, True):
            for T in (1, 8, 64, 512, 4096):
                x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
                logits = torch.randn((T, E), device="cuda", generator=gen)
                if skew:
                    # 30% of tokens: +8 on 8 hot experts, 2 per group in groups 0-3
                    hot = torch.tensor([0, 1, 32, 33, 64, 65, 96, 97], device="cuda")
                    sel = torch.rand(T, device="cuda", generator=gen) < 0.3
                    logits[sel.nonzero()[:, 0][:, None], hot[None, :]] += 8.0
                logits = logits.to(torch.bfloat16)

                def routed_part():
                    return moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "fp8_block")

                def shared():
                    from qmoe import _capi

                    xq, xs = ops.row_quant(x, "fp8", block=128)
                    a = ops.gemm(_capi.W8A8_BLK, xq.view(torch.uint8), sh13.view(torch.uint8), a_scale=xs,
                                 w_scale=ss13, ws_bn=128, activation="silu")
                    aq, as_ = ops.row_quant(a, "fp8", block=128)
                    return ops.gemm(_capi.W8A8_BLK, aq.view(torch.uint8), sh2.view(torch.uint8), a_scale=as_,
                                    w_scale=ss2, ws_bn=128)

                def full():
                    return routed_part() + shared()

                us = graph_time_us(full, iters=15)[0]
                _, ids = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=2.5,
                                       num_expert_group=8, topk_group=4)
                touched = int(torch.unique(ids).numel()) + 1
                nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
                out.append(dict(cfg=4, kind="moe_fp8blk_dsv3" + ("_skewed" if skew else ""), T=T,
                                experts_touched=touched, **roof(T * (k + 1) * 6.0 * H * I, nbytes, us, "fp8")))
                log(out[-1])
    return out


def profiled_traffic(m):
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 counters (profiles/, collected with `bench.py --profile`):
    FETCH_SIZE and WRITE_SIZE, each scaled by what it reads for a plain copy
    of known size in the same run. None when no profile matches the
    workload."""
    path = os.path.join(ROOT, "profiles", "tiled_gemm_fp8_w8a8_M4096_K4096_N14336.json")
    try:
        d = json.load(open(path))
    except (OSError, ValueError):
        return None
    if d.get("workload", {}).get("M") != m:
        return None
    cal = d["copy_calibration"]
    c = d["counters_kib_per_dispatch"]
    rd = c["FETCH_SIZE"] * cal["bytes"] / cal["FETCH_SIZE_kib"]
    wr = c["WRITE_SIZE"] * cal["bytes"] / cal["WRITE_SIZE_kib"]
    return int(rd + wr)


# ------------------------------------------------------------------ CPU baseline


def cpu_baseline():
    """The CPU oracle on a bounded sample of the headline workload: FP8 W8A8
    per-channel, K=4096, N=14336, M=256 (dynamic per-token quant + fp32
    dequantize-then-matmul), repeated for about 10-20 s."""
    sys.path.insert(0, ROOT)
    from oracle import codecs, linear, quant

    threads = os.cpu_count() or 1
    rng = np.random.default_rng(0)
    K, N, M = 4096, 14336, 256
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    linear.w8a8_per_channel(x, wq, ws, "fp8")  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        linear.w8a8_per_channel(x, wq, ws, "fp8")
        reps += 1
        el = time.perf_counter() - t0
        if el > 10.0 or reps >= 30:
            break
    dt = el / reps
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=round(2.0 * M * N * K / dt / 1e12, 4), unit="TFLOP/s", cores=threads,
                kind="port", sample=f"fp8 w8a8 per-channel M={M} K={K} N={N}, {reps} reps, "
                f"{dt * 1e3:.1f} ms each, numpy fp32 BLAS, {cpu_model}")


def profile_target(args):
    """Short run for rocprofv3 (kernel trace / counters): the dominant kernel
    of the headline step (FP8 W8A8 tiled GEMM, up projection, M=args.m), 10
    launches, plus a plain 256 MiB device copy (10 launches) whose known byte
    count calibrates FETCH_SIZE / WRITE_SIZE."""
    import torch

    from qmoe import _capi, ops

    gen = torch.Generator(device="cuda").manual_seed(0)
    M = args.m
    w_up, s_up = fp8_weights(14336, 4096, gen)
    x1 = torch.randn((M, 4096), device="cuda", generator=gen).to(torch.bfloat16)
    xq, xs = ops.row_quant(x1, "fp8")
    for _ in range(10):
        ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), w_up.view(torch.uint8), a_scale=xs, w_scale=s_up)
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile target done: gemm M={M} x10, copy 256MiB x10")


def profile_decode(args):
    """rocprofv3 target: 20 launches each of the decode linears at M=1 --
    cfg 0 MXFP4 (K 2880, N 5760), cfg 1 FP8 W8A8 up (K 4096, N 14336, incl.
    the activation quant), cfg 2 block FP8 (K 7168, N 24576) -- after 3
    warm-up calls."""
    import torch

    from qmoe.layers.linear_common import quantized_matmul, quantized_matmul_fp4

    gen = torch.Generator(device="cuda").manual_seed(1)
    codes, sc = mxfp4_weights((5760, 2880), gen)
    x0 = torch.randn((1, 2880), device="cuda", generator=gen).to(torch.bfloat16)
    w1, s1 = fp8_weights(14336, 4096, gen)
    x1 = torch.randn((1, 4096), device="cuda", generator=gen).to(torch.bfloat16)
    w2, s2 = fp8_weights(24576, 7168, gen, tiles=True)
    x2 = torch.randn((1, 7168), device="cuda", generator=gen).to(torch.bfloat16)
    for fn in (lambda: quantized_matmul_fp4(x0, codes, sc), lambda: quantized_matmul(x1, w1.t(), s1),
               lambda: quantized_matmul(x2, w2.t(), s2)):
        for _ in range(23):
            fn()
        torch.cuda.synchronize()
    log("profile target done: cfg0/cfg1/cfg2 M=1 x23 each")


def profile_moe(args):
    """rocprofv3 target: 20 MoE layers at T=1 each for cfg 3 (GPT-OSS,
    MXFP4) and cfg 4 (DeepSeek-V3 routed experts, 128x128 FP8), after 3
    warm-up layers."""
    import torch

    from qmoe.layers.fused_moe import moe_forward

    gen = torch.Generator(device="cuda").manual_seed(2)
    E, k, H, I = 128, 4, 2880, 2880
    w13, s13 = mxfp4_weights((E, 2 * I, H), gen)
    w2, s2 = mxfp4_weights((E, H, I), gen)
    x = torch.randn((1, H), device="cuda", generator=gen).to(torch.bfloat16)
    logits = torch.randn((1, E), device="cuda", generator=gen).to(torch.bfloat16)
    lcfg = moe_layer_cfg(k, "softmax", "swigluoai")
    for _ in range(23):
        moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "mxfp4")
    torch.cuda.synchronize()
    del w13, s13, w2, s2
    E, k, H, I = 256, 8, 7168, 2048
    w13 = torch.empty((E, 2 * I, H), device="cuda", dtype=torch.float8_e4m3fn)
    s13 = torch.empty((E, 2 * I // 128, H // 128), device="cuda", dtype=torch.float32)
    w2 = torch.empty((E, H, I), device="cuda", dtype=torch.float8_e4m3fn)
    s2 = torch.empty((E, H // 128, I // 128), device="cuda", dtype=torch.float32)
    for e in range(E):
        w13[e], s13[e] = fp8_weights(2 * I, H, gen, tiles=True)
        w2[e], s2[e] = fp8_weights(H, I, gen, tiles=True)
    bias = torch.randn(E, device="cuda", generator=gen) * 0.1
    x = torch.randn((1, H), device="cuda", generator=gen).to(torch.bfloat16)
    logits = torch.randn((1, E), device="cuda", generator=gen).to(torch.bfloat16)
    lcfg = moe_layer_cfg(k, "sigmoid", "silu", bias=bias, rsf=2.5, groups=(8, 4))
    for _ in range(23):
        moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "fp8_block")
    torch.cuda.synchronize()
    log("profile target done: cfg3 / cfg4 MoE T=1 x23 each")


def main():
    args = parse()
    if args.profile:
        {"headline": profile_target, "decode": profile_decode, "moe": profile_moe}[args.profile](args)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); "
              "sharding across GPUs is a design only in this build, not a measured path", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    h = headline(args)
    value = h["flops"] / h["dt"] / 1e12
    k_tf = h["k_flops"] / (h["k_us"] * 1e-6) / 1e12
    res = {
        "metric": "quant GEMM/MoE TFLOP/s + % MFMA/HBM roofline vs M; us per MoE layer",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["dt"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 x fp8_e4m3 -> f32 acc -> bf16",
        "data": "synthetic (seeded randn weights quantized per channel, randn bf16 activations)",
        "config": {"workload": "cfg1: FP8 W8A8 per-channel linear, Llama-3-8B MLP up (K4096,N14336) + "
                   f"down (K14336,N4096), M={args.m}, incl. per-token activation quant",
                   "M": args.m, "parallelism": "single GPU"},
        "roofline": {"kernel": "tiled W8A8 FP8 GEMM (up projection)", "bound": "mfma",
                     "achieved": round(k_tf, 2), "peak": PEAK["fp8"] / 1e12, "unit": "TFLOP/s",
                     "frac": round(k_tf / (PEAK["fp8"] / 1e12), 4), "traffic": profiled_traffic(args.m),
                     "us_per_launch": round(h["k_us"], 2),
                     "algorithmic_bytes": h["k_bytes"]},
    }
    only = [c for c in args.only.split(",") if c]
    if not args.no_sweep:
        res["sweep"] = sweep_linear(only) + sweep_moe(only) + sweep_nvfp4(only)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res))


if __name__ == "__main__":
    main()
