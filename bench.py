#!/usr/bin/env python3
"""Benchmark of the quantized-GEMM / fused-MoE hot path on one MI355X.

Headline (the JSON `value`): BASELINE config 1 -- the FP8 e4m3 W8A8 linear on
Llama-3-8B MLP shapes. One step = the up projection (K=4096 -> N=14336) and
the down projection (K=14336 -> N=4096) at M=4096 tokens, each with its
per-token dynamic activation quantization; `value` is TFLOP/s over the timed
steps (inputs resident in HBM).

The sweep times every BASELINE config point on the device
(CUDA-graph replays, HIP events): configs 0-2 as GEMM TFLOP/s and GB/s with
the fraction of the bounding roofline, configs 3-4 as microseconds per MoE
layer (routing + dispatch + both grouped GEMMs + combine, plus the shared
expert for config 4) against the HBM roofline of the experts actually routed.
Each point is logged to stderr as it finishes; the whole sweep (with the
read floor and per-point parity) is written to --sweep-out, and the final
stdout line carries only the headline fields plus `sweep_summary` (per
point: M or T, us, roofline fraction, parity ok), which keeps that line a
few KB long.

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
    ap.add_argument("--steps", type=int, default=50)
    # untimed steps before the timed ones: on a fresh MI355X the headline step
    # takes ~60 steps to reach its steady time (measured: 489, 469, then
    # 455-460 us per step over blocks of 20 steps)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--m", type=int, default=4096, help="tokens of the headline step")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep-out", default="gpurun_out/bench_sweep.json",
                    help="where the full sweep (every point, read floor, parity objects) is written")
    ap.add_argument("--only", default="", help="comma list of sweep configs to run (0-4; 5 = NVFP4 / INT4; "
                                                "6 = the decoder layers' other linears; "
                                                "v = hipBLASLt reference points)")
    ap.add_argument("--profile", nargs="?", const="headline", default=None,
                    choices=["headline", "decode", "moe", "vendor", "floor", "w4", "mx", "midm", "moet", "dec6"],
                    help="rocprofv3 targets: the headline kernel + a copy calibration (default), "
                         "the decode GEMMs (cfg 0/1/2 at M=1), the MoE layers at T=1 (cfg 3/4), "
                         "this build's FP8 GEMM beside hipBLASLt's (torch._scaled_mm) on both cfg 1 "
                         "shapes at M=4096, the plain-read floor (time vs size), the large-M MXFP4 "
                         "path (cfg 0 at M=8192, cfg 3 at T=8192), or the opt-in MX activation path "
                         "(cfg 0 at M=8192, cfg 3 at T=8192), the mid-M linears (cfg 0 M=128, cfg 1 "
                         "M=64 / 512, cfg 2 M=256), the cfg 4 MoE layers at T=512 / 4096, or config "
                         "6's linears at 4096 tokens")
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
    # weight codes + per-channel scales + bf16 x + bf16 y (the activation
    # quantization is not counted as algorithmic traffic)
    k_bytes = 14336 * 4096 + 14336 * 4 + 2 * M * 4096 + 2 * M * 14336
    return dict(dt=dt, flops=flops, k_us=k_us, k_flops=k_flops, k_bytes=k_bytes)


# ------------------------------------------------------------------ sweep


FLOOR = []  # plain-read floor curve of this run (read_floor), when measured


def roof(flops, nbytes, us, peak_key):
    """Throughput of one point against its bound. HBM-bound points also carry
    `floor_frac`: the plain read of the same bytes (this run's floor curve,
    launch included) over the point's time."""
    t = us * 1e-6
    tf = flops / t / 1e12
    gbs = nbytes / t / 1e9
    t_mem = nbytes / HBM_PEAK
    t_mfma = flops / PEAK[peak_key]
    bound = "hbm" if t_mem >= t_mfma else "mfma"
    frac = (t_mem if bound == "hbm" else t_mfma) / t
    r = dict(us=round(us, 2), tflops=round(tf, 2), gbs=round(gbs, 1), bound=bound,
             roofline_frac=round(frac, 3), t_roof_us=round(max(t_mem, t_mfma) * 1e6, 2))
    if bound == "hbm" and FLOOR:
        r["floor_frac"] = round(floor_us(FLOOR, nbytes) / us, 3)
    return r


def sweep_mx(codes, sc, host, gen):
    """Config 0 shape with the opt-in MX activations (W4A4: e2m1 + e8m0 per
    32 columns on both operands, K zero-padded 2880 -> 3072 for the MX
    kernel) at the large-M points: the whole linear (activation quant +
    GEMM) and the GEMM alone, against the dense FP4 peak. Flops count the
    layer's K (2880); the padded columns are overhead."""
    import torch

    from qmoe import _capi, ops
    from qmoe.layers.linear_common import pad_mxfp4_for_mx, quantized_matmul_mxfp4_a4

    N, K = codes.shape[0], codes.shape[1] * 2
    wp, wsp = pad_mxfp4_for_mx(codes, sc)
    kp = wp.shape[1] * 2
    hostp = (wp.cpu().numpy(), wsp.cpu().numpy()) if PAR.on else None
    out = []
    for M in (2048, 8192):
        x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
        us = graph_time_us(lambda: quantized_matmul_mxfp4_a4(x, wp, wsp, K))[0]
        q, s = ops.mx_quant(x, k_pad=kp)
        us_gemm = graph_time_us(lambda: ops.gemm(_capi.W4A4_MX, q, wp, a_scale=s, w_scale=wsp))[0]
        nbytes = N * kp // 2 + N * kp // 32 + 2 * M * K + 2 * M * N
        if PAR.on:
            olin, oq = oracle_mod("linear"), oracle_mod("quant")
            par = PAR.linear(quantized_matmul_mxfp4_a4(x, wp, wsp, K), x, M,
                             lambda xr: olin.w4a4_mxfp4(*oq.quantize_mx_fp4(xr, k_pad=kp), *hostp))
        else:
            par = {}
        flops = 2.0 * M * N * K
        pt = dict(cfg=0, kind="mxfp4_w4a4_mx", M=M, K=K, K_padded=kp, N=N, **roof(flops, nbytes, us, "fp4"),
                  fp4_peak_frac=round(flops / (us * 1e-6) / PEAK["fp4"], 4), gemm_us=round(us_gemm, 2),
                  gemm_fp4_peak_frac=round(flops / (us_gemm * 1e-6) / PEAK["fp4"], 4),
                  gemm_fp4_peak_frac_padded_k=round(2.0 * M * N * kp / (us_gemm * 1e-6) / PEAK["fp4"], 4), **par)
        out.append(pt)
        log(pt)
    return out


def sweep_linear(only):
    import torch

    from qmoe.layers.linear_common import quantized_matmul, quantized_matmul_fp4
    from qmoe import ops

    gen = torch.Generator(device="cuda").manual_seed(1)
    out = []
    if not only or "0" in only:
        K, N = 2880, 5760
        codes, sc = mxfp4_weights((N, K), gen)
        host = (codes.cpu().numpy(), sc.cpu().numpy()) if PAR.on else None
        for M in (1, 16, 128, 2048, 8192):
            x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
            us = graph_time_us(lambda: quantized_matmul_fp4(x, codes, sc))[0]
            nbytes = N * K // 2 + N * K // 32 + 2 * M * K + 2 * M * N
            par = PAR.linear(quantized_matmul_fp4(x, codes, sc), x, M,
                             lambda xr: oracle_mod("linear").w4a16_mxfp4(xr, *host)) if PAR.on else {}
            pt = dict(cfg=0, kind="mxfp4_w4a16", M=M, K=K, N=N, **roof(2.0 * M * N * K, nbytes, us, "bf16"), **par)
            if M >= 2048:
                # the W4A16 recipe runs bf16 MFMA; against the dense FP4 peak too
                pt["fp4_peak_frac"] = round(2.0 * M * N * K / (us * 1e-6) / PEAK["fp4"], 4)
            out.append(pt)
            log(out[-1])
        out.extend(sweep_mx(codes, sc, host, gen))
    if not only or "1" in only:
        for qd in ("fp8", "int8"):
            for K, N in ((4096, 14336), (14336, 4096)):
                w = torch.randn((N, K), device="cuda", generator=gen) * 0.02
                q, s = ops.row_quant(w, qd, mode="load")
                del w
                if PAR.on:
                    wq_h, ws_h = q.view(torch.uint8).cpu().numpy(), s.cpu().numpy()
                    if qd == "int8":
                        wq_h = wq_h.view(np.int8)
                for M in (1, 8, 64, 512, 4096):
                    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
                    us = graph_time_us(lambda: quantized_matmul(x, q.t(), s), iters=30)[0]
                    nbytes = N * K + 4 * N + 2 * M * K + 2 * M * N
                    par = PAR.linear(quantized_matmul(x, q.t(), s), x, M,
                                     lambda xr: oracle_mod("linear").w8a8_per_channel(xr, wq_h, ws_h, qd)[0],
                                     exact=qd == "int8") if PAR.on else {}
                    out.append(dict(cfg=1, kind=f"{qd}_w8a8_pc", M=M, K=K, N=N,
                                    **roof(2.0 * M * N * K, nbytes, us, qd), **par))
                    log(out[-1])
    if not only or "2" in only:
        K = 7168
        for N in (18432, 24576):
            q, s = fp8_weights(N, K, gen, tiles=True)
            if PAR.on:
                wq_h = q.view(torch.uint8).cpu().numpy()
                wsb_h = oracle_mod("linear").tile_scales_to_blocks(s.cpu().numpy(), N)
            for M in (1, 32, 256, 2048, 8192):
                x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
                us = graph_time_us(lambda: quantized_matmul(x, q.t(), s), iters=20)[0]
                nbytes = N * K + 4 * (N // 128) * (K // 128) + 2 * M * K + 2 * M * N
                par = PAR.linear(quantized_matmul(x, q.t(), s), x, M,
                                 lambda xr: oracle_mod("linear").w8a8_blockwise(xr, wq_h, wsb_h)[0],
                                 n=2) if PAR.on else {}
                out.append(dict(cfg=2, kind="fp8_w8a8_blk128", M=M, K=K, N=N,
                                **roof(2.0 * M * N * K, nbytes, us, "fp8"), **par))
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


def sweep_decoder(only):
    """Config "6": the other linears of the decoder layers the MoE configs
    come from, through the same entry points at their real shapes --
    DeepSeek-V3's attention projections (q_a, kv_a with the rope part, q_b,
    kv_b, o) as the FP8 method's default recipe (per-channel e4m3 weights,
    per-token activation codes, `layers/adapter/quantization/fp8.py:1669-1690`),
    Llama-3-8B's qkv and o, and DeepSeek-V3's bf16 router gate
    (`UnquantizedLinearMethod`, the W16A16 kind) -- at decode (1 token) and
    prefill (4096 tokens)."""
    import torch

    from qmoe import _capi, ops
    from qmoe.layers.linear_common import quantized_matmul

    if only and "6" not in only:
        return []
    gen = torch.Generator(device="cuda").manual_seed(6)
    out = []
    shapes = [("dsv3_q_a", 1536, 7168), ("dsv3_kv_a", 576, 7168), ("dsv3_q_b", 24576, 1536),
              ("dsv3_kv_b", 32768, 512), ("dsv3_o", 7168, 16384), ("llama3_qkv", 6144, 4096),
              ("llama3_o", 4096, 4096)]
    for name, N, K in shapes:
        w = torch.randn((N, K), device="cuda", generator=gen) * 0.02
        q, s = ops.row_quant(w, "fp8", mode="load")
        del w
        if PAR.on:
            wq_h, ws_h = q.view(torch.uint8).cpu().numpy(), s.cpu().numpy()
        for M in (1, 4096):
            x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
            us = graph_time_us(lambda: quantized_matmul(x, q.t(), s), iters=20)[0]
            nbytes = N * K + 4 * N + 2 * M * K + 2 * M * N
            par = PAR.linear(quantized_matmul(x, q.t(), s), x, M,
                             lambda xr: oracle_mod("linear").w8a8_per_channel(xr, wq_h, ws_h, "fp8")[0],
                             n=2) if PAR.on else {}
            out.append(dict(cfg=6, kind=f"fp8_pc_{name}", M=M, K=K, N=N, **roof(2.0 * M * N * K, nbytes, us, "fp8"),
                            **par))
            log(out[-1])
    N, K = 256, 7168
    wg = (torch.randn((N, K), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    wg_h = wg.float().cpu().numpy() if PAR.on else None
    for M in (1, 4096):
        x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
        us = graph_time_us(lambda: ops.gemm(_capi.W16A16, x, wg), iters=20)[0]
        nbytes = 2 * N * K + 2 * M * K + 2 * M * N
        par = PAR.linear(ops.gemm(_capi.W16A16, x, wg), x, M,
                         lambda xr: oracle_mod("linear").w16a16(xr, wg_h), n=2) if PAR.on else {}
        out.append(dict(cfg=6, kind="bf16_dsv3_router_gate", M=M, K=K, N=N,
                        **roof(2.0 * M * N * K, nbytes, us, "bf16"), **par))
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
            tw, ids = ops.moe_route(logits, k, "softmax", True)
            touched = int(torch.unique(ids).numel())
            nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
            par = {}
            if PAR.on:
                omoe, orouting = oracle_mod("moe"), oracle_mod("routing")
                _, ids_ref = orouting.select_experts(PAR._np(logits), k, True, "softmax")
                ew = omoe.ExpertWeights("mxfp4", _DevRows(w13), _DevRows(s13), _DevRows(w2), _DevRows(s2), keep=False)
                par = PAR.moe(layer(), T, lambda tk: omoe.fused_moe_tokens(
                    PAR._np(x[tk]), ew, PAR._np(tw[tk]), ids_ref[tk], "swigluoai", E),
                    np.array_equal(ids.cpu().numpy(), ids_ref))
            pt = dict(cfg=3, kind="moe_mxfp4_gptoss", T=T, experts_touched=touched,
                      **roof(T * k * 6.0 * H * I, nbytes, us, "bf16"), **par)
            if T >= 1024:
                pt["fp4_peak_frac"] = round(T * k * 6.0 * H * I / (us * 1e-6) / PEAK["fp4"], 4)
            out.append(pt)
            log(out[-1])
        # the opt-in MX activations (weight format mxfp4_mx: experts padded
        # along K 2880 -> 3072, tokens and intermediate MX-quantized) at the
        # large-T points; flops count the layer's K
        from qmoe.layers.quantization.mxfp4 import _pad_experts_for_mx

        w13p, s13p = _pad_experts_for_mx(w13, s13)
        w2p, s2p = _pad_experts_for_mx(w2, s2)
        for T in (1024, 8192):
            x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
            logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)

            def layer_mx():
                return moe_forward(lcfg, x, logits, w13p, w2p, s13p, s2p, None, None, "mxfp4_mx")

            us = graph_time_us(layer_mx, iters=20)[0]
            tw, ids = ops.moe_route(logits, k, "softmax", True)
            touched = int(torch.unique(ids).numel())
            nbytes = touched * per_expert * 3072 // 2880 + 2 * T * H * 2 + 2 * T * E
            par = {}
            if PAR.on:
                omoe, orouting = oracle_mod("moe"), oracle_mod("routing")
                _, ids_ref = orouting.select_experts(PAR._np(logits), k, True, "softmax")
                ew = omoe.ExpertWeights("mxfp4_mx", _DevRows(w13), _DevRows(s13), _DevRows(w2), _DevRows(s2),
                                        keep=False)
                par = PAR.moe(layer_mx(), T, lambda tk: omoe.fused_moe_tokens(
                    PAR._np(x[tk]), ew, PAR._np(tw[tk]), ids_ref[tk], "swigluoai", E),
                    np.array_equal(ids.cpu().numpy(), ids_ref))
            flops = T * k * 6.0 * H * I
            pt = dict(cfg=3, kind="moe_mxfp4_gptoss_mx_act", T=T, experts_touched=touched,
                      **roof(flops, nbytes, us, "fp4"), fp4_peak_frac=round(flops / (us * 1e-6) / PEAK["fp4"], 4),
                      **par)
            out.append(pt)
            log(out[-1])
        del w13, s13, w2, s2, w13p, s13p, w2p, s2p
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
                tw, ids = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=2.5,
                                        num_expert_group=8, topk_group=4)
                touched = int(torch.unique(ids).numel()) + 1
                nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
                par, ids_ok = {}, None
                if PAR.on:
                    omoe, orouting = oracle_mod("moe"), oracle_mod("routing")
                    _, ids_ref = orouting.grouped_topk(PAR._np(logits), k, True, 8, 4, "sigmoid", PAR._np(bias), 2.5)
                    ids_ok = np.array_equal(ids.cpu().numpy(), ids_ref)
                    # routed part only (the shared expert's GEMMs are
                    # checked at these shapes by the parity tests)
                    ew = omoe.ExpertWeights("fp8_block", _DevRows(w13.view(torch.uint8)), _DevRows(s13),
                                            _DevRows(w2.view(torch.uint8)), _DevRows(s2), keep=False)
                    par = PAR.moe(routed_part(), T, lambda tk: omoe.fused_moe_tokens(
                        PAR._np(x[tk]), ew, PAR._np(tw[tk]), ids_ref[tk], "silu", E), ids_ok, n=1)
                out.append(dict(cfg=4, kind="moe_fp8blk_dsv3" + ("_skewed" if skew else ""), T=T,
                                experts_touched=touched, **roof(T * (k + 1) * 6.0 * H * I, nbytes, us, "fp8"),
                                **par))
                log(out[-1])
                # an armed layer serves larger steps with the GMM path above
                if T > min(ops.DECODE_MAX_TOKENS, decode_op_tokens()):
                    continue

                def decode_layer():
                    # the fused decode op (shared + routed experts), routing
                    # the tokens itself; routed_scaling_factor moves into it
                    return ops.moe_decode_routed(x, logits, k, w13, w2, s13, s2, sh13, ss13, sh2, ss2, None,
                                                 scoring_func="sigmoid", renormalize=True, bias=bias,
                                                 routed_scaling_factor=1.0, num_expert_group=8, topk_group=4,
                                                 routed_scale=2.5, weight_blocks=128)[0]

                us = graph_time_us(decode_layer, iters=15)[0]
                par = {}
                if PAR.on:
                    odec = oracle_mod("decode")
                    tw1, ti1 = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=1.0,
                                             num_expert_group=8, topk_group=4)
                    sh = tuple(PAR._np(t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t)
                               for t in (sh13, ss13, sh2, ss2))
                    par = PAR.moe(decode_layer(), T, lambda tk: odec.fused_moe_decode(
                        PAR._np(x[tk]), _DevRows(w13.view(torch.uint8)), _DevRows(s13), _DevRows(w2.view(torch.uint8)),
                        _DevRows(s2), *sh, None, PAR._np(tw1[tk]), PAR._np(ti1[tk]), routed_scale=2.5,
                        weight_blocks=128), ids_ok, n=1)
                out.append(dict(cfg=4, kind="moe_fp8blk_dsv3_decode_op" + ("_skewed" if skew else ""), T=T,
                                experts_touched=touched, **roof(T * (k + 1) * 6.0 * H * I, nbytes, us, "fp8"),
                                **par))
                log(out[-1])
        out.extend(sweep_moe_default(lcfg, w13, s13, w2, s2, sh13, ss13, sh2, ss2, bias, gen))
    return out


def decode_op_tokens():
    """The most tokens an armed MoE layer serves with the fused decode op
    (the measured crossover to the GMM path)."""
    from qmoe import envs

    return envs.QMOE_DECODE_OP_MAX_TOKENS or 1 << 30


def sweep_moe_default(lcfg, w13, s13, w2, s2, sh13, ss13, sh2, ss2, bias, gen):
    """Config 4 through the FP8 MoE method's DEFAULT recipe (what a
    DeepSeek-V3 checkpoint runs without the opt-in native tiles,
    `layers/adapter/quantization/fp8.py:486-617`): the 128 x 128 tiles
    dequantized and requantized per output channel (e4m3, and int8 with
    MOE_REQUANTIZE_WEIGHT_DTYPE=int8), per-(token, 512) bf16-arithmetic
    activation codes before each grouped GEMM; the shared expert as the
    default dense recipe (per-channel weights, per-token activations, silu
    fused). For e4m3 at T <= 64 also the fused decode op on the same
    per-channel experts."""
    import torch

    from qmoe import _capi, ops
    from qmoe.layers.fused_moe import moe_forward
    from qmoe.layers.quantization.fp8 import dequantize_fp8_weight, requantize

    E, k, H, I = 256, 8, 7168, 2048
    out = []

    def per_channel(w, s, qd):
        q = torch.empty(w.shape, dtype=torch.float8_e4m3fn if qd == "fp8" else torch.int8, device=w.device)
        sc = torch.empty(w.shape[:-1], dtype=torch.float32, device=w.device)
        for e in range(w.shape[0] if w.dim() == 3 else 1):
            we, se = (w[e], s[e]) if w.dim() == 3 else (w, s)
            qe, sce = requantize(dequantize_fp8_weight(we, weight_scale_inv=se, block=(128, 128)),
                                 "float8_e4m3fn" if qd == "fp8" else "int8")
            if w.dim() == 3:
                q[e], sc[e] = qe, sce
            else:
                q, sc = qe, sce
        return q, sc

    per_expert = 3 * H * I + 4 * (2 * I + H)
    for qd in ("fp8", "int8"):
        q13, c13 = per_channel(w13, s13, qd)
        q2, c2 = per_channel(w2, s2, qd)
        qs13, cs13 = per_channel(sh13, ss13, qd)
        qs2, cs2 = per_channel(sh2, ss2, qd)
        wf = 0 if qd == "fp8" else 1
        for T in (1, 8, 64, 512, 4096):
            x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
            logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)

            def routed_part():
                return moe_forward(lcfg, x, logits, q13, q2, c13, c2, None, None, qd)

            def shared():
                xq, xs = ops.row_quant(x, qd)
                a = ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), qs13.view(torch.uint8), a_scale=xs,
                             w_scale=cs13, wfmt=wf, activation="silu")
                aq, as_ = ops.row_quant(a, qd)
                return ops.gemm(_capi.W8A8_PC, aq.view(torch.uint8), qs2.view(torch.uint8), a_scale=as_,
                                w_scale=cs2, wfmt=wf)

            def full():
                return routed_part() + shared()

            us = graph_time_us(full, iters=15)[0]
            tw, ids = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=2.5,
                                    num_expert_group=8, topk_group=4)
            touched = int(torch.unique(ids).numel()) + 1
            nbytes = touched * per_expert + 2 * T * H * 2 + 2 * T * E
            par, ids_ok = {}, None
            if PAR.on:
                omoe, orouting = oracle_mod("moe"), oracle_mod("routing")
                _, ids_ref = orouting.grouped_topk(PAR._np(logits), k, True, 8, 4, "sigmoid", PAR._np(bias), 2.5)
                ids_ok = np.array_equal(ids.cpu().numpy(), ids_ref)
                cv = (lambda t: t.view(torch.uint8)) if qd == "fp8" else (lambda t: t)  # noqa: E731
                ew = omoe.ExpertWeights(qd, _DevRows(cv(q13)), _DevRows(c13), _DevRows(cv(q2)), _DevRows(c2),
                                        keep=False)
                par = PAR.moe(routed_part(), T, lambda tk: omoe.fused_moe_tokens(
                    PAR._np(x[tk]), ew, PAR._np(tw[tk]), ids_ref[tk], "silu", E), ids_ok, n=1)
            out.append(dict(cfg=4, kind=f"moe_{qd}_pc_dsv3_default", T=T, experts_touched=touched,
                            **roof(T * (k + 1) * 6.0 * H * I, nbytes, us, qd), **par))
            log(out[-1])
            if qd != "fp8" or T > min(ops.DECODE_MAX_TOKENS, decode_op_tokens()):
                continue

            def decode_layer():
                return ops.moe_decode_routed(x, logits, k, q13, q2, c13, c2, qs13, cs13, qs2, cs2, None,
                                             scoring_func="sigmoid", renormalize=True, bias=bias,
                                             routed_scaling_factor=1.0, num_expert_group=8, topk_group=4,
                                             routed_scale=2.5)[0]

            us = graph_time_us(decode_layer, iters=15)[0]
            par = {}
            if PAR.on:
                odec = oracle_mod("decode")
                tw1, ti1 = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=1.0,
                                         num_expert_group=8, topk_group=4)
                sh = tuple(PAR._np(t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t)
                           for t in (qs13, cs13, qs2, cs2))
                par = PAR.moe(decode_layer(), T, lambda tk: odec.fused_moe_decode(
                    PAR._np(x[tk]), _DevRows(q13.view(torch.uint8)), _DevRows(c13), _DevRows(q2.view(torch.uint8)),
                    _DevRows(c2), *sh, None, PAR._np(tw1[tk]), PAR._np(ti1[tk]), routed_scale=2.5), ids_ok, n=1)
            out.append(dict(cfg=4, kind="moe_fp8_pc_dsv3_decode_op", T=T, experts_touched=touched,
                            **roof(T * (k + 1) * 6.0 * H * I, nbytes, us, "fp8"), **par))
            log(out[-1])
        del q13, c13, q2, c2, qs13, cs13, qs2, cs2
        torch.cuda.empty_cache()
    return out


def sweep_vendor():
    """Vendor reference points on the same box: hipBLASLt's FP8 GEMM
    (torch._scaled_mm) on the cfg 1 shapes at M 512 and 4096, same codes as
    this build's tiled GEMM, GEMM alone (no activation quantization), beside
    this build's GEMM alone."""
    import torch

    from qmoe import _capi, ops

    gen = torch.Generator(device="cuda").manual_seed(3)
    out = []
    for K, N in ((4096, 14336), (14336, 4096)):
        w, s = fp8_weights(N, K, gen)
        for M in (512, 4096):
            x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
            xq, xs = ops.row_quant(x, "fp8")
            ours = lambda: ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), w.view(torch.uint8),  # noqa: E731
                                    a_scale=xs, w_scale=s)
            vend, scaling = vendor_scaled_mm(xq, w, xs, s)
            nbytes = N * K + 4 * N + 2 * M * K + 2 * M * N
            for name, fn in (("qmoe_gemm_fp8_pc", ours), (f"hipblaslt_scaled_mm_{scaling.split()[0]}", vend)):
                us = graph_time_us(fn, iters=30)[0]
                out.append(dict(cfg=1, kind=name, M=M, K=K, N=N, **roof(2.0 * M * N * K, nbytes, us, "fp8")))
                log(out[-1])
        del w, s
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


# ------------------------------------------------------------------ CPU leg: per-point parity


class ParityLeg:
    """Per-point parity and CPU time, part of the CPU-baseline leg (the oracle
    is the checker here, never the thing timed on the GPU). For each sweep
    point a few output rows (tokens) are recomputed by the CPU oracle from
    the same device inputs:

    * `parity`: rows checked, max |err| / row max, cosine, and `pass` for the
      north-star bar (max |err| <= 2e-2 * row max, cosine >= 0.9995); INT8
      GEMMs also carry `exact` (integer accumulation is bit-exact); MoE points
      carry `ids_exact` (every token's routing ids against the oracle's);
    * `cpu_ms_est`: the oracle's time for the whole point, from its times on
      n and 2n sampled rows (fixed part + per-row part, linear in rows), or
      for MoE points the per-token time times T (the oracle loops over
      tokens); `cpu_ms_sample` is the measured time of the larger sample.

    Disabled (empty dicts) with --no-cpu."""

    def __init__(self, on):
        self.on = on
        self.threads = None
        if on:
            sys.path.insert(0, ROOT)

    @staticmethod
    def _np(t):
        return t.detach().float().cpu().numpy() if t.dtype in (_torch().bfloat16, _torch().float16) \
            else t.detach().cpu().numpy()

    @staticmethod
    def _rows(M, n):
        if M <= n:
            return np.arange(M)
        return np.unique(np.linspace(0, M - 1, n).round().astype(np.int64))

    @staticmethod
    def _stats(got, ref):
        got = np.asarray(got, np.float64).reshape(-1, np.asarray(got).shape[-1])
        ref = np.asarray(ref, np.float64).reshape(got.shape)
        err = np.abs(got - ref).max(axis=-1) / np.maximum(np.abs(ref).max(axis=-1), 1e-30)
        den = np.linalg.norm(got) * np.linalg.norm(ref)
        cos = float((got * ref).sum() / den) if den > 0 else 1.0
        ok = bool(np.isfinite(got).all() and err.max() <= 2e-2 and cos >= 0.9995)
        return dict(rows=int(got.shape[0]), max_err_rowmax=float(f"{err.max():.3g}"), cos=round(cos, 7), ok=ok)

    def linear(self, y, x, M, oracle_fn, n=4, exact=False):
        """oracle_fn(x_rows_f32) -> reference rows; y the device output."""
        if not self.on:
            return {}
        r1, r2 = self._rows(M, n), self._rows(M, 2 * n)
        t0 = time.perf_counter()
        oracle_fn(self._np(x[r1]))
        t1 = time.perf_counter()
        ref = oracle_fn(self._np(x[r2]))
        t2 = time.perf_counter()
        got = self._np(y[r2])
        st = self._stats(got, ref)
        if exact:
            st["exact"] = bool(np.array_equal(got, ref))
        ta, tb = t1 - t0, t2 - t1
        per_row = max(tb - ta, 0.0) / max(len(r2) - len(r1), 1)
        est = max(ta - len(r1) * per_row, 0.0) + M * per_row if len(r2) > len(r1) else tb
        return dict(parity=st, cpu_ms_sample=round(tb * 1e3, 1), cpu_ms_est=round(est * 1e3, 1))

    def moe(self, y, T, oracle_tokens, ids_exact, n=2):
        """oracle_tokens(token_idx) -> reference rows for those tokens."""
        if not self.on:
            return {}
        toks = self._rows(T, n)
        t0 = time.perf_counter()
        ref = oracle_tokens(toks)
        dt = time.perf_counter() - t0
        st = self._stats(self._np(y[toks]), ref)
        st["ids_exact"] = bool(ids_exact)
        return dict(parity=st, cpu_ms_sample=round(dt * 1e3, 1), cpu_ms_est=round(dt / len(toks) * T * 1e3, 1))


def _torch():
    import torch

    return torch


PAR = ParityLeg(False)


def oracle_mod(name):
    """An oracle module (the CPU leg's checker)."""
    import importlib

    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    return importlib.import_module(f"oracle.{name}")


class _DevRows:
    """[E, ...] device tensor read one expert at a time (the oracle indexes
    w[e])."""

    def __init__(self, t):
        self.t, self.shape = t, tuple(t.shape)

    def __getitem__(self, e):
        return self.t[int(e)].cpu().numpy()


# ------------------------------------------------------------------ CPU baseline


def cpu_baseline():
    """The CPU oracle on a bounded sample of the headline workload: FP8 W8A8
    per-channel, K=4096, N=14336, M=256 (dynamic per-token quant + fp32
    dequantize-then-matmul), at least 5 repetitions and up to about 10 s;
    the median repetition gives `value`. `cores` is the BLAS thread count
    numpy ran with (threadpoolctl), beside os.cpu_count() and
    torch.get_num_threads()."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import codecs, linear, quant

    rng = np.random.default_rng(0)
    K, N, M = 4096, 14336, 256
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, ws = quant.quantize_tensor(w, "fp8")
    x = codecs.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    linear.w8a8_per_channel(x, wq, ws, "fp8")  # warm-up
    times, t_start = [], time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < 10.0 and len(times) < 60):
        t0 = time.perf_counter()
        linear.w8a8_per_channel(x, wq, ws, "fp8")
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    blas_threads = None
    try:
        from threadpoolctl import threadpool_info

        blas = [i["num_threads"] for i in threadpool_info() if i.get("user_api") == "blas"]
        blas_threads = max(blas) if blas else None
    except Exception:  # threadpoolctl absent or unreadable: report os.cpu_count()
        blas_threads = None
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    cores = blas_threads or os.cpu_count() or 1
    return dict(value=round(2.0 * M * N * K / dt / 1e12, 4), unit="TFLOP/s", cores=cores,
                kind="port", sample=f"fp8 w8a8 per-channel M={M} K={K} N={N}: median of {len(times)} reps, "
                f"{dt * 1e3:.1f} ms each (p10 {np.percentile(times, 10) * 1e3:.1f}, p90 "
                f"{np.percentile(times, 90) * 1e3:.1f}), numpy fp32 BLAS with {cores} threads; "
                f"os.cpu_count() {os.cpu_count()}, torch.get_num_threads() {torch.get_num_threads()}; {cpu_model}")


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
    MXFP4) and cfg 4 (DeepSeek-V3 routed experts, 128x128 FP8), then 20 of
    cfg 4's fused decode op (routing inside its first launch, shared and
    routed experts), after 3 warm-up layers each."""
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
    # the fused decode op (shared expert + routed experts) on the same layer
    from qmoe import ops

    sh13, ss13 = fp8_weights(2 * I, H, gen, tiles=True)
    sh2, ss2 = fp8_weights(H, I, gen, tiles=True)
    for _ in range(23):
        ops.moe_decode_routed(x, logits, k, w13, w2, s13, s2, sh13, ss13, sh2, ss2, None, scoring_func="sigmoid",
                              renormalize=True, bias=bias, routed_scaling_factor=1.0, num_expert_group=8,
                              topk_group=4, routed_scale=2.5, weight_blocks=128)
    torch.cuda.synchronize()
    log("profile target done: cfg3 / cfg4 MoE T=1 x23 each, cfg4 decode op T=1 x23")


def vendor_scaled_mm(xq, wq, xs, ws):
    """hipBLASLt's FP8 GEMM through torch._scaled_mm on the same codes: row-wise
    scales ([M,1] x [1,N]) when this torch build takes them, else unit tensor
    scales. Returns (callable, scaling)."""
    import torch

    b = wq.t()  # [K, N] column-major view of the N-major weight
    out = torch.empty((xq.shape[0], wq.shape[0]), dtype=torch.bfloat16, device=xq.device)
    try:
        sa, sb = xs.reshape(-1, 1).float().contiguous(), ws.reshape(1, -1).float().contiguous()
        torch._scaled_mm(xq, b, sa, sb, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        return (lambda: torch._scaled_mm(xq, b, sa, sb, out_dtype=torch.bfloat16)), "rowwise"
    except (RuntimeError, ValueError):
        one = torch.ones((), dtype=torch.float32, device=xq.device)
        torch._scaled_mm(xq, b, one, one, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        return (lambda: torch._scaled_mm(xq, b, one, one, out_dtype=torch.bfloat16)), "tensorwise (unit)"
    finally:
        del out


def profile_vendor(args):
    """rocprofv3 target: 10 launches each of this build's tiled FP8 GEMM and
    of hipBLASLt's FP8 GEMM (torch._scaled_mm) on the two cfg 1 shapes at
    M=args.m (up K4096 N14336, down K14336 N4096), same codes, after 3
    warm-up calls; then a plain 256 MiB copy (10 launches) for the
    FETCH_SIZE / WRITE_SIZE calibration."""
    import torch

    from qmoe import _capi, ops

    gen = torch.Generator(device="cuda").manual_seed(0)
    M = args.m
    for K, N in ((4096, 14336), (14336, 4096)):
        w, s = fp8_weights(N, K, gen)
        x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
        xq, xs = ops.row_quant(x, "fp8")
        ours = lambda: ops.gemm(_capi.W8A8_PC, xq.view(torch.uint8), w.view(torch.uint8),  # noqa: E731
                                a_scale=xs, w_scale=s)
        vend, scaling = vendor_scaled_mm(xq, w, xs, s)
        for fn in (ours, vend):
            for _ in range(13):
                fn()
            torch.cuda.synchronize()
        log(f"profile target: K={K} N={N} M={M}: qmoe tiled FP8 x13, torch._scaled_mm ({scaling}) x13")
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("profile target done: copy 256MiB x10")


FLOOR_MB = (1, 2, 4, 8.8, 16, 32, 58.7, 128, 176, 352, 1024)


def read_floor():
    """Plain-read floor: `qmoe_stream_read` over buffers of FLOOR_MB
    megabytes, each timed like the sweep points (graph replays, so the
    launch gap inside a graph is included). Returns [{mb, us, gbs}]."""
    import torch

    from qmoe import ops

    big = torch.empty(int(max(FLOOR_MB) * 1e6) // 16 * 16, dtype=torch.uint8, device="cuda")
    big.random_(0, 255)
    sink = torch.empty(2048, dtype=torch.int32, device="cuda")
    out = []
    for mb in FLOOR_MB:
        n = int(mb * 1e6) // 16 * 16
        view = big[:n]
        us = graph_time_us(lambda: ops.stream_read(view, sink=sink), iters=30)[0]
        out.append(dict(mb=mb, us=round(us, 2), gbs=round(n / us / 1e3, 1)))
        log("read floor", out[-1])
    del big
    return out


def floor_us(floor, nbytes):
    """Plain-read time of `nbytes` interpolated (linear in bytes) on the
    measured floor curve."""
    pts = [(p["mb"] * 1e6, p["us"]) for p in floor]
    if nbytes <= pts[0][0]:
        return pts[0][1]
    for (b0, t0), (b1, t1) in zip(pts, pts[1:]):
        if nbytes <= b1:
            return t0 + (t1 - t0) * (nbytes - b0) / (b1 - b0)
    (b0, t0), (b1, t1) = pts[-2], pts[-1]
    return t1 + (t1 - t0) * (nbytes - b1) / (b1 - b0)


def profile_w4(args):
    """rocprofv3 target: the large-M MXFP4 (W4A16) path -- 8 launches of the
    dense cfg 0 linear at M=8192 (K 2880, N 5760) and 8 cfg 3 GPT-OSS MoE
    layers at T=8192 (128 experts, top-4, swigluoai), after 2 warm-up calls
    each; then a plain 256 MiB copy (10 launches) for the FETCH_SIZE /
    WRITE_SIZE calibration."""
    import torch

    from qmoe.layers.fused_moe import moe_forward
    from qmoe.layers.linear_common import quantized_matmul_fp4

    gen = torch.Generator(device="cuda").manual_seed(3)
    K, N, M = 2880, 5760, 8192
    codes, sc = mxfp4_weights((N, K), gen)
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    for _ in range(10):
        quantized_matmul_fp4(x, codes, sc)
    torch.cuda.synchronize()
    log("profile target: cfg0 MXFP4 M=8192 x10")
    E, k, H, I, T = 128, 4, 2880, 2880, 8192
    w13, s13 = mxfp4_weights((E, 2 * I, H), gen)
    w2, s2 = mxfp4_weights((E, H, I), gen)
    x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
    logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)
    lcfg = moe_layer_cfg(k, "softmax", "swigluoai")
    for _ in range(10):
        moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "mxfp4")
    torch.cuda.synchronize()
    log("profile target: cfg3 MoE T=8192 x10")
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("profile target done: copy 256MiB x10")


def profile_mx(args):
    """rocprofv3 target: the opt-in MX activation path at config 0's shape,
    M=8192 (K 2880 padded to 3072, N 5760): 10 activation quantizations
    and 10 MX GEMMs after 2 warm-up calls each; 10 config 3 GPT-OSS MoE
    layers at T=8192 with MX activations (experts padded to K 3072); then a
    plain 256 MiB copy (10 launches) for the FETCH_SIZE / WRITE_SIZE
    calibration."""
    import torch

    from qmoe import _capi, ops
    from qmoe.layers.linear_common import pad_mxfp4_for_mx

    gen = torch.Generator(device="cuda").manual_seed(3)
    K, N, M = 2880, 5760, 8192
    codes, sc = mxfp4_weights((N, K), gen)
    wp, wsp = pad_mxfp4_for_mx(codes, sc)
    kp = wp.shape[1] * 2
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    for _ in range(12):
        q, s = ops.mx_quant(x, k_pad=kp)
    for _ in range(12):
        ops.gemm(_capi.W4A4_MX, q, wp, a_scale=s, w_scale=wsp)
    torch.cuda.synchronize()
    log("profile target: cfg0 MX W4A4 M=8192 quant x12, gemm x12")
    from qmoe.layers.fused_moe import moe_forward
    from qmoe.layers.quantization.mxfp4 import _pad_experts_for_mx

    E, k, H, I, T = 128, 4, 2880, 2880, 8192
    w13, s13 = _pad_experts_for_mx(*mxfp4_weights((E, 2 * I, H), gen))
    w2, s2 = _pad_experts_for_mx(*mxfp4_weights((E, H, I), gen))
    x = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
    logits = torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16)
    lcfg = moe_layer_cfg(k, "softmax", "swigluoai")
    for _ in range(10):
        moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "mxfp4_mx")
    torch.cuda.synchronize()
    log("profile target: cfg3 MoE T=8192 with MX activations x10")
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("profile target done: copy 256MiB x10")


def profile_midm(args):
    """rocprofv3 target: the small- and mid-M linears, 23 launches each --
    cfg 0 MXFP4 at M=1, 16 and 128, cfg 1 FP8 W8A8 up / down at M=64 and 512
    (activation quant included), cfg 2 block FP8 (N 18432) at M=256."""
    import torch

    from qmoe.layers.linear_common import quantized_matmul, quantized_matmul_fp4

    gen = torch.Generator(device="cuda").manual_seed(1)
    codes, sc = mxfp4_weights((5760, 2880), gen)
    calls = []
    for M in (1, 16, 128):
        x0 = torch.randn((M, 2880), device="cuda", generator=gen).to(torch.bfloat16)
        calls.append((f"cfg0 M={M}", lambda x0=x0: quantized_matmul_fp4(x0, codes, sc)))
    for K, N in ((4096, 14336), (14336, 4096)):
        w, s = fp8_weights(N, K, gen)
        for M in (64, 512):
            x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
            calls.append((f"cfg1 K={K} M={M}", lambda x=x, w=w, s=s: quantized_matmul(x, w.t(), s)))
    w2, s2 = fp8_weights(18432, 7168, gen, tiles=True)
    x2 = torch.randn((256, 7168), device="cuda", generator=gen).to(torch.bfloat16)
    calls.append(("cfg2 M=256", lambda: quantized_matmul(x2, w2.t(), s2)))
    for name, fn in calls:
        for _ in range(23):
            fn()
        torch.cuda.synchronize()
        log(f"profile target: {name} x23")
    log("profile target done")


def profile_dec6(args):
    """rocprofv3 target: config 6's linears at 4096 tokens, 13 launches each
    after 3 warm-up calls -- DeepSeek-V3 q_a / kv_a / q_b / kv_b / o and
    Llama-3-8B qkv / o through `quantized_matmul` (activation quant
    included), and the bf16 router gate; then a plain 256 MiB copy (10
    launches) for the FETCH_SIZE / WRITE_SIZE calibration."""
    import torch

    from qmoe import _capi, ops
    from qmoe.layers.linear_common import quantized_matmul

    gen = torch.Generator(device="cuda").manual_seed(6)
    M = 4096
    for name, N, K in (("dsv3_q_a", 1536, 7168), ("dsv3_kv_a", 576, 7168), ("dsv3_q_b", 24576, 1536),
                       ("dsv3_kv_b", 32768, 512), ("dsv3_o", 7168, 16384), ("llama3_qkv", 6144, 4096),
                       ("llama3_o", 4096, 4096)):
        w, s = fp8_weights(N, K, gen)
        x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
        for _ in range(3):
            quantized_matmul(x, w.t(), s)
        torch.cuda.synchronize()
        log(f"profile target: {name} warm-up x3")
        for _ in range(13):
            quantized_matmul(x, w.t(), s)
        torch.cuda.synchronize()
        log(f"profile target: {name} M={M} K={K} N={N} x13")
        del w, s, x
    wg = (torch.randn((256, 7168), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn((M, 7168), device="cuda", generator=gen).to(torch.bfloat16)
    for _ in range(3):
        ops.gemm(_capi.W16A16, x, wg)
    torch.cuda.synchronize()
    for _ in range(13):
        ops.gemm(_capi.W16A16, x, wg)
    torch.cuda.synchronize()
    log(f"profile target: bf16 router gate M={M} K=7168 N=256 x13 (after 3 warm-up)")
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("profile target done: copy 256MiB x10")


def profile_moet(args):
    """rocprofv3 target: config 4 (DeepSeek-V3, 256 experts, top-8 grouped)
    routed MoE layers at T = 512 and 4096 -- 6 layers each with the native
    128 x 128 FP8 tiles (format fp8_block), then 6 each through the method's
    default recipe (per-channel e4m3 experts, per-(token, 512) activation
    codes, format fp8) -- after 2 warm-up layers each; then a plain 256 MiB
    copy (10 launches) for the FETCH_SIZE / WRITE_SIZE calibration."""
    import torch

    from qmoe.layers.fused_moe import moe_forward
    from qmoe.layers.quantization.fp8 import dequantize_fp8_weight, requantize

    gen = torch.Generator(device="cuda").manual_seed(4)
    E, k, H, I = 256, 8, 7168, 2048
    w13 = torch.empty((E, 2 * I, H), device="cuda", dtype=torch.float8_e4m3fn)
    s13 = torch.empty((E, 2 * I // 128, H // 128), device="cuda", dtype=torch.float32)
    w2 = torch.empty((E, H, I), device="cuda", dtype=torch.float8_e4m3fn)
    s2 = torch.empty((E, H // 128, I // 128), device="cuda", dtype=torch.float32)
    for e in range(E):
        w13[e], s13[e] = fp8_weights(2 * I, H, gen, tiles=True)
        w2[e], s2[e] = fp8_weights(H, I, gen, tiles=True)
    bias = torch.randn(E, device="cuda", generator=gen) * 0.1
    lcfg = moe_layer_cfg(k, "sigmoid", "silu", bias=bias, rsf=2.5, groups=(8, 4))
    inputs = {}
    for T in (512, 4096):
        inputs[T] = (torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16),
                     torch.randn((T, E), device="cuda", generator=gen).to(torch.bfloat16))
    from qmoe import ops

    for T, (x, logits) in inputs.items():
        for _ in range(8):
            moe_forward(lcfg, x, logits, w13, w2, s13, s2, None, None, "fp8_block")
        torch.cuda.synchronize()
        _, ids = ops.moe_route(logits, k, "sigmoid", True, bias=bias, routed_scaling_factor=2.5, num_expert_group=8,
                               topk_group=4)
        log(f"profile target: cfg4 fp8_block T={T} x8, {int(torch.unique(ids).numel())} experts routed")

    def per_channel(w, s):
        q = torch.empty(w.shape, dtype=torch.float8_e4m3fn, device=w.device)
        sc = torch.empty(w.shape[:-1], dtype=torch.float32, device=w.device)
        for e in range(w.shape[0]):
            q[e], sc[e] = requantize(dequantize_fp8_weight(w[e], weight_scale_inv=s[e], block=(128, 128)),
                                     "float8_e4m3fn")
        return q, sc

    q13, c13 = per_channel(w13, s13)
    del w13, s13
    q2, c2 = per_channel(w2, s2)
    del w2, s2
    for T, (x, logits) in inputs.items():
        for _ in range(8):
            moe_forward(lcfg, x, logits, q13, q2, c13, c2, None, None, "fp8")
        torch.cuda.synchronize()
        log(f"profile target: cfg4 fp8 default recipe T={T} x8")
    del q13, q2
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("profile target done: copy 256MiB x10")


def profile_floor(args):
    """rocprofv3 target: the plain-read floor curve (qmoe_stream_read over
    FLOOR_MB sizes), printed as one JSON line."""
    print(json.dumps({"read_floor": read_floor()}))


def main():
    args = parse()
    if args.profile:
        {"headline": profile_target, "decode": profile_decode, "moe": profile_moe, "vendor": profile_vendor,
         "floor": profile_floor, "w4": profile_w4, "mx": profile_mx, "midm": profile_midm, "dec6": profile_dec6,
         "moet": profile_moet}[args.profile](args)
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
    PAR.on = not args.no_cpu
    full = dict(res)
    if not args.no_sweep:
        FLOOR.extend(read_floor())
        full["read_floor"] = FLOOR
        full["sweep"] = sweep_linear(only) + sweep_moe(only) + sweep_nvfp4(only) + sweep_decoder(only)
        if not only or "v" in only:
            full["sweep"] += sweep_vendor()
        res["sweep_summary"] = compact_sweep(full["sweep"])
    if not args.no_cpu:
        res["cpu_baseline"] = full["cpu_baseline"] = cpu_baseline()
    if not args.no_sweep:
        res["sweep_file"] = write_sweep_file(full, args.sweep_out)
    line = json.dumps(res, separators=(",", ":"))
    # the driver keeps the last 16 KB of stdout: the headline must fit whole
    assert len(line) < 12000, f"headline line is {len(line)} bytes"
    print(line, flush=True)


def compact_sweep(sweep):
    """The sweep as the headline line carries it: per (config, kind, shape)
    a list of [M or T, us, roofline fraction, parity ok] rows, and per config
    the worst and best roofline fraction. The full points (GB/s, TFLOP/s,
    floor fractions, parity statistics, CPU estimates) are in the sweep
    file."""
    series, worst = {}, {}
    for p in sweep:
        key = f"cfg{p['cfg']} {p['kind']}" + (f" K{p['K']} N{p['N']}" if "K" in p else "")
        par = p.get("parity")
        row = [p.get("M", p.get("T")), p["us"], p["roofline_frac"], par.get("ok") if par else None]
        series.setdefault(key, []).append(row)
        if p["kind"].startswith("hipblaslt"):
            continue  # vendor reference points: not this build's kernels
        c = f"cfg{p['cfg']}"
        lo, hi = worst.get(c, (None, None))
        lo = p if lo is None or p["roofline_frac"] < lo["roofline_frac"] else lo
        hi = p if hi is None or p["roofline_frac"] > hi["roofline_frac"] else hi
        worst[c] = (lo, hi)

    def name(p):
        return f"{p['kind']} {'M' if 'M' in p else 'T'}={p.get('M', p.get('T'))}"

    per_cfg = {c: {"worst": [name(lo), lo["roofline_frac"], lo["bound"]],
                   "best": [name(hi), hi["roofline_frac"], hi["bound"]]} for c, (lo, hi) in worst.items()}
    checked = [p["parity"]["ok"] for p in sweep if p.get("parity")]
    return {"columns": ["M|T", "us", "roofline_frac", "parity_ok"], "series": series, "per_cfg": per_cfg,
            "parity_points": len(checked), "parity_all_ok": all(checked) if checked else None}


def write_sweep_file(full, path):
    """Every sweep point, the read floor and the per-point parity objects as
    one JSON document (relative paths are under the repository root).
    Returns the path written, or None when it cannot be written."""
    p = path if os.path.isabs(path) else os.path.join(ROOT, path)
    try:
        os.makedirs(os.path.dirname(p), exist_ok=True)
        with open(p, "w") as f:
            json.dump(full, f, indent=1)
    except OSError as e:
        log(f"bench.py: sweep file not written ({e})")
        return None
    return os.path.relpath(p, ROOT)


if __name__ == "__main__":
    main()
