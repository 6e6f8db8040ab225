"""Benchmark of the awq_inference_engine hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one ViT-L MLP pair of the VGGT aggregator at M = 8 x 1374 = 10992
tokens (BASELINE config 2a): W4A16 g128 fc1 1024->4096 with bias + GELU fused,
then W4A16 fc2 4096->1024 with bias, synthetic seeded inputs already resident
in HBM.  value = W4 GEMM TFLOP/s over the timed steps (2*M*N*K per GEMM).

Prints ONE JSON line on stdout; extra diagnostics go to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "W4 GEMM TFLOP/s & % MFMA peak; VGGT aggregator frames/s at S=32 (1 GPU)"
PEAK_FP16_TFLOPS = 2500.0      # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 0) for i in threadpool_info() if i.get("user_api") == "blas"]
        if n:
            return int(max(n))
    except Exception:
        pass
    return os.cpu_count() or 1


def synthetic_w4(M: int, K: int, N: int, seed: int, dev, group: int = 128):
    """Seeded synthetic W4A16 linear in the reference's buffer layout: x ~ N(0,1)
    fp16, qweight uniformly random int16 words (every int4 weight U{0..15}),
    fp16 scales U[0.005, 0.02], integer zeros U{0..15} -> scaled_zeros =
    -(s * z), group tables zero-padded to calculate_zeros_width(K) * 8 rows."""
    import torch

    from qvggt_amd.awq.qmodule import calculate_zeros_width

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).half() if M else None
    qw = torch.randint(-32768, 32768, (N // 4, K), generator=g, dtype=torch.int32).to(torch.int16)
    rows, G = calculate_zeros_width(K, group) * 8, K // group
    s = (torch.rand(G, N, generator=g) * 0.015 + 0.005).half()
    z = torch.randint(0, 16, (G, N), generator=g).float()
    scales = torch.zeros(rows, N, dtype=torch.float16)
    szeros = torch.zeros(rows, N, dtype=torch.float16)
    scales[:G] = s
    szeros[:G] = (-(s.float() * z)).half()
    to = (lambda t: t.to(dev) if t is not None else None)
    return to(x), to(qw), to(scales), to(szeros)


def cpu_baseline_mlp(x, w1, b1, w2, b2, y, M_sample: int = 2748, reps: int = 5):
    """CPU leg: the oracle (numpy dequantisation + fp32 matmul + erf-GELU) of
    fc1 -> GELU -> fc2 on the first M_sample tokens of the benchmark's own
    inputs (two frames, about 10 s of host work), timed on the host.  Also the
    checker: the GPU's timed output y on those tokens is compared with it.
    Returns (baseline dict, max|y - y_ref| / max|y_ref|)."""
    import numpy as np
    from math import sqrt

    from oracle import awq as O
    from scipy.special import erf

    xs = x[:M_sample].cpu().numpy()
    t1 = [t.cpu().numpy() for t in w1]
    t2 = [t.cpu().numpy() for t in w2]
    bb1, bb2 = b1.float().cpu().numpy(), b2.float().cpu().numpy()
    H, D = t1[0].shape[0] * 4, t1[0].shape[1]
    times = []
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        W1 = O.dequantize(t1[0], t1[1], t1[2], H, D).astype(np.float32)
        W2 = O.dequantize(t2[0], t2[1], t2[2], D, H).astype(np.float32)
        h = xs.astype(np.float32) @ W1.T + bb1
        h = 0.5 * h * (1.0 + erf(h / sqrt(2.0)))
        yr = h.astype(np.float16).astype(np.float32) @ W2.T + bb2
        times.append(time.perf_counter() - t0)
    t = sorted(times[1:])[len(times[1:]) // 2]
    flops = 2 * 2 * M_sample * D * H
    err = O.rel_err(y[:M_sample].float().cpu().numpy(), yr)
    return dict(value=flops / t / 1e12, unit="TFLOP/s", cores=blas_threads(), kind="port",
                sample=f"{M_sample // 1374} frames (M={M_sample}) of the benchmark's MLP pair: oracle numpy "
                       f"dequant + fp32 matmul + erf-GELU, median of {reps} after 1 warm-up, {t:.3f} s each; "
                       f"CPU: {cpu_model()}"), err


def aggregator_fps(dev, S: int = 32, reps: int = 3, w8a8: bool = False):
    """VGGT-1B aggregator (W4A16 g128 or W8A8 AA blocks, fp16 DINOv2-L/14-reg
    patch embed, seeded random-init weights) on S synthetic 518x518 frames
    U[0,1]: frames/s."""
    import torch

    from qvggt_amd import aggregator as AG

    agg = AG.Aggregator.random(w8a8=w8a8, seed=0, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    img = torch.rand(S, 3, AG.IMG, AG.IMG, generator=g, device=dev).half()
    agg(img)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        out, _ = agg(img)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    ok = bool(torch.isfinite(out.float()).all().item())
    del agg, out
    torch.cuda.empty_cache()
    return {"S": S, "frames_per_s": round(S / ms * 1e3, 2), "ms_per_forward": round(ms, 2), "reps": reps,
            "variant": ("W8A8 (per-token int8 activations, per-channel int8 weights)" if w8a8 else "W4A16 g128")
                       + " frame/global blocks (24+24), fp16 DINOv2-L/14-reg patch embed",
            "data": "seeded random-init weights, images U[0,1]", "finite": ok,
            "flop_per_forward": 2.816e14}


def _time_graph(fn, calls: int, reps: int = 3):
    """Capture `calls` invocations of fn(i) in one HIP graph, replay, return us per call.
    The graph is captured on the stream that ran the warm-up calls, so the ops'
    per-stream split-K workspaces already exist when capture starts."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(min(calls, 4)):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(calls):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * calls)


def kernel_suite(dev):
    """Per-kernel throughput at the benchmark shapes, HBM-bound kernels cold
    (every call touches a different buffer set; the sets span >= 1 GiB, beyond
    the 256 MiB Infinity Cache), launches replayed from a HIP graph."""
    import numpy as np
    import torch

    from qvggt_amd import awq_inference_engine as E

    r = {}
    f16 = dict(dtype=torch.float16, device=dev)
    # config 1: one W4A16 qkv linear on one frame (M = 1374, 1024 -> 3072, + bias)
    xq, qwq, sq, zq = synthetic_w4(1374, 1024, 3072, seed=3, dev=dev)
    bq_ = torch.zeros(3072, **f16)
    oq = torch.empty(1374, 3072, **f16)
    us = _time_graph(lambda i: E.w4a16_linear(xq, qwq, sq, zq, bias=bq_, epilogue=1, out=oq), 50)
    r["w4a16_qkv_M1374"] = {"us": round(us, 2), "TFLOP/s": round(2.0 * 1374 * 3072 * 1024 / us / 1e6, 1)}
    del xq, qwq, sq, zq, oq
    # configs 3 and 4: one W4A16 frame block at S = 8 and one global block at
    # S = 32 (LN, qkv, qk-norm + 2-D RoPE, attention, proj, LN, fc1 + GELU, fc2)
    from qvggt_amd import aggregator as AG
    agg1 = AG.Aggregator.random(w8a8=False, seed=4, device=dev, depth=1)
    tables = E.rope2d_tables(AG.GRID + 1, 100.0, device=dev)
    for name, S, blk, glob in (("frame_block_S8", 8, agg1.frame_blocks[0], False),
                               ("global_block_S32", 32, agg1.global_blocks[0], True)):
        Mb = S * AG.TOKENS
        xb = torch.randn(Mb, AG.DIM, **f16)
        ws = agg1._workspace(Mb, dev)
        posb = AG.vggt_positions(S, dev)
        us = _time_graph(lambda i: blk(xb, Mb if glob else AG.TOKENS, posb, tables, ws), 2 if glob else 10)
        r[name] = {"us": round(us, 1), "tokens": Mb}
        del xb
    del agg1
    agg1 = None
    M, D = 32 * 1374, 1024                                     # S = 32 tokens
    nb = 6                                                     # 6 x 180 MB rotating sets
    xs = [torch.randn(M, D, **f16) for _ in range(nb)]
    ys = [torch.empty(M, D, **f16) for _ in range(nb)]
    g, b = torch.ones(D, **f16), torch.zeros(D, **f16)
    us = _time_graph(lambda i: E.layer_norm(xs[i % nb], g, b, 1e-6, out=ys[i % nb]), 12)
    r["layernorm_S32"] = {"us": round(us, 1), "GB/s": round(4 * M * D / us / 1e3, 1)}
    q8 = [torch.empty(M, D, dtype=torch.int8, device=dev) for _ in range(nb)]
    sc = [torch.empty(M, **f16) for _ in range(nb)]
    us = _time_graph(lambda i: E.invoke_quant(q8[i % nb], xs[i % nb], sc[i % nb]), 12)
    r["quant_S32"] = {"us": round(us, 1), "GB/s": round((3 * M * D + 2 * M) / us / 1e3, 1)}
    us = _time_graph(lambda i: E.rms_norm_general(q8[i % nb], xs[i % nb], g, b, sc[i % nb], 1e-6, True), 12)
    r["layernorm_quant_S32"] = {"us": round(us, 1), "GB/s": round((3 * M * D + 2 * M) / us / 1e3, 1)}
    del ys, q8
    # W8A8 MLP hidden: GELU + per-token quant at M = 10992, D = 4096 (reads x,
    # writes int8 + the fp16 GELU copy + scales), 4 rotating sets of 450 MB
    Mh, Dh = 8 * 1374, 4096
    hx = [torch.randn(Mh, Dh, **f16) for _ in range(4)]
    hq = [torch.empty(Mh, Dh, dtype=torch.int8, device=dev) for _ in range(4)]
    ht = [torch.empty(Mh, Dh, **f16) for _ in range(4)]
    hs = torch.empty(Mh, **f16)
    us = _time_graph(lambda i: E.gelu_and_quant(hq[i % 4], hx[i % 4], hs, ht[i % 4]), 8)
    r["gelu_quant_M10992x4096"] = {"us": round(us, 1), "GB/s": round((5 * Mh * Dh + 2 * Mh) / us / 1e3, 1)}
    del hx, hq, ht
    qkv = [torch.randn(M, 3 * D, **f16) for _ in range(4)]    # 4 x 270 MB
    pos = torch.from_numpy(np.tile(np.array([[0, 0]] * 5 + [[i // 37 + 1, i % 37 + 1] for i in range(1369)],
                                             np.int32), (32, 1))).to(dev)
    ct, st = E.rope2d_tables(38, device=dev)
    us = _time_graph(lambda i: E.rope2d(qkv[i % 4], pos, ct, st, 16, out=qkv[i % 4]), 8)
    r["rope2d_S32"] = {"us": round(us, 1), "GB/s": round(8 * M * D / us / 1e3, 1)}
    gq = torch.ones(64, **f16)
    bq = torch.zeros(64, **f16)
    us = _time_graph(lambda i: E.qknorm_rope2d(qkv[i % 4], pos, ct, st, 16, gq, bq, gq, bq), 8)
    r["qknorm_rope2d_S32"] = {"us": round(us, 1), "GB/s": round(8 * M * D / us / 1e3, 1)}
    del qkv, xs
    # skinny M (the GEMV entry): aggregator qkv 1024 -> 3072 and the camera-head
    # fc1 / fc2 shapes, weights cold (rotating sets of ~1 GiB)
    for K, N in ((1024, 3072), (2048, 8192), (8192, 2048)):
        wbytes = N * K // 2
        nw = max(16, (1 << 30) // wbytes)
        _, qw0, scl, szs = synthetic_w4(0, K, N, seed=0, dev=dev)
        qw = [qw0.clone() for _ in range(nw)]
        for m in (1, 8, 32):
            x = torch.randn(m, K, **f16)
            out = torch.empty(m, N, **f16)
            us = _time_graph(lambda i: E.w4a16_linear(x, qw[i % nw], scl, szs, out=out), nw)
            byts = wbytes + 4 * (K // 128) * N + 2 * m * K + 2 * m * N
            r[f"w4_skinny_M{m}_{K}x{N}"] = {"us": round(us, 2), "GB/s": round(byts / us / 1e3, 1)}
        del qw
    # attention (MFMA-bound): frame S=8 and global S=32
    for name, Bq, L in (("attention_frame_S8", 8, 1374), ("attention_global_S32", 1, 32 * 1374)):
        qk = torch.randn(Bq * L, 3, 16, 64, **f16)
        o = torch.empty(Bq * L, 16, 64, **f16)
        us = _time_graph(lambda i: E.attention(qk[:, 0], qk[:, 1], qk[:, 2], L, out=o), 2, reps=2)
        r[name] = {"us": round(us, 1), "TFLOP/s": round(4.0 * Bq * 16 * L * L * 64 / us / 1e6, 1)}
        del qk, o
    # W8A8 GEMM (int8 MFMA), fc1 shape at M = 10992
    a = torch.randint(-128, 128, (10992, 1024), dtype=torch.int8, device=dev)
    w = torch.randint(-128, 128, (4096, 1024), dtype=torch.int8, device=dev)
    ws_, as_ = torch.rand(4096, **f16) * 0.01, torch.rand(10992, **f16) * 0.01
    o = torch.empty(10992, 4096, **f16)
    us = _time_graph(lambda i: E.w8a8_gemm_forward_cuda(a, w, ws_, as_, o), 10)
    r["w8a8_fc1_M10992"] = {"us": round(us, 1), "TOPS": round(2.0 * 10992 * 4096 * 1024 / us / 1e6, 1)}
    # W8A8 MLP pair (W8A8 variant): fc1 + bias, GELU + per-token
    # quant of the hidden activations, fc2 + bias
    x8 = torch.randint(-128, 128, (10992, 1024), dtype=torch.int8, device=dev)
    s8 = torch.rand(10992, **f16) * 0.01
    w2 = torch.randint(-128, 128, (1024, 4096), dtype=torch.int8, device=dev)
    ws2 = torch.rand(1024, **f16) * 0.01
    b1, b2 = torch.zeros(4096, **f16), torch.zeros(1024, **f16)
    hq = torch.empty(10992, 4096, dtype=torch.int8, device=dev)
    hs, ht = torch.empty(10992, **f16), torch.empty(10992, 4096, **f16)
    y8 = torch.empty(10992, 1024, **f16)

    def w8_pair(i):
        E.w8a8_gemm_fuse_bias_forward_cuda(x8, w, ws_, s8, o, b1)
        E.gelu_and_quant(hq, o, hs, ht)
        E.w8a8_gemm_fuse_bias_forward_cuda(hq, w2, ws2, hs, y8, b2)

    us = _time_graph(w8_pair, 5)
    r["w8a8_mlp_pair_M10992"] = {"us": round(us, 1), "TOPS": round(2 * 2.0 * 10992 * 4096 * 1024 / us / 1e6, 1)}
    return r


def camera_head_ms(dev, S=32, reps=50):
    """VGGT camera head (W4 trunk, 4 iterations) on S pose tokens, replayed from
    one HIP graph: wall ms per forward."""
    import torch

    from qvggt_amd.camera_head import CameraHead, GraphedCameraHead

    head = GraphedCameraHead(CameraHead.random(seed=0, device=dev), S)
    t = torch.randn(S, 2048, device=dev).half()
    for _ in range(5):
        head(t)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        head(t)
    torch.cuda.synchronize()
    return {"S": S, "ms_per_forward": round((time.perf_counter() - t0) * 1e3 / reps, 3), "graph": True}


def profiled_traffic():
    """HBM bytes per launch of the fc1 kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated); None if absent."""
    p = ROOT / "profiles" / "w4a16_stream32_fc1_M10992_traffic.txt"
    try:
        for line in p.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1])), str(p.relative_to(ROOT))
    except OSError:
        pass
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prewarm-s", type=float, default=1.0,
                    help="seconds of untimed steps before the warm-up steps (clock ramp)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-aggregator", action="store_true")
    ap.add_argument("--no-kernel-suite", action="store_true")
    ap.add_argument("--no-camera-head", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path is measured on one GPU's share of the work, and sharding across GPUs "
              "is not implemented", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS, QV_EPI_BIAS_GELU

    dev = torch.device("cuda:0")
    M = 8 * 1374
    D, H = 1024, 4096
    x, *w1 = synthetic_w4(M, D, H, seed=0, dev=dev)
    _, *w2 = synthetic_w4(0, H, D, seed=10, dev=dev)
    b1 = torch.from_numpy((np.random.default_rng(5).standard_normal(H) * 0.1).astype(np.float16)).to(dev)
    b2 = torch.from_numpy((np.random.default_rng(6).standard_normal(D) * 0.1).astype(np.float16)).to(dev)
    h = torch.empty(M, H, dtype=torch.float16, device=dev)
    y = torch.empty(M, D, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step(evs=None):
        if evs is not None:
            evs[0].record(stream)
        E.w4a16_linear(x, *w1, bias=b1, epilogue=QV_EPI_BIAS_GELU, out=h)
        if evs is not None:
            evs[1].record(stream)
        E.w4a16_linear(h, *w2, bias=b2, epilogue=QV_EPI_BIAS, out=y)
        if evs is not None:
            evs[2].record(stream)

    # Untimed: first bring the GPU to its sustained clock (an idle MI355X takes
    # a few hundred ms of load to get there), then the W warm-up steps.
    t_end = time.perf_counter() + args.prewarm_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    fc1_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    fc2_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    ms_per_step = wall * 1e3 / args.steps
    flop_gemm = 2.0 * M * D * H
    value = 2 * flop_gemm / (ms_per_step / 1e3) / 1e12
    fc1_tflops = flop_gemm / (fc1_ms / 1e3) / 1e12
    fc2_tflops = flop_gemm / (fc2_ms / 1e3) / 1e12
    log(f"[bench] MLP pair M={M}: {ms_per_step:.4f} ms/step, {value:.1f} TFLOP/s; "
        f"fc1 {fc1_ms * 1e3:.1f} us ({fc1_tflops:.1f} TFLOP/s), fc2 {fc2_ms * 1e3:.1f} us ({fc2_tflops:.1f} TFLOP/s)")

    kernels = None
    if not args.no_kernel_suite:
        kernels = kernel_suite(dev)
        for k, v in kernels.items():
            log(f"[bench] {k}: {v}")

    agg = agg8 = None
    if not args.no_aggregator:
        agg = aggregator_fps(dev)
        log(f"[bench] aggregator S={agg['S']}: {agg['ms_per_forward']:.1f} ms/forward, "
            f"{agg['frames_per_s']:.1f} frames/s")
        agg8 = aggregator_fps(dev, w8a8=True)
        log(f"[bench] aggregator W8A8 S={agg8['S']}: {agg8['ms_per_forward']:.1f} ms/forward, "
            f"{agg8['frames_per_s']:.1f} frames/s")

    cam = None
    if not args.no_camera_head:
        cam = camera_head_ms(dev)
        log(f"[bench] camera head S={cam['S']} (HIP graph): {cam['ms_per_forward']:.3f} ms/forward")

    cpu, err = None, None
    if not args.no_cpu_baseline:
        cpu, err = cpu_baseline_mlp(x, w1, b1, w2, b2, y)
        log(f"[bench] cpu baseline: {cpu['value']:.4f} TFLOP/s ({cpu['sample']})")
        log(f"[bench] timed output vs oracle on the CPU sample: rel err {err:.3e}")
    traffic, traffic_src = profiled_traffic()

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded: x~N(0,1) fp16, int4 U{0..15} in AWQ-v2 int16 words, fp16 scales U[0.005,0.02], zeros U{0..15})",
        "config": {"workload": "W4A16 g128 ViT-L MLP pair fc1(1024->4096)+bias+GELU, fc2(4096->1024)+bias, "
                               "M=8x1374=10992 tokens (BASELINE config 2a)",
                   "M": M, "K_N": [[D, H], [H, D]], "group_size": 128,
                   "pct_fp16_mfma_peak": round(100 * value / PEAK_FP16_TFLOPS, 2),
                   "fc1_us": round(fc1_ms * 1e3, 2), "fc2_us": round(fc2_ms * 1e3, 2),
                   "rel_err_vs_oracle": err},
        "aggregator": agg,
        "aggregator_w8a8": agg8,
        "camera_head": cam,
        "kernels": kernels,
        "roofline": {"bound": "mfma", "achieved": round(fc1_tflops, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(fc1_tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": "w4a16_stream32_kernel (fc1 launch, 2*M*N*K = %.4g FLOP)" % flop_gemm},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
