"""Fixed workloads for rocprofv3 runs (kernel traces and PMC counters).

    python qvggt_amd/profiling.py copy                 # traffic calibration
    python qvggt_amd/profiling.py gemm M K N [--gelu] [--reps R]
    python qvggt_amd/profiling.py aggregator [--frames S] [--w8a8]
    python qvggt_amd/profiling.py attention [--frames S] [--global] [--reps R]
    python qvggt_amd/profiling.py camera [--frames S] [--reps R] [--graph]
    python qvggt_amd/profiling.py dense M K N [--bias | --int8]
    python qvggt_amd/profiling.py sdpa [--frames S] [--global]

``copy`` launches one elementwise kernel that reads 512 MiB and writes
512 MiB, three times: the FETCH_SIZE / WRITE_SIZE it reports per dispatch
calibrate those counters against known byte counts.  ``gemm`` runs the W4A16
linear (optionally with the fused bias + GELU epilogue) on seeded synthetic
data; ``aggregator`` runs the VGGT aggregator forward twice (the first call
warms up); ``attention`` runs frame (S sequences of 1374 tokens) or global
(one sequence of S x 1374 tokens) attention over 16 heads on seeded data;
``gemm`` and ``attention`` first run 1 s of untimed fp16 matmuls so their
launches see the sustained clock.  ``camera`` runs the W4-trunk camera head (4 iterations) on S seeded pose
tokens, eager or replayed from a HIP graph, and prints the mean wall time per
forward.  ``dense`` and ``sdpa`` time the vendor-library counterparts on the
same shapes, for scale: an unquantised fp16 ``torch.mm`` / ``torch.addmm``
(hipBLASLt), an int8 x int8 -> int32 ``torch._int_mm`` (hipBLASLt, the W8A8
counterpart) and torch's ``scaled_dot_product_attention``, each replayed
from a HIP graph after a 1 s warm-up.  Every mode prints one line when done.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))


def _copy():
    import torch
    a = torch.randn(256 * 1024 * 1024, dtype=torch.float16, device="cuda")  # 512 MiB
    b = torch.empty_like(a)
    for _ in range(3):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    print("copy: 3 launches, each 512 MiB read + 512 MiB written", flush=True)


def _prewarm(seconds=1.0):
    """Untimed fp16 matmuls (hipBLASLt, a kernel of its own in the trace) for
    `seconds`, so that the traced launches run at the sustained clock rather
    than on the ramp from idle."""
    import time

    import torch

    a = torch.randn(4096, 4096, device="cuda:0", dtype=torch.float16)
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            a @ a
        torch.cuda.synchronize()


def _gemm(M, K, N, gelu, reps):
    import torch

    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS_GELU, QV_EPI_NONE
    from qvggt_amd.awq.qmodule import calculate_zeros_width

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    x = torch.randn(M, K, generator=g).half().to(dev)
    qw = torch.randint(-32768, 32768, (N // 4, K), generator=g, dtype=torch.int32).to(torch.int16).to(dev)
    rows = calculate_zeros_width(K, 128) * 8
    s = (torch.rand(rows, N, generator=g) * 0.015 + 0.005).half().to(dev)
    z = (-(s.float() * torch.randint(0, 16, (rows, N), generator=g).float().to(dev))).half()
    b = torch.zeros(N, dtype=torch.float16, device=dev)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    _prewarm()
    for _ in range(reps):
        E.w4a16_linear(x, qw, s, z, bias=b, epilogue=QV_EPI_BIAS_GELU if gelu else QV_EPI_NONE, out=out)
    torch.cuda.synchronize()
    print(f"gemm: M={M} K={K} N={N} gelu={gelu}, {reps} launches", flush=True)


def _aggregator(S, w8a8):
    import torch

    from qvggt_amd import aggregator as AG

    dev = torch.device("cuda:0")
    agg = AG.Aggregator.random(w8a8=w8a8, seed=0, device=dev)
    img = torch.rand(S, 3, AG.IMG, AG.IMG, generator=torch.Generator().manual_seed(1)).half().to(dev)
    for _ in range(2):
        agg(img)
        torch.cuda.synchronize()
    print(f"aggregator: S={S} w8a8={w8a8}, 2 forwards", flush=True)


def _attention(S, glob, reps):
    import torch

    from qvggt_amd import awq_inference_engine as E

    dev = torch.device("cuda:0")
    L = S * 1374 if glob else 1374
    qkv = torch.randn(S * 1374, 3, 16, 64, generator=torch.Generator().manual_seed(0)).half().to(dev)
    out = torch.empty(S * 1374, 16, 64, dtype=torch.float16, device=dev)
    _prewarm()
    for _ in range(reps):
        E.attention(qkv[:, 0], qkv[:, 1], qkv[:, 2], L, out=out)
    torch.cuda.synchronize()
    print(f"attention: S={S} global={glob}, {reps} launches", flush=True)


def _camera(S, reps, graph):
    import time

    import torch

    from qvggt_amd.camera_head import CameraHead, GraphedCameraHead

    dev = torch.device("cuda:0")
    head = CameraHead.random(seed=0, device=dev)
    if graph:
        head = GraphedCameraHead(head, S)
    t = torch.randn(S, 2048, generator=torch.Generator().manual_seed(1)).half().to(dev)
    head(t)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        head(t)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    print(f"camera: S={S} graph={graph}, {reps} forwards, {ms:.3f} ms per forward", flush=True)


def _replay_us(fn, reps=20, rounds=5):
    import time

    import torch
    a = torch.randn(4096, 4096, device="cuda", dtype=torch.float16)
    t0 = time.time()
    while time.time() - t0 < 1.0:
        a @ a
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(rounds):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * rounds)


def _dense(M, K, N, bias, int8=False):
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    if int8:
        xi = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
        wi = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
        us = _replay_us(lambda: torch._int_mm(xi, wi.t()))
        print(f"dense int8 _int_mm (int32 out): M={M} K={K} N={N}, {us:.1f} us, "
              f"{2 * M * N * K / us / 1e6:.1f} TOPS", flush=True)
        return
    x = torch.randn(M, K, generator=g).half().to(dev)
    w = torch.randn(N, K, generator=g).half().to(dev)
    b = torch.randn(N, generator=g).half().to(dev)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    fn = (lambda: torch.addmm(b, x, w.t(), out=out)) if bias else (lambda: torch.mm(x, w.t(), out=out))
    us = _replay_us(fn)
    print(f"dense fp16 {'addmm' if bias else 'mm'}: M={M} K={K} N={N}, {us:.1f} us, "
          f"{2 * M * N * K / us / 1e6:.1f} TFLOP/s", flush=True)


def _sdpa(S, glob):
    import torch
    import torch.nn.functional as F
    dev = torch.device("cuda:0")
    B, L = (1, S * 1374) if glob else (S, 1374)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, 16, L, 64, generator=g).half().to(dev) for _ in range(3))
    us = _replay_us(lambda: F.scaled_dot_product_attention(q, k, v), reps=2 if glob else 10, rounds=3)
    print(f"sdpa fp16: S={S} global={glob} (B={B}, L={L}, 16 heads x 64), {us:.1f} us, "
          f"{4 * B * 16 * L * L * 64 / us / 1e6:.1f} TFLOP/s", flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="mode", required=True)
    sub.add_parser("copy")
    g = sub.add_parser("gemm")
    g.add_argument("M", type=int)
    g.add_argument("K", type=int)
    g.add_argument("N", type=int)
    g.add_argument("--gelu", action="store_true")
    g.add_argument("--reps", type=int, default=3)
    a = sub.add_parser("aggregator")
    a.add_argument("--frames", type=int, default=32)
    a.add_argument("--w8a8", action="store_true")
    t = sub.add_parser("attention")
    t.add_argument("--frames", type=int, default=8)
    t.add_argument("--global", dest="glob", action="store_true")
    t.add_argument("--reps", type=int, default=5)
    c = sub.add_parser("camera")
    c.add_argument("--frames", type=int, default=32)
    c.add_argument("--reps", type=int, default=10)
    c.add_argument("--graph", action="store_true")
    d = sub.add_parser("dense")
    d.add_argument("M", type=int)
    d.add_argument("K", type=int)
    d.add_argument("N", type=int)
    d.add_argument("--bias", action="store_true")
    d.add_argument("--int8", action="store_true")
    q = sub.add_parser("sdpa")
    q.add_argument("--frames", type=int, default=8)
    q.add_argument("--global", dest="glob", action="store_true")
    args = ap.parse_args(argv)
    if args.mode == "copy":
        _copy()
    elif args.mode == "gemm":
        _gemm(args.M, args.K, args.N, args.gelu, args.reps)
    elif args.mode == "attention":
        _attention(args.frames, args.glob, args.reps)
    elif args.mode == "camera":
        _camera(args.frames, args.reps, args.graph)
    elif args.mode == "dense":
        _dense(args.M, args.K, args.N, args.bias, args.int8)
    elif args.mode == "sdpa":
        _sdpa(args.frames, args.glob)
    else:
        _aggregator(args.frames, args.w8a8)


if __name__ == "__main__":
    main()
