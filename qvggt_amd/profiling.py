"""Fixed workloads for rocprofv3 runs (kernel traces and PMC counters).

    python qvggt_amd/profiling.py copy                 # traffic calibration
    python qvggt_amd/profiling.py gemm M K N [--gelu] [--reps R]
    python qvggt_amd/profiling.py aggregator [--frames S] [--w8a8]
    python qvggt_amd/profiling.py attention [--frames S] [--global] [--reps R]
    python qvggt_amd/profiling.py camera [--frames S] [--reps R] [--graph]
    python qvggt_amd/profiling.py dense M K N [--bias | --int8]
    python qvggt_amd/profiling.py sdpa [--frames S] [--global]
    python qvggt_amd/profiling.py rows [--reps R]
    python qvggt_amd/profiling.py w8a8 M K N [--reps R] [--packed]
    python qvggt_amd/profiling.py trace-summary KERNEL_TRACE_CSV [--match NAME] [--grid G] [--run RUN --last N]
    python qvggt_amd/profiling.py pmc-summary COUNTER_COLLECTION_CSV [--match NAME]

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
from a HIP graph after a 1 s warm-up.  ``rows`` runs each HBM-bound row
kernel at its benchmark shape -- LayerNorm, per-token quant, LN + quant, T5
RMSNorm and rotate-half RoPE (fused_rope_with_pos, 16 heads of 64 with fp32
angles) on S = 32 tokens (43968 x 1024), GELU + quant on the MLP hidden (10992 x 4096),
2-D RoPE and qk-norm + 2-D RoPE on the S = 32 qkv (43968 x 3072) -- R times,
each launch on its own buffer set (so no launch finds its data in the
caches).  ``w8a8`` runs the W8A8 GEMM with bias (int8 MFMA) on random int8
operands (``--packed``: on the packed weight layout, packed before the
timed launches).  Every mode above prints one line when done.

``trace-summary`` reads a rocprofv3 kernel-trace CSV and prints the dispatch
count, mean and median duration of the kernels whose name contains NAME
(and, with ``--grid``, whose grid size in work-items is G).  With ``--run``
and ``--last N`` it keeps only the last N such dispatches of the first
uninterrupted run of dispatches whose names contain RUN: for ``bench.py``,
whose first launches are its MLP steps (pre-warm, warm-up, then the timed
steps) and nothing else, those are the timed steps.  ``pmc-summary`` reads a
rocprofv3 ``--pmc`` counter-collection CSV and prints, per kernel (name
containing NAME) and counter, the value of every dispatch and their mean.
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


def _rows(reps):
    import numpy as np
    import torch

    from qvggt_amd import awq_inference_engine as E

    dev = torch.device("cuda:0")
    f16 = dict(dtype=torch.float16, device=dev)
    M, D = 32 * 1374, 1024
    _prewarm()
    xs = [torch.randn(M, D, **f16) for _ in range(reps)]
    ys = [torch.empty(M, D, **f16) for _ in range(reps)]
    q8 = [torch.empty(M, D, dtype=torch.int8, device=dev) for _ in range(reps)]
    sc = [torch.empty(M, **f16) for _ in range(reps)]
    g, b = torch.ones(D, **f16), torch.zeros(D, **f16)
    for i in range(reps):
        E.layer_norm(xs[i], g, b, 1e-6, out=ys[i])
    for i in range(reps):
        E.invoke_quant(q8[i], xs[i], sc[i])
    for i in range(reps):
        E.rms_norm_general(q8[i], xs[i], g, b, sc[i], 1e-6, True)
    for i in range(reps):
        E.layernorm_forward_cuda(xs[i].view(32, 1374, D), g, ys[i].view(32, 1374, D), 1e-6)
    fr = [torch.rand(1, M, 64, device=dev) * 40 - 20 for _ in range(reps)]
    for i in range(reps):
        E.fused_rope_with_pos_forward_func(xs[i].view(M, 1, 16, 64), fr[i], False)
    torch.cuda.synchronize()
    del xs, ys, q8, sc, fr
    Mh, Dh = 8 * 1374, 4096
    for i in range(reps):
        hx = torch.randn(Mh, Dh, **f16)
        hq = torch.empty(Mh, Dh, dtype=torch.int8, device=dev)
        ht = torch.empty(Mh, Dh, **f16)
        E.gelu_and_quant(hq, hx, torch.empty(Mh, **f16), ht)
        torch.cuda.synchronize()
    del ht
    for i in range(reps):   # the form the W8A8 blocks call: no fp16 copy stored
        hx = torch.randn(Mh, Dh, **f16)
        E.gelu_and_quant(hq, hx, torch.empty(Mh, **f16), None)
        torch.cuda.synchronize()
    del hx, hq
    pos = torch.from_numpy(np.tile(np.array([[0, 0]] * 5 + [[i // 37 + 1, i % 37 + 1] for i in range(1369)],
                                            np.int32), (32, 1))).to(dev)
    ct, st = E.rope2d_tables(38, device=dev)
    qkv = [torch.randn(M, 3 * D, **f16) for _ in range(reps)]
    for i in range(reps):
        E.rope2d(qkv[i], pos, ct, st, 16, out=qkv[i])
    gq, bq = torch.ones(64, **f16), torch.zeros(64, **f16)
    for i in range(reps):
        E.qknorm_rope2d(qkv[i], pos, ct, st, 16, gq, bq, gq, bq)
    torch.cuda.synchronize()
    print(f"rows: layernorm, quant, ln+quant, rmsnorm, rope_with_pos (S=32), gelu+quant (10992x4096, with and "
          f"without the fp16 copy), rope2d, "
          f"qknorm_rope2d (S=32), {reps} launches each", flush=True)


def _w8a8(M, K, N, reps, packed):
    import torch

    from qvggt_amd import awq_inference_engine as E

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    ws = (torch.rand(N, generator=g) * 0.01).half().to(dev)
    as_ = (torch.rand(M, generator=g) * 0.01).half().to(dev)
    b = torch.zeros(N, dtype=torch.float16, device=dev)
    o = torch.empty(M, N, dtype=torch.float16, device=dev)
    wp = E.w8a8_pack_weight(w) if packed else None
    _prewarm()
    for _ in range(reps):
        if packed:
            E.w8a8_gemm_packed(a, wp, N, ws, as_, o, bias=b)
        else:
            E.w8a8_gemm_fuse_bias_forward_cuda(a, w, ws, as_, o, b)
    torch.cuda.synchronize()
    print(f"w8a8: M={M} K={K} N={N} + bias{' (packed weights)' if packed else ''}, {reps} launches", flush=True)


def _trace_summary(path, match, grid, run, last):
    import csv
    import statistics

    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))

    def hit(r):
        g = r.get("Grid_Size", r.get("Grid_Size_X"))   # rocprofv3 names it Grid_Size_X in newer releases
        return match in r["Kernel_Name"] and (grid is None or int(g) == grid)

    if run:
        first = next(i for i, r in enumerate(rows) if run in r["Kernel_Name"])
        end = next((i for i in range(first, len(rows)) if run not in rows[i]["Kernel_Name"]), len(rows))
        rows = rows[first:end]
    sel = [r for r in rows if hit(r)]
    if last:
        sel = sel[-last:]
    us = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in sel]
    names = sorted({r["Kernel_Name"] for r in sel})
    print(f"{len(us)} dispatches of {names}: mean {statistics.mean(us):.2f} us, "
          f"median {statistics.median(us):.2f} us, min {min(us):.2f}, max {max(us):.2f}", flush=True)


def _pmc_summary(path, match):
    import csv
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(float))   # (kernel, counter) -> dispatch -> value
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if match in r["Kernel_Name"]:
                vals[(r["Kernel_Name"], r["Counter_Name"])][int(r["Dispatch_Id"])] += float(r["Counter_Value"])
    for (name, ctr), d in sorted(vals.items()):
        v = [d[k] for k in sorted(d)]
        print(f"{name.split('(')[0]} | {ctr} | dispatches {len(v)} | mean {sum(v) / len(v):.6g} | "
              f"values {', '.join(f'{x:.6g}' for x in v)}", flush=True)


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
    r = sub.add_parser("rows")
    r.add_argument("--reps", type=int, default=3)
    w = sub.add_parser("w8a8")
    w.add_argument("M", type=int)
    w.add_argument("K", type=int)
    w.add_argument("N", type=int)
    w.add_argument("--reps", type=int, default=3)
    w.add_argument("--packed", action="store_true")
    ts = sub.add_parser("trace-summary")
    ts.add_argument("csv")
    ts.add_argument("--match", default="")
    ts.add_argument("--grid", type=int, default=None)
    ps = sub.add_parser("pmc-summary")
    ps.add_argument("csv")
    ps.add_argument("--match", default="")
    ts.add_argument("--run", default="")
    ts.add_argument("--last", type=int, default=0)
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
    elif args.mode == "rows":
        _rows(args.reps)
    elif args.mode == "w8a8":
        _w8a8(args.M, args.K, args.N, args.reps, args.packed)
    elif args.mode == "pmc-summary":
        _pmc_summary(args.csv, args.match)
    elif args.mode == "trace-summary":
        _trace_summary(args.csv, args.match, args.grid, args.run, args.last)
    else:
        _aggregator(args.frames, args.w8a8)


if __name__ == "__main__":
    main()
