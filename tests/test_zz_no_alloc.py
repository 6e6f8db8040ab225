"""qv_w4a16_gemm_noalloc: the W4A16 GEMM entry that allocates nothing (its
split-K partials and counters live in a fixed device array), checked through
the C ABI against qv_w4a16_gemm, whose skinny path uses a library-allocated
workspace.  Same kernels and the same split plan, so the outputs must be
bit-identical: two calls in a row (the second with a smaller input, so stale
scratch contents from the first call would show), the large-M path (no
scratch), a size the split counters do not cover (run unsplit), and HIP-graph capture on a stream that never ran
the library (where the allocating entry may not allocate), replayed with
eager work in between."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import awq as O

pytestmark = pytest.mark.gpu


def _fns():
    from qvggt_amd import _lib
    lib = _lib.load()
    return lib, {name: getattr(lib, name) for name in ("qv_w4a16_gemm", "qv_w4a16_gemm_noalloc")}


def _problem(gpu, M, K, N, seed):
    p = O.make_w4_problem(M, K, N, seed=seed)
    t = {k: torch.from_numpy(p[k]).to(gpu) for k in ("x", "qweight", "scales", "scaled_zeros")}
    t["bias"] = torch.from_numpy((np.random.default_rng(seed).standard_normal(N) * 0.2).astype(np.float16)).to(gpu)
    return p, t


def _call(f, t, out, M, N, K, epi, stream):
    ptr = lambda v: C.c_void_p(v.data_ptr())
    return f(ptr(t["x"]), ptr(t["qweight"]), ptr(t["scales"]), ptr(t["scaled_zeros"]), ptr(t["bias"]), ptr(out),
             M, N, K, 0, epi, C.c_void_p(stream.cuda_stream))


def test_noalloc_matches_allocating_entry(gpu):
    from qvggt_amd._lib import QV_EPI_BIAS, QV_EPI_BIAS_GELU
    lib, fns = _fns()
    st = torch.cuda.current_stream()
    # 1) split path (32 x 8192 -> 2048: 4 splits), 2) a smaller split call after it,
    # 3) an unsplit skinny call, 4) the large-M path, which uses no scratch
    for (M, K, N, epi) in ((32, 8192, 2048, QV_EPI_BIAS_GELU), (8, 8192, 1024, QV_EPI_BIAS), (4, 1024, 512, QV_EPI_BIAS),
                           (300, 1024, 1024, QV_EPI_BIAS_GELU)):
        p, t = _problem(gpu, M, K, N, seed=M + K + N)
        want = torch.empty(M, N, dtype=torch.float16, device=gpu)
        got = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
        assert _call(fns["qv_w4a16_gemm"], t, want, M, N, K, epi, st) == 0
        assert _call(fns["qv_w4a16_gemm_noalloc"], t, got, M, N, K, epi, st) == 0, lib.qv_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, K, N)
        W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
        ref = O.gemm_ref(p["x"], W) + t["bias"].float().cpu().numpy()
        if epi == QV_EPI_BIAS_GELU:
            from scipy.special import erf
            ref = 0.5 * ref * (1 + erf(ref / np.sqrt(2)))
        assert O.rel_err(got.float().cpu().numpy(), ref) <= 1e-2


def test_noalloc_serves_n_beyond_the_split_counters(gpu):
    """N above 4096 channel blocks of 16 is more than the scratch has counters
    for; such a shape is never split (the split plan needs fewer than 256
    blocks), so the entry runs it unsplit, as the allocating entry does: the
    same bits, and the oracle's values."""
    lib, fns = _fns()
    M, K, N = 1, 128, 65536 + 16
    p, t = _problem(gpu, M, K, N, seed=1)
    want = torch.empty(M, N, dtype=torch.float16, device=gpu)
    got = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
    st = torch.cuda.current_stream()
    assert _call(fns["qv_w4a16_gemm"], t, want, M, N, K, 0, st) == 0
    assert _call(fns["qv_w4a16_gemm_noalloc"], t, got, M, N, K, 0, st) == 0, lib.qv_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    assert O.rel_err(got.float().cpu().numpy(), O.gemm_ref(p["x"], W)) <= 1e-2


def test_noalloc_in_a_graph_captured_on_a_fresh_stream(gpu):
    """Captured on a stream the library has never seen, the no-allocation entry
    still splits K; three replays on changing inputs, with eager work and
    synchronisation between them, each equal to the allocating entry's eager
    output on the same input.  One eager call comes first, as the entry's
    first call on a device resolves the scratch address."""
    from qvggt_amd._lib import QV_EPI_BIAS
    lib, fns = _fns()
    M, K, N = 24, 8192, 2048
    p, t = _problem(gpu, M, K, N, seed=5)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    assert _call(fns["qv_w4a16_gemm_noalloc"], t, out, M, N, K, QV_EPI_BIAS, torch.cuda.current_stream()) == 0
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert _call(fns["qv_w4a16_gemm_noalloc"], t, out, M, N, K, QV_EPI_BIAS, s) == 0
    gen = torch.Generator(device=gpu).manual_seed(1)
    for i in range(3):
        t["x"].copy_(torch.randn(M, K, generator=gen, device=gpu).half())
        want = torch.empty(M, N, dtype=torch.float16, device=gpu)
        assert _call(fns["qv_w4a16_gemm"], t, want, M, N, K, QV_EPI_BIAS, torch.cuda.current_stream()) == 0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
