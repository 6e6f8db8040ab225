"""GPU parity of the W4A16 path against the oracle (oracle/awq.py).

Bars: dequantisation bit-exact; GEMM/GEMV fp16 outputs within
max|y - y_ref| / max|y_ref| <= 1e-2 of the fp32 dequant reference (the
tolerance stated for this path), plus absolute error reported.
"""
import numpy as np
import pytest
import torch

from oracle import awq as O

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _to_dev(p, dev, dtype=torch.float16):
    t = {
        "x": torch.from_numpy(p["x"]).to(dev),
        "qweight": torch.from_numpy(p["qweight"]).to(dev),
        "scales": torch.from_numpy(p["scales"]).to(dev),
        "scaled_zeros": torch.from_numpy(p["scaled_zeros"]).to(dev),
    }
    return t


def _bf16_problem(p):
    """bf16 copy of a problem: scales rounded to bf16, sz = -bf16(s*z)."""
    N = p["s"].shape[0]
    K = p["x"].shape[1]
    s_bits = O.f64_to_bf16_bits(p["s"].astype(np.float64))
    s = O.bf16_bits_to_f32(s_bits).astype(np.float64)
    sz_bits = O.f64_to_bf16_bits(-(s * p["z"]))
    rows = O.scale_rows(K)
    sc = np.zeros((rows, N), np.uint16)
    sz = np.zeros((rows, N), np.uint16)
    sc[: s.shape[1]] = s_bits.T
    sz[: s.shape[1]] = sz_bits.T
    x_bits = O.f64_to_bf16_bits(p["x"].astype(np.float64))
    return x_bits, sc, sz


@pytest.mark.parametrize("N,K", [(64, 128), (3072, 1024), (4096, 1024), (1024, 4096)])
def test_dequant_bit_exact_fp16(gpu, N, K):
    from qvggt_amd import awq_inference_engine as E
    p = O.make_w4_problem(1, K, N, seed=N + K)
    t = _to_dev(p, gpu)
    W = E.w4a16_dequantize(t["qweight"], t["scales"], t["scaled_zeros"], K)
    ref = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    assert np.array_equal(W.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("N,K", [(64, 256), (3072, 1024)])
def test_dequant_bit_exact_bf16(gpu, N, K):
    from qvggt_amd import awq_inference_engine as E
    p = O.make_w4_problem(1, K, N, seed=3)
    _, sc, sz = _bf16_problem(p)
    qw = torch.from_numpy(p["qweight"]).to(gpu)
    sct = torch.from_numpy(sc.view(np.int16)).to(gpu).view(torch.bfloat16)
    szt = torch.from_numpy(sz.view(np.int16)).to(gpu).view(torch.bfloat16)
    W = E.w4a16_dequantize(qw, sct, szt, K)
    ref = O.dequantize_bf16_bits(p["qweight"], sc, sz, N, K)
    assert np.array_equal(W.cpu().view(torch.int16).numpy().view(np.uint16), ref)


def _check_gemm(y, p, N, K, tol=TOL):
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    ref = O.gemm_ref(p["x"], W)
    got = y.float().cpu().numpy().reshape(ref.shape)
    err = O.rel_err(got, ref)
    assert np.isfinite(got).all()
    assert err <= tol, f"rel err {err:.3e}, abs {np.abs(got - ref).max():.3e}"
    return err


@pytest.mark.parametrize("M,N,K", [
    (1374, 3072, 1024),   # config 1: VGGT qkv on one frame
    (17, 3072, 1024), (129, 256, 1024), (200, 48, 128), (1, 16, 128), (33, 1024, 4096),
    (2748, 4096, 1024),
])
def test_gemm_forward_cuda_new_parity(gpu, M, N, K):
    from qvggt_amd import awq_inference_engine as E
    p = O.make_w4_problem(M, K, N, seed=M + N + K)
    t = _to_dev(p, gpu)
    y = E.gemm_forward_cuda_new(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
    assert y.shape == (M, N) and y.dtype == torch.float16
    _check_gemm(y, p, N, K)


def test_gemm_mlp_shapes(gpu):
    """config 2a shapes at full M: fc1 1024->4096 and fc2 4096->1024, M = 10992."""
    from qvggt_amd import awq_inference_engine as E
    for (N, K) in [(4096, 1024), (1024, 4096)]:
        p = O.make_w4_problem(10992, K, N, seed=N)
        t = _to_dev(p, gpu)
        y = E.gemm_forward_cuda_new(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
        _check_gemm(y, p, N, K)


def test_gemm_3d_input_and_determinism(gpu):
    from qvggt_amd import awq_inference_engine as E
    p = O.make_w4_problem(2 * 300, 1024, 512, seed=1)
    t = _to_dev(p, gpu)
    x3 = t["x"].view(2, 300, 1024)
    y1 = E.gemm_forward_cuda_new(x3, t["qweight"], t["scales"], t["scaled_zeros"])
    y2 = E.gemm_forward_cuda_new(x3, t["qweight"], t["scales"], t["scaled_zeros"])
    assert y1.shape == (2, 300, 512)
    assert torch.equal(y1, y2), "re-run is not bitwise identical"
    _check_gemm(y1, p, 512, 1024)


@pytest.mark.parametrize("M", [300, 40, 6])
def test_gemm_bf16(gpu, M):
    """bf16 on the MFMA GEMM (M = 300) and the skinny kernel (M = 40, 6)."""
    from qvggt_amd import awq_inference_engine as E
    N, K = 512, 1024
    p = O.make_w4_problem(M, K, N, seed=21)
    xb, sc, sz = _bf16_problem(p)
    x = torch.from_numpy(xb.view(np.int16)).to(gpu).view(torch.bfloat16).view(M, K)
    qw = torch.from_numpy(p["qweight"]).to(gpu)
    sct = torch.from_numpy(sc.view(np.int16)).to(gpu).view(torch.bfloat16)
    szt = torch.from_numpy(sz.view(np.int16)).to(gpu).view(torch.bfloat16)
    y = E.gemm_forward_cuda_new(x, qw, sct, szt)
    W = O.bf16_bits_to_f32(O.dequantize_bf16_bits(p["qweight"], sc, sz, N, K))
    ref = O.bf16_bits_to_f32(xb) @ W.T
    err = O.rel_err(y.float().cpu().numpy(), ref)
    assert err <= TOL, err


@pytest.mark.parametrize("M,N,K", [(24, 2048, 8192), (48, 6144, 2048), (64, 1024, 1024), (61, 48, 256),
                                   (32, 8192, 2048), (12, 4112, 256), (7, 8192, 1024)])
def test_skinny_range(gpu, M, N, K):
    """M <= 64 runs the skinny MFMA kernel: channels across the grid, 128-k
    groups across the waves (several per wave at K = 8192), tokens past M
    read as zero, partial sums reduced through LDS."""
    from qvggt_amd import awq_inference_engine as E
    p = O.make_w4_problem(M, K, N, seed=7 * M + K)
    t = _to_dev(p, gpu)
    y = E.gemm_forward_cuda_new(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
    _check_gemm(y, p, N, K)


@pytest.mark.parametrize("m", list(range(1, 8)))
def test_gemv_forward_cuda_new_parity(gpu, m):
    from qvggt_amd import awq_inference_engine as E
    N, K = 3072, 1024
    p = O.make_w4_problem(m, K, N, seed=m)
    t = _to_dev(p, gpu)
    y = E.gemv_forward_cuda_new(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], m, N, K, 128)
    assert y.shape == (m, N)
    _check_gemm(y, p, N, K)


@pytest.mark.parametrize("M,N,K", [(1, 1024, 4096), (8, 3072, 1024), (16, 4096, 1024), (12, 64, 128)])
def test_linear_small_m_routes_and_matches(gpu, M, N, K):
    from qvggt_amd import awq_inference_engine as E
    p = O.make_w4_problem(M, K, N, seed=100 + M)
    t = _to_dev(p, gpu)
    y = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
    _check_gemm(y, p, N, K)


@pytest.mark.parametrize("M", [3, 5, 50, 700])
def test_epilogues_bias_gelu(gpu, M):
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS, QV_EPI_BIAS_GELU
    N, K = 1024, 1024
    p = O.make_w4_problem(M, K, N, seed=M)
    t = _to_dev(p, gpu)
    b = (np.random.default_rng(1).standard_normal(N) * 0.5).astype(np.float16)
    bt = torch.from_numpy(b).to(gpu)
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    ref = O.gemm_ref(p["x"], W) + b.astype(np.float32)
    y = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=bt, epilogue=QV_EPI_BIAS)
    assert O.rel_err(y.float().cpu().numpy(), ref) <= TOL
    from math import erf
    gelu = np.vectorize(lambda v: 0.5 * v * (1 + erf(v / np.sqrt(2))))
    y = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=bt, epilogue=QV_EPI_BIAS_GELU)
    assert O.rel_err(y.float().cpu().numpy(), gelu(ref.astype(np.float64))) <= TOL


@pytest.mark.parametrize("M", [1, 200])
def test_gelu_epilogue_pointwise(gpu, M):
    """x = 0 makes the output GELU(bias): the epilogue's GELU on every finite
    fp16 value (GEMV path at M = 1, MFMA GEMM at M = 200) is within one fp16
    ulp of the float64 erf GELU rounded to fp16."""
    from scipy.special import erf
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS_GELU
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    b = b[np.isfinite(b)]
    N, K = b.size, 128            # 63488 channels, a multiple of 16
    p = O.make_w4_problem(M, K, N, seed=3)
    t = _to_dev(p, gpu)
    x = torch.zeros(M, K, dtype=torch.float16, device=gpu)
    y = E.w4a16_linear(x, t["qweight"], t["scales"], t["scaled_zeros"], bias=torch.from_numpy(b).to(gpu),
                       epilogue=QV_EPI_BIAS_GELU).cpu().numpy()
    b64 = b.astype(np.float64)
    ref = (0.5 * b64 * (1 + erf(b64 / np.sqrt(2)))).astype(np.float16)
    ulp = np.spacing(np.abs(ref)).astype(np.float64)
    assert np.all(np.abs(y.astype(np.float64) - ref.astype(np.float64)) <= ulp[None, :]), "GELU off by > 1 ulp"


def test_wqlinear_forward(gpu):
    from qvggt_amd.awq import WQLinear
    M, N, K = 400, 3072, 1024
    p = O.make_w4_problem(M, K, N, seed=77)
    q = WQLinear(4, 128, K, N, True, gpu)
    q.qweight.copy_(torch.from_numpy(p["qweight"]))
    q.scales.copy_(torch.from_numpy(p["scales"]))
    q.scaled_zeros.copy_(torch.from_numpy(p["scaled_zeros"]))
    b = np.linspace(-1, 1, N).astype(np.float16)
    q.bias.copy_(torch.from_numpy(b))
    x = torch.from_numpy(p["x"]).to(gpu)
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    ref = O.gemm_ref(p["x"], W) + b.astype(np.float32)
    for xin in (x, x[:3]):   # GEMM path and GEMV path (M < 8)
        y = q(xin)
        assert O.rel_err(y.float().cpu().numpy(), ref[: xin.shape[0]]) <= TOL


@pytest.mark.parametrize("M,N,K", [(1, 1024, 4096), (40, 1024, 1024), (300, 1024, 4096), (1374, 1024, 1024),
                                   (10992, 1024, 4096)])
def test_linear_residual_matches_unfused(gpu, M, N, K):
    """residual += gamma * fp16(x W^T + b) in the GEMM epilogue (skinny kernel at
    M <= 64, stream tiles above) equals the linear followed by the fp32
    update, to one fp16 ulp (fma contraction of the update may differ)."""
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS
    p = O.make_w4_problem(M, K, N, seed=M + 3)
    t = _to_dev(p, gpu)
    g = torch.Generator(device=gpu).manual_seed(M)
    bias = (torch.randn(N, generator=g, device=gpu) * 0.1).half()
    gamma = (torch.rand(N, generator=g, device=gpu) + 0.5).half()
    resid = torch.randn(M, N, generator=g, device=gpu).half()
    o = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=bias, epilogue=QV_EPI_BIAS)
    want = (resid.float() + o.float() * gamma.float()).half()
    got = resid.clone()
    E.w4a16_linear_residual(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias, gamma, got)
    torch.cuda.synchronize()
    d = (got.float() - want.float()).abs()
    ulp = torch.from_numpy(np.spacing(np.abs(want.cpu().numpy())).astype(np.float32)).to(gpu)
    assert torch.isfinite(got.float()).all() and bool((d <= ulp).all()), d.max().item()
    with pytest.raises(RuntimeError):
        E.w4a16_linear_residual(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias, gamma[:16], got)


@pytest.mark.parametrize("M", [4, 300])
def test_noncontiguous_activations_match_contiguous(gpu, M):
    """The ops read the activations through a contiguous copy when given a
    strided view (the reference reads raw data_ptr whatever the strides): a
    column slice of a wider tensor gives the same bits as its contiguous copy,
    on the GEMV (M = 4) and GEMM (M = 300) entries."""
    from qvggt_amd import awq_inference_engine as E
    N, K = 1024, 1024
    p = O.make_w4_problem(M, K, N, seed=11 + M)
    t = _to_dev(p, gpu)
    wide = torch.zeros(M, 2 * K, dtype=torch.float16, device=gpu)
    wide[:, K // 2:K // 2 + K] = t["x"]
    view = wide[:, K // 2:K // 2 + K]
    assert not view.is_contiguous()
    if M <= 7:
        got = E.gemv_forward_cuda_new(view, t["qweight"], t["scales"], t["scaled_zeros"], M, N, K, 128)
        want = E.gemv_forward_cuda_new(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], M, N, K, 128)
    else:
        got = E.gemm_forward_cuda_new(view, t["qweight"], t["scales"], t["scaled_zeros"])
        want = E.gemm_forward_cuda_new(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_bench_mlp_pair_instance(gpu):
    """The exact launches bench.py times (config 2a, M = 8 x 1374): fc1
    1024 -> 4096 with the bias + erf-GELU epilogue on the 128-row stream tile,
    then fc2 4096 -> 1024 + bias from the GPU's own fc1 output, each against
    the fp32 dequantised reference (+ float64 erf GELU)."""
    from scipy.special import erf
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS, QV_EPI_BIAS_GELU
    M = 10992
    p1 = O.make_w4_problem(M, 1024, 4096, seed=0)
    p2 = O.make_w4_problem(M, 4096, 1024, seed=1)
    b1 = (np.random.default_rng(5).standard_normal(4096) * 0.1).astype(np.float16)
    b2 = (np.random.default_rng(6).standard_normal(1024) * 0.1).astype(np.float16)
    t1, t2 = _to_dev(p1, gpu), _to_dev(p2, gpu)
    h = E.w4a16_linear(t1["x"], t1["qweight"], t1["scales"], t1["scaled_zeros"], bias=torch.from_numpy(b1).to(gpu),
                       epilogue=QV_EPI_BIAS_GELU)
    y = E.w4a16_linear(h, t2["qweight"], t2["scales"], t2["scaled_zeros"], bias=torch.from_numpy(b2).to(gpu),
                       epilogue=QV_EPI_BIAS)
    torch.cuda.synchronize()
    W1 = O.dequantize(p1["qweight"], p1["scales"], p1["scaled_zeros"], 4096, 1024)
    pre = (O.gemm_ref(p1["x"], W1) + b1.astype(np.float32)).astype(np.float64)
    ref1 = 0.5 * pre * (1.0 + erf(pre / np.sqrt(2.0)))
    hn = h.float().cpu().numpy()
    assert np.isfinite(hn).all() and O.rel_err(hn, ref1) <= TOL
    W2 = O.dequantize(p2["qweight"], p2["scales"], p2["scaled_zeros"], 1024, 4096)
    ref2 = O.gemm_ref(h.cpu().numpy(), W2) + b2.astype(np.float32)
    assert O.rel_err(y.float().cpu().numpy(), ref2) <= TOL


def test_noncontiguous_tables_match_contiguous(gpu):
    """Transposed-view scales, zeros, bias (and LayerNorm / qk-norm weights)
    give the same bits as their contiguous copies: each strided argument is
    copied to a buffer that stays alive until the kernel has been launched."""
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS
    M, N, K = 300, 1024, 1024
    p = O.make_w4_problem(M, K, N, seed=31)
    t = _to_dev(p, gpu)
    sT = t["scales"].t().contiguous().t()        # same shape, column-major
    zT = t["scaled_zeros"].t().contiguous().t()
    assert not sT.is_contiguous() and not zT.is_contiguous()
    bias = torch.linspace(-1, 1, 2 * N, device=gpu).half()[::2]
    for m in (M, 5):
        want = E.w4a16_linear(t["x"][:m], t["qweight"], t["scales"], t["scaled_zeros"], bias=bias.contiguous(),
                              epilogue=QV_EPI_BIAS)
        got = E.w4a16_linear(t["x"][:m], t["qweight"], sT, zT, bias=bias, epilogue=QV_EPI_BIAS)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    xg = torch.randn(64, 1024, generator=torch.Generator().manual_seed(0)).half().to(gpu)
    w = torch.linspace(0.5, 1.5, 2048, device=gpu).half()[::2]
    b = torch.linspace(-0.5, 0.5, 2048, device=gpu).half()[1::2]
    assert torch.equal(E.layer_norm(xg, w, b), E.layer_norm(xg, w.contiguous(), b.contiguous()))
    q1, q2 = (torch.empty(64, 1024, dtype=torch.int8, device=gpu) for _ in range(2))
    s1, s2 = (torch.empty(64, dtype=torch.float16, device=gpu) for _ in range(2))
    E.rms_norm_general(q1, xg, w, b, s1, 1e-6, True)
    E.rms_norm_general(q2, xg, w.contiguous(), b.contiguous(), s2, 1e-6, True)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(s1, s2)


def test_output_must_be_16_byte_aligned(gpu):
    """The stream GEMM's epilogue stores 16-byte row pieces: an output view
    offset by 8 bytes is refused with a clear error (by the Python op and by
    the C ABI itself), never written misaligned."""
    import ctypes as C
    from qvggt_amd import _lib
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_NONE, QV_F16
    M, N, K = 300, 1024, 1024
    p = O.make_w4_problem(M, K, N, seed=41)
    t = _to_dev(p, gpu)
    buf = torch.zeros(M * N + 4, dtype=torch.float16, device=gpu)
    bad = buf[4:].view(M, N)
    assert bad.data_ptr() % 16 == 8
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], out=bad)
    ptr = lambda v: C.c_void_p(v.data_ptr())
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _lib.call("qv_w4a16_gemm", ptr(t["x"]), ptr(t["qweight"]), ptr(t["scales"]), ptr(t["scaled_zeros"]),
                  C.c_void_p(0), ptr(bad), M, N, K, QV_F16, QV_EPI_NONE, C.c_void_p(0))
    torch.cuda.synchronize()
    assert not buf.any()


@pytest.mark.parametrize("M,N,K", [(1, 2048, 8192), (8, 2048, 8192), (32, 2048, 8192), (40, 1024, 8192),
                                   (64, 1024, 16384)])
def test_skinny_split_k(gpu, M, N, K):
    """Long-K skinny shapes split K across workgroups (fp32 partials, the last
    split to arrive sums them in split order): parity with the fp32 reference
    for the plain, bias + GELU and LayerScale-residual epilogues, and bitwise
    equal re-runs (the sum order does not depend on arrival order)."""
    from math import erf
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS_GELU
    p = O.make_w4_problem(M, K, N, seed=M * 31 + K)
    t = _to_dev(p, gpu)
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    ref = O.gemm_ref(p["x"], W)
    runs = [E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"]) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    assert O.rel_err(runs[0].float().cpu().numpy(), ref) <= TOL
    b = (np.random.default_rng(M).standard_normal(N) * 0.3).astype(np.float16)
    bt = torch.from_numpy(b).to(gpu)
    y = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=bt, epilogue=QV_EPI_BIAS_GELU)
    pre = (ref + b.astype(np.float32)).astype(np.float64)
    gelu = np.vectorize(lambda v: 0.5 * v * (1 + erf(v / np.sqrt(2))))(pre)
    assert O.rel_err(y.float().cpu().numpy(), gelu) <= TOL
    gamma = torch.linspace(0.5, 1.5, N, device=gpu).half()
    resid = torch.randn(M, N, generator=torch.Generator(device=gpu).manual_seed(M), device=gpu).half()
    o = torch.from_numpy(ref + b.astype(np.float32)).to(gpu).half()   # the linear's fp16 output
    want = resid.float() + o.float() * gamma.float()
    got = resid.clone()
    E.w4a16_linear_residual(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bt, gamma, got)
    torch.cuda.synchronize()
    assert ((got.float() - want).abs().max() / want.abs().max()).item() <= TOL


def test_skinny_split_k_bf16(gpu):
    from qvggt_amd import awq_inference_engine as E
    M, N, K = 24, 2048, 8192
    p = O.make_w4_problem(M, K, N, seed=23)
    xb, sc, sz = _bf16_problem(p)
    x = torch.from_numpy(xb.view(np.int16)).to(gpu).view(torch.bfloat16).view(M, K)
    qw = torch.from_numpy(p["qweight"]).to(gpu)
    sct = torch.from_numpy(sc.view(np.int16)).to(gpu).view(torch.bfloat16)
    szt = torch.from_numpy(sz.view(np.int16)).to(gpu).view(torch.bfloat16)
    y = E.gemm_forward_cuda_new(x, qw, sct, szt)
    W = O.bf16_bits_to_f32(O.dequantize_bf16_bits(p["qweight"], sc, sz, N, K))
    assert O.rel_err(y.float().cpu().numpy(), O.bf16_bits_to_f32(xb) @ W.T) <= TOL


def test_skinny_split_k_captured_on_a_fresh_stream_matches_eager(gpu):
    """A split-K skinny call captured into a graph on a stream the library has
    never run on takes the same split plan as an eager call (it uses the
    device scratch, since capture cannot allocate), so every replay equals
    the eager output bit for bit; eager calls on the capture stream and on
    the current stream run between the replays.  One eager call comes first:
    a device's first split-K call sets the device scratch up, outside
    capture."""
    from qvggt_amd import awq_inference_engine as E
    M, N, K = 32, 2048, 8192
    p = O.make_w4_problem(M, K, N, seed=77)
    t = _to_dev(p, gpu)
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], out=out)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], out=out)
    gen = torch.Generator(device=gpu).manual_seed(3)
    for i in range(3):
        t["x"].copy_(torch.randn(M, K, generator=gen, device=gpu).half())
        want = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
        with torch.cuda.stream(s):
            other = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want) and torch.equal(other, want), i
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    assert O.rel_err(out.float().cpu().numpy(), O.gemm_ref(t["x"].cpu().numpy(), W)) <= TOL


@pytest.mark.parametrize("M", [1374, 2748, 300, 40])
def test_qkv_qknorm_rope_fused_matches_two_step(gpu, M):
    """qv_w4a16_gemm_qkrope (the qkv projection with its q/k LayerNorm and 2-D
    RoPE in the GEMM epilogue) against the two-step path it replaces,
    qv_w4a16_gemm + qv_qknorm_rope2d, both of which are pinned bit-exact
    elsewhere.  The v heads are the same GEMM epilogue (bit-identical); the q
    and k heads sum the LayerNorm statistics in another order, so their
    LayerNorm outputs may differ by an fp16 rounding step.  M = 40 takes the skinny path, where the
    entry runs the two steps itself (bit-identical)."""
    from oracle import rope as R
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd._lib import QV_EPI_BIAS
    H, K = 16, 1024
    N = 3 * H * 64
    p = O.make_w4_problem(M, K, N, seed=M)
    t = _to_dev(p, gpu)
    rng = np.random.default_rng(M)
    bias = torch.from_numpy((rng.standard_normal(N) * 0.5).astype(np.float16)).to(gpu)
    if M % 1374 == 0:
        pos = R.vggt_positions(M // 1374)
    else:
        pos = rng.integers(0, 38, size=(M, 2)).astype(np.int32)
    pt = torch.from_numpy(pos).to(gpu)
    ct, st = E.rope2d_tables(38, device=gpu)
    qg, qb, kg, kb = (torch.from_numpy(((1 if i % 2 == 0 else 0) + 0.1 * rng.standard_normal(64)).astype(np.float16))
                      .to(gpu) for i in range(4))
    fused = E.w4a16_linear_qkrope(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias, pt, ct, st, H,
                                  qg, qb, kg, kb, eps=1e-6)
    two = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=bias, epilogue=QV_EPI_BIAS)
    E.qknorm_rope2d(two, pt, ct, st, H, qg, qb, kg, kb, eps=1e-6)
    torch.cuda.synchronize()
    f = fused.view(M, 3, H, 64).cpu().numpy().astype(np.float64)
    w = two.view(M, 3, H, 64).cpu().numpy().astype(np.float64)
    assert np.isfinite(f).all()
    assert np.array_equal(f[:, 2], w[:, 2]), "v heads"
    if M <= 64:
        assert np.array_equal(f, w)
    # The LayerNorm outputs may differ by one fp16 rounding step; the rotation
    # a c -/+ b s then carries that into its result, which can cancel to far
    # below the inputs' magnitude, so the bound is in ulps of each head row's
    # largest value: 2 input steps plus the output rounding.
    row_max = np.maximum(np.abs(f[:, :2]), np.abs(w[:, :2])).max(axis=-1, keepdims=True)
    ulp = np.spacing(row_max.astype(np.float16)).astype(np.float64)
    worst = (np.abs(f[:, :2] - w[:, :2]) / ulp).max()
    print(f"[qkrope] M={M}: max |fused - two-step| = {worst:.2f} ulp of the head row's max", flush=True)
    assert worst <= 3.0, f"q/k heads differ by {worst} fp16 ulp of the head row's largest value"


@pytest.mark.parametrize("M", [1374, 2748])
def test_qkv_qknorm_rope_fused_matches_oracle(gpu, M):
    """qv_w4a16_gemm_qkrope against the oracle directly: the fp32-dequantised
    projection plus bias (float64 from the dequantised weights), rounded to
    fp16 as the epilogue stores it, then oracle.rope.qknorm_rope2d (the
    reference q/k LayerNorm + 2-D RoPE) on the q and k heads; v heads are the
    projection itself.  Tolerance: max |out - ref| <= 1e-2 of max |ref| per
    part, and the q / k values within a few fp16 steps of their head row's
    largest value (the GEMM's fp32 sum may round y to the neighbouring fp16
    value, which the LayerNorm and rotation then carry)."""
    from oracle import rope as R
    from qvggt_amd import awq_inference_engine as E
    H, K = 16, 1024
    N = 3 * H * 64
    p = O.make_w4_problem(M, K, N, seed=M + 5)
    t = _to_dev(p, gpu)
    rng = np.random.default_rng(M + 5)
    bias = (rng.standard_normal(N) * 0.5).astype(np.float16)
    pos = R.vggt_positions(M // 1374)
    ct, st = E.rope2d_tables(38, device=gpu)
    prm = [((1 if i % 2 == 0 else 0) + 0.1 * rng.standard_normal(64)).astype(np.float16) for i in range(4)]
    got = E.w4a16_linear_qkrope(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], torch.from_numpy(bias).to(gpu),
                                torch.from_numpy(pos).to(gpu), ct, st, H, *(torch.from_numpy(v).to(gpu) for v in prm),
                                eps=1e-6)
    torch.cuda.synchronize()
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K).astype(np.float64)
    y = (p["x"].astype(np.float64) @ W.T + bias.astype(np.float64)).astype(np.float16).reshape(M, 3, H, 64)
    c, s = R.rope2d_tables(38)
    qk = R.qknorm_rope2d(y[:, :2], pos, c, s, *prm, eps=1e-6).astype(np.float64)
    g = got.view(M, 3, H, 64).cpu().numpy().astype(np.float64)
    for part, ref in ((0, qk[:, 0]), (1, qk[:, 1]), (2, y[:, 2].astype(np.float64))):
        err = np.abs(g[:, part] - ref).max() / np.abs(ref).max()
        assert np.isfinite(g[:, part]).all() and err <= 1e-2, (part, err)
    row_max = np.abs(qk).max(axis=-1, keepdims=True)
    ulp = np.spacing(row_max.astype(np.float16)).astype(np.float64)
    worst = (np.abs(g[:, :2] - qk) / ulp).max()
    print(f"[qkrope] M={M}: max |fused - oracle| = {worst:.2f} ulp of the head row's max", flush=True)
    assert worst <= 8.0, worst


# Shapes whose launch covers the rows in two ranges of different tile heights
# (the tile planner picks 96- then 64-row tiles for 2748 x 3072, 128- then
# 96-row tiles for the others), with the epilogue each runs with in the model.
@pytest.mark.parametrize("M,N,K,epi_name,dt", [(2748, 3072, 1024, "BIAS", "f16"), (10992, 4096, 1024, "BIAS_GELU", "f16"),
                                               (5496, 4096, 1024, "BIAS_GELU", "f16"), (10992, 3072, 1024, "BIAS", "f16"),
                                               (21984, 1024, 4096, "BIAS", "f16"), (10992, 3072, 1024, "BIAS", "bf16")])
def test_two_range_launch_matches_row_slices(gpu, M, N, K, epi_name, dt):
    """A tile's results do not depend on its height or on which range of the
    launch it sits in: the whole launch equals, bit for bit, the same linear
    run on two row slices (each slice gets a plan of its own), and sampled
    rows stay within the tolerance of the fp32 dequantised reference."""
    from scipy.special import erf
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd import _lib
    epi = getattr(_lib, "QV_EPI_" + epi_name)
    p = O.make_w4_problem(M, K, N, seed=M + N)
    bias = (np.random.default_rng(M).standard_normal(N) * 0.1).astype(np.float16)
    if dt == "bf16":
        x_bits, sc, sz = _bf16_problem(p)
        x = torch.from_numpy(x_bits.view(np.int16)).to(gpu).view(torch.bfloat16)
        scales = torch.from_numpy(sc.view(np.int16)).to(gpu).view(torch.bfloat16)
        zeros = torch.from_numpy(sz.view(np.int16)).to(gpu).view(torch.bfloat16)
        b = torch.from_numpy(bias).to(gpu).to(torch.bfloat16)
    else:
        t = _to_dev(p, gpu)
        x, scales, zeros = t["x"], t["scales"], t["scaled_zeros"]
        b = torch.from_numpy(bias).to(gpu)
    qw = torch.from_numpy(p["qweight"]).to(gpu)
    whole = E.w4a16_linear(x, qw, scales, zeros, bias=b, epilogue=epi)
    cut = 1000
    parts = torch.cat([E.w4a16_linear(x[:cut], qw, scales, zeros, bias=b, epilogue=epi),
                       E.w4a16_linear(x[cut:], qw, scales, zeros, bias=b, epilogue=epi)])
    torch.cuda.synchronize()
    plans = [E.w4a16_plan(m, N, K, epi) for m in (M, cut, M - cut)]
    assert plans[0]["kernel"] == "stream" and plans[0]["tile2"] > 0, plans[0]
    if all(pl["kernel"] in ("stream", "stream_k128") for pl in plans):
        assert torch.equal(whole, parts)
    else:
        # a slice small enough for one tile per CU sums K in two halves: the
        # fp32 sums differ in rounding only -- one 16-bit step of the value,
        # plus the fp32 accumulation error (a few 2^-24 of the row's partial
        # sums), which spans many steps only where the sum cancels to ~0
        w, pt = whole.float(), parts.float()
        step = torch.maximum(w.abs(), pt.abs()) * (2.0 ** -7 if dt == "bf16" else 2.0 ** -10)
        slack = 2.0 ** -20 * w.abs().max().item()
        assert ((w - pt).abs() <= step + slack).all(), (w - pt).abs().max().item()
    rows = np.random.default_rng(1).choice(M, 256, replace=False)
    xr = x[torch.from_numpy(rows).to(gpu)].float().cpu().numpy()
    if dt == "bf16":
        W = O.bf16_bits_to_f32(O.dequantize_bf16_bits(p["qweight"], sc, sz, N, K))
    else:
        W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    ref = (O.gemm_ref(xr, W) + b.float().cpu().numpy()).astype(np.float64)
    if epi_name == "BIAS_GELU":
        ref = 0.5 * ref * (1.0 + erf(ref / np.sqrt(2.0)))
    got = whole[torch.from_numpy(rows).to(gpu)].float().cpu().numpy()
    assert np.isfinite(got).all() and O.rel_err(got, ref) <= TOL


# Launches of at most one tile per CU: K split between two wave groups of one
# workgroup, or 128-k pipeline stages (one case per tile height, with the
# epilogues the model uses).
@pytest.mark.parametrize("M,N,K,epi_name,tile,kind", [
    (1374, 1024, 4096, "BIAS", 32, "stream_ksplit"), (1374, 512, 1024, "NONE", 32, "stream_ksplit"),
    (2748, 1024, 4096, "BIAS", 64, "stream_ksplit"), (2000, 2048, 2048, "BIAS_GELU", 64, "stream_ksplit"),
    (4000, 2048, 2048, "BIAS", 128, "stream_ksplit"), (300, 256, 256, "GELU", 32, "stream_ksplit"),
    (2500, 2048, 2048, "BIAS", 96, "stream_ksplit"),
    (1374, 3072, 1024, "BIAS", 96, "stream_k128"), (1000, 3072, 1024, "NONE", 64, "stream_k128"),
    (1374, 4096, 1024, "BIAS_GELU", 96, "stream_k128"), (2000, 3072, 256, "GELU", 96, "stream_k128"),
    (1500, 2048, 512, "BIAS", 64, "stream_k128")])
def test_one_round_launch_matches_oracle(gpu, M, N, K, epi_name, tile, kind):
    """The one-round launch (plan checked) against the fp32 dequantised
    reference: every row within the tolerance, a re-run bitwise identical."""
    from scipy.special import erf
    from qvggt_amd import awq_inference_engine as E
    from qvggt_amd import _lib
    epi = getattr(_lib, "QV_EPI_" + epi_name)
    plan = E.w4a16_plan(M, N, K, epi)
    assert plan["kernel"] == kind and plan["tile"] == tile, plan
    p = O.make_w4_problem(M, K, N, seed=M + 3 * N + K)
    t = _to_dev(p, gpu)
    bias = (np.random.default_rng(N).standard_normal(N) * 0.1).astype(np.float16)
    b = torch.from_numpy(bias).to(gpu)
    y = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=b, epilogue=epi)
    y2 = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=b, epilogue=epi)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    ref = O.gemm_ref(p["x"], W).astype(np.float64)
    if epi_name in ("BIAS", "BIAS_GELU"):
        ref = ref + bias.astype(np.float64)
    if epi_name in ("BIAS_GELU", "GELU"):
        ref = 0.5 * ref * (1.0 + erf(ref / np.sqrt(2.0)))
    got = y.float().cpu().numpy()
    err = O.rel_err(got, ref)
    print(f"[{kind}] M={M} N={N} K={K} {epi_name} tile {tile}: rel err {err:.3e}", flush=True)
    assert np.isfinite(got).all() and err <= TOL, err


def test_ksplit_residual_matches_unfused(gpu):
    """The residual epilogue on a K-split launch (M = 1374, one frame's proj)
    against the same op chain run unfused: the plain linear (also K-split)
    followed by torch's residual update, within 2 fp16 steps."""
    from qvggt_amd import awq_inference_engine as E
    M, K = 1374, 1024
    assert E.w4a16_plan(M, 1024, K, 1)["kernel"] == "stream_ksplit"
    rng = np.random.default_rng(11)
    # residual: r + ls * linear(x)
    p = O.make_w4_problem(M, K, 1024, seed=5)
    t = _to_dev(p, gpu)
    b = torch.from_numpy((rng.standard_normal(1024) * 0.1).astype(np.float16)).to(gpu)
    gam = torch.from_numpy((rng.standard_normal(1024) * 0.5).astype(np.float16)).to(gpu)
    r0 = torch.from_numpy(rng.standard_normal((M, 1024)).astype(np.float16)).to(gpu)
    r = r0.clone()
    E.w4a16_linear_residual(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], b, gam, r)
    lin = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=b, epilogue=1)
    want = r0.clone().addcmul_(lin, gam)
    torch.cuda.synchronize()
    step = want.float().abs() * 2.0 ** -10
    assert ((r.float() - want.float()).abs() <= 2 * step + 1e-7).all()


def test_k128_bf16_and_residual(gpu):
    """128-k stages with bf16 operands (1000 x 1024 -> 3072) against the bf16
    dequantised reference, and the residual epilogue on a 128-k launch
    (5496 x 1024 -> 1024) against the unfused chain, within 2 16-bit steps."""
    from qvggt_amd import awq_inference_engine as E
    M, N, K = 1000, 3072, 1024
    assert E.w4a16_plan(M, N, K, 0)["kernel"] == "stream_k128"
    p = O.make_w4_problem(M, K, N, seed=77)
    xb, sc, sz = _bf16_problem(p)
    x = torch.from_numpy(xb.view(np.int16)).to(gpu).view(torch.bfloat16).view(M, K)
    qw = torch.from_numpy(p["qweight"]).to(gpu)
    sct = torch.from_numpy(sc.view(np.int16)).to(gpu).view(torch.bfloat16)
    szt = torch.from_numpy(sz.view(np.int16)).to(gpu).view(torch.bfloat16)
    y = E.gemm_forward_cuda_new(x, qw, sct, szt)
    W = O.bf16_bits_to_f32(O.dequantize_bf16_bits(p["qweight"], sc, sz, N, K))
    ref = O.bf16_bits_to_f32(xb) @ W.T
    err = O.rel_err(y.float().cpu().numpy(), ref)
    assert err <= TOL, err
    M, N = 5496, 1024
    assert E.w4a16_plan(M, N, K, 1)["kernel"] == "stream_k128"
    rng = np.random.default_rng(3)
    p = O.make_w4_problem(M, K, N, seed=6)
    t = _to_dev(p, gpu)
    b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float16)).to(gpu)
    gam = torch.from_numpy((rng.standard_normal(N) * 0.5).astype(np.float16)).to(gpu)
    r0 = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float16)).to(gpu)
    r = r0.clone()
    E.w4a16_linear_residual(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], b, gam, r)
    lin = E.w4a16_linear(t["x"], t["qweight"], t["scales"], t["scaled_zeros"], bias=b, epilogue=1)
    want = r0.clone().addcmul_(lin, gam)
    torch.cuda.synchronize()
    step = want.float().abs() * 2.0 ** -10
    assert ((r.float() - want.float()).abs() <= 2 * step + 1e-7).all()
