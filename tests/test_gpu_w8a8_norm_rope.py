"""GPU parity of the W8A8, normalisation and RoPE ops against the oracle.

Bars: int32 accumulators, int8 codes, per-token scales and every fp16 output
of the row kernels bit-exact (the kernels and oracle/w8a8.py share the
arithmetic contract and reduction order); fused_rope_with_pos within one
fp16 ulp (its cos/sin of arbitrary fp32 angles go through fp64 library calls
on both sides); rope2d bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import rope as R
from oracle import w8a8 as Q

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy()
    return t.numpy()


def _rng(seed):
    return np.random.default_rng(seed)


_TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _as(x, dt: str) -> np.ndarray:
    """fp32 values of storage type ``dt`` (exactly representable in it)."""
    return Q.round_store(np.asarray(x, np.float32), dt)


def _dev(x32: np.ndarray, dt: str, gpu) -> torch.Tensor:
    """A device tensor of type ``dt`` holding the fp32 values x32 exactly."""
    return torch.from_numpy(np.ascontiguousarray(x32, np.float32)).to(_TORCH_DT[dt]).to(gpu)


def _vals(t: torch.Tensor) -> np.ndarray:
    """fp32 values of a device tensor (exact for fp16 / bf16 / fp32)."""
    return t.detach().float().cpu().numpy()


# ----------------------------------------------------------- quantisation
@pytest.mark.parametrize("M,D,dt", [(1374, 1024, "f16"), (10992, 1024, "f16"), (300, 4096, "f32"),
                                    (5, 8, "f16"), (64, 8192, "f16"), (777, 1024, "bf16"), (3, 4096, "bf16")])
def test_invoke_quant_bit_exact(gpu, M, D, dt):
    """quantization.cu:87-95 dispatches float, half and bfloat16."""
    from qvggt_amd import awq_inference_engine as E
    x = _as(_rng(M + D).standard_normal((M, D)) * 3, dt)
    x[0] = 0  # amax = 0 row
    xt = _dev(x, dt, gpu)
    q = torch.empty(M, D, dtype=torch.int8, device=gpu)
    s = torch.empty(M, dtype=torch.float16, device=gpu)
    E.invoke_quant(q, xt, s)
    qr, sr = Q.quant_per_token(x)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(_bits(s), sr.view(np.int16))


# ------------------------------------------------------------------ GEMM
# K = 64, 128, 192 and 256 cover one to four 64-k stages (the pipeline's
# prologue and last-stage paths); (4100, 4112) and (3001, 4624) walk the tiles in column groups of 6 and 5
# whose last group is narrower (17 and 19 tile columns); (10992, 4096) in two
# groups of 8; the others in whole rows.
@pytest.mark.parametrize("M,N,K", [(10992, 4096, 1024), (10992, 1024, 4096), (300, 3072, 1024), (1, 48, 64),
                                   (50, 64, 128), (37, 272, 192), (200, 512, 256), (4100, 4112, 1024),
                                   (3001, 4624, 1024)])
def test_w8a8_int32_bit_exact(gpu, M, N, K):
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(M * 7 + N)
    a = rng.integers(-128, 128, (M, K)).astype(np.int8)
    b = np.clip(np.rint(rng.standard_normal((N, K)) * 32), -128, 127).astype(np.int8)
    acc = E.w8a8_gemm_int32(torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu))
    assert np.array_equal(acc.cpu().numpy(), Q.w8a8_int32(a, b))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M,N,K", [(2748, 4096, 1024), (129, 1024, 4096), (4100, 4112, 1024)])
def test_w8a8_gemm_fp16_bit_exact(gpu, M, N, K, bias):
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    a, as_ = Q.quant_per_token(x)
    b = np.clip(np.rint(rng.standard_normal((N, K)) * 32), -128, 127).astype(np.int8)
    ws = rng.uniform(0.001, 0.01, N).astype(np.float16)
    bb = (rng.standard_normal(N) * 0.1).astype(np.float16) if bias else None
    out = torch.empty(M, N, dtype=torch.float16, device=gpu)
    args = [torch.from_numpy(v).to(gpu) for v in (a, b, ws, as_)] + [out]
    if bias:
        E.w8a8_gemm_fuse_bias_forward_cuda(*args, torch.from_numpy(bb).to(gpu))
    else:
        E.w8a8_gemm_forward_cuda(*args)
    ref = Q.w8a8_epilogue(Q.w8a8_int32(a, b), ws, as_, bb)
    assert np.array_equal(_bits(out), ref.view(np.int16))


@pytest.mark.parametrize("M,N,K", [(10992, 1024, 4096), (1374, 1024, 1024), (129, 1040, 1024)])
def test_w8a8_linear_residual_bit_exact(gpu, M, N, K):
    """qv_w8a8_gemm_residual: residual = fp16(residual + gamma * o), o the bit-exact
    fp16 epilogue of the GEMM with bias; o * gamma is exact in fp32, so the
    result is one rounding of residual + o * gamma.  The 10992 x 4096 -> 1024
    shape takes 128-row tiles (epilogue operands prefetched), the others
    64-row tiles; N = 1040 leaves a partial column tile."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(M * 7 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    a, as_ = Q.quant_per_token(x)
    b = np.clip(np.rint(rng.standard_normal((N, K)) * 32), -128, 127).astype(np.int8)
    ws = rng.uniform(0.0005, 0.005, N).astype(np.float16)
    bb = (rng.standard_normal(N) * 0.1).astype(np.float16)
    g = rng.uniform(0.005, 1.5, N).astype(np.float16)
    r0 = rng.standard_normal((M, N)).astype(np.float16)
    resid = torch.from_numpy(r0).to(gpu)
    t = [torch.from_numpy(v).to(gpu) for v in (a, b, ws, as_, bb, g)]
    E.w8a8_linear_residual(*t, resid)
    o = Q.w8a8_epilogue(Q.w8a8_int32(a, b), ws, as_, bb)
    ref = (r0.astype(np.float32) + o.astype(np.float32) * g.astype(np.float32)).astype(np.float16)
    assert np.array_equal(_bits(resid), ref.view(np.int16))


# ------------------------------------------------------ packed weights
def _pack_mirror(b: np.ndarray) -> np.ndarray:
    """The packed layout from its definition: 16-byte chunk
    ((cb * KS + ks) * 2 + s) * 64 + L = bytes [64 ks + 32 s + 16 (L // 32), +16)
    of row 32 cb + L % 32, rows past N zero."""
    N, K = b.shape
    KS, CB = K // 64, (N + 31) // 32
    bp = np.zeros((CB * 32, K), np.int8)
    bp[:N] = b
    # (cb, r, ks, s, half, 16) -> (cb, ks, s, half, r, 16): lane L = 32 half + r
    v = bp.reshape(CB, 32, KS, 2, 2, 16).transpose(0, 2, 3, 4, 1, 5)
    return np.ascontiguousarray(v).reshape(-1)


@pytest.mark.parametrize("N,K", [(4096, 1024), (272, 192), (48, 64)])
def test_w8a8_pack_weight_layout(gpu, N, K):
    from qvggt_amd import awq_inference_engine as E
    b = _rng(N + K).integers(-128, 128, (N, K)).astype(np.int8)
    p = E.w8a8_pack_weight(torch.from_numpy(b).to(gpu))
    assert p.numel() == E.w8a8_packed_bytes(N, K) == (N + 31) // 32 * 32 * K
    assert np.array_equal(p.cpu().numpy(), _pack_mirror(b))


# (37, 272, 192): three k stages (odd: the last loop iteration multiplies zero
# weights) and N = 272, which the layout pads to 288; (50, 1040, 64) one stage;
# (129, 1040, 320) five; (10992, 4096, 1024) and (10992, 1024, 4096) the
# 128-row tiles of the benchmark's MLP pair; (4100, 4112, 1024) column groups
# with a narrower last group.
@pytest.mark.parametrize("mode", ["plain", "bias", "residual"])
@pytest.mark.parametrize("M,N,K", [(10992, 4096, 1024), (10992, 1024, 4096), (1374, 3072, 1024), (37, 272, 192),
                                   (50, 1040, 64), (129, 1040, 320), (4100, 4112, 1024)])
def test_w8a8_gemm_packed_bit_exact(gpu, M, N, K, mode):
    """qv_w8a8_gemm_packed against the oracle, as the unpacked GEMM is held."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(M * 3 + N + K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    a, as_ = Q.quant_per_token(x)
    b = np.clip(np.rint(rng.standard_normal((N, K)) * 32), -128, 127).astype(np.int8)
    ws = rng.uniform(0.0005, 0.005, N).astype(np.float16)
    bb = (rng.standard_normal(N) * 0.1).astype(np.float16) if mode != "plain" else None
    g = rng.uniform(0.005, 1.5, N).astype(np.float16)
    ta, tb, tws, tas = (torch.from_numpy(v).to(gpu) for v in (a, b, ws, as_))
    tbb = torch.from_numpy(bb).to(gpu) if bb is not None else None
    p = E.w8a8_pack_weight(tb)
    o = Q.w8a8_epilogue(Q.w8a8_int32(a, b), ws, as_, bb)
    if mode == "residual":
        r0 = rng.standard_normal((M, N)).astype(np.float16)
        out = torch.from_numpy(r0).to(gpu)
        E.w8a8_gemm_packed(ta, p, N, tws, tas, out, bias=tbb, gamma=torch.from_numpy(g).to(gpu))
        ref = (r0.astype(np.float32) + o.astype(np.float32) * g.astype(np.float32)).astype(np.float16)
    else:
        out = torch.empty(M, N, dtype=torch.float16, device=gpu)
        E.w8a8_gemm_packed(ta, p, N, tws, tas, out, bias=tbb)
        ref = o
    assert np.array_equal(_bits(out), ref.view(np.int16))


def test_w8a8_linear_repacks_a_changed_weight(gpu):
    """W8A8Linear runs on a packed copy of its weight; writing the weight in
    place must re-make the copy (the module's output follows the weight)."""
    from qvggt_amd import aggregator as AG
    rng = _rng(5)
    M, N, K = 200, 512, 256
    m = AG.W8A8Linear(K, N, bias=True, dev=gpu)
    x = rng.standard_normal((M, K)).astype(np.float16)
    a, as_ = Q.quant_per_token(x)
    ta, tas = torch.from_numpy(a).to(gpu), torch.from_numpy(as_).to(gpu)
    ws = rng.uniform(0.0005, 0.005, N).astype(np.float16)
    bb = (rng.standard_normal(N) * 0.1).astype(np.float16)
    m.wscales.copy_(torch.from_numpy(ws))
    m.bias.copy_(torch.from_numpy(bb))
    for seed in (1, 2):
        b = _rng(seed).integers(-128, 128, (N, K)).astype(np.int8)
        m.weight.copy_(torch.from_numpy(b))
        out = m(ta, tas)
        ref = Q.w8a8_epilogue(Q.w8a8_int32(a, b), ws, as_, bb)
        assert np.array_equal(_bits(out), ref.view(np.int16)), seed


# ------------------------------------------------------- LN + quant
@pytest.mark.parametrize("M,D,dt", [(10992, 1024, "f16"), (33, 4096, "f16"), (7, 1000, "f16"), (1001, 2048, "f16"), (18, 512, "f16"),
                                    (1374, 1024, "bf16"), (65, 4096, "bf16"), (300, 1024, "f32"), (9, 2048, "f32")])
def test_rms_norm_general_per_token_bit_exact(gpu, M, D, dt):
    """layernorm.cu:166-190 dispatches float, half and bfloat16."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(M + D)
    x = _as(rng.standard_normal((M, D)) * 2 + 0.5, dt)
    g = _as(1 + 0.1 * rng.standard_normal(D), dt)
    b = _as(0.1 * rng.standard_normal(D), dt)
    q = torch.empty(M, D, dtype=torch.int8, device=gpu)
    s = torch.empty(M, dtype=torch.float16, device=gpu)
    E.rms_norm_general(q, _dev(x, dt, gpu), _dev(g, dt, gpu), _dev(b, dt, gpu), s, 1e-6, True)
    qr, sr = Q.layernorm_quant(x, g, b, 1e-6, dt)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(_bits(s), sr.view(np.int16))


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_rms_norm_general_per_tensor_bit_exact(gpu, dt):
    """Per-tensor scale (layernorm.cu:100-123): a nonzero beta is passed and
    must be ignored (the host passes nullptr, layernorm.cu:180-187).  Random
    rows against the oracle; rows with a closed-form LayerNorm (eps = 0,
    [4, -4, ...] -> +-gamma and [2, -2, 0, 0, ...] -> +-sqrt 2 rounded to the
    storage type) against their known codes."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(9)
    M, D = 500, 1024
    x = _as(rng.standard_normal((M, D)), dt)
    g = _as(1 + 0.1 * rng.standard_normal(D), dt)
    beta = _dev(_as(0.5 + rng.standard_normal(D), dt), dt, gpu)
    sc = np.array([24.0], np.float16)
    q = torch.empty(M, D, dtype=torch.int8, device=gpu)
    E.rms_norm_general(q, _dev(x, dt, gpu), _dev(g, dt, gpu), beta, torch.from_numpy(sc).to(gpu), 1e-6, False)
    assert np.array_equal(q.cpu().numpy(), Q.layernorm_quant_per_tensor(x, g, 1e-6, sc[0], dt))
    # closed-form rows
    xk = np.stack([np.tile(np.array([4.0, -4.0], np.float32), D // 2),
                   np.tile(np.array([2.0, -2.0, 0.0, 0.0], np.float32), D // 4)])
    gk = _as(np.linspace(-40, 40, D), dt)
    gk[0::4] = 1.0        # columns 0 and 1 of the sqrt-2 row see gamma 1
    gk[1::4] = 1.0
    # an fp16 scale at which rint(T(sqrt 2) * s) != rint(sqrt(2) * s) for T = fp16 / bf16
    cand = np.unique(np.arange(1.0, 89.0, 2 ** -8).astype(np.float16)).astype(np.float64)
    sck = np.array([cand[np.rint(1.4140625 * cand) != np.rint(np.sqrt(2.0) * cand)][0]], np.float16)
    qk = torch.empty(2, D, dtype=torch.int8, device=gpu)
    E.rms_norm_general(qk, _dev(xk, dt, gpu), _dev(gk, dt, gpu), beta, torch.from_numpy(sck).to(gpu), 0.0, False)
    got = qk.cpu().numpy()
    sign = np.where(np.arange(D) % 2 == 0, 1.0, -1.0)
    want0 = np.clip(np.rint(sign * gk.astype(np.float64) * float(sck[0])), -128, 127)
    assert np.array_equal(got[0], want0.astype(np.int8))
    s32 = np.float32(sck[0])
    if dt == "f32":   # fp32 keeps LN = 2 * fp32(1/fp32(sqrt 2)); the product rounds in fp32
        ln = np.float32(2.0) * (np.float32(1.0) / np.sqrt(np.float32(2.0)))
        want = np.rint(np.float32(ln * s32))
    else:             # fp16 and bf16 both round sqrt 2 to 1.4140625
        want = np.rint(1.4140625 * float(s32))
        assert want != np.rint(np.sqrt(2.0) * float(s32))
    assert got[1, 0] == want and got[1, 1] == -want and got[1, 2] == 0 and got[1, 3] == 0
    assert np.array_equal(got, Q.layernorm_quant_per_tensor(xk, gk, 0.0, sck[0], dt))


@pytest.mark.parametrize("M,D", [(2748, 4096), (3, 64)])
def test_gelu_and_quant_bit_exact(gpu, M, D):
    from qvggt_amd import awq_inference_engine as E
    x = (_rng(M) .standard_normal((M, D)) * 2).astype(np.float16)
    q = torch.empty(M, D, dtype=torch.int8, device=gpu)
    s = torch.empty(M, dtype=torch.float16, device=gpu)
    tmp = torch.empty(M, D, dtype=torch.float16, device=gpu)
    E.gelu_and_quant(q, torch.from_numpy(x).to(gpu), s, tmp)
    qr, sr, tr = Q.gelu_and_quant(x)
    assert np.array_equal(_bits(tmp), tr.view(np.int16))
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)
    # tmp = None (no fp16 copy stored): the same codes and scales
    q2 = torch.zeros_like(q)
    s2 = torch.zeros_like(s)
    E.gelu_and_quant(q2, torch.from_numpy(x).to(gpu), s2, None)
    assert torch.equal(q2, q) and torch.equal(s2, s)


def test_gelu_and_quant_rows_near_the_fold_floor(gpu):
    """Rows whose largest |GELU| sits just below, at and just above fp16(1e-4)
    (the act.cu:47-48 fold floor) and around the smallest maximum for which
    fp16(127 / amax) is finite, rows whose maximum comes from a negative
    value, and an all-zero row, bit for bit against the oracle: the kernel
    takes a shortcut only for rows with a finite maximum above the floor and
    a finite multiplier."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(11)
    D = 1024
    rows = []
    for top in (1.5e-4, 2.0e-4, 2.0003e-4, 2.0004e-4, 2.1e-4, 3e-4, 1e-2):   # GELU(x) ~ x / 2 here
        rows.append(rng.uniform(0, top, D))
        rows.append(-rng.uniform(0, top, D))
        r = rng.uniform(0, top / 4, D)
        r[rng.integers(D)] = -top
        rows.append(r)
    big_neg = rng.uniform(0, 1.5e-4, D)
    big_neg[::97] = -3.0                   # maximum from GELU(-3) ~ -0.004
    rows += [big_neg, np.zeros(D)]
    x = np.stack(rows).astype(np.float16)
    # x = 0x0A8E, 0x0A8F, 0x0A90 (and negated) give |GELU| = fp16(1e-4) and
    # the next two fp16 values up; x = 0x1BEA .. 0x1BEC and 0x9BF6 .. 0x9BF8
    # give |GELU| = 0x17F0 .. 0x17F2 around 0x17F1, the smallest row maximum
    # whose fp16(127 / amax) is finite: one such element in a row of smaller ones
    edge = []
    for b in (0x0A8E, 0x0A8F, 0x0A90, 0x8A8E, 0x8A8F, 0x8A90, 0x1BEA, 0x1BEB, 0x1BEC, 0x9BF6, 0x9BF7, 0x9BF8):
        r = rng.uniform(-1e-4, 1e-4, D).astype(np.float16)
        r[rng.integers(D)] = np.uint16(b).view(np.float16)
        edge.append(r)
    x = np.concatenate([x, np.stack(edge)])
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], dtype=torch.float16, device=gpu)
    E.gelu_and_quant(q, torch.from_numpy(x).to(gpu), s, None)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        qr, sr, _ = Q.gelu_and_quant(x)
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)


def test_gelu_every_finite_fp16_input(gpu):
    """The fp16 GELU (and its tanh table) on all 63488 finite fp16 values,
    bit for bit against the oracle."""
    from qvggt_amd import awq_inference_engine as E
    bits = np.arange(0x10000, dtype=np.uint16)
    x = bits.view(np.float16)
    x = x[np.isfinite(x)].reshape(62, 1024)
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], dtype=torch.float16, device=gpu)
    tmp = torch.empty(x.shape, dtype=torch.float16, device=gpu)
    E.gelu_and_quant(q, torch.from_numpy(x).to(gpu), s, tmp)
    with np.errstate(over="ignore", invalid="ignore"):
        qr, sr, tr = Q.gelu_and_quant(x)
    assert np.array_equal(_bits(tmp), tr.view(np.int16))
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)


def test_per_token_quant_and_ln_quant_with_nan_rows_match_oracle(gpu):
    """A NaN element in some rows, bit for bit against the oracle: it stays out
    of the row maximum (per-token quant) or turns the whole row NaN (LN)."""
    from qvggt_amd import awq_inference_engine as E
    x = (_rng(6).standard_normal((4, 1024))).astype(np.float16)
    x[0, 17] = np.nan
    x[2, 1000] = np.nan
    xd = torch.from_numpy(x).to(gpu)
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], dtype=torch.float16, device=gpu)
    E.invoke_quant(q, xd, s)
    with np.errstate(invalid="ignore"):
        qr, sr = Q.quant_per_token(x)
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)
    g = (1 + 0.1 * _rng(7).standard_normal(1024)).astype(np.float16)
    b = (0.1 * _rng(8).standard_normal(1024)).astype(np.float16)
    E.rms_norm_general(q, xd, torch.from_numpy(g).to(gpu), torch.from_numpy(b).to(gpu), s, 1e-6, True)
    with np.errstate(invalid="ignore"):
        qr, sr = Q.layernorm_quant(x, g, b, 1e-6)
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)


def test_quant_and_ln_quant_row_edge_cases_match_oracle(gpu):
    """Rows at the edges of the kernels' row-level checks, bit for bit against
    the oracle: +-inf, a row of fp16 subnormals, a maximum of +-65504, a single
    non-zero element (per-token quant); LayerNorm outputs so small that amax
    falls below the smallest normal fp16, and rows with inf (LN + quant)."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(12)
    D = 1024
    x = (rng.standard_normal((8, D)) * 2).astype(np.float16)
    x[0, 3] = np.inf
    x[1, 9] = -np.inf
    x[2] = (rng.integers(-1023, 1024, D) * 2.0 ** -24).astype(np.float16)   # subnormals
    x[3, 100] = 65504
    x[4, 200] = -65504
    x[5] = 0
    x[5, 7] = -3.0
    xd = torch.from_numpy(x).to(gpu)
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], dtype=torch.float16, device=gpu)
    E.invoke_quant(q, xd, s)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        qr, sr = Q.quant_per_token(x)
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)
    # LN + quant: gamma / beta of 1e-5 .. 1e-3 scale the outputs to around and
    # below fp16's smallest normal (6.1e-5); rows 0 and 1 hold an inf
    for gs in (1e-5, 3e-5, 1e-4, 1e-3):
        g = (gs * (1 + 0.1 * rng.standard_normal(D))).astype(np.float16)
        b = (0.1 * gs * rng.standard_normal(D)).astype(np.float16)
        E.rms_norm_general(q, xd, torch.from_numpy(g).to(gpu), torch.from_numpy(b).to(gpu), s, 1e-6, True)
        with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
            qr, sr = Q.layernorm_quant(x, g, b, 1e-6)
        assert np.array_equal(_bits(s), sr.view(np.int16)), gs
        assert np.array_equal(q.cpu().numpy(), qr), gs


def test_gelu_non_finite_inputs_match_oracle(gpu):
    """+-inf and NaN in some rows (others finite), bit for bit against the
    oracle: the GELU output, the per-row scale and the int8 values."""
    from qvggt_amd import awq_inference_engine as E
    x = (_rng(5).standard_normal((5, 1024)) * 2).astype(np.float16)
    x[0, :3] = [np.inf, -np.inf, np.nan]
    x[1, 7] = np.inf
    x[2, 100] = -np.inf
    x[3, 1023] = np.nan
    q = torch.empty(x.shape, dtype=torch.int8, device=gpu)
    s = torch.empty(x.shape[0], dtype=torch.float16, device=gpu)
    tmp = torch.empty(x.shape, dtype=torch.float16, device=gpu)
    E.gelu_and_quant(q, torch.from_numpy(x).to(gpu), s, tmp)
    with np.errstate(over="ignore", invalid="ignore"):
        qr, sr, tr = Q.gelu_and_quant(x)
    assert np.array_equal(_bits(tmp), tr.view(np.int16))
    assert np.array_equal(_bits(s), sr.view(np.int16))
    assert np.array_equal(q.cpu().numpy(), qr)


# ------------------------------------------------------- normalisation
@pytest.mark.parametrize("shape,dt", [((4, 300, 1024), "f16"), ((2, 7, 4096), "f16"), ((1, 1, 64), "f16"),
                                      ((3, 333, 1024), "bf16"), ((1, 5, 4096), "bf16")])
def test_layernorm_forward_cuda_rmsnorm_bit_exact(gpu, shape, dt):
    """layernorm/layernorm.cu:8-19 dispatches half and bfloat16 (the half
    output is clamped, the bfloat16 one is not)."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(sum(shape))
    x = _as(rng.standard_normal(shape) * (1 if dt == "f16" else 3), dt)
    g = _as(rng.uniform(0.5, 1.5, shape[-1]), dt)
    if dt == "bf16":
        g[:4] = 1e5 * np.array([1, -1, 3, -3], np.float32)   # beyond the fp16 range: no clamp for bf16
        g = _as(g, dt)
    out = torch.empty(shape, dtype=_TORCH_DT[dt], device=gpu)
    E.layernorm_forward_cuda(_dev(x, dt, gpu), _dev(g, dt, gpu), out, 1e-6)
    ref = Q.rmsnorm(x.reshape(-1, shape[-1]), g, 1e-6, dt).reshape(shape)
    if dt == "f16":
        assert np.array_equal(_bits(out), ref.view(np.int16))
    else:
        assert np.array_equal(_vals(out).view(np.int32), ref.astype(np.float32).view(np.int32))
        assert np.abs(_vals(out)).max() > 65504


@pytest.mark.parametrize("M", [10992, 1374, 1])
def test_vggt_layer_norm_bit_exact(gpu, M):
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(M)
    D = 1024
    x = (rng.standard_normal((M, D)) * 1.5 + 0.3).astype(np.float16)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    b = (0.1 * rng.standard_normal(D)).astype(np.float16)
    y = E.layer_norm(torch.from_numpy(x).to(gpu), torch.from_numpy(g).to(gpu), torch.from_numpy(b).to(gpu), 1e-6)
    assert np.array_equal(_bits(y), Q.layernorm(x, g, b, 1e-6).view(np.int16))


# ------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("dt", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("transpose_out", [False, True])
@pytest.mark.parametrize("shape", [(37, 3, 16, 64, 48), (7, 2, 16, 128, 128), (5, 2, 3, 40, 20), (3, 1, 2, 1040, 1032),
                                   (2, 2, 1, 1040, 1024)],
                         ids=["vec", "vec_two_items", "elementwise", "wide_elementwise", "wide_vec"])
def test_fused_rope_with_pos(gpu, transpose_out, dt, shape):
    """fused_rope_with_pos.cu:155-161 dispatches float, half and bfloat16.
    fp16 / bf16 within one ulp of the oracle's rounding (and equal in more
    than 99.9 % of elements), fp32 within 2e-6 relative.  The shapes take the
    kernel's paths: 16-byte chunks (d2/2 and d - d2 multiples of 8; fewer
    (head, chunk) items than lanes with pass-through dims, and two items per
    lane with a two-pass angle table), element accesses (d2/2 = 10;
    d2/2 = 516), and d2 > 512, where the cos / sin of the angles are
    evaluated per element instead of once per position."""
    from qvggt_amd import awq_inference_engine as E
    rng = _rng(3)
    S, B, H, D, D2 = shape
    base = rng.standard_normal((B, S, H, D)).astype(np.float32)
    freqs = rng.uniform(-20, 20, (B, S, D2)).astype(np.float32)
    xt = torch.from_numpy(base).to(gpu).to(dt).transpose(0, 1)   # (S,B,H,D), non-contiguous
    y = E.fused_rope_with_pos_forward_func(xt, torch.from_numpy(freqs).to(gpu), transpose_out)
    assert y.shape == (S, B, H, D) and y.dtype == dt
    if dt == torch.bfloat16:
        ref = R.rope_with_pos(_vals(xt), freqs, "bf16")
        got = _vals(y)
        ulp = np.abs(ref) * 2.0 ** -7          # one bf16 ulp is at most 2**-7 of the value
        assert (np.abs(got - ref) <= np.maximum(ulp, 1e-30)).all()
        assert (got == ref).mean() > 0.999
    elif dt == torch.float16:
        ref = R.rope_with_pos(xt.cpu().numpy(), freqs)
        got = y.cpu().numpy()
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
        assert (np.abs(got.astype(np.float32) - ref.astype(np.float32)) <= ulp).all()
        assert (got == ref).mean() > 0.999
    else:
        ref = R.rope_with_pos(xt.cpu().numpy(), freqs)
        got = y.cpu().numpy()
        assert np.abs(got - ref).max() <= 2e-6 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("inplace,H,S", [(False, 16, 2), (True, 16, 2), (False, 6, 2), (True, 1, 2), (False, 48, 1),
                                         (True, 32, 1)])
def test_rope2d_bit_exact(gpu, inplace, H, S):
    """H a multiple of 16 takes the token-block kernel (H = 48: the q / k
    boundary inside a 32-row block; S = 1: a last workgroup with idle
    waves), other H the per-row kernel; H = 16 and 1 (powers of two) index
    rows by shifts, H = 6 and 48 by division."""
    from qvggt_amd import awq_inference_engine as E
    pos = R.vggt_positions(S)
    T = pos.shape[0]
    qkv = _rng(4).standard_normal((T, 3 * H * 64)).astype(np.float16)
    c, s = R.rope2d_tables(38)
    ct, st = E.rope2d_tables(38, device=gpu)
    assert np.array_equal(ct.cpu().numpy(), c) and np.array_equal(st.cpu().numpy(), s)
    qt = torch.from_numpy(qkv).to(gpu)
    pt = torch.from_numpy(pos).to(gpu)
    if inplace:
        E.rope2d(qt, pt, ct, st, H, out=qt)
        got = qt.view(T, 3, H, 64)[:, :2].cpu().numpy()
        assert np.array_equal(qt.view(T, 3, H, 64)[:, 2].cpu().numpy(), qkv.reshape(T, 3, H, 64)[:, 2])
    else:
        got = E.rope2d(qt, pt, ct, st, H).cpu().numpy()
    x = qkv.reshape(T, 3, H, 64)
    for part in range(2):
        ref = R.rope2d(x[:, part], pos, c, s)
        assert np.array_equal(got[:, part].view(np.int16), ref.view(np.int16))


@pytest.mark.parametrize("H,S", [(16, 2), (6, 2), (48, 1), (32, 1)])
def test_qknorm_rope2d_bit_exact(gpu, H, S):
    """H = 16, 48, 32: the token-block kernel (q and k rows in one 32-row
    block at 16 and 48); H = 6: the per-row kernel."""
    from qvggt_amd import awq_inference_engine as E
    pos = R.vggt_positions(S)
    T = pos.shape[0]
    rng = _rng(11)
    qkv = (rng.standard_normal((T, 3 * H * 64)) * 2 + 0.3).astype(np.float16)
    qg, qb, kg, kb = ((1 + 0.1 * rng.standard_normal(64)).astype(np.float16) if i % 2 == 0
                      else (0.1 * rng.standard_normal(64)).astype(np.float16) for i in range(4))
    c, s = R.rope2d_tables(38)
    ct, st = E.rope2d_tables(38, device=gpu)
    qt = torch.from_numpy(qkv.copy()).to(gpu)
    E.qknorm_rope2d(qt, torch.from_numpy(pos).to(gpu), ct, st, H,
                    *[torch.from_numpy(v).to(gpu) for v in (qg, qb, kg, kb)], eps=1e-6)
    got = qt.view(T, 3, H, 64).cpu().numpy()
    x = qkv.reshape(T, 3, H, 64)
    ref = R.qknorm_rope2d(x[:, :2], pos, c, s, qg, qb, kg, kb, 1e-6)
    assert np.array_equal(got[:, :2].view(np.int16), ref.view(np.int16))
    assert np.array_equal(got[:, 2], x[:, 2])
