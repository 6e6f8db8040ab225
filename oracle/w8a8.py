"""Oracle: W8A8 quantisation, LayerNorm/RMSNorm and activation semantics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference files followed (paths under
``qvggt/runtime/awq_inference_engine/csrc/``):

* ``w8a8/quantization.cu:42-96`` per-token quantisation: amax = max|x| (fp32),
  scale = fp16_rn(amax / 127.0f), q = sat_s8(rint(x * (127.0f / amax)))
  (``utils.cuh:75-80``: cvt.rni.sat -- round half to even, saturate, NaN -> 0).
* ``w8a8/w8a8_gemm_cuda.cu:535-561, 851-878`` int32 accumulation, epilogue
  fp16_rn((float(acc) * ws[n]) * as[m]) (+ bias[n]).
* ``w8a8/layernorm.cu:20-151`` LayerNorm (Sum x, Sum x^2 in fp32,
  var = E[x^2] - mean^2, rs = rsqrt(var + eps)) fused with per-token int8:
  amax over the fp16-rounded outputs, floor fp16(1e-6); int8 from the fp32
  LayerNorm value * (127 / amax); scale = fp16_rn(amax / 127).
* ``w8a8/act.cu:22-75`` gelu_fast in fp16 arithmetic + per-token quant that
  multiplies (half)(127/amax) * tmp in fp16.
* ``layernorm/layernorm.cu:31-57`` (+ ``reduction.cuh:60-71``) T5 RMSNorm,
  output clamped to +-(65504 - 1000) before the fp16 conversion.

Arithmetic contract shared with the GPU kernels (so results are bit-exact):
IEEE fp32 operations, one rounding each, no fused multiply-add except where
the product is exact; IEEE division and square root (the reference was built
with --use_fast_math, whose approximations are not reproduced); tanh of the
GELU evaluated in float64 and rounded to fp32.  Row reductions use the
kernel's fixed order (``row_sum_f32``): element chunks of 8 are dealt to 64
lanes (lane l owns chunks l, l+64, ...), each lane sums its elements in
order, then a butterfly over lane distances 1, 2, 4, 8, 16, 32.

Pinning (tests/test_oracle_w8a8.py): known answers (x = k*amax/127 -> k,
amax = 0 -> 0, saturation, half-even ties), float64 LayerNorm/RMSNorm within
fp32 rounding, reduction order against math.fsum, exact int64 matmul against
brute-force loops, gelu_fast against the closed-form tanh-GELU in float64.
"""
from __future__ import annotations

import numpy as np

from .awq import bf16_bits_to_f32, f64_to_bf16_bits

F32 = np.float32
F16 = np.float16
DTYPES = ("f16", "bf16", "f32")


def round_store(t, dtype: str = "f16") -> np.ndarray:
    """fp32 values rounded (nearest even) to a kernel's storage type T and read
    back as fp32: the ``cuda_cast<T>(...)`` of a float in the reference kernels,
    which dispatch half, bfloat16 and float (dispatch_utils.h)."""
    t = np.asarray(t, F32)
    if dtype == "f16":
        return t.astype(F16).astype(F32)
    if dtype == "bf16":
        with np.errstate(invalid="ignore"):
            return bf16_bits_to_f32(f64_to_bf16_bits(t.astype(np.float64)))
    if dtype == "f32":
        return t
    raise ValueError(dtype)


# --------------------------------------------------------------- rounding
def sat_s8(v: np.ndarray) -> np.ndarray:
    """cvt.rni.sat.s8.f32: round half to even, saturate to [-128, 127], NaN -> 0."""
    v = np.asarray(v, np.float64)
    r = np.rint(v)
    r = np.where(np.isnan(r), 0.0, r)
    return np.clip(r, -128, 127).astype(np.int8)


# ------------------------------------------------------ reduction order
LANES = 64
CHUNK = 8


def row_sum_f32(v: np.ndarray) -> np.ndarray:
    """fp32 row sums of v (M, D) in the kernels' fixed order (see module doc)."""
    v = np.asarray(v, F32)
    M, D = v.shape
    per = LANES * CHUNK
    J = -(-D // per)
    pad = np.zeros((M, J * per), F32)
    pad[:, :D] = v
    p = pad.reshape(M, J, LANES, CHUNK)
    acc = np.zeros((M, LANES), F32)
    for j in range(J):
        for e in range(CHUNK):
            acc = (acc + p[:, j, :, e]).astype(F32)
    lane = np.arange(LANES)
    for off in (1, 2, 4, 8, 16, 32):
        acc = (acc + acc[:, lane ^ off]).astype(F32)
    return acc[:, 0]


# ------------------------------------------------------------ quantisation
def quant_per_token(x: np.ndarray):
    """invoke_quant (quantization.cu:42-96): returns (int8 (M,K), fp16 scale (M,))."""
    xf = np.asarray(x).astype(F32)
    # quantization.cu:49-56: `if (val > amax_val) amax_val = val` from 0, so a
    # NaN never enters the maximum (fmax skips it)
    amax = np.fmax.reduce(np.abs(xf), axis=1, initial=F32(0.0)).astype(F32)
    scale = (amax / F32(127.0)).astype(F32).astype(F16)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (F32(127.0) / amax).astype(F32)
        q = sat_s8((xf * inv[:, None]).astype(F32))
    return q, scale


# ----------------------------------------------------------------- GEMM
def w8a8_int32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators a (M,K) int8 . b (N,K)^T int8.

    Uses a float64 BLAS product: every partial sum is an integer of magnitude
    <= K * 2**14 < 2**53, so float64 represents it exactly and the result is
    the exact integer dot product (checked against int64 loops in tests)."""
    a = np.asarray(a)
    K = a.shape[1]
    assert K * 128 * 128 < 2 ** 53
    r = np.asarray(a, np.float64) @ np.asarray(b, np.float64).T
    return r.astype(np.int64).astype(np.int32)


def w8a8_epilogue(acc: np.ndarray, ws: np.ndarray, as_: np.ndarray, bias=None) -> np.ndarray:
    """fp16_rn((float(acc) * ws[n]) * as[m] (+ bias[n])), fp32 ops, one rounding each."""
    t = (acc.astype(F32) * np.asarray(ws).astype(F32)[None, :]).astype(F32)
    t = (t * np.asarray(as_).astype(F32)[:, None]).astype(F32)
    if bias is not None:
        t = (t + np.asarray(bias).astype(F32)[None, :]).astype(F32)
    return t.astype(F16)


# ---------------------------------------------------------- normalisation
def _mean_rs_diffsq(xf: np.ndarray, eps: float):
    D = xf.shape[1]
    s = row_sum_f32(xf)
    s2 = row_sum_f32((xf * xf).astype(F32))
    mean = (s / F32(D)).astype(F32)
    var = ((s2 / F32(D)).astype(F32) - (mean * mean).astype(F32)).astype(F32)
    rs = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    return mean, rs


def layernorm_quant(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float, dtype: str = "f16"):
    """rms_norm_general with use_per_token_quant=True (w8a8/layernorm.cu:20-151).

    ``dtype`` is the input's storage type T ("f16", "bf16", "f32"; x, gamma
    and beta hold values of that type): amax runs over T(y) from a floor of
    T(1e-6) (layernorm.cu:103-113).  Returns (int8 (M,D), fp16 scale (M,))."""
    xf = np.asarray(x).astype(F32)
    g = np.asarray(gamma).astype(F32)[None, :]
    b = np.asarray(beta).astype(F32)[None, :]
    mean, rs = _mean_rs_diffsq(xf, eps)
    t = ((xf - mean[:, None]).astype(F32) * rs[:, None]).astype(F32)
    t = (t * g).astype(F32)
    t = (t + b).astype(F32)
    yT = round_store(t, dtype)
    # layernorm.cu:103-113: amax = cuda_max(|y|, amax) from 1e-6 in the input
    # type; that max keeps the non-NaN operand, so NaN never enters it
    floor = round_store(np.array([1e-6], F32), dtype)[0]
    amax = np.fmax.reduce(np.abs(yT), axis=1, initial=floor).astype(F32)
    dyn = (F32(127.0) / amax).astype(F32)
    q = sat_s8((t * dyn[:, None]).astype(F32))
    scale = (amax / F32(127.0)).astype(F32).astype(F16)
    return q, scale


def layernorm_quant_per_tensor(x, gamma, eps, scale_fp16, dtype: str = "f16"):
    """rms_norm_general with use_per_token_quant=False (layernorm.cu:100-123,
    host layernorm.cu:180-187 passes beta = nullptr): no beta,
    int8 = sat(rint(float(T(LN * gamma)) * float(scale))), T the input's
    storage type, scale the fp16 per-tensor scale."""
    xf = np.asarray(x).astype(F32)
    g = np.asarray(gamma).astype(F32)[None, :]
    mean, rs = _mean_rs_diffsq(xf, eps)
    t = ((xf - mean[:, None]).astype(F32) * rs[:, None]).astype(F32)
    t = (t * g).astype(F32)
    yT = round_store(t, dtype)
    return sat_s8((yT * F32(np.float16(scale_fp16))).astype(F32))


def rmsnorm(x: np.ndarray, gamma: np.ndarray, eps: float, dtype: str = "f16") -> np.ndarray:
    """T5 RMSNorm (layernorm/layernorm.cu:31-57): (x * rs) * g, for half
    clamped to +-(65504 - 1000) before the conversion (reduction.cuh:60-71,
    clamp_inf_for_half; the bfloat16 instantiation converts unclamped).
    Returns fp16 for dtype "f16", else fp32 values of the storage type."""
    xf = np.asarray(x).astype(F32)
    D = xf.shape[1]
    s2 = row_sum_f32((xf * xf).astype(F32))
    rs = (F32(1.0) / np.sqrt(((s2 / F32(D)).astype(F32) + F32(eps)).astype(F32))).astype(F32)
    t = ((xf * rs[:, None]).astype(F32) * np.asarray(gamma).astype(F32)[None, :]).astype(F32)
    if dtype == "f16":
        t = np.clip(t, F32(-65504.0 + 1000.0), F32(65504.0 - 1000.0))
        return t.astype(F16)
    return round_store(t, dtype)


def layernorm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """VGGT LayerNorm (torch.nn.LayerNorm semantics, fp32 statistics, two-pass
    variance): ((x - mean) * rs) * g + b -> fp16.  Not in the reference (the
    model graph lives in the absent vggt-hf); restated from nn.LayerNorm."""
    xf = np.asarray(x).astype(F32)
    D = xf.shape[1]
    mean = (row_sum_f32(xf) / F32(D)).astype(F32)
    d = (xf - mean[:, None]).astype(F32)
    var = (row_sum_f32((d * d).astype(F32)) / F32(D)).astype(F32)
    rs = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    t = (d * rs[:, None]).astype(F32)
    t = (t * np.asarray(gamma).astype(F32)[None, :]).astype(F32)
    t = (t + np.asarray(beta).astype(F32)[None, :]).astype(F32)
    return t.astype(F16)


# ------------------------------------------------------------- activations
def _h(v):
    """Round to fp16 (every fp16 operation of act.cu is one rounding)."""
    return np.asarray(v, np.float64).astype(F16)


def gelu_fast_f16(x: np.ndarray) -> np.ndarray:
    """act.cu:22-28 with T = half, evaluated as fp16 operations:
    f = x; a = f*0.79788456; b = (0.044715*f)*x; c = 1 + b; u = a*c;
    t = fp16(fp32(tanh(u))); y = (0.5*x) * (1 + t)."""
    x = np.asarray(x, F16).astype(np.float64)
    c1 = float(F16(0.79788456))
    c2 = float(F16(0.044715))
    a = _h(x * c1).astype(np.float64)
    b = _h(_h(c2 * x).astype(np.float64) * x).astype(np.float64)
    c = _h(1.0 + b).astype(np.float64)
    u = _h(a * c).astype(np.float64)
    t = np.tanh(u).astype(F32).astype(F16).astype(np.float64)
    y = _h(_h(0.5 * x).astype(np.float64) * _h(1.0 + t).astype(np.float64))
    return y


def gelu_and_quant(x: np.ndarray):
    """gelu_and_quant (act.cu:30-90): returns (int8 (M,d), fp16 scale (M,), tmp fp16 (M,d))."""
    tmp = gelu_fast_f16(x)
    t32 = tmp.astype(F32)
    zero = F32(F16(0.0001))
    folded = np.where(t32 > zero, t32, -t32)   # act.cu:47-48: not a plain abs
    # act.cu:49-50: `if ((float)t > amax_val) amax_val = (float)t` from 0, so a
    # NaN never enters the maximum (fmax skips it)
    amax = np.fmax.reduce(folded, axis=1, initial=F32(0.0)).astype(F32)
    # the strict comparison from +0 never takes a -0 (a zero t folds to -0):
    # a row with no folded value above zero keeps amax = +0
    amax = np.where(amax > 0, amax, F32(0.0)).astype(F32)
    scale = (amax / F32(127.0)).astype(F32).astype(F16)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        inv = (F32(127.0) / amax).astype(F32).astype(F16).astype(np.float64)
        prod = (inv[:, None] * tmp.astype(np.float64)).astype(F16).astype(F32)
    return sat_s8(prod), scale, tmp


def gelu_tanh_f64(x: np.ndarray) -> np.ndarray:
    """Closed-form tanh-GELU in float64 (for pinning gelu_fast_f16)."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))
