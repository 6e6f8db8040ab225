"""Oracle: AWQ-v2 W4A16 group-128 layout, dequantisation and GEMM/GEMV semantics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference files followed (paths under ``qvggt/runtime/``):

* ``awq/qmodule.py:9-41``   make_divisible / calculate_zeros_width
* ``awq/qmodule.py:43-99``  pack_intweight (interleave=4, kstride=64)
* ``awq/qmodule.py:147-211`` scales / scaled_zeros buffer shapes
* ``awq/qmodule.py:255-327`` from_linear: q = round((W + z*s)/s), scales
  padded and transposed, scaled_zeros = -(s*z) cast to the model dtype
* ``awq_inference_engine/csrc/quantization_new/dequantize.cuh:8-51``
  nibble -> fp16 (exact), then ``hfma2(q, s, sz)`` at
  ``gemm/gemm_cuda.cu:302-307,911-916`` and ``gemv/gemv_cuda.cu:113-133``:
  one fused fp16 FMA, one rounding.
* ``gemm/gemm_cuda.cu:1125-1235`` and ``gemv/gemv_cuda.cu:197-281``:
  y[m, n] = sum_k x[m, k] * w[n, k].

How each function is pinned (tests/test_oracle_awq.py):

* ``calculate_zeros_width``: known answers (K=1024 -> 8 rows, K=4096 -> 32,
  G=64 doubling, G=-1) and the closed form ceil(ceil(K/G)/8)*8 for G>=128.
* ``pack_intweight``: (1) an emulation of the reference GEMV's per-thread
  index arithmetic (gemv_cuda.cu:83-140, a different derivation of where
  each nibble goes) reconstructs x @ W^T from the packed words; (2) a
  bit-level emulation of the lop3/magic-number nibble order of
  dequantize.cuh:15-50; (3) round trip and bijectivity.
* ``dequantize``: exhaustive over q in 0..15 against a float64 product-sum
  rounded once, plus the special cases q == z -> 0 and s = 1, sz = 0 -> q.
* ``gemm_ref``: brute-force triple loop on tiny shapes, q == z -> y == 0,
  one-hot activations read back single weight columns.
* ``quantize_intweight``: weights on an exactly representable grid
  W = s (q - z) give back q; half-way cases round to even; and the same
  expression evaluated with torch's own fp16 / bf16 tensor ops (a second
  engine for the per-op rounding) agrees element for element.
"""
from __future__ import annotations

import numpy as np

GROUP = 128
INTERLEAVE = 4
KSTRIDE = 64


# ---------------------------------------------------------------- table sizes
def make_divisible(c: int, divisor: int) -> int:
    """Ceiling division (qmodule.py:9-11)."""
    return (c + divisor - 1) // divisor


def calculate_zeros_width(in_features: int, group_size: int = 128, pack_num: int = 8) -> int:
    """Number of packed 8-wide columns of the scale table (qmodule.py:13-41).

    The scales / scaled_zeros buffers have ``calculate_zeros_width(K, G) * 8``
    rows (qmodule.py:169-211).
    """
    if group_size == -1:
        group_size = in_features
        mult = 1
    elif group_size >= 128:
        mult = 1
    elif group_size == 64:
        mult = 2
    elif group_size == 32:
        mult = 4
    else:
        raise NotImplementedError(group_size)
    base = make_divisible(in_features // group_size, pack_num)
    return make_divisible(base, mult) * mult


def scale_rows(in_features: int, group_size: int = 128) -> int:
    return calculate_zeros_width(in_features, group_size) * 8


# ------------------------------------------------------------------- packing
def _layout_axes(N: int, K: int):
    """Closed form of the AWQ-v2 layout.

    For weight (n, k): rg = n//4, r = n%4, kb = k//64, c = (k%64)//32,
    j = k%32, h = j//8, f = (j%8)//2, e = j%2.  The nibble sits in
    qweight[rg, 64*kb + 16*r + 8*c + 2*f + e] at bit offset 4*h.
    Equivalently: a little-endian u32 at int16 columns
    (64kb + 16r + 8c + 2f, +1) holds nibble i = 4e + h for
    k = 64kb + 32c + 8h + 2f + e.
    """
    assert N % INTERLEAVE == 0 and K % KSTRIDE == 0
    return (N // 4, 4, K // 64, 2, 4, 4, 2)  # (rg, r, kb, c, h, f, e)


def pack_intweight(U: np.ndarray) -> np.ndarray:
    """Pack unsigned int4 values U (N, K) into the AWQ-v2 int16 (N/4, K) layout.

    Semantics of qmodule.py:43-99 with interleave=4, kstride=64, derived as the
    closed form documented in ``_layout_axes``.
    """
    U = np.asarray(U)
    N, K = U.shape
    if U.min() < 0 or U.max() > 15:
        raise ValueError("int4 values must be in 0..15")
    V = U.astype(np.uint16).reshape(_layout_axes(N, K))
    # -> (rg, kb, r, c, f, e, h): h is the nibble slot inside one int16
    V = V.transpose(0, 2, 1, 3, 5, 6, 4)
    packed = V[..., 0] | (V[..., 1] << 4) | (V[..., 2] << 8) | (V[..., 3] << 12)
    return packed.reshape(N // 4, K).view(np.int16)


def unpack_intweight(qweight: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of ``pack_intweight``: int16 (N/4, K) -> uint8 (N, K)."""
    q = np.asarray(qweight).view(np.uint16).reshape(N // 4, K // 64, 4, 2, 4, 2)
    nib = np.stack([(q >> (4 * h)) & 0xF for h in range(4)], axis=-1)  # (rg,kb,r,c,f,e,h)
    nib = nib.transpose(0, 2, 1, 3, 6, 4, 5)  # (rg, r, kb, c, h, f, e)
    return nib.reshape(N, K).astype(np.uint8)


def quantize_intweight(W: np.ndarray, s: np.ndarray, z: np.ndarray, group_size: int = 128,
                       dtype=np.float16) -> np.ndarray:
    """Integer weights of ``from_linear`` (qmodule.py:255-315):
    q = round((W + z*s) / s) evaluated as the reference's 16-bit tensor ops do,
    each op in float32 and rounded to ``dtype`` (fp16, or "bf16" given as
    float32 values), torch.round = round half to even.  W (N, K); s, z
    (N, K / group).  Returns int32 (N, K)."""
    if dtype == np.float16:
        r = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    else:
        r = lambda a: bf16_bits_to_f32(f64_to_bf16_bits(np.asarray(a, np.float32).astype(np.float64)))
    W, s, z = (r(a) for a in (W, s, z))
    K = W.shape[1]
    gidx = np.arange(K) // (K if group_size == -1 else group_size)
    sz = r(z * s)
    t = r(W + sz[:, gidx])
    u = r(t / s[:, gidx])
    return np.rint(u).astype(np.int32)


# ---------------------------------------------------------- scale / zero tables
def build_tables(s: np.ndarray, z: np.ndarray, in_features: int, group_size: int = 128,
                 dtype=np.float16):
    """scales / scaled_zeros buffers from per-(n, group) s and integer z.

    qmodule.py:255-283 (scales zero-padded to ``scale_rows`` then transposed)
    and qmodule.py:317-327 (scaled_zeros = -(float(s) * z) cast to dtype).
    s, z: (N, K/G).  Returns two (rows, N) arrays of ``dtype``.
    """
    N, G = s.shape
    rows = scale_rows(in_features, group_size)
    s_d = np.asarray(s).astype(dtype)
    scales = np.zeros((N, rows), dtype)
    scales[:, :G] = s_d
    sz = np.zeros((N, rows), dtype)
    sz[:, :G] = (-(s_d.astype(np.float32) * np.asarray(z).astype(np.float32))).astype(dtype)
    return np.ascontiguousarray(scales.T), np.ascontiguousarray(sz.T)


# ----------------------------------------------------------------- dequantise
def _round_to(x64: np.ndarray, dtype) -> np.ndarray:
    if dtype == np.float16:
        return x64.astype(np.float16)
    if dtype == "bfloat16":
        return f64_to_bf16_bits(x64)
    raise ValueError(dtype)


def f64_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float64 -> bfloat16 (nearest-even, one rounding); uint16 bit patterns.

    Rounds the significand to 8 bits directly in float64 (frexp/rint), so no
    intermediate float32 rounding is involved.  Normal range only.
    """
    x = np.asarray(x, np.float64)
    m, e = np.frexp(x)                       # x = m * 2**e, 0.5 <= |m| < 1
    r = np.ldexp(np.rint(np.ldexp(m, 8)), e - 8)   # exact in float32 now
    return (r.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequantize(qweight: np.ndarray, scales: np.ndarray, scaled_zeros: np.ndarray,
               N: int, K: int, group_size: int = 128) -> np.ndarray:
    """Dequantised fp16 weights W (N, K): w = fp16_rn(q*s + sz), one rounding.

    dequantize.cuh:8-51 makes q exact; the hfma2 (gemm_cuda.cu:911-916) is a
    fused multiply-add with a single rounding.  q*s + sz is exact in float64
    (an 11-bit by 4-bit product plus an fp16), so rounding the float64 sum
    once to fp16 reproduces the fused operation bit for bit.
    """
    U = unpack_intweight(qweight, N, K).astype(np.float64)
    g = np.arange(K) // group_size
    s = np.asarray(scales, np.float16)[g, :].T.astype(np.float64)      # (N, K)
    sz = np.asarray(scaled_zeros, np.float16)[g, :].T.astype(np.float64)
    return (U * s + sz).astype(np.float16)


def dequantize_bf16_bits(qweight, scales_bits, zeros_bits, N, K, group_size=128):
    """bf16 variant: inputs/outputs as uint16 bf16 bit patterns (dequantize.cuh:53-89)."""
    U = unpack_intweight(qweight, N, K).astype(np.float64)
    g = np.arange(K) // group_size
    s = bf16_bits_to_f32(np.asarray(scales_bits)[g, :].T).astype(np.float64)
    sz = bf16_bits_to_f32(np.asarray(zeros_bits)[g, :].T).astype(np.float64)
    return f64_to_bf16_bits(U * s + sz)


def gemm_ref(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """fp32 reference y = x @ w^T for the W4A16 GEMM/GEMV (gemm_cuda.cu:1125-1235)."""
    x32 = np.asarray(x).reshape(-1, np.asarray(x).shape[-1]).astype(np.float32)
    return x32 @ np.asarray(w).astype(np.float32).T


def rel_err(y: np.ndarray, y_ref: np.ndarray) -> float:
    """max|y - y_ref| / max|y_ref| -- the tolerance metric for fp16 outputs."""
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    den = max(np.abs(y_ref).max(), 1e-30)
    return float(np.abs(y - y_ref).max() / den)


# --------------------------------------------------------- synthetic inputs
def make_w4_problem(M: int, K: int, N: int, seed: int = 0, group_size: int = 128):
    """Seeded synthetic W4A16 linear as specified for the qkv / MLP configs.

    activations fp16 ~ N(0,1) (seed), int4 weights U{0..15} (seed+1),
    fp16 scales U[0.005, 0.02] (seed+2), int zeros U{0..15} (seed+3).
    """
    x = np.random.default_rng(seed).standard_normal((M, K), dtype=np.float32).astype(np.float16)
    U = np.random.default_rng(seed + 1).integers(0, 16, size=(N, K), dtype=np.uint8)
    G = K // group_size
    s = np.random.default_rng(seed + 2).uniform(0.005, 0.02, size=(N, G)).astype(np.float16)
    z = np.random.default_rng(seed + 3).integers(0, 16, size=(N, G))
    qweight = pack_intweight(U)
    scales, szeros = build_tables(s, z, K, group_size)
    return dict(x=x, U=U, s=s, z=z, qweight=qweight, scales=scales, scaled_zeros=szeros)
