"""Pins the W4A16 oracle (oracle/awq.py) with checks that do not restate it.

* pack layout: an emulation of the reference GEMV's per-thread index
  arithmetic (gemv_cuda.cu:83-140) -- a second derivation of which k each
  nibble multiplies -- must reproduce x @ W^T from the packed words;
* nibble order: a bit-level emulation of dequantize.cuh:15-50 (lop3 with the
  0x64006400 magic, sub / fma by 1/16 and -64);
* dequant rounding: exact rational arithmetic with a hand-written
  round-to-nearest-even to fp16 (no numpy float conversion involved);
* GEMM: brute-force loops and the special cases q == z and one-hot inputs.
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import awq as O


# ------------------------------------------------------------ table widths
@pytest.mark.parametrize("K,G,expect", [
    (1024, 128, 1), (4096, 128, 4), (2048, 128, 2), (8192, 128, 8), (9 * 128, 128, 2),
    (1024, 64, 2), (1024, 32, 4), (1024, -1, 1), (128, 128, 1),
])
def test_calculate_zeros_width_known_answers(K, G, expect):
    assert O.calculate_zeros_width(K, G) == expect


def test_scale_rows_closed_form():
    for K in range(128, 128 * 40, 128):
        assert O.scale_rows(K, 128) == -(-(-(-K // 128)) // 8) * 8
    assert O.scale_rows(1024) == 8 and O.scale_rows(4096) == 32


# ------------------------------------------------------------ pack layout
def _ref_gemv_consumer(x, qweight, N, K):
    """Emulate gemv_cuda.cu:83-140 index arithmetic with exact integer weights.

    NPerBlock=2, kInterleave=4, kElemsPerThread=32, kThreadsNumPerTile=2,
    BlockSize=256.  Thread tid of block b reads 16 bytes (4 u32) of qweight row
    2b+idx at int16 column tid*8 (+ 8192*it), splits each u32 into the
    half2 pairs (n_i, n_{i+4}) of dequantize.cuh, re-shuffles them with
    (i + 4j) -> position (i*4 + j)*2 + e and multiplies by the 32 activations
    at act_k_offset = tid//8*64 + (tid%2)*32.  The output channel is
    8b + 4*idx + (tid//2)%4.
    """
    M = x.shape[0]
    words = np.asarray(qweight).view(np.uint16).reshape(N // 4, K).astype(np.uint32)
    y = np.zeros((M, N), np.int64)
    for b in range(N // 8):
        for tid in range(256):
            thd_row = (tid // 2) % 4
            for it in range(0, (K * 4) // 8192 + 1):
                kk = tid * 32 + it * 8192
                if kk >= K * 4:
                    continue
                act_k = (tid // 8) * 64 + (tid % 2) * 32 + it * (256 * 32 // 4)
                for idx in range(2):
                    row = 2 * b + idx
                    col16 = kk // 4
                    u32 = [int(words[row, col16 + 2 * w]) | (int(words[row, col16 + 2 * w + 1]) << 16)
                           for w in range(4)]
                    buf = []
                    for w in u32:  # dequantize_s4_to_fp16x2 output order
                        nib = [(w >> (4 * i)) & 0xF for i in range(8)]
                        buf += [nib[0], nib[4], nib[1], nib[5], nib[2], nib[6], nib[3], nib[7]]
                    deq = [0] * 32
                    for i in range(4):
                        for j in range(4):
                            pos = (i + j * 4) * 2
                            deq[(i * 4 + j) * 2 + 0] = buf[pos]
                            deq[(i * 4 + j) * 2 + 1] = buf[pos + 1]
                    n = 8 * b + 4 * idx + thd_row
                    for m in range(M):
                        y[m, n] += sum(int(x[m, act_k + t]) * deq[t] for t in range(32))
    return y


@pytest.mark.parametrize("N,K", [(8, 64), (16, 128), (8, 256)])
def test_pack_matches_reference_gemv_consumer(N, K):
    rng = np.random.default_rng(N * 1000 + K)
    U = rng.integers(0, 16, size=(N, K))
    x = rng.integers(-3, 4, size=(2, K))
    y = _ref_gemv_consumer(x, O.pack_intweight(U), N, K)
    assert np.array_equal(y, x @ U.T)


def test_pack_roundtrip_and_bijection():
    rng = np.random.default_rng(7)
    for N, K in [(4, 64), (12, 192), (64, 512), (3072, 1024)]:
        U = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
        P = O.pack_intweight(U)
        assert P.shape == (N // 4, K) and P.dtype == np.int16
        assert np.array_equal(O.unpack_intweight(P, N, K), U)
    # every nibble position is hit exactly once: pack one-hot index patterns
    N, K = 8, 128
    seen = np.zeros((N // 4, K, 4), int)
    for n in range(N):
        for k in range(K):
            U = np.zeros((N, K), np.uint8)
            U[n, k] = 15
            p = O.pack_intweight(U).view(np.uint16)
            r, c = np.nonzero(p)
            assert len(r) == 1
            shift = int(np.log2(int(p[r[0], c[0]]) // 15)) // 4 * 4
            assert int(p[r[0], c[0]]) == 15 << shift
            seen[r[0], c[0], shift // 4] += 1
    assert (seen == 1).all()


def test_pack_closed_form_examples():
    # k = 64*kb + 32*c + 8*h + 2*f + e  -> int16 column 64*kb + 16*r + 8*c + 2*f + e, bits 4h
    N, K = 8, 128
    for (n, k) in [(0, 0), (1, 0), (5, 1), (3, 9), (0, 31), (7, 127), (2, 66)]:
        U = np.zeros((N, K), np.uint8)
        U[n, k] = 1
        p = O.pack_intweight(U).view(np.uint16)
        kb, c, j = k // 64, (k % 64) // 32, k % 32
        h, f, e = j // 8, (j % 8) // 2, j % 2
        col = 64 * kb + 16 * (n % 4) + 8 * c + 2 * f + e
        assert p[n // 4, col] == 1 << (4 * h), (n, k)


# --------------------------------------------- nibble order (dequantize.cuh)
def _f16_bits_to_float(b):
    return float(np.array([b], np.uint16).view(np.float16)[0])


def _emulate_dequantize_s4(i4s: int):
    """Bit-level emulation of dequantize.cuh:15-50 (fp16 path)."""
    def lop3(a, mask, magic):  # immLut (0xf0 & 0xcc) | 0xaa = (a & b) | c
        return (a & mask) | magic
    top = i4s >> 8
    h = [lop3(i4s, 0x000F000F, 0x64006400), lop3(i4s, 0x00F000F0, 0x64006400),
         lop3(top, 0x000F000F, 0x64006400), lop3(top, 0x00F000F0, 0x64006400)]
    out = []
    for idx, v in enumerate(h):
        lo, hi = _f16_bits_to_float(v & 0xFFFF), _f16_bits_to_float(v >> 16)
        if idx % 2 == 0:   # sub.f16x2 by 0x6400 (1024)
            out += [lo - 1024.0, hi - 1024.0]
        else:              # fma.rn.f16x2 by 1/16 and -64
            out += [lo / 16.0 - 64.0, hi / 16.0 - 64.0]
    return out


def test_dequantize_nibble_order_matches_bit_emulation():
    rng = np.random.default_rng(3)
    for w in list(rng.integers(0, 2**32, size=200, dtype=np.uint64)) + [0, 0xFFFFFFFF, 0x76543210]:
        w = int(w)
        nib = [(w >> (4 * i)) & 0xF for i in range(8)]
        got = _emulate_dequantize_s4(w)
        assert got == [nib[0], nib[4], nib[1], nib[5], nib[2], nib[6], nib[3], nib[7]]


# ------------------------------------------------------- dequant rounding
def _round_fraction_to_f16(v: Fraction) -> float:
    """Round an exact rational to the nearest fp16 (ties to even), by hand."""
    if v == 0:
        return 0.0
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    e = max(e, -14)                      # subnormal range shares exponent -14
    scaled = abs(v) / Fraction(2) ** (e - 10)   # 10 fraction bits
    q, r = divmod(scaled.numerator, scaled.denominator)
    rem = Fraction(r, scaled.denominator)
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and q % 2 == 1):
        q += 1
    return sign * float(Fraction(q) * Fraction(2) ** (e - 10))


def test_dequantize_single_rounding_exhaustive_q():
    rng = np.random.default_rng(11)
    s = rng.uniform(0.005, 0.02, size=40).astype(np.float16)
    z = rng.integers(0, 16, size=40)
    N, K = 16, 128
    for i in range(0, 40, 16):
        ss = np.resize(s[i:i + 16], 16)[:, None]
        zz = np.resize(z[i:i + 16], 16)[:, None]
        U = np.tile(np.arange(16, dtype=np.uint8), (N, K // 16))
        scales, szeros = O.build_tables(ss, zz, K)
        W = O.dequantize(O.pack_intweight(U), scales, szeros, N, K)
        for n in range(N):
            sv = Fraction(float(scales[0, n]))
            zv = Fraction(float(szeros[0, n]))
            for q in range(16):
                assert float(W[n, q]) == _round_fraction_to_f16(q * sv + zv)


def test_dequantize_special_cases():
    N, K = 32, 256
    rng = np.random.default_rng(5)
    z = rng.integers(0, 16, size=(N, K // 128))
    s = rng.uniform(0.005, 0.02, size=(N, K // 128)).astype(np.float16)
    # q == z  ->  w = fp16(z*s - fp16(s*z)): only the rounding residual of sz,
    # at most half an fp16 ulp of s*z
    U = np.repeat(z, 128, axis=1).astype(np.uint8)
    sc, sz = O.build_tables(s, z, K)
    W = O.dequantize(O.pack_intweight(U), sc, sz, N, K).astype(np.float64)
    sz_exact = np.repeat(s.astype(np.float64) * z, 128, axis=1)
    half_ulp = np.spacing(np.abs(sz_exact).astype(np.float16)).astype(np.float64) / 2
    assert np.all(np.abs(W) <= half_ulp + 1e-12)
    # s = 1, sz = 0 -> w = q
    U = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    sc, sz = O.build_tables(np.ones((N, 2), np.float16), np.zeros((N, 2), int), K)
    assert np.array_equal(O.dequantize(O.pack_intweight(U), sc, sz, N, K), U.astype(np.float16))


def test_scaled_zero_table_layout():
    N, K = 8, 384
    s = (np.arange(N * 3).reshape(N, 3) + 1).astype(np.float16) / 64
    z = np.arange(N * 3).reshape(N, 3) % 16
    sc, sz = O.build_tables(s, z, K)
    assert sc.shape == (8, N) and sz.shape == (8, N)
    assert np.all(sc[3:] == 0) and np.all(sz[3:] == 0)
    assert np.array_equal(sc[:3], s.T)
    assert np.array_equal(sz[:3], (-(s.astype(np.float32) * z)).astype(np.float16).T)


def test_bf16_rounding_helper():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-9, 1.0 + 2**-9, -3.5, 1e-3, 255.5, 256.5])
    bits = O.f64_to_bf16_bits(vals)
    back = O.bf16_bits_to_f32(bits).astype(np.float64)
    # nearest-even to 8 significant bits
    assert back[0] == 1.0 and back[1] == 1.0 and back[2] == 1.0 + 2**-7
    assert back[3] == 1.0 and back[4] == -3.5
    assert back[6] == 256.0 and back[7] == 256.0
    assert abs(back[5] - 1e-3) <= 1e-3 * 2**-8


# ------------------------------------------------------------------- GEMM
def test_gemm_ref_brute_force_and_special_cases():
    rng = np.random.default_rng(2)
    M, N, K = 3, 8, 128
    p = O.make_w4_problem(M, K, N, seed=9)
    W = O.dequantize(p["qweight"], p["scales"], p["scaled_zeros"], N, K)
    y = O.gemm_ref(p["x"], W)
    for m in range(M):
        for n in range(N):
            ref = sum(float(p["x"][m, k]) * float(W[n, k]) for k in range(K))
            assert abs(y[m, n] - ref) <= 1e-5 * max(1.0, abs(ref))
    # one-hot activation reads back one weight column
    x = np.zeros((K, K), np.float16)
    x[np.arange(K), np.arange(K)] = 1
    assert np.array_equal(O.gemm_ref(x, W), W.T.astype(np.float32))
    # q == z everywhere -> y is only the sz rounding residue (|w| < 1e-5 here)
    U = np.repeat(p["z"], 128, axis=1).astype(np.uint8)
    W0 = O.dequantize(O.pack_intweight(U), p["scales"], p["scaled_zeros"], N, K)
    assert np.abs(O.gemm_ref(p["x"], W0)).max() < 1e-5 * K * np.abs(p["x"].astype(np.float32)).max()


def test_rel_err_metric():
    assert O.rel_err(np.array([1.0, 2.0]), np.array([1.0, 2.0])) == 0
    assert abs(O.rel_err(np.array([1.0, 2.1]), np.array([1.0, 2.0])) - 0.05) < 1e-12


# The W4A16 epilogue's GELU: max(v,0) - |v| * 2^P(|v|), P the degree-5 fit of
# log2 Phi(-a) on [0, 6] used by gelu_erf in qvggt_amd/csrc/common.h.
GELU_P = [-2.016825019e-04, 4.467580467e-03, -4.283261672e-02, -4.727858603e-01, -1.144399643e+00,
          -1.000531793e+00]


def _gelu_poly_f32(v, exp2_rel=0.0):
    v = np.asarray(v, np.float32)
    a = np.abs(v)
    p = np.full_like(a, np.float32(GELU_P[0]))
    for c in GELU_P[1:]:
        p = (p.astype(np.float64) * a + np.float32(c)).astype(np.float32)   # fma: one rounding
    with np.errstate(over="ignore", invalid="ignore"):
        e = (np.exp2(p.astype(np.float64)) * (1 + exp2_rel)).astype(np.float32)
    return (np.maximum(v, 0).astype(np.float64) - a.astype(np.float64) * e).astype(np.float32)


def test_gelu_polynomial_matches_erf_gelu():
    """The kernel's GELU (emulated in float32, exp2 also off by +-2 fp32 ulps)
    rounded to fp16 is within one ulp of the correctly rounded float64 erf
    GELU for every finite fp16 input -- including v < -90, where the product
    must round to -0 -- and exact zero / identity far out."""
    from scipy.special import erf
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = v[np.isfinite(v)].astype(np.float32)
    v64 = v.astype(np.float64)
    ref = (0.5 * v64 * (1 + erf(v64 / np.sqrt(2)))).astype(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    for rel in (-2 * 2.0 ** -23, 0.0, 2 * 2.0 ** -23):
        got = _gelu_poly_f32(v, rel).astype(np.float16).astype(np.float64)
        assert np.all(np.abs(got - ref) <= ulp), rel
    # the fit itself: |P - log2 Phi(-a)| <= 5.4e-4 on [0, 6], no turning point beyond
    from scipy.special import log_ndtr
    t = np.linspace(0, 6, 60001)
    assert np.abs(np.polyval(GELU_P, t) - log_ndtr(-t) / np.log(2)).max() <= 5.4e-4
    assert np.all(np.diff(np.polyval(GELU_P, np.linspace(0, 1e4, 100001))) < 0)
    assert _gelu_poly_f32(np.float32(0.0)) == 0.0
    assert _gelu_poly_f32(np.float32(25.0)) == np.float32(25.0)
    assert abs(_gelu_poly_f32(np.float32(-25.0))) < 1e-7


def test_quantize_intweight_recovers_exact_grid():
    rng = np.random.default_rng(5)
    N, K = 32, 256
    q = rng.integers(0, 16, (N, K))
    s = (2.0 ** -rng.integers(4, 9, (N, K // 128))).astype(np.float32)      # exact in fp16
    z = rng.integers(0, 16, (N, K // 128)).astype(np.float32)
    gidx = np.arange(K) // 128
    W = ((q - z[:, gidx]) * s[:, gidx]).astype(np.float16)                  # exact
    assert np.array_equal(O.quantize_intweight(W, s, z), q)


def test_quantize_intweight_rounds_half_to_even():
    W = np.array([[0.5, 1.5, 2.5, 3.5, -0.5, 4.5] + [0.0] * 58], np.float16)
    q = O.quantize_intweight(W, np.ones((1, 1), np.float16), np.zeros((1, 1), np.float16), group_size=64)
    assert q[0, :6].tolist() == [0, 2, 2, 4, 0, 4]


def test_quantize_intweight_matches_torch_16bit_ops():
    """The per-op roundings, cross-checked against torch's fp16 / bf16 tensor
    arithmetic running the from_linear expression (qmodule.py:296-305)."""
    import torch
    rng = np.random.default_rng(6)
    N, K, gs = 48, 384, 64
    W32 = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    s32 = rng.uniform(0.002, 0.02, (N, K // gs)).astype(np.float32)
    z32 = rng.integers(0, 16, (N, K // gs)).astype(np.float32)
    gidx = torch.arange(K) // gs
    for tdt, odt in ((torch.float16, np.float16), (torch.bfloat16, "bf16")):
        Wt, st, zt = (torch.from_numpy(a).to(tdt) for a in (W32, s32, z32))
        ref = torch.round((Wt + (zt * st)[:, gidx]) / st[:, gidx]).to(torch.int32).numpy()
        got = O.quantize_intweight(Wt.float().numpy(), st.float().numpy(), zt.float().numpy(), gs, dtype=odt)
        assert np.array_equal(got, ref), tdt
