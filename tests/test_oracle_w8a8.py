"""Pins oracle/w8a8.py and oracle/rope.py with independent checks: known
answers, float64 closed forms, exact-sum references and brute force."""
import math

import numpy as np
import pytest

from oracle import rope as R
from oracle import w8a8 as Q


# ------------------------------------------------------------ rounding
def test_sat_s8_known_answers():
    v = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 127.4, 127.5, 200.0, -128.5, -300.0, np.nan, np.inf, -np.inf])
    assert Q.sat_s8(v).tolist() == [0, 2, 2, 0, -2, 127, 127, 127, -128, -128, 0, 127, -128]


def test_quant_known_answers():
    amax = 3.0
    k = np.arange(-127, 128)
    x = np.zeros((1, 256), np.float32)
    x[0, :255] = k * (amax / 127.0)
    x[0, 255] = amax
    q, s = Q.quant_per_token(x)
    assert np.array_equal(q[0, :255], k.astype(np.int8))
    assert q[0, 255] == 127
    assert s[0] == np.float16(np.float32(amax) / np.float32(127))
    # all-zero row: scale 0, codes 0 (0 * inf is NaN -> 0)
    q0, s0 = Q.quant_per_token(np.zeros((2, 16), np.float16))
    assert not q0.any() and not s0.any()


def test_quant_roundtrip_error_bound():
    x = np.random.default_rng(0).standard_normal((64, 1024)).astype(np.float16)
    q, s = Q.quant_per_token(x)
    amax = np.abs(x.astype(np.float64)).max(axis=1, keepdims=True)
    err = np.abs(q * (amax / 127.0) - x.astype(np.float64))
    assert (err <= amax / 127.0 * 0.5 * (1 + 1e-5)).all()


# ------------------------------------------------------- reductions
def test_row_sum_order_close_to_fsum():
    rng = np.random.default_rng(1)
    for D in (8, 1024, 4096, 1000 * 8):
        v = rng.standard_normal((4, D)).astype(np.float32)
        got = Q.row_sum_f32(v)
        for r in range(4):
            exact = math.fsum(v[r].astype(np.float64))
            assert abs(got[r] - exact) <= 1e-6 * np.abs(v[r]).sum()


def test_row_sum_order_is_the_lane_tree():
    # chunk c of 8 goes to lane c % 64; a sum whose rounding depends on order:
    v = np.zeros((1, 1024), np.float32)
    v[0, 0] = 1e8      # lane 0, first element
    v[0, 8] = 1.0      # lane 1
    v[0, 512] = -1e8   # lane 0, second pass (chunk 64)
    # lane 0 sums 1e8 + (-1e8) = 0 exactly, lane 1 holds 1 -> total 1
    assert Q.row_sum_f32(v)[0] == 1.0


# ------------------------------------------------------- normalisations
def _ln64(x, g, b, eps):
    x = x.astype(np.float64)
    m = x.mean(1, keepdims=True)
    v = ((x - m) ** 2).mean(1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


def test_layernorm_matches_float64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 1024)).astype(np.float16)
    g = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float16)
    b = (0.1 * rng.standard_normal(1024)).astype(np.float16)
    y = Q.layernorm(x, g, b, 1e-6).astype(np.float64)
    ref = _ln64(x, g.astype(np.float64), b.astype(np.float64), 1e-6)
    assert np.abs(y - ref).max() <= 2 ** -10 * np.abs(ref).max()
    # identity affine: zero mean, unit variance (up to fp16)
    y1 = Q.layernorm(x, np.ones(1024, np.float16), np.zeros(1024, np.float16)).astype(np.float64)
    assert np.abs(y1.mean(1)).max() < 2e-3 and np.abs(y1.std(1) - 1).max() < 2e-3


def test_layernorm_quant_matches_float64_and_bounds():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 1024)).astype(np.float16)
    g = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float16)
    b = (0.1 * rng.standard_normal(1024)).astype(np.float16)
    q, s = Q.layernorm_quant(x, g, b, 1e-6)
    ref = _ln64(x, g.astype(np.float64), b.astype(np.float64), 1e-6)
    amax = np.abs(ref).max(1, keepdims=True)
    assert np.abs(s.astype(np.float64)[:, None] - amax / 127).max() <= 1e-3 * amax.max()
    # half an LSB per row, plus slack for amax being taken over fp16-rounded values
    assert (np.abs(q * (amax / 127) - ref) <= 0.55 * amax / 127).all()
    assert np.abs(q).max(1).min() >= 126   # the largest magnitude maps to +-127


def test_rmsnorm_matches_float64_and_clamps():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 512)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, 512).astype(np.float16)
    y = Q.rmsnorm(x, g, 1e-6).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * g
    assert np.abs(y - ref).max() <= 2 ** -10 * np.abs(ref).max()
    xb = np.zeros((1, 64), np.float16)
    xb[0, 0], xb[0, 1] = 8, -8          # rms = sqrt(128/64); y = +-8/sqrt(2)*60000 overflows fp16
    big = Q.rmsnorm(xb, np.full(64, 60000, np.float16), 1e-6)
    assert float(big[0, 0]) == float(np.float16(64504.0)) == -float(big[0, 1])
    assert np.isfinite(big.astype(np.float32)).all()


def _sqrt2_scales():
    """fp16 scales s in [1, 89] for which rint(fp16(sqrt 2) * s) differs from
    rint(sqrt(2) * s): the int8 code then tells whether the LayerNorm value was
    rounded to fp16 before the multiply."""
    r16 = 1.4140625                       # fp16(sqrt 2): 1448 * 2**-10
    cands = np.arange(1.0, 89.0, 2 ** -8).astype(np.float16)
    cands = np.unique(cands).astype(np.float64)
    hit = cands[np.rint(r16 * cands) != np.rint(math.sqrt(2.0) * cands)]
    assert hit.size >= 3
    return hit


def test_layernorm_quant_per_tensor_known_answers():
    """rms_norm_general with a per-tensor scale (w8a8/layernorm.cu:100-123;
    the host passes beta = nullptr, layernorm.cu:180-187):
    q = sat(rint(float(fp16(LN(x) * gamma)) * scale)), no beta, no amax.

    Rows with a closed-form LayerNorm (eps = 0):
    * [4, -4, 4, -4, ...]: mean 0, variance 16, LN = +-1 exactly, so
      q = sat(rint(+-gamma * scale)) -- gamma is applied, the scale multiplies
      (dividing would give rint(gamma / scale)), ties go to even and codes
      saturate at 127 / -128;
    * [2, -2, 0, 0, ...]: LN = +-sqrt(2), 0; fp16 rounds sqrt 2 to 1.4140625,
      and at the scales of ``_sqrt2_scales`` only the fp16-rounded value gives
      the oracle's code."""
    D = 1024
    x1 = np.tile(np.array([4.0, -4.0], np.float32), D // 2)[None]
    gam = np.float16(np.linspace(-40, 40, D)).astype(np.float32)
    for sc in (4.5, 0.25, 3.0):
        q = Q.layernorm_quant_per_tensor(x1, gam, 0.0, np.float16(sc))[0]
        sign = np.where(np.arange(D) % 2 == 0, 1.0, -1.0)
        want = np.clip(np.rint(sign * gam.astype(np.float64) * sc), -128, 127)
        assert np.array_equal(q, want.astype(np.int8)), sc
    # a tie: gamma 3 * scale 4.5 = 13.5 -> 14 (even), 2.5 * 1 = 2.5 -> 2
    g2 = np.full(D, 3.0, np.float32)
    g2[1::2] = 2.5
    q = Q.layernorm_quant_per_tensor(x1, g2, 0.0, np.float16(4.5))[0]
    assert q[0] == 14 and q[2] == 14 and q[1] == -11   # -2.5 * 4.5 = -11.25 -> -11
    q = Q.layernorm_quant_per_tensor(x1, g2, 0.0, np.float16(1.0))[0]
    assert q[0] == 3 and q[1] == -2                      # -2.5 -> -2 (even)
    x2 = np.tile(np.array([2.0, -2.0, 0.0, 0.0], np.float32), D // 4)[None]
    ones = np.ones(D, np.float32)
    for sc in _sqrt2_scales()[:8]:
        q = Q.layernorm_quant_per_tensor(x2, ones, 0.0, np.float16(sc))[0]
        assert q[0] == np.rint(1.4140625 * sc) != np.rint(math.sqrt(2.0) * sc), sc
        assert q[1] == -q[0] and q[2] == 0 and q[3] == 0


def test_layernorm_quant_storage_types():
    """bf16 / fp32 inputs (layernorm.cu dispatches half, bfloat16, float): the
    LayerNorm value is rounded to the input type before the per-tensor int8
    conversion and before the per-token amax, whose floor is T(1e-6)."""
    D = 1024
    x2 = np.tile(np.array([2.0, -2.0, 0.0, 0.0], np.float32), D // 4)[None]
    ones = np.ones(D, np.float32)
    # bf16(sqrt 2) = 1.4140625 as well (8 significant bits: 181 * 2**-7); fp32 keeps sqrt 2
    sc = float(_sqrt2_scales()[0])
    assert Q.layernorm_quant_per_tensor(x2, ones, 0.0, sc, "bf16")[0, 0] == np.rint(1.4140625 * sc)
    assert Q.layernorm_quant_per_tensor(x2, ones, 0.0, sc, "f32")[0, 0] == np.rint(
        np.float32(np.float32(2.0) * np.float32(1.0) / np.sqrt(np.float32(2.0))) * np.float32(sc))
    # per-token floor: an all-equal row has LN = 0 everywhere, so amax = T(1e-6);
    # fp32 1e-6 is 0x358637BD, which bf16 truncates (low half < 0x8000) to 0x35860000
    assert np.float32(1e-6).view(np.uint32) == 0x358637BD
    flat = np.full((1, 64), 3.0, np.float32)
    for dt, floor in (("f16", np.float32(np.float16(1e-6))), ("f32", np.float32(1e-6)),
                      ("bf16", np.uint32(0x35860000).view(np.float32))):
        q, s = Q.layernorm_quant(flat, np.ones(64, np.float32), np.zeros(64, np.float32), 1e-6, dt)
        assert not q.any() and s[0] == np.float16(floor / np.float32(127.0)), dt


def test_round_store_known_answers():
    v = np.array([1.0, 1.00390625, 1.005859375, 1.0029296875, -3.0, 65520.0, 1e-6], np.float32)
    # bf16 keeps 8 significant bits: ties to even at 1 + 2**-8, 1 + 3*2**-9 rounds up
    assert Q.round_store(v[:5], "bf16").tolist() == [1.0, 1.0, 1.0078125, 1.0, -3.0]
    assert Q.round_store(v, "f16").tolist()[:5] == [1.0, 1.00390625, 1.005859375, 1.0029296875, -3.0]
    with np.errstate(over="ignore"):
        assert np.isinf(Q.round_store(v[5:6], "f16")[0])   # past the fp16 range
    assert Q.round_store(v, "f32").tolist() == v.tolist()


# ------------------------------------------------------------- GELU
def test_gelu_fast_close_to_closed_form():
    x = np.linspace(-6, 6, 4097).astype(np.float16)
    y = Q.gelu_fast_f16(x).astype(np.float64)
    ref = Q.gelu_tanh_f64(x.astype(np.float64))
    assert np.abs(y - ref).max() <= 8e-3 * max(1.0, np.abs(ref).max())
    assert Q.gelu_fast_f16(np.array([0.0], np.float16))[0] == 0


def test_gelu_and_quant_scale_semantics():
    x = np.random.default_rng(5).standard_normal((4, 256)).astype(np.float16)
    q, s, tmp = Q.gelu_and_quant(x)
    amax = np.abs(tmp.astype(np.float32)).max(1)
    assert np.array_equal(s, (amax / np.float32(127)).astype(np.float16))
    assert (np.abs(q).max(1) == 127).all()


def test_gelu_and_quant_amax_skips_nan_like_the_reference_loop():
    """act.cu:44-50 keeps amax with `if ((float)t > amax) amax = t` from 0, so a
    NaN GELU output (from NaN or -inf input) never enters the maximum, and a
    row whose values all fold to zero or below (all zeros: the fold gives -0;
    tiny positives: they fold negative) keeps amax = +0, scale +0."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 64)).astype(np.float16)
    x[0, 5] = np.nan
    x[1, 9] = -np.inf
    x[2, 0] = np.inf
    x[3] = 0.0
    x[4] = rng.uniform(0, 1.5e-4, 64).astype(np.float16)     # GELU in (0, 1e-4]
    x[5] = -x[4]
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        q, s, tmp = Q.gelu_and_quant(x)
    assert s[3].view(np.uint16) == 0 and s[4].view(np.uint16) == 0 and (q[3] == 0).all()
    zero = np.float32(np.float16(0.0001))
    for r in range(6):
        amax = np.float32(0.0)
        for t in tmp[r].astype(np.float32):
            f = t if t > zero else -t
            if f > amax:
                amax = f
        with np.errstate(over="ignore"):
            want = (amax / np.float32(127)).astype(np.float16)
        assert s[r].view(np.int16) == want.view(np.int16), r
    assert np.isnan(tmp[0, 5]) and np.isnan(tmp[1, 9]) and np.isinf(s[2])


def test_per_token_amax_skips_nan_like_the_reference_loops():
    """quantization.cu:49-56 and layernorm.cu:103-113 keep the row maximum with
    updates that never take a NaN: a NaN element leaves the other rows' and
    elements' results alone, and a row that is NaN throughout keeps the floor."""
    x = np.random.default_rng(11).standard_normal((3, 64)).astype(np.float16)
    x[0, 3] = np.nan
    with np.errstate(invalid="ignore"):
        q, s = Q.quant_per_token(x)
    for r in range(3):
        amax = np.float32(0.0)
        for v in np.abs(x[r].astype(np.float32)):
            if v > amax:
                amax = v
        assert s[r].view(np.int16) == (amax / np.float32(127)).astype(np.float16).view(np.int16), r
    assert q[0, 3] == 0
    g = np.ones(64, np.float16)
    b = np.zeros(64, np.float16)
    with np.errstate(invalid="ignore"):
        q2, s2 = Q.layernorm_quant(x, g, b, 1e-6)
    # row 0's mean is NaN, so every y is NaN and amax stays at fp16(1e-6)
    want0 = (np.float32(np.float16(1e-6)) / np.float32(127)).astype(np.float16)
    assert s2[0].view(np.int16) == want0.view(np.int16)
    assert (q2[0] == 0).all()
    assert np.isfinite(s2[1:].astype(np.float32)).all()


# ------------------------------------------------------------- GEMM
def test_w8a8_int32_brute_force_and_epilogue():
    rng = np.random.default_rng(6)
    a = rng.integers(-128, 128, (5, 64)).astype(np.int8)
    b = rng.integers(-128, 128, (7, 64)).astype(np.int8)
    acc = Q.w8a8_int32(a, b)
    for m in range(5):
        for n in range(7):
            assert acc[m, n] == sum(int(a[m, k]) * int(b[n, k]) for k in range(64))
    ws = rng.uniform(0.001, 0.01, 7).astype(np.float16)
    as_ = rng.uniform(0.001, 0.05, 5).astype(np.float16)
    y = Q.w8a8_epilogue(acc, ws, as_).astype(np.float64)
    ref = acc * ws.astype(np.float64)[None] * as_.astype(np.float64)[:, None]
    assert np.abs(y - ref).max() <= 2 ** -10 * np.abs(ref).max()
    # extreme accumulators stay exact in int32
    big = np.full((1, 4096), -128, np.int8)
    assert Q.w8a8_int32(big, big)[0, 0] == 4096 * 128 * 128


# ------------------------------------------------------------- RoPE
def test_rope_with_pos_pairs_rotate_like_complex_numbers():
    rng = np.random.default_rng(7)
    S, B, H, D, D2 = 5, 3, 2, 40, 32
    x = rng.standard_normal((S, B, H, D)).astype(np.float32)
    f = rng.uniform(-5, 5, (B, S, D2 // 2)).astype(np.float32)
    freqs = np.concatenate([f, f], axis=-1)
    y = R.rope_with_pos(x, freqs).astype(np.float64)
    z = (x[..., :16] + 1j * x[..., 16:32]).astype(np.complex128)
    th = f.transpose(1, 0, 2)[:, :, None, :].astype(np.float64)
    ref = z * np.exp(1j * th)
    assert np.abs(y[..., :16] - ref.real).max() < 1e-5
    assert np.abs(y[..., 16:32] - ref.imag).max() < 1e-5
    assert np.array_equal(y[..., 32:], x[..., 32:])
    # zero angles: identity
    assert np.array_equal(R.rope_with_pos(x, np.zeros((B, S, D2), np.float32)), x)


def test_rope2d_is_two_1d_ropes_and_specials_unrotated():
    rng = np.random.default_rng(8)
    T, H = 42, 3
    x = rng.standard_normal((T, H, 64)).astype(np.float16)
    pos = R.vggt_positions(1, grid=6, specials=6)
    c, s = R.rope2d_tables(8)
    y = R.rope2d(x, pos, c, s)
    assert np.array_equal(y[:6], x[:6])           # position 0 = identity
    for half in range(2):
        p = pos[:, half]
        ang = np.arccos(np.clip(c[p], -1, 1)).astype(np.float64)
        ang = np.where(s[p] < 0, -ang, ang)
        fr = np.concatenate([ang, ang], axis=-1).astype(np.float32)   # (T, 32)
        sub = x[:, :, 32 * half:32 * half + 32].transpose(0, 1, 2)[:, None]  # (T,1,H,32)
        ref = R.rope_with_pos(sub.astype(np.float32), fr[None].transpose(0, 1, 2).reshape(1, T, 32))
        assert np.abs(ref[:, 0].astype(np.float64) - y[:, :, 32 * half:32 * half + 32]).max() < 2e-3
    assert pos.shape == (42, 2) and pos[:6].sum() == 0 and pos[6:].min() == 1


def test_qknorm_rope2d_is_float64_layernorm_then_complex_rotation():
    """Independent restatement: float64 per-head LayerNorm, then each 2-D RoPE
    half as a complex rotation by p * base**(-i/16) (base 100)."""
    rng = np.random.default_rng(9)
    T, H = 41, 2
    qk = (rng.standard_normal((T, 2, H, 64)) * 3 + 0.5).astype(np.float16)
    g = [(1 + 0.1 * rng.standard_normal(64)).astype(np.float16) for _ in range(2)]
    b = [(0.1 * rng.standard_normal(64)).astype(np.float16) for _ in range(2)]
    pos = R.vggt_positions(1, grid=6, specials=5)
    c, s = R.rope2d_tables(8)
    y = R.qknorm_rope2d(qk, pos, c, s, g[0], b[0], g[1], b[1]).astype(np.float64)
    x = qk.astype(np.float64)
    ln = (x - x.mean(-1, keepdims=True)) / np.sqrt(x.var(-1, keepdims=True) + 1e-6)
    ln = ln * np.stack(g).astype(np.float64)[None, :, None] + np.stack(b).astype(np.float64)[None, :, None]
    freq = 100.0 ** (-np.arange(16) / 16.0)
    for half in range(2):
        th = pos[:, half].astype(np.float64)[:, None] * freq[None]          # (T, 16)
        z = ln[..., 32 * half:32 * half + 16] + 1j * ln[..., 32 * half + 16:32 * half + 32]
        r = z * np.exp(1j * th)[:, None, None, :]
        tol = 2e-3 * np.abs(ln).max()
        assert np.abs(y[..., 32 * half:32 * half + 16] - r.real).max() < tol
        assert np.abs(y[..., 32 * half + 16:32 * half + 32] - r.imag).max() < tol
    # specials (position 0) are the bare fp16 LayerNorm
    assert np.abs(y[:5] - ln[:5]).max() < 2e-3 * np.abs(ln).max()


def _rne(q, mant_bits: int, emin: int):
    """Round the rational q to the nearest binary float with ``mant_bits``
    fraction bits and minimum normal exponent ``emin`` (ties to even,
    subnormals below 2**emin, no overflow handling needed here), exactly."""
    from fractions import Fraction
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(Fraction(q))
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (max(e, emin) - mant_bits)
    n, r = divmod(a, ulp)
    if r > ulp / 2 or (r == ulp / 2 and n % 2 == 1):
        n += 1
    return sign * n * ulp


def test_gelu_fast_f16_rounding_order_known_answers():
    """act.cu:22-28 with T = half fixes the order and the rounding of every
    operation: a = h(f * c1), b = h(h(c2 * f) * x), c = h(1 + b), u = h(a * c),
    t = h(fp32(tanh u)), y = h(h(0.5 * x) * h(1 + t)), h = round to fp16.
    Restated here in exact rational arithmetic with its own round-to-nearest-
    even (not numpy's float16), over every 3rd fp16 value in [-8, 8].  The
    inputs are also evaluated with three plausible mistakes -- one rounding at
    the end, the product reassociated as c2 * h(f * x), and 1 + b left
    unrounded inside u -- each of which must disagree with the reference order
    somewhere, so the oracle's agreement pins its order."""
    import math
    from fractions import Fraction as Fr
    h = lambda q: _rne(q, 10, -14)
    f32 = lambda q: _rne(q, 23, -126)
    bits = np.arange(0x8000, dtype=np.uint32).astype(np.uint16)
    vals = np.concatenate([bits.view(np.float16), (bits | 0x8000).view(np.float16)])
    vals = vals[np.isfinite(vals) & (np.abs(vals.astype(np.float64)) <= 8)][::3]
    c1, c2 = Fr(float(np.float16(0.79788456))), Fr(float(np.float16(0.044715)))
    half, one = Fr(1, 2), Fr(1)

    def tanh16(u):
        return h(f32(Fr(math.tanh(float(u)))))

    def ref(x):
        a = h(x * c1)
        b = h(h(c2 * x) * x)
        u = h(a * h(one + b))
        return h(h(half * x) * h(one + tanh16(u)))

    def one_rounding(x):
        u = x * c1 * (one + c2 * x * x)
        return h(half * x * (one + Fr(math.tanh(float(u)))))

    def reassoc(x):
        a = h(x * c1)
        b = h(c2 * h(x * x))
        u = h(a * h(one + b))
        return h(h(half * x) * h(one + tanh16(u)))

    def unrounded_sum(x):
        a = h(x * c1)
        b = h(h(c2 * x) * x)
        u = h(a * (one + b))
        return h(h(half * x) * h(one + tanh16(u)))

    xs = [Fr(float(v)) for v in vals]
    want = np.array([float(ref(x)) for x in xs])
    got = Q.gelu_fast_f16(vals).astype(np.float64)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]
    for alt in (one_rounding, reassoc, unrounded_sum):
        other = np.array([float(alt(x)) for x in xs])
        assert (other != want).any(), alt.__name__
