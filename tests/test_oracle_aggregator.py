"""Pins oracle/aggregator.py (the fp32 VGGT block composition) with closed
forms that do not go through its own code path: zeroed projections reduce a
block to its LayerScaled biases, and one-token sequences reduce attention to
the value rows."""
import numpy as np
from scipy.special import erf

from oracle import aggregator as OA
from oracle import awq as A
from oracle import rope as R

DIM = 1024


def _w4_params(rng, name, K, N, zero=False):
    U = np.zeros((N, K), np.uint8) if zero else rng.integers(0, 16, (N, K)).astype(np.uint8)
    s = rng.uniform(0.005, 0.02, (N, K // 128)).astype(np.float16)
    z = rng.integers(0, 16, (N, K // 128))
    if zero:
        z = np.zeros_like(z)
    sc, sz = A.build_tables(s, z, K)
    return {f"{name}.qweight": A.pack_intweight(U), f"{name}.scales": sc, f"{name}.scaled_zeros": sz,
            f"{name}.bias": (0.1 * rng.standard_normal(N)).astype(np.float16)}


def _params(rng, zero_out=False):
    p = {}
    p.update(_w4_params(rng, "attn.qkv", DIM, 3 * DIM))
    p.update(_w4_params(rng, "attn.proj", DIM, DIM, zero=zero_out))
    p.update(_w4_params(rng, "mlp.fc1", DIM, 4 * DIM))
    p.update(_w4_params(rng, "mlp.fc2", 4 * DIM, DIM, zero=zero_out))
    for n in ("norm1", "norm2"):
        p[f"{n}.weight"] = (1 + 0.1 * rng.standard_normal(DIM)).astype(np.float16)
        p[f"{n}.bias"] = (0.1 * rng.standard_normal(DIM)).astype(np.float16)
    for n in ("attn.q_norm", "attn.k_norm"):
        p[f"{n}.weight"] = np.ones(64, np.float16)
        p[f"{n}.bias"] = np.zeros(64, np.float16)
    p["ls1.gamma"] = rng.uniform(0.5, 1.5, DIM).astype(np.float32)
    p["ls2.gamma"] = rng.uniform(0.5, 1.5, DIM).astype(np.float32)
    return p


def _ln64(x, g, b):
    m = x.mean(-1, keepdims=True)
    return (x - m) / np.sqrt(x.var(-1, keepdims=True) + 1e-6) * g + b


def test_zero_projections_leave_layerscaled_biases():
    rng = np.random.default_rng(0)
    p = _params(rng, zero_out=True)
    x = rng.standard_normal((6, DIM)).astype(np.float16)
    pos = R.vggt_positions(1, grid=1, specials=5)
    c, s = R.rope2d_tables(4)
    d = OA.aa_block_delta(x, p, 6, pos, c, s, np.arange(6))
    ref = p["ls1.gamma"].astype(np.float64) * p["attn.proj.bias"] + p["ls2.gamma"] * p["mlp.fc2.bias"].astype(np.float64)
    assert np.abs(d - ref[None]).max() < 1e-6


def test_single_token_sequences_reduce_attention_to_values():
    """seq_len = 1: softmax over one key is 1, so attention returns v; the rest
    is written here directly in float64 from the dequantised weights."""
    rng = np.random.default_rng(1)
    p = _params(rng)
    x = rng.standard_normal((3, DIM)).astype(np.float16)
    pos = np.array([[0, 0], [1, 2], [3, 1]], np.int32)
    c, s = R.rope2d_tables(4)
    d = OA.aa_block_delta(x, p, 1, pos, c, s, np.arange(3))

    def lin(v, n, K, N):
        W = A.dequantize(p[f"{n}.qweight"], p[f"{n}.scales"], p[f"{n}.scaled_zeros"], N, K).astype(np.float64)
        return v @ W.T + p[f"{n}.bias"].astype(np.float64)

    x64 = x.astype(np.float64)
    h = _ln64(x64, p["norm1.weight"].astype(np.float64), p["norm1.bias"].astype(np.float64))
    v = lin(h, "attn.qkv", DIM, 3 * DIM)[:, 2 * DIM:]
    xr = x64 + p["ls1.gamma"] * lin(v, "attn.proj", DIM, DIM)
    h2 = _ln64(xr, p["norm2.weight"].astype(np.float64), p["norm2.bias"].astype(np.float64))
    f = lin(h2, "mlp.fc1", DIM, 4 * DIM)
    f = 0.5 * f * (1 + erf(f / np.sqrt(2)))
    ref = xr + p["ls2.gamma"] * lin(f, "mlp.fc2", 4 * DIM, DIM) - x64
    assert np.abs(d - ref).max() <= 1e-4 * np.abs(ref).max()
