"""Oracle: VGGT aggregator blocks in fp32 (floating-point reference).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The VGGT model graph is not in the reference (vggt-hf is external, no pinned
version: loader.py:27,154,158,284), so this restates the public VGGT block
with the same assumptions as the product (qk-norm, LayerScale, 2-D RoPE base
100, exact-erf GELU in the W4 path, tanh GELU + per-token int8 in the W8A8
path).  Parity vs vggt-hf itself is unpinned; parity of the GPU path is
pinned against this fp32 composition of the pinned oracle pieces
(oracle.awq dequantisation, oracle.w8a8 quantisation, oracle.rope tables,
oracle.attention), with no fp16 rounding of intermediates (the "fp32
dequantised reference" of the W4 path).

Parameters come in as dicts of numpy arrays named like the module tree
(``norm1.weight``, ``attn.qkv.qweight`` ...).
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from . import awq as A
from . import w8a8 as Q
from .attention import attention_ref

DIM, HEADS, HD = 1024, 16, 64


def _ln(x, g, b, eps=1e-6):
    x = np.asarray(x, np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * np.asarray(g, np.float64) + np.asarray(b, np.float64)


def _w4(x, p, name):
    N = p[f"{name}.qweight"].shape[0] * 4
    K = p[f"{name}.qweight"].shape[1]
    W = A.dequantize(p[f"{name}.qweight"], p[f"{name}.scales"], p[f"{name}.scaled_zeros"], N, K)
    return np.asarray(x, np.float32) @ W.astype(np.float32).T + p[f"{name}.bias"].astype(np.float32)


def _w8(x, p, name):
    """Reference W8A8 linear: per-token int8 quantisation of x, exact int32
    accumulation, dequantisation by ws * as, + bias, all in fp32."""
    q, s = Q.quant_per_token(np.asarray(x, np.float32))
    acc = Q.w8a8_int32(q, p[f"{name}.weight"]).astype(np.float64)
    return (acc * p[f"{name}.wscales"].astype(np.float64)[None] * s.astype(np.float64)[:, None]
            + p[f"{name}.bias"].astype(np.float64)[None])


def _rope(x, pos, cos_t, sin_t):
    """fp32 2-D RoPE of x (T, H, 64) with the fp32 tables."""
    out = np.empty_like(x)
    for half in range(2):
        c = cos_t[pos[:, half]][:, None, :].astype(np.float64)
        s = sin_t[pos[:, half]][:, None, :].astype(np.float64)
        a = x[..., 32 * half:32 * half + 16]
        b = x[..., 32 * half + 16:32 * half + 32]
        out[..., 32 * half:32 * half + 16] = a * c - b * s
        out[..., 32 * half + 16:32 * half + 32] = b * c + a * s
    return out


def aa_block_delta(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8=False):
    """Residual update x_out - x_in of one AA block, for the token ``rows``
    (every row still attends to all keys of its sequence).  float64 result."""
    x = np.asarray(x, np.float64)
    M = x.shape[0]
    lin = (lambda v, n: _w8(v, p, n)) if w8a8 else (lambda v, n: _w4(v, p, n))
    # attention: q/k/v for all tokens (keys), normalised and rotated
    h = _ln(x, p["norm1.weight"], p["norm1.bias"])
    qkv = np.asarray(lin(h, "attn.qkv"), np.float64).reshape(M, 3, HEADS, HD)
    q = _ln(qkv[:, 0], p["attn.q_norm.weight"], p["attn.q_norm.bias"])
    k = _ln(qkv[:, 1], p["attn.k_norm.weight"], p["attn.k_norm.bias"])
    q, k = _rope(q, pos, cos_t, sin_t), _rope(k, pos, cos_t, sin_t)
    att = attention_ref(q, k, qkv[:, 2], M // seq_len, seq_len, rows=rows).reshape(len(rows), DIM)
    o = np.asarray(lin(att, "attn.proj"), np.float64)
    xr = x[rows] + p["ls1.gamma"].astype(np.float64) * o
    h2 = _ln(xr, p["norm2.weight"], p["norm2.bias"])
    f = np.asarray(lin(h2, "mlp.fc1"), np.float64)
    if w8a8:
        f = Q.gelu_tanh_f64(f)
    else:
        f = 0.5 * f * (1.0 + erf(f / np.sqrt(2.0)))
    o2 = np.asarray(lin(f, "mlp.fc2"), np.float64)
    return xr + p["ls2.gamma"].astype(np.float64) * o2 - x[rows]
