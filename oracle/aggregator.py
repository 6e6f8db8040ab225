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


def _ln(x, g, b, eps=1e-6, dtype=np.float64):
    """LayerNorm over the last axis in ``dtype`` (float64 for the checked rows;
    float32, the reference's own precision, for the all-token key path)."""
    x = np.asarray(x, dtype)
    m = x.mean(-1, keepdims=True, dtype=dtype)
    d = x - m
    v = np.mean(d * d, axis=-1, keepdims=True, dtype=dtype)
    d *= (1.0 / np.sqrt(v + dtype(eps))).astype(dtype)
    d *= np.asarray(g, dtype)
    d += np.asarray(b, dtype)
    return d


def _dequant(p, name):
    N = p[f"{name}.qweight"].shape[0] * 4
    K = p[f"{name}.qweight"].shape[1]
    return A.dequantize(p[f"{name}.qweight"], p[f"{name}.scales"], p[f"{name}.scaled_zeros"], N, K)


def _w4(x, p, name, cols=None):
    """x @ W^T + b in fp32 with the dequantised fp16 weights; ``cols`` selects
    output channels."""
    W = _dequant(p, name).astype(np.float32)
    b = p[f"{name}.bias"].astype(np.float32)
    if cols is not None:
        W, b = W[cols], b[cols]
    return np.asarray(x, np.float32) @ W.T + b


def _w8(x, p, name, cols=None):
    """Reference W8A8 linear: per-token int8 quantisation of x, exact int32
    accumulation, dequantisation by ws * as, + bias, all in fp32."""
    q, s = Q.quant_per_token(np.asarray(x, np.float32))
    W, ws, b = p[f"{name}.weight"], p[f"{name}.wscales"], p[f"{name}.bias"]
    if cols is not None:
        W, ws, b = W[cols], ws[cols], b[cols]
    acc = Q.w8a8_int32(q, W).astype(np.float64)
    return (acc * ws.astype(np.float64)[None] * s.astype(np.float64)[:, None]
            + b.astype(np.float64)[None])


def _rope(x, pos, cos_t, sin_t):
    """2-D RoPE of x (T, H, 64) with the fp32 tables, in x's precision."""
    out = np.empty_like(x)
    for half in range(2):
        c = cos_t[pos[:, half]][:, None, :].astype(x.dtype)
        s = sin_t[pos[:, half]][:, None, :].astype(x.dtype)
        a = x[..., 32 * half:32 * half + 16]
        b = x[..., 32 * half + 16:32 * half + 32]
        out[..., 32 * half:32 * half + 16] = a * c - b * s
        out[..., 32 * half + 16:32 * half + 32] = b * c + a * s
    return out


def aa_block_attention(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8=False, eps=1e-6):
    """The attention half of one AA block for the token ``rows``: returns
    ``o`` = proj(attention(...)) (float64, (len(rows), 1024)), every row
    attending to all keys of its sequence.  q is formed for the rows only; the
    keys and values of every token go through LayerNorm, k-norm and RoPE in
    float32."""
    x = np.asarray(x, np.float32)
    M = x.shape[0]
    rows = np.asarray(rows)
    lin = (lambda v, n, c=None: _w8(v, p, n, c)) if w8a8 else (lambda v, n, c=None: _w4(v, p, n, c))
    h = _ln(x, p["norm1.weight"], p["norm1.bias"], eps, np.float32)
    if w8a8:   # the per-token quantisation of h is per row, so column subsets are exact
        kv = np.asarray(lin(h, "attn.qkv", np.arange(DIM, 3 * DIM)), np.float32).reshape(M, 2, HEADS, HD)
    else:
        kv = lin(h, "attn.qkv", np.arange(DIM, 3 * DIM)).reshape(M, 2, HEADS, HD)
    qr = np.asarray(lin(h[rows], "attn.qkv", np.arange(DIM)), np.float64).reshape(len(rows), HEADS, HD)
    q = _rope(_ln(qr, p["attn.q_norm.weight"], p["attn.q_norm.bias"], eps), pos[rows], cos_t, sin_t)
    k = _rope(_ln(kv[:, 0], p["attn.k_norm.weight"], p["attn.k_norm.bias"], eps, np.float32), pos, cos_t, sin_t)
    att = attention_ref(q, k, kv[:, 1], M // seq_len, seq_len, rows=rows, q_rows=True).reshape(len(rows), DIM)
    return np.asarray(lin(att, "attn.proj"), np.float64)


def aa_block_finish(x_rows, o, p, w8a8=False, eps=1e-6, ls1=None, ls2=None):
    """The rest of the block for the same rows: the LayerScale residual of the
    attention output ``o``, then LayerNorm -> fc1 -> GELU -> fc2 -> LayerScale
    residual.  ``ls1`` / ``ls2`` override the block's LayerScale gammas.
    Returns the residual update x_out - x_in (float64)."""
    x_rows = np.asarray(x_rows, np.float64)
    g1 = np.asarray(p["ls1.gamma"] if ls1 is None else ls1, np.float64)
    g2 = np.asarray(p["ls2.gamma"] if ls2 is None else ls2, np.float64)
    lin = (lambda v, n: _w8(v, p, n)) if w8a8 else (lambda v, n: _w4(v, p, n))
    xr = x_rows + g1 * o
    h2 = _ln(xr, p["norm2.weight"], p["norm2.bias"], eps)
    f = np.asarray(lin(h2, "mlp.fc1"), np.float64)
    if w8a8:
        f = Q.gelu_tanh_f64(f)
    else:
        f = 0.5 * f * (1.0 + erf(f / np.sqrt(2.0)))
    o2 = np.asarray(lin(f, "mlp.fc2"), np.float64)
    return xr + g2 * o2 - x_rows


def aa_block_delta(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8=False, eps=1e-6):
    """Residual update x_out - x_in of one AA block, for the token ``rows``
    (every row still attends to all keys of its sequence); ``eps`` of the four
    LayerNorms (norm1, norm2, q_norm, k_norm).  float64 result."""
    o = aa_block_attention(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8, eps)
    return aa_block_finish(np.asarray(x)[np.asarray(rows)], o, p, w8a8, eps)
