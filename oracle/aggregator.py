"""Oracle: VGGT aggregator blocks (floating-point reference).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The VGGT model graph is not in the reference (vggt-hf is external, no pinned
version: loader.py:27,154,158,284), so this restates the public VGGT block
with the same assumptions as the product (qk-norm, LayerScale, 2-D RoPE base
100, exact-erf GELU in the W4 path, tanh GELU + per-token int8 in the W8A8
path).  Parity vs vggt-hf itself is unpinned; parity of the GPU path is
pinned against compositions of the pinned oracle pieces (oracle.awq
dequantisation, oracle.w8a8 quantisation and W8A8 GEMM, oracle.rope,
oracle.attention):

* W4A16 blocks: an fp32 composition with no fp16 rounding of intermediates
  (the "fp32 dequantised reference").
* W8A8 blocks: the reference's W8A8 op chain, in which every op takes and
  returns 16-bit tensors (pybind.cpp:29-36: rms_norm_general,
  w8a8_gemm_fuse_bias_forward_cuda, invoke_quant, gelu_and_quant all read and
  write half): LayerNorm + per-token int8 (layernorm.cu:20-151) -> W8A8 qkv
  with its fp16 epilogue (w8a8_gemm_cuda.cu:851-878) -> q/k LayerNorm + 2-D
  RoPE on the stored fp16 q/k -> attention (float64) stored as fp16 ->
  invoke_quant (quantization.cu:42-96) -> W8A8 proj -> fp16 LayerScale
  residual -> LayerNorm + int8 -> W8A8 fc1 -> gelu_and_quant
  (act.cu:30-90) -> W8A8 fc2 -> fp16 residual.  Each quantiser thus sees the
  fp16 tensor the previous op stores, as in the reference.

Parameters come in as dicts of numpy arrays named like the module tree
(``norm1.weight``, ``attn.qkv.qweight`` ...).
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from . import awq as A
from . import rope as R
from . import w8a8 as Q
from .attention import attention_ref

DIM, HEADS, HD = 1024, 16, 64
F16, F32 = np.float16, np.float32


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


def _w8(q, s, p, name, cols=None):
    """W8A8 linear of the reference (w8a8_gemm_fuse_bias_forward_cuda): int8
    codes q (M, K) with their per-token fp16 scales s, exact int32
    accumulation, epilogue fp16_rn((acc * ws) * as + bias).  Returns fp16."""
    W, ws, b = p[f"{name}.weight"], p[f"{name}.wscales"], p[f"{name}.bias"]
    if cols is not None:
        W, ws, b = W[cols], ws[cols], b[cols]
    return Q.w8a8_epilogue(Q.w8a8_int32(q, W), ws, s, b)


def _addcmul16(x, o, g):
    """torch's in-place x.addcmul_(o, g) on fp16 tensors: x + o * g in fp32,
    one rounding to fp16."""
    t = (np.asarray(o, F32) * np.asarray(g, F32)[None, :]).astype(F32)
    return (np.asarray(x, F32) + t).astype(F32).astype(F16)


def _qknorm_rope16(t16, part, pos, cos_t, sin_t, p, eps):
    """qknorm_rope2d of the stored fp16 q (part 0) or k (part 1) heads
    (T, H, 64): per-head LayerNorm with the q_norm / k_norm parameters, fp16,
    then the 2-D RoPE (oracle.rope.qknorm_rope2d, pinned bit-exact)."""
    qk = np.stack([t16, t16], axis=1)
    out = R.qknorm_rope2d(qk, pos, cos_t, sin_t, p["attn.q_norm.weight"], p["attn.q_norm.bias"],
                          p["attn.k_norm.weight"], p["attn.k_norm.bias"], eps)
    return out[:, part]


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


def aa_block_attention(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8=False, eps=1e-6, att_out=None):
    """The attention half of one AA block for the token ``rows``: returns
    ``o`` = proj(attention(...)) ((len(rows), 1024); float64 for W4A16, the
    fp16 values of the W8A8 chain for W8A8), every row attending to all keys
    of its sequence.  W4A16: q is formed for the rows only; the keys and
    values of every token go through LayerNorm, k-norm and RoPE in float32.
    ``att_out``, a dict, receives the attention output of the rows before the
    projection ("att": float64; W8A8 stores it as fp16 before quantising)."""
    x = np.asarray(x, np.float32)
    M = x.shape[0]
    rows = np.asarray(rows)
    if w8a8:
        q8, s8 = Q.layernorm_quant(x.astype(F16), p["norm1.weight"], p["norm1.bias"], eps)
        kv = _w8(q8, s8, p, "attn.qkv", np.arange(DIM, 3 * DIM)).reshape(M, 2, HEADS, HD)
        qr = _w8(q8[rows], s8[rows], p, "attn.qkv", np.arange(DIM)).reshape(len(rows), HEADS, HD)
        q = _qknorm_rope16(qr, 0, pos[rows], cos_t, sin_t, p, eps)
        k = _qknorm_rope16(kv[:, 0], 1, pos, cos_t, sin_t, p, eps)
        att = attention_ref(q, k, kv[:, 1], M // seq_len, seq_len, rows=rows, q_rows=True).reshape(len(rows), DIM)
        if att_out is not None:
            att_out["att"] = att
        qa, sa = Q.quant_per_token(att.astype(F16))
        return _w8(qa, sa, p, "attn.proj").astype(np.float64)
    h = _ln(x, p["norm1.weight"], p["norm1.bias"], eps, np.float32)
    kv = _w4(h, p, "attn.qkv", np.arange(DIM, 3 * DIM)).reshape(M, 2, HEADS, HD)
    qr = np.asarray(_w4(h[rows], p, "attn.qkv", np.arange(DIM)), np.float64).reshape(len(rows), HEADS, HD)
    q = _rope(_ln(qr, p["attn.q_norm.weight"], p["attn.q_norm.bias"], eps), pos[rows], cos_t, sin_t)
    k = _rope(_ln(kv[:, 0], p["attn.k_norm.weight"], p["attn.k_norm.bias"], eps, np.float32), pos, cos_t, sin_t)
    att = attention_ref(q, k, kv[:, 1], M // seq_len, seq_len, rows=rows, q_rows=True).reshape(len(rows), DIM)
    if att_out is not None:
        att_out["att"] = att
    return np.asarray(_w4(att, p, "attn.proj"), np.float64)


def w8a8_block_from_attention(x_rows, att16, p, eps=1e-6, ls1=None, ls2=None):
    """The W8A8 chain from a given fp16 attention output of the rows on:
    invoke_quant -> W8A8 proj -> fp16 LayerScale residual -> the MLP half
    (``aa_block_finish``).  Returns the residual update (float64)."""
    qa, sa = Q.quant_per_token(np.asarray(att16, F16))
    o = _w8(qa, sa, p, "attn.proj")
    return aa_block_finish(x_rows, o, p, True, eps, ls1, ls2)


def aa_block_finish(x_rows, o, p, w8a8=False, eps=1e-6, ls1=None, ls2=None):
    """The rest of the block for the same rows: the LayerScale residual of the
    attention output ``o``, then LayerNorm -> fc1 -> GELU -> fc2 -> LayerScale
    residual.  ``ls1`` / ``ls2`` override the block's LayerScale gammas.
    Returns the residual update x_out - x_in (float64)."""
    g1 = np.asarray(p["ls1.gamma"] if ls1 is None else ls1, np.float64)
    g2 = np.asarray(p["ls2.gamma"] if ls2 is None else ls2, np.float64)
    if w8a8:
        x16 = np.asarray(x_rows, np.float32).astype(F16)
        xr = _addcmul16(x16, np.asarray(o, F16), g1)
        q8, s8 = Q.layernorm_quant(xr, p["norm2.weight"], p["norm2.bias"], eps)
        f = _w8(q8, s8, p, "mlp.fc1")
        qf, sf, _ = Q.gelu_and_quant(f)
        xo = _addcmul16(xr, _w8(qf, sf, p, "mlp.fc2"), g2)
        return xo.astype(np.float64) - x16.astype(np.float64)
    x_rows = np.asarray(x_rows, np.float64)
    xr = x_rows + g1 * o
    h2 = _ln(xr, p["norm2.weight"], p["norm2.bias"], eps)
    f = np.asarray(_w4(h2, p, "mlp.fc1"), np.float64)
    f = 0.5 * f * (1.0 + erf(f / np.sqrt(2.0)))
    o2 = np.asarray(_w4(f, p, "mlp.fc2"), np.float64)
    return xr + g2 * o2 - x_rows


def aa_block_delta(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8=False, eps=1e-6):
    """Residual update x_out - x_in of one AA block, for the token ``rows``
    (every row still attends to all keys of its sequence); ``eps`` of the four
    LayerNorms (norm1, norm2, q_norm, k_norm).  float64 result."""
    o = aa_block_attention(x, p, seq_len, pos, cos_t, sin_t, rows, w8a8, eps)
    return aa_block_finish(np.asarray(x)[np.asarray(rows)], o, p, w8a8, eps)


# ------------------------------------------------------- DINOv2 patch embed
# The aggregator's patch embed is DINOv2 ViT-L/14 with 4 register tokens in
# fp16, unquantised (loader.py:346 leaves ``patch_embed`` in floating point);
# restated from the public DINOv2 / VGGT design in float64.

GRID, PATCH, N_REG = 37, 14, 4
SPECIALS = 1 + N_REG


def dino_patch_project(images, weight, bias):
    """patch_embed.proj, a Conv2d(3, 1024, 14, stride 14) of (S, 3, 518, 518)
    images, as (S, 1369, 1024) float64: token (i, j) of the 37 x 37 grid is the
    dot product of the 3 x 14 x 14 pixel block at (14 i, 14 j) with each
    output channel's kernel, plus its bias."""
    x = np.asarray(images, np.float64)
    S = x.shape[0]
    blocks = x.reshape(S, 3, GRID, PATCH, GRID, PATCH)                 # s, c, i, y, j, x
    w = np.asarray(weight, np.float64)                                  # (D, 3, 14, 14)
    out = np.einsum("sciyjx,dcyx->sijd", blocks, w, optimize=True)
    return out.reshape(S, GRID * GRID, -1) + np.asarray(bias, np.float64)


def dino_tokens(patches, cls_token, register_tokens, pos_embed):
    """DINOv2 token assembly for (S, 1369, D) patch projections: per frame
    [cls + pos_embed[0], the 4 registers (no position), patches +
    pos_embed[1:]] -> (S, 1374, D) float64."""
    p = np.asarray(patches, np.float64)
    S, _, D = p.shape
    pe = np.asarray(pos_embed, np.float64).reshape(1 + GRID * GRID, D)
    x = np.empty((S, SPECIALS + GRID * GRID, D))
    x[:, 0] = np.asarray(cls_token, np.float64).reshape(D) + pe[0]
    x[:, 1:SPECIALS] = np.asarray(register_tokens, np.float64).reshape(N_REG, D)
    x[:, SPECIALS:] = p + pe[1:]
    return x


def _lin64(x, p, name):
    return np.asarray(x, np.float64) @ np.asarray(p[f"{name}.weight"], np.float64).T + \
        np.asarray(p[f"{name}.bias"], np.float64)


def dino_block_delta(x, p, rows, seq_len, eps=1e-6, ls1=None, ls2=None):
    """Residual update of one DINOv2 block (pre-norm ViT: LayerNorm -> qkv ->
    16-head attention over the token's own frame -> proj -> LayerScale
    residual; LayerNorm -> fc1 -> exact-erf GELU -> fc2 -> LayerScale
    residual) for the token ``rows`` of x (T, D), in float64 from the fp16
    weights.  ``ls1`` / ``ls2`` override the LayerScale gammas."""
    x = np.asarray(x, np.float64)
    rows = np.asarray(rows)
    g1 = np.asarray(p["ls1.gamma"] if ls1 is None else ls1, np.float64)
    g2 = np.asarray(p["ls2.gamma"] if ls2 is None else ls2, np.float64)
    h = _ln(x, p["norm1.weight"], p["norm1.bias"], eps)
    W = np.asarray(p["attn.qkv.weight"], np.float64)
    b = np.asarray(p["attn.qkv.bias"], np.float64)
    kv = (h @ W[DIM:].T + b[DIM:]).reshape(-1, 2, HEADS, HD)
    q = (h[rows] @ W[:DIM].T + b[:DIM]).reshape(len(rows), HEADS, HD)
    att = attention_ref(q, kv[:, 0], kv[:, 1], x.shape[0] // seq_len, seq_len, rows=rows,
                        q_rows=True).reshape(len(rows), DIM)
    xr = x[rows] + g1 * _lin64(att, p, "attn.proj")
    f = _lin64(_ln(xr, p["norm2.weight"], p["norm2.bias"], eps), p, "mlp.fc1")
    f = 0.5 * f * (1.0 + erf(f / np.sqrt(2.0)))
    return xr + g2 * _lin64(f, p, "mlp.fc2") - x[rows]


def dino_final(x, weight, bias, S, eps=1e-6):
    """The patch embed's output: the final LayerNorm of the (S * 1374, D)
    tokens, without the cls and register tokens -> (S, 1369, D) float64."""
    y = _ln(np.asarray(x, np.float64), weight, bias, eps).reshape(S, SPECIALS + GRID * GRID, -1)
    return y[:, SPECIALS:]


def aggregator_tokens(patch_tokens, camera_token, register_token):
    """The aggregator's AA input: per frame [camera token, 4 register tokens,
    the patch embed's 1369 tokens], frame 0 with token set 0 of
    camera_token (1, 2, 1, D) / register_token (1, 2, 4, D) and every other
    frame with set 1 -> (S * 1374, D) float64."""
    pt = np.asarray(patch_tokens, np.float64)
    S, _, D = pt.shape
    cam = np.asarray(camera_token, np.float64).reshape(2, D)
    reg = np.asarray(register_token, np.float64).reshape(2, N_REG, D)
    x = np.empty((S, SPECIALS + GRID * GRID, D))
    for f in range(S):
        t = 0 if f == 0 else 1
        x[f, 0] = cam[t]
        x[f, 1:SPECIALS] = reg[t]
    x[:, SPECIALS:] = pt
    return x.reshape(S * (SPECIALS + GRID * GRID), D)
