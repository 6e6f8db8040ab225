"""Oracle: rotary position embeddings.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``rope_with_pos`` follows ``rope_new/fused_rope_with_pos.cu:19-57``:
  for d < d2/2: out = x[d]*cos(f[d]) + (-x[d + d2/2])*sin(f[d]);
  for d2/2 <= d < d2: out = x[d]*cos(f[d]) + x[d - d2/2]*sin(f[d]);
  d >= d2 copied; f = freqs[b][s][:] (fp32).  fp32 arithmetic, one rounding
  per operation; cos/sin of the fp32 angle evaluated in float64 and rounded
  to fp32 (the reference's fast-math sincosf is not reproduced).
* ``rope2d`` is the VGGT 2-D RoPE (not in the reference; restated from the
  public VGGT design): head dims [0,32) use the y position, [32,64) the x
  position; inside each 32-dim half the same rotate-half as above with
  d2 = 32 and angle p * base**(-i/16), i = d % 16, from fp32 tables.

Pinning (tests/test_oracle_rope.py): rotation preserves the norm of every
(d, d + d2/2) pair; angle 0 is the identity; the result equals multiplying
the complex number (x[d] + i x[d+d2/2]) by exp(i theta) (closed form in
float64); the 2-D variant reduces to two 1-D calls on the half-views.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def cos_sin_f32(theta: np.ndarray):
    t = np.asarray(theta, F32).astype(np.float64)
    return np.cos(t).astype(F32), np.sin(t).astype(F32)


def rope_with_pos(x: np.ndarray, freqs: np.ndarray, out_dtype=None) -> np.ndarray:
    """x (S, B, H, D) (float array of any float dtype), freqs (B, S, D2) fp32.
    ``out_dtype`` "bf16" returns fp32 values rounded to bfloat16 (x then holds
    bfloat16 values as fp32)."""
    x = np.asarray(x)
    out_dtype = out_dtype or x.dtype
    S, B, H, D = x.shape
    D2 = freqs.shape[-1]
    half = D2 // 2
    xf = x.astype(F32)
    f = np.asarray(freqs, F32).reshape(B, S, D2).transpose(1, 0, 2)[:, :, None, :]  # (S,B,1,D2)
    c, s = cos_sin_f32(f)
    a = xf[..., :half]
    p = xf[..., half:D2]
    first = ((a * c[..., :half]).astype(F32) + ((-p) * s[..., :half]).astype(F32)).astype(F32)
    second = ((p * c[..., half:]).astype(F32) + (a * s[..., half:]).astype(F32)).astype(F32)
    out = xf.copy()
    out[..., :half] = first
    out[..., half:D2] = second
    if isinstance(out_dtype, str) and out_dtype == "bf16":
        from .w8a8 import round_store
        return round_store(out, "bf16")
    return out.astype(out_dtype)


def rope2d_tables(max_position: int, base: float = 100.0):
    """fp32 (P, 16) cos/sin tables: angle = p * fp32(base**(-i/16)) in float64."""
    p = np.arange(max_position, dtype=np.float64)[:, None]
    inv = (base ** (-np.arange(16, dtype=np.float64) / 16.0)).astype(F32).astype(np.float64)
    ang = p * inv[None, :]
    return np.cos(ang).astype(F32), np.sin(ang).astype(F32)


def rope2d(x: np.ndarray, pos: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray) -> np.ndarray:
    """x (T, H, 64) fp16, pos (T, 2) int (y, x) -> rotated fp16 (T, H, 64)."""
    xf = np.asarray(x).astype(F32)
    out = np.empty_like(xf)
    for half in range(2):
        p = np.asarray(pos)[:, half]
        c = cos_t[p][:, None, :]   # (T,1,16)
        s = sin_t[p][:, None, :]
        a = xf[..., 32 * half:32 * half + 16]
        b = xf[..., 32 * half + 16:32 * half + 32]
        out[..., 32 * half:32 * half + 16] = ((a * c).astype(F32) - (b * s).astype(F32)).astype(F32)
        out[..., 32 * half + 16:32 * half + 32] = ((b * c).astype(F32) + (a * s).astype(F32)).astype(F32)
    return out.astype(np.float16)


def vggt_positions(S: int, grid: int = 37, specials: int = 5) -> np.ndarray:
    """(S*T, 2) int32 positions of VGGT tokens: per frame `specials` tokens at
    (0, 0) then the grid x grid patches at (y+1, x+1), row-major."""
    yy, xx = np.meshgrid(np.arange(grid), np.arange(grid), indexing="ij")
    patch = np.stack([yy.ravel() + 1, xx.ravel() + 1], axis=1)
    frame = np.concatenate([np.zeros((specials, 2), np.int64), patch], axis=0)
    return np.tile(frame, (S, 1)).astype(np.int32)


def _lane8_sum_f32(v: np.ndarray) -> np.ndarray:
    """fp32 sum over the last axis (64) in the kernel's order: lane j (0..7)
    sums elements 8j..8j+7 in index order, then a butterfly over lanes j ^ 1,
    j ^ 2, j ^ 4 (pairwise adds; every lane ends with the same value)."""
    v = np.asarray(v, F32).reshape(np.shape(v)[:-1] + (8, 8))     # [..., lane j, element e]
    lanes = np.zeros(v.shape[:-1], F32)
    for e in range(8):
        lanes = (lanes + v[..., e]).astype(F32)
    idx = np.arange(8)
    for off in (1, 2, 4):
        lanes = (lanes + lanes[..., idx ^ off]).astype(F32)
    return lanes[..., 0]


def qknorm_rope2d(qk: np.ndarray, pos, cos_t, sin_t, qg, qb, kg, kb, eps: float = 1e-6) -> np.ndarray:
    """VGGT attention prologue: per-head LayerNorm of q and k (affine over the
    64 head dims, fp32 statistics summed in the kernel's 8-lane order
    (``_lane8_sum_f32``), two-pass variance),
    rounded to fp16, then ``rope2d``.  qk: (T, 2, H, 64) fp16 -> same shape."""
    x = np.asarray(qk).astype(F32)
    mean = (_lane8_sum_f32(x) / F32(64)).astype(F32)
    d = (x - mean[..., None]).astype(F32)
    var = (_lane8_sum_f32((d * d).astype(F32)) / F32(64)).astype(F32)
    rs = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    g = np.stack([np.asarray(qg), np.asarray(kg)]).astype(F32)[None, :, None, :]
    b = np.stack([np.asarray(qb), np.asarray(kb)]).astype(F32)[None, :, None, :]
    t = ((d * rs[..., None]).astype(F32) * g).astype(F32)
    t = (t + b).astype(F32).astype(np.float16)
    out = np.empty_like(t)
    for part in range(2):
        out[:, part] = rope2d(t[:, part], pos, cos_t, sin_t)
    return out
