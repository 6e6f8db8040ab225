"""Oracle: VGGT camera head with a W4A16 trunk, in float64.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference quantises the camera head's trunk linears
(qvggt/inference/loader.py:204-206 infers ``camera_head.trunk.*`` from the
``.qweight`` keys, loader.py:338-344 selects every trunk linear that is not a
norm) but the head itself is in the external vggt-hf (no pinned version,
loader.py:27,154).  This restates the public VGGT camera head with the
product's assumptions: 4 refinement iterations, adaLN modulation of the
LayerNorm'd camera tokens, a 4-block trunk (dim 2048, 16 heads of 128, MLP
8192, exact-erf GELU, LayerScale, no qk-norm or RoPE), ``pose_branch``
2048 -> 1024 -> GELU -> 9, absT_quaR_FoV activation (linear, linear, ReLU).
LayerNorm eps 1e-5 except ``adaln_norm`` (1e-6, no affine).  Trunk linears are
dequantised with ``oracle.awq.dequantize``; everything else is float64 with no
fp16 rounding of intermediates.

Pinned by tests/test_oracle_camera_head.py through properties the design
fixes, each chosen so a plausible slip fails it: permutation equivariance over
frames (no positional term; a head/frame axis mix-up breaks it), S identical
frames reproducing the single-frame result (attention over identical keys
returns v), the zero-trunk / zero-modulation closed form
``pred_i = (i + 1) * delta`` (iteration accumulation and the residual path),
and the activation.  Parity with vggt-hf itself is unpinned (no copy of the
model or its outputs exists here), and the CICT token the loader can attach
(loader.py:224-246) has no public definition and is not modelled: parity
unpinned for both.

Parameters: a dict of numpy arrays named like the module tree under
``camera_head.`` (``trunk.0.attn.qkv.qweight``, ``token_norm.weight``,
``poseLN_modulation.1.weight``, ``pose_branch.fc1.weight`` ...).
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from . import awq as A

DIM, HEADS, HD, POSE_DIM = 2048, 16, 128, 9
TRUNK_DEPTH = 4


def _ln(x, g=None, b=None, eps=1e-5):
    x = np.asarray(x, np.float64)
    m = x.mean(-1, keepdims=True)
    y = (x - m) / np.sqrt(((x - m) ** 2).mean(-1, keepdims=True) + eps)
    if g is not None:
        y = y * np.asarray(g, np.float64) + np.asarray(b, np.float64)
    return y


def _gelu(x):
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def linear(x, p, name):
    """x @ W^T + b; W dequantised from the W4 tables when ``name`` is a W4 layer."""
    if f"{name}.qweight" in p:
        qw = p[f"{name}.qweight"]
        N, K = qw.shape[0] * 4, qw.shape[1]
        W = A.dequantize(qw, p[f"{name}.scales"], p[f"{name}.scaled_zeros"], N, K).astype(np.float64)
    else:
        W = np.asarray(p[f"{name}.weight"], np.float64)
    y = np.asarray(x, np.float64) @ W.T
    if f"{name}.bias" in p:
        y = y + np.asarray(p[f"{name}.bias"], np.float64)
    return y


def trunk_block(x, p, i):
    """One trunk block over the S pose tokens (S, 2048): attention mixes frames."""
    pre = f"trunk.{i}."
    S = x.shape[0]
    h = _ln(x, p[pre + "norm1.weight"], p[pre + "norm1.bias"])
    qkv = linear(h, p, pre + "attn.qkv").reshape(S, 3, HEADS, HD)
    q, k, v = (qkv[:, j].transpose(1, 0, 2) for j in range(3))        # (H, S, 128)
    s = q @ k.transpose(0, 2, 1) / np.sqrt(HD)
    s = np.exp(s - s.max(-1, keepdims=True))
    att = (s / s.sum(-1, keepdims=True)) @ v                          # (H, S, 128)
    o = linear(att.transpose(1, 0, 2).reshape(S, DIM), p, pre + "attn.proj")
    x = x + np.asarray(p[pre + "ls1.gamma"], np.float64) * o
    h = _ln(x, p[pre + "norm2.weight"], p[pre + "norm2.bias"])
    f = _gelu(linear(h, p, pre + "mlp.fc1"))
    return x + np.asarray(p[pre + "ls2.gamma"], np.float64) * linear(f, p, pre + "mlp.fc2")


def activate(enc):
    """absT_quaR_FoV: translation and quaternion linear, field of view ReLU."""
    out = np.array(enc, np.float64)
    out[..., 7:] = np.maximum(out[..., 7:], 0.0)
    return out


def camera_head(tokens, p, num_iterations: int = 4, depth: int = TRUNK_DEPTH):
    """tokens: (S, 2048) camera tokens of the last aggregator layer.  Returns
    the activated pose encodings (S, 9) of every iteration, float64."""
    pose = _ln(tokens, p["token_norm.weight"], p["token_norm.bias"])
    adaln = _ln(pose, eps=1e-6)
    S = pose.shape[0]
    pred, outs = None, []
    for _ in range(num_iterations):
        src = (np.broadcast_to(np.asarray(p["empty_pose_tokens"], np.float64).reshape(1, POSE_DIM), (S, POSE_DIM))
               if pred is None else pred)
        e = linear(src, p, "embed_pose")
        mod = linear(e / (1.0 + np.exp(-e)), p, "poseLN_modulation.1")
        shift, scale, gate = mod[:, :DIM], mod[:, DIM:2 * DIM], mod[:, 2 * DIM:]
        x = gate * (adaln * (1.0 + scale) + shift) + pose
        for i in range(depth):
            x = trunk_block(x, p, i)
        h = _ln(x, p["trunk_norm.weight"], p["trunk_norm.bias"])
        delta = linear(_gelu(linear(h, p, "pose_branch.fc1")), p, "pose_branch.fc2")
        pred = delta if pred is None else pred + delta
        outs.append(activate(pred))
    return outs
