"""GPU parity of the flash attention kernel against the float64 oracle.

Tolerance: max|y - y_ref| / max|y_ref| <= 1e-2 (fp16 outputs; P is rounded
to fp16 before the PV product, as in every fp16 flash attention).
"""
import numpy as np
import pytest
import torch

from oracle.attention import attention_ref

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _qkv(T, H, seed):
    x = np.random.default_rng(seed).standard_normal((T, 3, H, 64)).astype(np.float16)
    return x


@pytest.mark.parametrize("B,L,H", [(2, 1374, 16), (1, 64, 1), (3, 100, 2), (1, 1, 4), (1, 200, 16)])
def test_attention_small_full_check(gpu, B, L, H):
    from qvggt_amd import awq_inference_engine as E
    x = _qkv(B * L, H, B * L + H)
    xt = torch.from_numpy(x).to(gpu)
    out = E.attention(xt[:, 0], xt[:, 1], xt[:, 2], L)
    rows = np.arange(B * L) if B * L <= 600 else np.random.default_rng(0).choice(B * L, 600, replace=False)
    ref = attention_ref(x[:, 0], x[:, 1], x[:, 2], B, L, rows=rows)
    got = out.float().cpu().numpy()[rows]
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert np.isfinite(got).all() and err <= TOL, err


def test_frame_attention_s8(gpu):
    """config 3: frame attention, S = 8 frames of 1374 tokens, 16 heads."""
    from qvggt_amd import awq_inference_engine as E
    S, L, H = 8, 1374, 16
    x = _qkv(S * L, H, 1)
    xt = torch.from_numpy(x).to(gpu)
    out = E.attention(xt[:, 0], xt[:, 1], xt[:, 2], L)
    rows = np.random.default_rng(1).choice(S * L, 256, replace=False)
    ref = attention_ref(x[:, 0], x[:, 1], x[:, 2], S, L, rows=rows)
    got = out.float().cpu().numpy()[rows]
    assert np.abs(got - ref).max() / np.abs(ref).max() <= TOL


def test_global_attention_s32_sampled_rows(gpu):
    """config 4: global attention over 32 x 1374 = 43,968 tokens, 16 heads,
    checked on sampled query rows (each attends to all keys)."""
    from qvggt_amd import awq_inference_engine as E
    L, H = 32 * 1374, 16
    x = _qkv(L, H, 2)
    xt = torch.from_numpy(x).to(gpu)
    out = E.attention(xt[:, 0], xt[:, 1], xt[:, 2], L)
    rows = np.random.default_rng(2).choice(L, 48, replace=False)
    ref = attention_ref(x[:, 0], x[:, 1], x[:, 2], 1, L, rows=rows)
    got = out.float().cpu().numpy()[rows]
    assert np.abs(got - ref).max() / np.abs(ref).max() <= TOL


def test_attention_separate_buffers_and_determinism(gpu):
    from qvggt_amd import awq_inference_engine as E
    B, L, H = 2, 300, 4
    x = _qkv(B * L, H, 3)
    q = torch.from_numpy(np.ascontiguousarray(x[:, 0])).to(gpu)
    kv = torch.from_numpy(np.ascontiguousarray(x[:, 1:])).to(gpu)   # (T, 2, H, 64)
    o1 = E.attention(q, kv[:, 0], kv[:, 1], L)
    o2 = E.attention(q, kv[:, 0], kv[:, 1], L)
    assert torch.equal(o1, o2)
    ref = attention_ref(x[:, 0], x[:, 1], x[:, 2], B, L)
    assert np.abs(o1.float().cpu().numpy() - ref).max() / np.abs(ref).max() <= TOL
