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


def _w8_params(rng, name, K, N, zero=False):
    W = np.zeros((N, K), np.int8) if zero else rng.integers(-127, 128, (N, K)).astype(np.int8)
    return {f"{name}.weight": W, f"{name}.wscales": rng.uniform(0.5e-3, 2e-3, N).astype(np.float16),
            f"{name}.bias": (0.1 * rng.standard_normal(N)).astype(np.float16)}


def _params_w8(rng, zero_out=False):
    p = {k: v for k, v in _params(rng).items() if not k.startswith(("attn.qkv", "attn.proj", "mlp."))}
    p.update(_w8_params(rng, "attn.qkv", DIM, 3 * DIM))
    p.update(_w8_params(rng, "attn.proj", DIM, DIM, zero=zero_out))
    p.update(_w8_params(rng, "mlp.fc1", DIM, 4 * DIM))
    p.update(_w8_params(rng, "mlp.fc2", 4 * DIM, DIM, zero=zero_out))
    return p


def test_w8a8_zero_projections_leave_fp16_layerscaled_biases():
    """W8A8 chain with zero proj / fc2 weights: each epilogue returns its
    fp16 bias exactly, so the block output is fp16(fp16(x + b_proj * g1) +
    b_fc2 * g2) -- the two fp16 residual updates of the chain, in closed form."""
    rng = np.random.default_rng(2)
    p = _params_w8(rng, zero_out=True)
    x = rng.standard_normal((6, DIM)).astype(np.float16)
    pos = R.vggt_positions(1, grid=1, specials=5)
    c, s = R.rope2d_tables(4)
    d = OA.aa_block_delta(x, p, 6, pos, c, s, np.arange(6), w8a8=True)
    f32 = np.float32
    xr = (x.astype(f32) + (p["attn.proj.bias"].astype(f32) * p["ls1.gamma"].astype(f32))).astype(np.float16)
    xo = (xr.astype(f32) + (p["mlp.fc2.bias"].astype(f32) * p["ls2.gamma"].astype(f32))).astype(np.float16)
    assert np.array_equal(d, xo.astype(np.float64) - x.astype(np.float64))


def test_w8a8_single_token_attention_returns_the_stored_v():
    """seq_len = 1: the chain's attention output is the fp16 v of the W8A8 qkv
    projection (columns 2048..3071, not q or k), computed here from the int8
    codes of the LayerNorm + quant step with an int64 loop product."""
    from oracle import w8a8 as Q
    rng = np.random.default_rng(3)
    p = _params_w8(rng)
    x = rng.standard_normal((3, DIM)).astype(np.float16)
    pos = np.array([[0, 0], [1, 2], [3, 1]], np.int32)
    c, s = R.rope2d_tables(4)
    got = {}
    OA.aa_block_attention(x, p, 1, pos, c, s, np.arange(3), w8a8=True, att_out=got)
    q8, s8 = Q.layernorm_quant(x, p["norm1.weight"], p["norm1.bias"], 1e-6)
    W = p["attn.qkv.weight"][2 * DIM:].astype(np.int64)
    acc = np.array([[int(np.dot(q8[m].astype(np.int64), W[n])) for n in range(DIM)] for m in range(3)])
    v = Q.w8a8_epilogue(acc, p["attn.qkv.wscales"][2 * DIM:], s8, p["attn.qkv.bias"][2 * DIM:])
    assert np.array_equal(got["att"], v.astype(np.float64))


# ------------------------------------------------------- DINOv2 patch embed
def _dino_params(rng, zero_out=False):
    def lin(name, K, N, zero=False):
        return {f"{name}.weight": (np.zeros((N, K)) if zero else 0.02 * rng.standard_normal((N, K))).astype(np.float16),
                f"{name}.bias": (0.1 * rng.standard_normal(N)).astype(np.float16)}
    p = {}
    p.update(lin("attn.qkv", DIM, 3 * DIM))
    p.update(lin("attn.proj", DIM, DIM, zero_out))
    p.update(lin("mlp.fc1", DIM, 4 * DIM))
    p.update(lin("mlp.fc2", 4 * DIM, DIM, zero_out))
    for n in ("norm1", "norm2"):
        p[f"{n}.weight"] = (1 + 0.1 * rng.standard_normal(DIM)).astype(np.float16)
        p[f"{n}.bias"] = (0.1 * rng.standard_normal(DIM)).astype(np.float16)
    p["ls1.gamma"] = rng.uniform(0.5, 1.5, DIM).astype(np.float16)
    p["ls2.gamma"] = rng.uniform(0.5, 1.5, DIM).astype(np.float16)
    return p


def test_dino_patch_project_is_the_strided_convolution():
    """The unfolded-patch product equals torch's float64 Conv2d(3, D, 14,
    stride 14) on a random image (a library routine, not this code)."""
    import torch
    rng = np.random.default_rng(4)
    img = rng.uniform(-2, 2, (2, 3, 518, 518))
    w = rng.standard_normal((8, 3, 14, 14))
    b = rng.standard_normal(8)
    got = OA.dino_patch_project(img, w, b)
    ref = torch.nn.functional.conv2d(torch.from_numpy(img), torch.from_numpy(w), torch.from_numpy(b), stride=14)
    ref = ref.flatten(2).transpose(1, 2).numpy()                    # (S, 1369, D), row-major grid
    assert got.shape == (2, 1369, 8) and np.abs(got - ref).max() <= 1e-10 * np.abs(ref).max()


def test_dino_and_aggregator_token_assembly():
    """Known answers with distinct values per slot: DINOv2 [cls + pos 0,
    registers, patches + pos 1..]; aggregator [camera, registers, patch
    tokens] with token set 0 for frame 0 only."""
    S, D = 3, 4
    patches = np.arange(S * 1369 * D, dtype=np.float64).reshape(S, 1369, D)
    cls = np.full((1, 1, D), 1000.0)
    reg = 2000.0 + np.arange(4 * D, dtype=np.float64).reshape(1, 4, D)
    pos = 0.5 * np.arange(1370 * D, dtype=np.float64).reshape(1, 1370, D)
    x = OA.dino_tokens(patches, cls, reg, pos)
    assert x.shape == (S, 1374, D)
    assert np.array_equal(x[:, 0], np.broadcast_to(1000.0 + pos[0, 0], (S, D)))
    assert np.array_equal(x[:, 1:5], np.broadcast_to(reg[0], (S, 4, D)))
    assert np.array_equal(x[:, 5:], patches + pos[0, 1:])
    cam = np.array([1.0, 2.0])[None, :, None, None] * np.ones((1, 2, 1, D))
    regs = np.array([10.0, 20.0])[None, :, None, None] * np.ones((1, 2, 4, D))
    a = OA.aggregator_tokens(patches, cam, regs).reshape(S, 1374, D)
    assert (a[0, 0] == 1).all() and (a[1:, 0] == 2).all()
    assert (a[0, 1:5] == 10).all() and (a[1:, 1:5] == 20).all()
    assert np.array_equal(a[:, 5:], patches)


def test_dino_block_zero_projections_and_single_token_sequences():
    """Zero proj / fc2 weights leave the LayerScaled biases; with one-token
    sequences attention returns v, and the block is written out here
    directly in float64."""
    rng = np.random.default_rng(5)
    p = _dino_params(rng, zero_out=True)
    x = rng.standard_normal((6, DIM)).astype(np.float16)
    d = OA.dino_block_delta(x, p, np.arange(6), 6)
    g1, g2 = p["ls1.gamma"].astype(np.float64), p["ls2.gamma"].astype(np.float64)
    ref = g1 * p["attn.proj.bias"].astype(np.float64) + g2 * p["mlp.fc2.bias"].astype(np.float64)
    assert np.abs(d - ref[None]).max() < 1e-12
    p = _dino_params(rng)
    d = OA.dino_block_delta(x, p, np.arange(6), 1)
    x64 = x.astype(np.float64)
    f64 = {k: v.astype(np.float64) for k, v in p.items()}
    lin = lambda v, n: v @ f64[f"{n}.weight"].T + f64[f"{n}.bias"]
    h = _ln64(x64, f64["norm1.weight"], f64["norm1.bias"])
    v = lin(h, "attn.qkv")[:, 2 * DIM:]
    xr = x64 + f64["ls1.gamma"] * lin(v, "attn.proj")
    f = lin(_ln64(xr, f64["norm2.weight"], f64["norm2.bias"]), "mlp.fc1")
    ref = xr + f64["ls2.gamma"] * lin(0.5 * f * (1 + erf(f / np.sqrt(2))), "mlp.fc2") - x64
    assert np.abs(d - ref).max() <= 1e-9 * np.abs(ref).max()


def test_dino_final_norm_drops_the_specials():
    """Final LayerNorm against torch's float64 layer_norm, cls and registers
    dropped per frame."""
    import torch
    rng = np.random.default_rng(6)
    S, D = 2, 16
    x = rng.standard_normal((S * 1374, D))
    w, b = rng.standard_normal(D), rng.standard_normal(D)
    got = OA.dino_final(x, w, b, S)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (D,), torch.from_numpy(w), torch.from_numpy(b),
                                         1e-6).numpy().reshape(S, 1374, D)[:, 5:]
    assert np.abs(got - ref).max() <= 1e-12
