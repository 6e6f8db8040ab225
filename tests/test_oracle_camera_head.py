"""Pins oracle/camera_head.py (VGGT camera head, float64) with properties the
design fixes and with library routines in place of its hand-written pieces:

* frames carry no positional term, so permuting the input frames permutes
  every output row (a head / frame axis mix-up in the trunk attention fails);
* S identical frames reproduce the one-frame result (softmax over identical
  keys averages identical values);
* zero trunk linears and zero modulation leave the trunk input equal to the
  LayerNorm'd tokens, so every iteration adds the same delta:
  ``out_i = activate((i + 1) * delta)``, delta from torch's layer_norm / gelu;
* one trunk block equals torch's ``nn.MultiheadAttention`` (its own head split,
  scaling and softmax) + ``F.layer_norm`` + ``F.gelu`` composition.

Plain float weights (``.weight``) stand in for the W4 tables here; the W4
dequantisation itself is pinned in test_oracle_awq.py.  Trunk depth 1 keeps
the float64 weights small.
"""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import camera_head as OC

D = OC.DIM


def _lin(p, rng, name, k, n, zero=False, scale=0.02):
    p[f"{name}.weight"] = np.zeros((n, k), np.float32) if zero else (scale * rng.standard_normal((n, k))).astype(np.float32)
    p[f"{name}.bias"] = np.zeros(n, np.float32) if zero else (scale * rng.standard_normal(n)).astype(np.float32)


def _params(rng, depth=1, zero_trunk=False, zero_mod=False):
    p = {}
    for i in range(depth):
        pre = f"trunk.{i}."
        _lin(p, rng, pre + "attn.qkv", D, 3 * D, zero_trunk)
        _lin(p, rng, pre + "attn.proj", D, D, zero_trunk)
        _lin(p, rng, pre + "mlp.fc1", D, 4 * D, zero_trunk)
        _lin(p, rng, pre + "mlp.fc2", 4 * D, D, zero_trunk)
        for n in ("norm1", "norm2"):
            p[pre + n + ".weight"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
            p[pre + n + ".bias"] = (0.1 * rng.standard_normal(D)).astype(np.float32)
        p[pre + "ls1.gamma"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
        p[pre + "ls2.gamma"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
    for n in ("token_norm", "trunk_norm"):
        p[n + ".weight"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        p[n + ".bias"] = (0.1 * rng.standard_normal(D)).astype(np.float32)
    p["empty_pose_tokens"] = (0.1 * rng.standard_normal((1, 1, 9))).astype(np.float32)
    _lin(p, rng, "embed_pose", 9, D, scale=0.3)
    _lin(p, rng, "poseLN_modulation.1", D, 3 * D, zero_mod, scale=0.05)
    _lin(p, rng, "pose_branch.fc1", D, D // 2, scale=0.05)
    _lin(p, rng, "pose_branch.fc2", D // 2, 9, scale=0.05)
    return p


def test_frames_are_permutation_equivariant():
    rng = np.random.default_rng(0)
    p = _params(rng)
    t = rng.standard_normal((5, D))
    perm = np.array([3, 0, 4, 1, 2])
    a = OC.camera_head(t, p, num_iterations=2, depth=1)
    b = OC.camera_head(t[perm], p, num_iterations=2, depth=1)
    for x, y in zip(a, b):
        assert np.abs(x[perm] - y).max() < 1e-10
    # and the frames do interact: a different companion frame changes row 0
    c = OC.camera_head(np.concatenate([t[:1], rng.standard_normal((4, D))]), p, num_iterations=1, depth=1)
    assert np.abs(c[0][0] - a[0][0]).max() > 1e-6


def test_identical_frames_reproduce_one_frame():
    rng = np.random.default_rng(1)
    p = _params(rng)
    t = rng.standard_normal((1, D))
    one = OC.camera_head(t, p, num_iterations=3, depth=1)
    many = OC.camera_head(np.repeat(t, 4, 0), p, num_iterations=3, depth=1)
    for x, y in zip(one, many):
        assert np.abs(y - x).max() < 1e-10


def test_zero_trunk_and_modulation_accumulate_one_delta():
    rng = np.random.default_rng(2)
    p = _params(rng, zero_trunk=True, zero_mod=True)
    p["pose_branch.fc2.bias"][7], p["pose_branch.fc2.bias"][8] = -20.0, 20.0  # FoV: one clamped, one kept
    t = rng.standard_normal((3, D))
    outs = OC.camera_head(t, p, num_iterations=4, depth=1)
    T = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    pose = F.layer_norm(T(t), (D,), T(p["token_norm.weight"]), T(p["token_norm.bias"]), 1e-5)
    h = F.layer_norm(pose, (D,), T(p["trunk_norm.weight"]), T(p["trunk_norm.bias"]), 1e-5)
    f = F.gelu(F.linear(h, T(p["pose_branch.fc1.weight"]), T(p["pose_branch.fc1.bias"])))
    delta = F.linear(f, T(p["pose_branch.fc2.weight"]), T(p["pose_branch.fc2.bias"])).numpy()
    assert (delta[:, 7] < 0).all() and (delta[:, 8] > 0).all()
    for i, o in enumerate(outs):
        want = (i + 1) * delta
        assert np.abs(o[:, :7] - want[:, :7]).max() < 1e-9
        assert (o[:, 7] == 0).all()
        assert np.abs(o[:, 8] - want[:, 8]).max() < 1e-9


def test_trunk_block_matches_torch_multihead_attention():
    rng = np.random.default_rng(3)
    p = _params(rng)
    S = 6
    x = rng.standard_normal((S, D))
    got = OC.trunk_block(x, p, 0)
    T = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    mha = torch.nn.MultiheadAttention(D, OC.HEADS, bias=True, dtype=torch.float64)
    with torch.no_grad():
        mha.in_proj_weight.copy_(T(p["trunk.0.attn.qkv.weight"]))
        mha.in_proj_bias.copy_(T(p["trunk.0.attn.qkv.bias"]))
        mha.out_proj.weight.copy_(T(p["trunk.0.attn.proj.weight"]))
        mha.out_proj.bias.copy_(T(p["trunk.0.attn.proj.bias"]))
        xt = T(x)
        h = F.layer_norm(xt, (D,), T(p["trunk.0.norm1.weight"]), T(p["trunk.0.norm1.bias"]), 1e-5)
        a, _ = mha(h[:, None], h[:, None], h[:, None], need_weights=False)     # (S, batch 1, D)
        xt = xt + T(p["trunk.0.ls1.gamma"]) * a[:, 0]
        h = F.layer_norm(xt, (D,), T(p["trunk.0.norm2.weight"]), T(p["trunk.0.norm2.bias"]), 1e-5)
        f = F.gelu(F.linear(h, T(p["trunk.0.mlp.fc1.weight"]), T(p["trunk.0.mlp.fc1.bias"])))
        ref = xt + T(p["trunk.0.ls2.gamma"]) * F.linear(f, T(p["trunk.0.mlp.fc2.weight"]), T(p["trunk.0.mlp.fc2.bias"]))
    assert np.abs(got - ref.numpy()).max() < 1e-9
