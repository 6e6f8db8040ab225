"""VGGT camera head with a W4A16 trunk: the small-M consumer of the GEMV path.

QVGGT quantises the camera head's trunk linears (``camera_head.trunk.*``,
loader.py:204-206, 338-344) and keeps the rest in floating point; the head
itself lives in the external vggt-hf, so this restates the public VGGT camera
head under the same module names:

* pose tokens = the camera token of every frame from the last aggregator
  output ([frame | global], 2048 wide), LayerNorm'd (``token_norm``);
* 4 refinement iterations: the current pose encoding (9 values: translation 3,
  quaternion 4, field of view 2; ``empty_pose_tokens`` on the first pass) is
  embedded (``embed_pose``), turned into adaLN shift / scale / gate
  (``poseLN_modulation`` = SiLU + Linear) that modulate the normalised pose
  tokens (``adaln_norm``, no affine), a residual is added, the 4-block trunk
  runs (dim 2048, 16 heads of 128, MLP 8192, LayerScale, no qk-norm / RoPE),
  then ``trunk_norm`` and ``pose_branch`` (2048 -> 1024 -> GELU -> 9) predict a
  delta that is accumulated; translation and quaternion are passed through,
  the field of view through ReLU.

LayerNorm eps: 1e-5 (torch's default) for ``token_norm``, ``trunk_norm`` and
the trunk blocks, 1e-6 for ``adaln_norm``.

Per frame there is one pose token, so the trunk linears run at M = S: every
S <= 64 runs on the skinny-M MFMA kernel (through the GEMV entry for
S <= 16 and the GEMM entry above).  Attention over S tokens with
head_dim 128 is a few kFLOP and runs in fp32 through torch.
``GraphedCameraHead`` records the whole forward as one HIP graph.  The CICT token
QVGGT's loader can attach (loader.py:224-246) has no public definition and is
not modelled.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import awq_inference_engine as E
from ._lib import QV_EPI_BIAS, QV_EPI_BIAS_GELU
from .aggregator import LayerScale, Mlp, _linear, _linear_residual, quantize_w4

DIM = 2048
HEADS = 16
HEAD_DIM = DIM // HEADS      # 128
MLP_DIM = 4 * DIM
TRUNK_DEPTH = 4
POSE_DIM = 9                 # absT (3) + quaternion (4) + FoV (2)
LN_EPS = 1e-5               # token_norm, trunk_norm, trunk blocks (torch's default)
ADALN_EPS = 1e-6


class TrunkBlock(nn.Module):
    """Camera-head trunk block: LN -> qkv -> attention over the frames -> proj ->
    LayerScale residual; LN -> fc1 -> GELU -> fc2 -> LayerScale residual."""

    def __init__(self, qkv, proj, fc1, fc2, dev=None):
        super().__init__()
        kw = dict(device=dev, dtype=torch.float16)
        self.norm1 = nn.LayerNorm(DIM, eps=LN_EPS, **kw)
        self.attn = nn.Module()
        self.attn.qkv, self.attn.proj = qkv, proj
        self.ls1 = LayerScale(DIM, 0.01, dev)
        self.norm2 = nn.LayerNorm(DIM, eps=LN_EPS, **kw)
        self.mlp = Mlp(fc1, fc2)
        self.ls2 = LayerScale(DIM, 0.01, dev)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        S = x.shape[0]
        h = E.layer_norm(x, self.norm1.weight, self.norm1.bias, LN_EPS)
        qkv = _linear(self.attn.qkv, h, QV_EPI_BIAS, torch.empty(S, 3 * DIM, dtype=x.dtype, device=x.device))
        q, k, v = qkv.float().view(S, 3, HEADS, HEAD_DIM).permute(1, 2, 0, 3)   # (H, S, 128) each
        a = torch.softmax(torch.bmm(q, k.transpose(1, 2).contiguous()) * HEAD_DIM ** -0.5, dim=-1) @ v
        att = a.permute(1, 0, 2).reshape(S, DIM).half()
        _linear_residual(self.attn.proj, att, self.ls1.gamma, x, torch.empty(S, DIM, dtype=x.dtype, device=x.device))
        h = E.layer_norm(x, self.norm2.weight, self.norm2.bias, LN_EPS)
        f = _linear(self.mlp.fc1, h, QV_EPI_BIAS_GELU, torch.empty(S, MLP_DIM, dtype=x.dtype, device=x.device))
        _linear_residual(self.mlp.fc2, f, self.ls2.gamma, x, torch.empty(S, DIM, dtype=x.dtype, device=x.device))
        return x


class CameraHead(nn.Module):
    """Iterative camera-pose head (module names as in the checkpoint, under
    ``camera_head.``).  ``forward(tokens)``: tokens (S, 2048) fp16 camera tokens;
    returns the activated pose encodings (S, 9) fp32 of every iteration."""

    def __init__(self, trunk_layers, dev=None):
        super().__init__()
        kw = dict(device=dev, dtype=torch.float16)
        self.trunk = nn.Sequential(*[TrunkBlock(*layers, dev=dev) for layers in trunk_layers])
        self.token_norm = nn.LayerNorm(DIM, eps=LN_EPS, **kw)
        self.trunk_norm = nn.LayerNorm(DIM, eps=LN_EPS, **kw)
        self.empty_pose_tokens = nn.Parameter(torch.zeros(1, 1, POSE_DIM, **kw), requires_grad=False)
        self.embed_pose = nn.Linear(POSE_DIM, DIM, **kw)
        self.poseLN_modulation = nn.Sequential(nn.SiLU(), nn.Linear(DIM, 3 * DIM, **kw))
        self.pose_branch = Mlp(nn.Linear(DIM, DIM // 2, **kw), nn.Linear(DIM // 2, POSE_DIM, **kw))
        self.register_buffer("_ones", torch.ones(DIM, **kw), persistent=False)
        self.register_buffer("_zeros", torch.zeros(DIM, **kw), persistent=False)

    @classmethod
    def empty(cls, device="cuda"):
        """fp16 ``nn.Linear`` trunk (the loader swaps the quantised ones)."""
        dev = torch.device(device)

        def lin(k, n):
            return nn.Linear(k, n, device=dev, dtype=torch.float16)

        return cls([(lin(DIM, 3 * DIM), lin(DIM, DIM), lin(DIM, MLP_DIM), lin(MLP_DIM, DIM))
                    for _ in range(TRUNK_DEPTH)], dev)

    @classmethod
    @torch.no_grad()
    def random(cls, seed: int = 0, device="cuda", w4: bool = True):
        """Seeded random weights (N(0, 0.02) linears); trunk linears W4 g128."""
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)

        def lin(k, n):
            l = nn.Linear(k, n, device=dev, dtype=torch.float16)
            l.weight.copy_((torch.randn(n, k, generator=g, device=dev) * 0.02).half())
            l.bias.copy_((torch.randn(n, generator=g, device=dev) * 0.02).half())
            return quantize_w4(l) if w4 else l

        layers = [(lin(DIM, 3 * DIM), lin(DIM, DIM), lin(DIM, MLP_DIM), lin(MLP_DIM, DIM)) for _ in range(TRUNK_DEPTH)]
        head = cls(layers, dev)
        for blk in head.trunk:
            for ln in (blk.norm1, blk.norm2):
                ln.weight.copy_((1 + 0.1 * torch.randn(DIM, generator=g, device=dev)).half())
                ln.bias.copy_((0.1 * torch.randn(DIM, generator=g, device=dev)).half())
            blk.ls1.gamma.copy_((0.5 + torch.rand(DIM, generator=g, device=dev)).half())
            blk.ls2.gamma.copy_((0.5 + torch.rand(DIM, generator=g, device=dev)).half())
        for ln in (head.token_norm, head.trunk_norm):
            ln.weight.copy_((1 + 0.1 * torch.randn(DIM, generator=g, device=dev)).half())
            ln.bias.copy_((0.1 * torch.randn(DIM, generator=g, device=dev)).half())
        for l in (head.embed_pose, head.poseLN_modulation[1], head.pose_branch.fc1, head.pose_branch.fc2):
            l.weight.copy_((torch.randn(l.weight.shape, generator=g, device=dev) * 0.02).half())
            l.bias.copy_((torch.randn(l.bias.shape, generator=g, device=dev) * 0.02).half())
        head.empty_pose_tokens.copy_((torch.randn(1, 1, POSE_DIM, generator=g, device=dev) * 0.02).half())
        return head

    @staticmethod
    def pose_tokens(layer_out: torch.Tensor) -> torch.Tensor:
        """Camera token (token 0) of every frame of a (S, tokens, 2048)
        [frame | global] aggregator output: the head's input."""
        return layer_out[:, 0].contiguous()

    @staticmethod
    def activate(enc: torch.Tensor) -> torch.Tensor:
        """absT_quaR_FoV with linear translation / quaternion and ReLU field of view."""
        return torch.cat([enc[..., :7], F.relu(enc[..., 7:])], dim=-1)

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, num_iterations: int = 4):
        S = tokens.shape[0]
        pose = E.layer_norm(tokens.contiguous(), self.token_norm.weight, self.token_norm.bias, LN_EPS)
        adaln = E.layer_norm(pose, self._ones, self._zeros, ADALN_EPS)
        pred, outs = None, []
        for _ in range(num_iterations):
            src = self.empty_pose_tokens.view(1, POSE_DIM).expand(S, POSE_DIM) if pred is None else pred.half()
            mod = self.poseLN_modulation(self.embed_pose(src))
            shift, scale, gate = mod.chunk(3, dim=-1)
            x = (gate * (adaln * (1 + scale) + shift) + pose).contiguous()
            for blk in self.trunk:
                blk(x)
            h = E.layer_norm(x, self.trunk_norm.weight, self.trunk_norm.bias, LN_EPS)
            delta = self.pose_branch.fc2(F.gelu(self.pose_branch.fc1(h))).float()
            pred = delta if pred is None else pred + delta
            outs.append(self.activate(pred))
        return outs


class GraphedCameraHead:
    """``CameraHead.forward`` for a fixed frame count S, recorded once as a HIP
    graph and replayed: the head is ~400 small launches per call (4 iterations
    x 4 trunk blocks of LayerNorm, four W4 linears at M = S, attention and
    residual updates), so replay removes the host launch cost that otherwise
    dominates at small S.  ``__call__(tokens)`` copies ``tokens`` (S, 2048)
    into the graph's input buffer, replays, and returns the graph's output
    tensors (overwritten by the next call; clone to keep them)."""

    def __init__(self, head: CameraHead, S: int, num_iterations: int = 4):
        dev = head.token_norm.weight.device
        self.head, self.S = head, S
        self.tokens = torch.zeros(S, DIM, dtype=torch.float16, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                head(self.tokens, num_iterations)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        # The eager calls above made every shape's tile plan; the W4 ops'
        # split-K launches in the graph use the device's scratch array (never
        # an eager stream's workspace), so replays may run on any stream, but
        # two graphs with split launches must not replay concurrently.
        with torch.cuda.graph(self.graph, stream=side):
            self.outs = head(self.tokens, num_iterations)

    @torch.no_grad()
    def __call__(self, tokens: torch.Tensor):
        if tokens.shape != self.tokens.shape:
            raise ValueError(f"GraphedCameraHead: recorded for {tuple(self.tokens.shape)} tokens, got {tuple(tokens.shape)}")
        self.tokens.copy_(tokens)
        self.graph.replay()
        return self.outs
