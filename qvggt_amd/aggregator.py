"""VGGT-1B aggregator on the MI355X kernels (W4A16 or W8A8 alternating-attention blocks).

The reference holds no model graph (it lives in the external vggt-hf fork,
loaded by qvggt/inference/loader.py:27,152-154); this is a restatement of the
public VGGT aggregator for the quantised hot path, with the module names the
reference's loader uses for the quantised layers
(``aggregator.frame_blocks.{i}.attn.qkv.qweight`` ..., loader.py:190-212,
346-392):

* patch embed: DINOv2 ViT-L/14 with 4 registers, fp16, unquantised
  (loader.py:346 keeps ``patch_embed`` linears in floating point);
* tokens per frame: camera token + 4 register tokens + 37 x 37 patches = 1374;
  the first frame uses token set 0, the others set 1;
* 24 x (frame block, global block); each block: LayerNorm -> qkv -> per-head
  qk LayerNorm -> 2-D RoPE (base 100, specials unrotated) -> attention ->
  proj -> LayerScale residual; LayerNorm -> fc1 -> GELU -> fc2 -> LayerScale
  residual.  Frame attention runs per frame (1374 tokens), global attention
  over all frames jointly.

Assumptions taken from the public VGGT design where the reference and the
benchmark configs are silent: qk-norm on, LayerScale init 0.01 (AA blocks) and
1e-5 (DINOv2), exact-erf GELU in the W4 path (the W8A8 path uses the
reference's tanh gelu_and_quant).  LayerNorm eps, depth and the RoPE base
come from ``AggregatorConfig`` (a checkpoint's config.json); its defaults are
the benchmark configuration's LayerNorm(1024, eps 1e-6) and 24 + 24 blocks.

Every hot op runs on libqvggt_hip.so, the AA blocks' LayerScale residual
updates included (fused into the proj / fc2 GEMMs); only the DINOv2 fp16
linears and the patch projection (plain GEMMs: hipBLASLt through torch), its
GELU and its LayerScale residual updates use torch.
"""
from __future__ import annotations

import dataclasses
import json
import math
from pathlib import Path

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import awq_inference_engine as E
from ._lib import QV_EPI_BIAS, QV_EPI_BIAS_GELU
from .awq.qmodule import WQLinear

GRID = 37
PATCH = 14
IMG = GRID * PATCH           # 518
DIM = 1024
HEADS = 16
HEAD_DIM = 64
MLP_DIM = 4096
N_REG = 4
SPECIALS = 1 + N_REG         # camera + registers
TOKENS = SPECIALS + GRID * GRID   # 1374
DEPTH = 24
LN_EPS = 1e-6                 # default DINOv2 patch-embed LayerNorm eps
BLOCK_LN_EPS = 1e-6           # default AA-block norm1 / norm2 / q_norm / k_norm eps
HEAD_LAYERS = (4, 11, 17, 23)     # intermediate outputs VGGT's heads consume


@dataclasses.dataclass(frozen=True)
class AggregatorConfig:
    """Model parameters of the aggregator, read from the checkpoint's model
    config as the reference builds its model from ``VGGTConfig`` (loader.py:146-162:
    ``VGGTConfig.from_pretrained(dirname(model_path))``, defaults otherwise).

    The defaults are the benchmark configuration (
    LayerNorm(1024, eps 1e-6), 24 + 24 blocks).  VGGT's published blocks build
    their norms with torch's default eps 1e-5, so a real checkpoint's config
    decides.  The kernels fix dim 1024, 16 heads of 64, MLP 4096 and the
    37 x 37 patch grid; other values are refused."""
    depth: int = DEPTH                 # AA iterations (one frame + one global block each)
    block_ln_eps: float = BLOCK_LN_EPS  # norm1 / norm2 / q_norm / k_norm of the AA blocks
    dino_depth: int = DEPTH            # DINOv2 patch-embed blocks
    dino_ln_eps: float = LN_EPS        # DINOv2 norms
    embed_dim: int = DIM
    num_heads: int = HEADS
    mlp_dim: int = MLP_DIM
    patch_size: int = PATCH
    img_size: int = IMG
    num_register_tokens: int = N_REG
    rope_base: float = 100.0

    # config.json keys accepted for each field (the vggt-hf VGGTConfig is
    # external and unpinned, so common Hugging Face spellings are all read)
    _ALIASES = {
        "depth": ("aa_depth", "depth", "num_hidden_layers"),
        "block_ln_eps": ("aa_layer_norm_eps", "block_layer_norm_eps", "layer_norm_eps", "norm_eps"),
        "dino_depth": ("patch_embed_depth", "dino_depth"),
        "dino_ln_eps": ("patch_embed_layer_norm_eps", "dino_layer_norm_eps"),
        "embed_dim": ("embed_dim", "hidden_size"),
        "num_heads": ("num_heads", "num_attention_heads"),
        "mlp_dim": ("mlp_dim", "intermediate_size"),
        "patch_size": ("patch_size",),
        "img_size": ("img_size", "image_size"),
        "num_register_tokens": ("num_register_tokens",),
        "rope_base": ("rope_freq", "rope_theta", "rope_base"),
    }

    def __post_init__(self):
        fixed = dict(embed_dim=DIM, num_heads=HEADS, mlp_dim=MLP_DIM, patch_size=PATCH, img_size=IMG,
                     num_register_tokens=N_REG)
        bad = {k: getattr(self, k) for k, v in fixed.items() if getattr(self, k) != v}
        if bad:
            raise ValueError(f"AggregatorConfig: unsupported model parameters {bad} (the kernels are built for {fixed})")
        if self.depth < 1 or self.dino_depth < 0 or not (self.block_ln_eps >= 0 and self.dino_ln_eps >= 0):
            raise ValueError(f"AggregatorConfig: bad depth / eps in {self}")

    @classmethod
    def from_dict(cls, d: dict) -> "AggregatorConfig":
        """Fields from a model-config dict; missing keys keep their defaults,
        and ``mlp_ratio`` gives ``mlp_dim``.  Top-level keys and those of a
        nested ``aggregator_config`` / ``aggregator`` section (which win) set
        any field.  A nested ``patch_embed_config`` section describes the
        DINOv2 patch embed only: its keys set ``dino_depth`` and
        ``dino_ln_eps`` (its plain ``depth`` / ``layer_norm_eps`` included) and
        never the aggregator's own blocks."""
        flat = dict(d)
        for sec in ("aggregator_config", "aggregator"):
            if isinstance(d.get(sec), dict):
                flat.update(d[sec])
        kw = {}
        for field, keys in cls._ALIASES.items():
            for k in keys:
                if k in flat and flat[k] is not None:
                    kw[field] = type(getattr(cls(), field))(flat[k])
                    break
        pe = d.get("patch_embed_config")
        if isinstance(pe, dict):
            for field, keys in (("dino_depth", cls._ALIASES["dino_depth"] + cls._ALIASES["depth"]),
                                ("dino_ln_eps", cls._ALIASES["dino_ln_eps"] + cls._ALIASES["block_ln_eps"])):
                for k in keys:
                    if pe.get(k) is not None:
                        kw[field] = type(getattr(cls(), field))(pe[k])
                        break
        if "mlp_dim" not in kw and flat.get("mlp_ratio") is not None:
            kw["mlp_dim"] = int(round(float(flat["mlp_ratio"]) * kw.get("embed_dim", DIM)))
        return cls(**kw)

    @classmethod
    def from_pretrained(cls, path) -> "AggregatorConfig":
        """``config.json`` of a checkpoint directory (or of the directory of a
        checkpoint file), read as JSON; defaults when there is none."""
        p = Path(path)
        cfg = (p if p.is_dir() else p.parent) / "config.json"
        if not cfg.exists():
            return cls()
        return cls.from_dict(json.loads(cfg.read_text()))


IMAGENET_MEAN = (0.485, 0.456, 0.406)
IMAGENET_STD = (0.229, 0.224, 0.225)


def vggt_positions(S: int, device=None) -> torch.Tensor:
    """(S*1374, 2) int32 (y, x) RoPE positions: specials at 0, patch (i, j) at (i+1, j+1)."""
    yy, xx = torch.meshgrid(torch.arange(GRID), torch.arange(GRID), indexing="ij")
    patch = torch.stack([yy.reshape(-1) + 1, xx.reshape(-1) + 1], 1)
    frame = torch.cat([torch.zeros(SPECIALS, 2, dtype=torch.long), patch], 0)
    return frame.repeat(S, 1).to(torch.int32).to(device)


# ------------------------------------------------------------ W8A8 linear
class W8A8Linear(nn.Module):
    """int8 per-output-channel weights; input is (int8 codes, per-token fp16 scales).

    forward(q, s) = fp16(float(q . W^T) * wscale[n] * s[m] + bias[n]), what the
    w8a8_gemm_fuse_bias_forward_cuda op computes.  (No such module exists in
    the reference; it pairs the W8A8 ops of csrc/w8a8 the way their signatures
    imply, pybind.cpp:29-36.)  The GEMM runs on a packed copy of ``weight``
    (``w8a8_pack_weight``), made on first use and again whenever ``weight``
    is replaced or written in place; results are bit for bit those of the
    op on ``weight``.
    """

    def __init__(self, in_features, out_features, bias=True, dev=None):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.register_buffer("weight", torch.zeros(out_features, in_features, dtype=torch.int8, device=dev))
        self.register_buffer("wscales", torch.zeros(out_features, dtype=torch.float16, device=dev))
        self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16, device=dev) if bias else None)
        self._packed, self._packed_key = None, None

    def packed_weight(self) -> torch.Tensor:
        """The packed copy of ``weight``, re-made when ``weight`` changed."""
        w = self.weight
        key = (w.data_ptr(), w._version, w.device)
        if self._packed_key != key:
            self._packed, self._packed_key = E.w8a8_pack_weight(w), key
        return self._packed

    @classmethod
    def from_linear(cls, linear: nn.Linear):
        W = linear.weight.data.float()
        m = cls(linear.in_features, linear.out_features, linear.bias is not None, W.device)
        ws = (W.abs().amax(1) / 127.0).clamp_min(1e-8)
        m.weight.copy_(torch.round(W / ws[:, None]).clamp(-128, 127).to(torch.int8))
        m.wscales.copy_(ws.half())
        if linear.bias is not None:
            m.bias.copy_(linear.bias.data.half())
        return m

    def forward(self, q: torch.Tensor, s: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        M = q.shape[0]
        out = torch.empty(M, self.out_features, dtype=torch.float16, device=q.device) if out is None else out
        E.w8a8_gemm_packed(q, self.packed_weight(), self.out_features, self.wscales, s, out, bias=self.bias)
        return out

    def forward_residual(self, q: torch.Tensor, s: torch.Tensor, gamma: torch.Tensor,
                         resid: torch.Tensor) -> torch.Tensor:
        """resid += gamma * forward(q, s), in place: fused into the GEMM's
        store loop when the layer has a bias, else the GEMM then torch's
        addcmul (the same single rounding of resid + gamma * o)."""
        if self.bias is not None:
            E.w8a8_gemm_packed(q, self.packed_weight(), self.out_features, self.wscales, s, resid,
                               bias=self.bias, gamma=gamma)
            return resid
        return resid.addcmul_(self.forward(q, s), gamma)


def quantize_w4(linear: nn.Linear, group: int = 128) -> WQLinear:
    """Asymmetric min/max int4 group quantisation of an fp16 ``nn.Linear`` into the
    AWQ-v2 ``WQLinear`` layout (scales s = (max-min)/15, integer zeros
    z = round(-min/s)), packed by ``WQLinear.from_linear`` (qmodule.py:225-329)."""
    W = linear.weight.data.float()
    N, K = W.shape
    Wg = W.view(N, K // group, group)
    wmin = Wg.amin(-1).clamp(max=0)
    wmax = Wg.amax(-1).clamp(min=0)
    s = ((wmax - wmin) / 15.0).clamp_min(1e-6)
    z = torch.round(-wmin / s).clamp(0, 15)
    return WQLinear.from_linear(linear, 4, group, scales=s.half(), zeros=z.half())


def _linear_residual(layer, x: torch.Tensor, gamma: torch.Tensor, resid: torch.Tensor, out: torch.Tensor):
    """resid += gamma * layer(x): a block's proj / fc2 with its LayerScale
    residual update, fused into the W4A16 epilogue when the layer is a
    ``WQLinear`` with a bias; otherwise the linear, then torch's addcmul."""
    if isinstance(layer, WQLinear) and layer.bias is not None:
        E.w4a16_linear_residual(x, layer.qweight, layer.scales, layer.scaled_zeros, layer.bias, gamma, resid)
        return resid
    o = _linear(layer, x, QV_EPI_BIAS if layer.bias is not None else 0, out)
    return resid.addcmul_(o, gamma)


def _linear(layer, x: torch.Tensor, epilogue: int, out: torch.Tensor) -> torch.Tensor:
    """One linear of an AA block: ``WQLinear`` on the W4A16 kernels with the
    bias (+ GELU) fused, or an unquantised fp16 ``nn.Linear`` (blocks a
    checkpoint leaves in floating point, loader.py:320-362) through torch."""
    if isinstance(layer, WQLinear):
        return E.w4a16_linear(x, layer.qweight, layer.scales, layer.scaled_zeros, bias=layer.bias,
                              epilogue=epilogue, out=out)
    if layer.bias is not None:
        y = torch.addmm(layer.bias, x, layer.weight.t(), out=out)
    else:
        y = torch.mm(x, layer.weight.t(), out=out)
    if epilogue == QV_EPI_BIAS_GELU:
        y.copy_(F.gelu(y))
    return y


def _with_depth(cfg: AggregatorConfig, depth: int | None) -> AggregatorConfig:
    return cfg if depth is None else dataclasses.replace(cfg, depth=depth, dino_depth=depth)


# ------------------------------------------------------------------ blocks
class LayerScale(nn.Module):
    def __init__(self, dim, init, dev=None):
        super().__init__()
        self.gamma = nn.Parameter(torch.full((dim,), init, dtype=torch.float16, device=dev), requires_grad=False)


class AAAttention(nn.Module):
    def __init__(self, qkv, proj, dev=None, eps: float = BLOCK_LN_EPS):
        super().__init__()
        self.qkv, self.proj = qkv, proj
        self.q_norm = nn.LayerNorm(HEAD_DIM, eps=eps, device=dev, dtype=torch.float16)
        self.k_norm = nn.LayerNorm(HEAD_DIM, eps=eps, device=dev, dtype=torch.float16)


class Mlp(nn.Module):
    def __init__(self, fc1, fc2):
        super().__init__()
        self.fc1, self.fc2 = fc1, fc2


class AABlock(nn.Module):
    """Frame or global block with W4A16 (``WQLinear``) or W8A8 linears; in the
    W4 form any of the four linears may also be an fp16 ``nn.Linear``."""

    def __init__(self, qkv, proj, fc1, fc2, w8a8: bool, dev=None, eps: float = BLOCK_LN_EPS):
        super().__init__()
        self.w8a8 = w8a8
        self.eps = float(eps)
        self.norm1 = nn.LayerNorm(DIM, eps=eps, device=dev, dtype=torch.float16)
        self.attn = AAAttention(qkv, proj, dev, eps)
        self.ls1 = LayerScale(DIM, 0.01, dev)
        self.norm2 = nn.LayerNorm(DIM, eps=eps, device=dev, dtype=torch.float16)
        self.mlp = Mlp(fc1, fc2)
        self.ls2 = LayerScale(DIM, 0.01, dev)

    @torch.no_grad()
    def forward(self, x: torch.Tensor, seq_len: int, pos: torch.Tensor, tables, ws: dict) -> torch.Tensor:
        """x: (M, 1024) fp16, updated in place.  ws: scratch buffers keyed by name."""
        M = x.shape[0]
        a = self.attn
        eps = self.eps
        if not self.w8a8 and isinstance(a.qkv, WQLinear) and a.qkv.bias is not None:
            # the qkv projection with its q/k LayerNorm and 2-D RoPE in the GEMM epilogue
            h = E.layer_norm(x, self.norm1.weight, self.norm1.bias, eps, out=ws["h"])
            qkv = E.w4a16_linear_qkrope(h, a.qkv.qweight, a.qkv.scales, a.qkv.scaled_zeros, a.qkv.bias, pos,
                                        tables[0], tables[1], HEADS, a.q_norm.weight, a.q_norm.bias,
                                        a.k_norm.weight, a.k_norm.bias, eps, out=ws["qkv"])
        else:
            if not self.w8a8:
                h = E.layer_norm(x, self.norm1.weight, self.norm1.bias, eps, out=ws["h"])
                qkv = _linear(a.qkv, h, QV_EPI_BIAS, ws["qkv"])
            else:
                E.rms_norm_general(ws["q8"], x, self.norm1.weight, self.norm1.bias, ws["s8"], eps, True)
                qkv = a.qkv(ws["q8"], ws["s8"], out=ws["qkv"])
            E.qknorm_rope2d(qkv, pos, tables[0], tables[1], HEADS, a.q_norm.weight, a.q_norm.bias,
                            a.k_norm.weight, a.k_norm.bias, eps)
        v3 = qkv.view(M, 3, HEADS, HEAD_DIM)
        att = E.attention(v3[:, 0], v3[:, 1], v3[:, 2], seq_len, out=ws["att"].view(M, HEADS, HEAD_DIM))
        att = att.view(M, DIM)
        if not self.w8a8:
            _linear_residual(a.proj, att, self.ls1.gamma, x, ws["o"])
        else:
            E.invoke_quant(ws["q8"], att, ws["s8"])
            a.proj.forward_residual(ws["q8"], ws["s8"], self.ls1.gamma, x)
        m = self.mlp
        if not self.w8a8:
            h = E.layer_norm(x, self.norm2.weight, self.norm2.bias, eps, out=ws["h"])
            f = _linear(m.fc1, h, QV_EPI_BIAS_GELU, ws["f"])
            _linear_residual(m.fc2, f, self.ls2.gamma, x, ws["o"])
        else:
            E.rms_norm_general(ws["q8"], x, self.norm2.weight, self.norm2.bias, ws["s8"], eps, True)
            f = m.fc1(ws["q8"], ws["s8"], out=ws["f"])
            E.gelu_and_quant(ws["q8f"], f, ws["s8"], None)   # the fp16 GELU copy is not needed
            m.fc2.forward_residual(ws["q8f"], ws["s8"], self.ls2.gamma, x)
        return x


class DinoBlock(nn.Module):
    """DINOv2 ViT-L block in fp16 (linears through hipBLASLt, LN/attention on our kernels)."""

    def __init__(self, dev=None, eps: float = LN_EPS):
        super().__init__()
        kw = dict(device=dev, dtype=torch.float16)
        self.eps = float(eps)
        self.norm1 = nn.LayerNorm(DIM, eps=eps, **kw)
        self.attn = nn.Module()
        self.attn.qkv = nn.Linear(DIM, 3 * DIM, **kw)
        self.attn.proj = nn.Linear(DIM, DIM, **kw)
        self.ls1 = LayerScale(DIM, 1e-5, dev)
        self.norm2 = nn.LayerNorm(DIM, eps=eps, **kw)
        self.mlp = Mlp(nn.Linear(DIM, MLP_DIM, **kw), nn.Linear(MLP_DIM, DIM, **kw))
        self.ls2 = LayerScale(DIM, 1e-5, dev)

    @torch.no_grad()
    def forward(self, x: torch.Tensor, ws: dict) -> torch.Tensor:
        M = x.shape[0]
        h = E.layer_norm(x, self.norm1.weight, self.norm1.bias, self.eps, out=ws["h"])
        qkv = torch.addmm(self.attn.qkv.bias, h, self.attn.qkv.weight.t(), out=ws["qkv"])
        v3 = qkv.view(M, 3, HEADS, HEAD_DIM)
        att = E.attention(v3[:, 0], v3[:, 1], v3[:, 2], TOKENS, out=ws["att"].view(M, HEADS, HEAD_DIM))
        o = torch.addmm(self.attn.proj.bias, att.view(M, DIM), self.attn.proj.weight.t(), out=ws["o"])
        x.addcmul_(o, self.ls1.gamma)
        h = E.layer_norm(x, self.norm2.weight, self.norm2.bias, self.eps, out=ws["h"])
        f = torch.addmm(self.mlp.fc1.bias, h, self.mlp.fc1.weight.t(), out=ws["f"])
        f = F.gelu(f)
        o = torch.addmm(self.mlp.fc2.bias, f, self.mlp.fc2.weight.t(), out=ws["o"])
        x.addcmul_(o, self.ls2.gamma)
        return x


class DinoPatchEmbed(nn.Module):
    """DINOv2 ViT-L/14 with 4 registers; returns the normalised patch tokens."""

    def __init__(self, dev=None, depth: int = DEPTH, eps: float = LN_EPS):
        super().__init__()
        kw = dict(device=dev, dtype=torch.float16)
        self.eps = float(eps)
        self.patch_embed = nn.Module()
        self.patch_embed.proj = nn.Conv2d(3, DIM, PATCH, PATCH, **kw)
        self.cls_token = nn.Parameter(torch.zeros(1, 1, DIM, **kw), requires_grad=False)
        self.register_tokens = nn.Parameter(torch.zeros(1, N_REG, DIM, **kw), requires_grad=False)
        self.pos_embed = nn.Parameter(torch.zeros(1, 1 + GRID * GRID, DIM, **kw), requires_grad=False)
        self.blocks = nn.ModuleList([DinoBlock(dev, eps) for _ in range(depth)])
        self.norm = nn.LayerNorm(DIM, eps=eps, **kw)

    @torch.no_grad()
    def project(self, images: torch.Tensor) -> torch.Tensor:
        """patch_embed.proj (a 14x14, stride-14 nn.Conv2d) of (S, 3, 518, 518)
        images as (S, 1369, D) tokens.  The convolution is a GEMM over the
        non-overlapping patches: each patch unfolds to its (channel, y, x)
        vector -- the order of the flattened conv weight (D, 3, 14, 14) -- and
        is multiplied in one addmm (M = S * 1369, K = 588, N = 1024,
        hipBLASLt), so no convolution solver is searched or picked per shape
        (in a benchmark trace MIOpen's naive direct kernel took 25.6 ms per
        call on average, most of it on the first calls)."""
        S = images.shape[0]
        proj = self.patch_embed.proj
        patches = (images.reshape(S, 3, GRID, PATCH, GRID, PATCH).permute(0, 2, 4, 1, 3, 5)
                   .reshape(S * GRID * GRID, 3 * PATCH * PATCH))
        return torch.addmm(proj.bias, patches, proj.weight.reshape(DIM, -1).t()).view(S, GRID * GRID, DIM)

    @torch.no_grad()
    def forward(self, images: torch.Tensor, ws: dict) -> torch.Tensor:
        S = images.shape[0]
        p = self.project(images)                                             # (S, 1369, D)
        x = torch.empty(S, TOKENS, DIM, dtype=torch.float16, device=images.device)
        x[:, :1] = self.cls_token + self.pos_embed[:, :1]
        x[:, 1:SPECIALS] = self.register_tokens
        torch.add(p, self.pos_embed[:, 1:], out=x[:, SPECIALS:])
        x = x.view(S * TOKENS, DIM)
        for blk in self.blocks:
            blk(x, ws)
        return E.layer_norm(x, self.norm.weight, self.norm.bias, self.eps).view(S, TOKENS, DIM)[:, SPECIALS:]


class Aggregator(nn.Module):
    """VGGT aggregator with quantised alternating-attention blocks.

    ``Aggregator.random(w8a8=False, seed=0, device=...)`` builds seeded random
    weights (fp16 masters quantised to W4 g128 or W8A8).  ``forward(images)``
    takes (S, 3, 518, 518) fp16 in [0, 1] and returns the final tokens
    (S*1374, 1024) plus the per-layer [frame | global] outputs VGGT's heads use.
    """

    def __init__(self, frame_blocks, global_blocks, w8a8: bool, dev=None, config: AggregatorConfig | None = None):
        super().__init__()
        self.config = config or AggregatorConfig(depth=len(frame_blocks))
        self.w8a8 = w8a8
        self.patch_embed = DinoPatchEmbed(dev, self.config.dino_depth, self.config.dino_ln_eps)
        self.camera_token = nn.Parameter(torch.zeros(1, 2, 1, DIM, dtype=torch.float16, device=dev),
                                         requires_grad=False)
        self.register_token = nn.Parameter(torch.zeros(1, 2, N_REG, DIM, dtype=torch.float16, device=dev),
                                           requires_grad=False)
        self.frame_blocks = nn.ModuleList(frame_blocks)
        self.global_blocks = nn.ModuleList(global_blocks)
        self.register_buffer("img_mean", torch.tensor(IMAGENET_MEAN, dtype=torch.float16, device=dev).view(1, 3, 1, 1))
        self.register_buffer("img_std", torch.tensor(IMAGENET_STD, dtype=torch.float16, device=dev).view(1, 3, 1, 1))
        self._tables = None
        self._ws = {}

    # ---------------------------------------------------------- construction
    @classmethod
    @torch.no_grad()
    def empty(cls, device="cuda", depth: int | None = None, config: AggregatorConfig | None = None):
        """fp16 aggregator with zero weights and plain ``nn.Linear`` AA linears,
        the starting point of checkpoint loading (qvggt_amd.loader swaps the
        quantised layers for ``WQLinear`` before the state dict goes in).
        ``depth`` overrides both depths of ``config``."""
        cfg = _with_depth(config or AggregatorConfig(), depth)
        dev = torch.device(device)

        def lin(k, n):
            return nn.Linear(k, n, device=dev, dtype=torch.float16)

        def block():
            return AABlock(lin(DIM, 3 * DIM), lin(DIM, DIM), lin(DIM, MLP_DIM), lin(MLP_DIM, DIM), False, dev,
                           cfg.block_ln_eps)

        return cls([block() for _ in range(cfg.depth)], [block() for _ in range(cfg.depth)], False, dev, cfg)

    @classmethod
    @torch.no_grad()
    def random(cls, w8a8: bool = False, seed: int = 0, device="cuda", depth: int | None = None,
               config: AggregatorConfig | None = None, layerscale: float = 0.01):
        """Seeded random-init weights (trunc-normal-like N(0, 0.02) linears), the
        AA linears quantised to W4 g128 (default) or W8A8; AA LayerScale
        ``layerscale`` (VGGT's init value 0.01 by default).  ``depth``
        overrides both depths of ``config``."""
        cfg = _with_depth(config or AggregatorConfig(), depth)
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)

        def lin(k, n):
            l = nn.Linear(k, n, device=dev, dtype=torch.float16)
            l.weight.copy_((torch.randn(n, k, generator=g, device=dev) * 0.02).half())
            l.bias.copy_((torch.randn(n, generator=g, device=dev) * 0.02).half())
            return l

        def q(l):
            return W8A8Linear.from_linear(l) if w8a8 else quantize_w4(l)

        def block():
            b = AABlock(q(lin(DIM, 3 * DIM)), q(lin(DIM, DIM)), q(lin(DIM, MLP_DIM)), q(lin(MLP_DIM, DIM)), w8a8, dev,
                        cfg.block_ln_eps)
            b.ls1.gamma.fill_(layerscale)
            b.ls2.gamma.fill_(layerscale)
            for ln in (b.norm1, b.norm2):
                ln.weight.copy_((1 + 0.1 * torch.randn(DIM, generator=g, device=dev)).half())
                ln.bias.copy_((0.1 * torch.randn(DIM, generator=g, device=dev)).half())
            for ln in (b.attn.q_norm, b.attn.k_norm):
                ln.weight.copy_((1 + 0.1 * torch.randn(HEAD_DIM, generator=g, device=dev)).half())
                ln.bias.copy_((0.1 * torch.randn(HEAD_DIM, generator=g, device=dev)).half())
            return b

        frame = [block() for _ in range(cfg.depth)]
        glob = [block() for _ in range(cfg.depth)]
        agg = cls(frame, glob, w8a8, dev, cfg)
        pe = agg.patch_embed
        pe.patch_embed.proj.weight.copy_((torch.randn(pe.patch_embed.proj.weight.shape, generator=g, device=dev) * 0.02).half())
        pe.patch_embed.proj.bias.zero_()
        pe.cls_token.copy_((torch.randn(1, 1, DIM, generator=g, device=dev) * 0.02).half())
        pe.register_tokens.copy_((torch.randn(1, N_REG, DIM, generator=g, device=dev) * 0.02).half())
        pe.pos_embed.copy_((torch.randn(1, 1 + GRID * GRID, DIM, generator=g, device=dev) * 0.02).half())
        for blk in pe.blocks:
            for name in ("qkv", "proj"):
                l = lin(DIM, 3 * DIM if name == "qkv" else DIM)
                getattr(blk.attn, name).weight.copy_(l.weight)
                getattr(blk.attn, name).bias.copy_(l.bias)
            for name, (k, n) in (("fc1", (DIM, MLP_DIM)), ("fc2", (MLP_DIM, DIM))):
                l = lin(k, n)
                getattr(blk.mlp, name).weight.copy_(l.weight)
                getattr(blk.mlp, name).bias.copy_(l.bias)
        agg.camera_token.copy_((torch.randn(1, 2, 1, DIM, generator=g, device=dev) * 0.02).half())
        agg.register_token.copy_((torch.randn(1, 2, N_REG, DIM, generator=g, device=dev) * 0.02).half())
        return agg

    # --------------------------------------------------------------- forward
    def _workspace(self, M: int, dev) -> dict:
        key = (M, str(dev))
        if self._ws.get("key") != key:
            f16 = dict(dtype=torch.float16, device=dev)
            self._ws = {
                "key": key,
                "h": torch.empty(M, DIM, **f16), "qkv": torch.empty(M, 3 * DIM, **f16),
                "att": torch.empty(M, DIM, **f16), "o": torch.empty(M, DIM, **f16),
                "f": torch.empty(M, MLP_DIM, **f16),
            }
            if self.w8a8:
                self._ws.update({
                    "q8": torch.empty(M, DIM, dtype=torch.int8, device=dev),
                    "q8f": torch.empty(M, MLP_DIM, dtype=torch.int8, device=dev),
                    "s8": torch.empty(M, **f16),
                })
        return self._ws

    @torch.no_grad()
    def forward(self, images: torch.Tensor, return_layers=HEAD_LAYERS):
        S = images.shape[0]
        dev = images.device
        M = S * TOKENS
        ws = self._workspace(M, dev)
        if self._tables is None or self._tables[0].device != dev:
            self._tables = E.rope2d_tables(GRID + 1, self.config.rope_base, device=dev)
        pos = vggt_positions(S, dev)
        x_img = (images - self.img_mean) / self.img_std
        patches = self.patch_embed(x_img, ws)                                   # (S, 1369, D)
        x = torch.empty(S, TOKENS, DIM, dtype=torch.float16, device=dev)
        x[:1, :1] = self.camera_token[:, 0]
        x[1:, :1] = self.camera_token[:, 1]
        x[:1, 1:SPECIALS] = self.register_token[:, 0]
        x[1:, 1:SPECIALS] = self.register_token[:, 1]
        x[:, SPECIALS:] = patches
        x = x.view(M, DIM)
        outputs = {}
        for i in range(len(self.frame_blocks)):
            self.frame_blocks[i](x, TOKENS, pos, self._tables, ws)
            keep = return_layers is not None and i in return_layers
            if keep:
                fr = x.clone()
            self.global_blocks[i](x, M, pos, self._tables, ws)
            if keep:
                outputs[i] = torch.cat([fr, x], dim=-1).view(S, TOKENS, 2 * DIM)
        return x, outputs
