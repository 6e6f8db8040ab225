"""Quantised linear module with the reference's API and buffer layout.

Mirrors qvggt/runtime/awq/qmodule.py: ``WQLinear`` has the same constructor
signature, the same buffers (names, dtypes, shapes) and the same
``from_linear`` recipe, so state dicts written for the reference load
unchanged.  ``forward`` runs on the MI355X kernels of libqvggt_hip.so; the
bias add of qmodule.py:367 is fused into the GEMM/GEMV epilogue.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

from .. import awq_inference_engine as engine
from .._lib import QV_EPI_BIAS, QV_EPI_NONE


def make_divisible(c: int, divisor: int) -> int:
    """Ceiling division (qmodule.py:9-11)."""
    return (c + divisor - 1) // divisor


def calculate_zeros_width(in_features: int, group_size: int = 128, pack_num: int = 8) -> int:
    """Packed width of the scale tables (qmodule.py:13-41)."""
    if group_size == -1:
        group_size, size_multiplier = in_features, 1
    elif group_size >= 128:
        size_multiplier = 1
    elif group_size == 64:
        size_multiplier = 2
    elif group_size == 32:
        size_multiplier = 4
    else:
        raise NotImplementedError
    base_width = make_divisible(in_features // group_size, pack_num)
    return make_divisible(base_width, size_multiplier) * size_multiplier


def pack_intweight(unpacked_qweight: torch.Tensor, interleave: int, kstride: int) -> torch.Tensor:
    """AWQ-v2 int4 packing, (N, K) int values 0..15 -> int16 (N/interleave, K).

    Same output as qmodule.py:43-99.  Formulated per 64-k block: output row
    n//4 holds, for each block, 16 int16 of row 4*(n//4)+0, then +1, +2, +3;
    inside a row's 32-k half c, int16 (2f + e) carries the nibbles of
    k = 32c + 8h + 2f + e at bit 4h.  Runs on the tensor's device.
    """
    if interleave != 4 or kstride != 64:
        raise NotImplementedError("only interleave=4, kstride=64 (the AWQ-v2 layout) is supported")
    U = unpacked_qweight
    N, K = U.shape
    if N % 4 or K % 64:
        raise ValueError(f"shape {(N, K)} not divisible by (4, 64)")
    V = U.to(torch.int32).reshape(N // 4, 4, K // 64, 2, 4, 4, 2)  # (rg, r, kb, c, h, f, e)
    V = V.permute(0, 2, 1, 3, 5, 6, 4)                             # (rg, kb, r, c, f, e, h)
    packed = V[..., 0] | (V[..., 1] << 4) | (V[..., 2] << 8) | (V[..., 3] << 12)
    packed = packed.reshape(N // 4, K)
    # two's-complement int16 view of the 16-bit patterns
    packed = torch.where(packed >= 32768, packed - 65536, packed)
    return packed.to(torch.int16).contiguous()


class ScaledActivation(nn.Module):
    """act(x) / scales (qmodule.py:101-113)."""

    def __init__(self, module, scales):
        super().__init__()
        self.act = module
        self.scales = nn.Parameter(scales.data)

    def forward(self, x):
        return self.act(x) / self.scales.view(1, 1, -1).to(x.device)


class WQLinear(nn.Module):
    """W4A16 linear (qmodule.py:115-389), forward on gfx950."""

    def __init__(self, w_bit, group_size, in_features, out_features, bias, dev,
                 dtype=torch.float16):
        super().__init__()
        if w_bit not in [4]:
            raise NotImplementedError("Only 4-bit are supported for now.")
        self.in_features = in_features
        self.out_features = out_features
        self.w_bit = w_bit
        self.group_size = group_size if group_size != -1 else in_features
        self.split_k_iters = 8
        self.interleave = 4
        assert self.in_features % self.group_size == 0
        assert out_features % (32 // self.w_bit) == 0
        pack_num = 32 // self.w_bit
        int16_pack_num = 16 // self.w_bit
        assert out_features % self.interleave == 0
        rows = calculate_zeros_width(in_features, self.group_size) * pack_num
        self.register_buffer("qweight", torch.zeros(
            (out_features // self.interleave, in_features // int16_pack_num * self.interleave),
            dtype=torch.int16, device=dev))
        self.register_buffer("scales", torch.zeros((rows, out_features), dtype=dtype, device=dev))
        self.register_buffer("scaled_zeros", torch.zeros((rows, out_features), dtype=dtype, device=dev))
        if bias:
            self.register_buffer("bias", torch.zeros((out_features), dtype=dtype, device=dev))
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear, w_bit, group_size, init_only=False, scales=None, zeros=None):
        """Quantise + pack an ``nn.Linear`` (qmodule.py:225-329).

        scales, zeros: (out_features, in_features/group).  q = round((W + z*s)/s)
        per column (vectorised; element-wise identical to the reference loop).
        On a GPU with weight, scales and zeros all fp16 (or all bf16) the whole
        recipe runs as one HIP pass (``w4a16_pack``); otherwise in torch ops.
        """
        awq_linear = cls(w_bit, group_size, linear.in_features, linear.out_features,
                         linear.bias is not None, linear.weight.device,
                         dtype=linear.weight.data.dtype)
        if init_only:
            return awq_linear
        assert scales is not None and zeros is not None
        W = linear.weight.data
        if (W.is_cuda and W.dtype in (torch.float16, torch.bfloat16) and scales.dtype == W.dtype
                and zeros.dtype == W.dtype and W.shape[1] % 64 == 0):
            awq_linear.qweight, awq_linear.scales, awq_linear.scaled_zeros = engine.w4a16_pack(
                W, scales, zeros, group_size)
            if linear.bias is not None:
                awq_linear.bias = linear.bias.clone().to(W.dtype)
            return awq_linear
        scale_zeros = zeros * scales
        dtype = scales.dtype
        gs = group_size if group_size != -1 else linear.in_features
        pack_num = 32 // awq_linear.w_bit
        qscales = torch.zeros((scales.shape[0], calculate_zeros_width(linear.in_features, group_size) * pack_num),
                              dtype=dtype, device=scales.device)
        qscales[:, : scales.shape[1]] = scales
        awq_linear.scales = qscales.transpose(1, 0).contiguous()
        if linear.bias is not None:
            awq_linear.bias = linear.bias.clone().to(dtype)
        gidx = torch.arange(awq_linear.in_features, device=scales.device) // gs
        intweight = torch.round((linear.weight.data + scale_zeros[:, gidx]) / qscales[:, gidx]).to(torch.int)
        intweight = intweight.to(dtype=torch.int32)
        awq_linear.qweight = pack_intweight(intweight.contiguous(), interleave=4, kstride=64)
        zeros = zeros.to(dtype=torch.int32)
        scaled_zeros = torch.zeros_like(qscales)
        scaled_zeros[:, : scales.shape[1]] = -(qscales[:, : scales.shape[1]] * (zeros.to(torch.float32))).to(dtype)
        awq_linear.scaled_zeros = scaled_zeros.transpose(1, 0).contiguous()
        return awq_linear

    @torch.no_grad()
    def forward(self, x):
        if self.group_size != 128:
            raise RuntimeError(f"WQLinear.forward: group size {self.group_size} unsupported "
                               "(the reference kernels hard-code 128)")
        epi = QV_EPI_BIAS if self.bias is not None else QV_EPI_NONE
        return engine.w4a16_linear(x, self.qweight, self.scales, self.scaled_zeros,
                                   bias=self.bias, epilogue=epi)

    def extra_repr(self) -> str:
        return "in_features={}, out_features={}, bias={}, w_bit={}, group_size={}".format(
            self.in_features, self.out_features, self.bias is not None, self.w_bit, self.group_size)
