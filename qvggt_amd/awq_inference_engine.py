"""Drop-in ``awq_inference_engine`` for MI355X (gfx950).

Same op names, argument order and meaning as the reference extension's
pybind module (qvggt/runtime/awq_inference_engine/csrc/pybind.cpp:16-37).
Each op validates its tensors on the host, then calls the C ABI of
libqvggt_hip.so (include/qvggt_hip.h) on the current HIP stream of the
input's device.  There is no CPU path: CPU tensors and a missing native
library raise.

Differences from the reference, all deliberate:
* launches go to ``torch.cuda.current_stream()`` (the reference GEMM/GEMV use
  the legacy default stream, gemm_cuda.cu:1229-1230, gemv_cuda.cu:237-268);
* non-contiguous inputs are made contiguous (the reference reads raw
  ``data_ptr`` regardless of strides);
* unsupported shapes raise ``RuntimeError`` instead of silently skipping a
  tail (gemm_cuda.cu:1224) or returning an uninitialised output
  (gemm_cuda.cu:1219-1223).
"""
from __future__ import annotations

import contextlib
import ctypes as C

import torch

from . import _lib
from ._lib import QV_BF16, QV_F16, QV_EPI_NONE

__all__ = [
    "layernorm_forward_cuda", "gemm_forward_cuda", "gemv_forward_cuda",
    "gemm_forward_cuda_new", "gemv_forward_cuda_new", "rotary_embedding_neox",
    "single_query_attention", "fused_rope_with_pos_forward_func",
    "w8a8_gemm_forward_cuda", "w8a8_gemm_fuse_bias_forward_cuda", "invoke_quant",
    "rms_norm_general", "silu_and_mul", "gelu_and_quant",
]

GROUP_SIZE = 128


# ----------------------------------------------------------------- helpers
def _fail(msg: str):
    raise RuntimeError(msg)


def _dtype_code(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.float16:
        return QV_F16
    if t.dtype == torch.bfloat16:
        return QV_BF16
    _fail(f"{what}: failed to dispatch data type {t.dtype} (expected float16 or bfloat16)")


def _on_gpu(*tensors: torch.Tensor, what: str):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            _fail(f"{what}: expected a tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            _fail(f"{what}: tensor on {t.device}; this op runs on the GPU only (no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            _fail(f"{what}: tensors on different devices ({dev} vs {t.device})")
    return dev


def _ptr(t: torch.Tensor | None):
    return C.c_void_p(t.data_ptr()) if t is not None else C.c_void_p(0)


def _stream(dev: torch.device):
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


_NULLCTX = contextlib.nullcontext()


def _device(dev: torch.device):
    """Device guard; free when ``dev`` is already the current device."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _NULLCTX
    return torch.cuda.device(dev)


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _check_w4_tables(kernel, scales, zeros, N, K, dt, what):
    if kernel.dtype not in (torch.int16, torch.int32):
        _fail(f"{what}: packed weight must be int16 (AWQ-v2 layout), got {kernel.dtype}")
    if kernel.numel() * kernel.element_size() != N * K // 2:
        _fail(f"{what}: packed weight holds {kernel.numel() * kernel.element_size()} bytes, "
              f"expected N*K/2 = {N * K // 2}")
    for name, t in (("scales", scales), ("zeros", zeros)):
        if t.dtype != dt:
            _fail(f"{what}: {name} dtype {t.dtype} != input dtype {dt}")
        if t.dim() != 2 or t.shape[1] != N or t.shape[0] < K // GROUP_SIZE:
            _fail(f"{what}: {name} must be (rows >= K/128 = {K // GROUP_SIZE}, N = {N}), "
                  f"got {tuple(t.shape)}")


# ----------------------------------------------------------- W4A16 GEMM/GEMV
def w4a16_linear(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                 scaled_zeros: torch.Tensor, bias: torch.Tensor | None = None,
                 epilogue: int = QV_EPI_NONE, out: torch.Tensor | None = None) -> torch.Tensor:
    """W4A16 g128 linear with an optional fused epilogue (bias, bias+GELU).

    Routes M <= 16 to the wavefront-reduction GEMV kernel and larger M to the
    MFMA GEMM.  Used by ``WQLinear`` to fuse qmodule.py:367's bias add.
    """
    what = "w4a16_linear"
    dev = _on_gpu(x, qweight, scales, scaled_zeros, bias, what=what)
    dt = _dtype_code(x, what)
    x = _contig(x)
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = qweight.shape[0] * 4
    _check_w4_tables(qweight, scales, scaled_zeros, N, K, x.dtype, what)
    if bias is not None and (bias.dtype != x.dtype or bias.numel() != N):
        _fail(f"{what}: bias must be ({N},) {x.dtype}")
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
    with _device(dev):
        args = (_ptr(x), _ptr(_contig(qweight)), _ptr(_contig(scales)), _ptr(_contig(scaled_zeros)),
                _ptr(bias), _ptr(out))
        if 1 <= M <= 16:
            _lib.call("qv_w4a16_gemv", *args, M, N, K, GROUP_SIZE, dt, epilogue, _stream(dev))
        else:
            _lib.call("qv_w4a16_gemm", *args, M, N, K, dt, epilogue, _stream(dev))
    return out


def gemm_forward_cuda_new(in_feats: torch.Tensor, kernel: torch.Tensor, scales: torch.Tensor,
                          zeros: torch.Tensor) -> torch.Tensor:
    """out[..., N] = in_feats[..., K] @ dequant(kernel)^T; N = kernel.size(0) * 4.

    Reference: quantization_new/gemm/gemm_cuda.cu:1125-1235 (group 128).
    """
    what = "gemm_forward_cuda_new"
    dt = _dtype_code(in_feats, what)
    K = in_feats.shape[-1]
    N = kernel.shape[0] * 4
    M = in_feats.numel() // K if K else 0
    _check_w4_tables(kernel, scales, zeros, N, K, in_feats.dtype, what)
    dev = _on_gpu(in_feats, kernel, scales, zeros, what=what)
    x = _contig(in_feats)
    out = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
    if M == 0:
        return out
    with _device(dev):
        _lib.call("qv_w4a16_gemm", _ptr(x), _ptr(_contig(kernel)), _ptr(_contig(scales)),
                  _ptr(_contig(zeros)), C.c_void_p(0), _ptr(out), M, N, K, dt, QV_EPI_NONE,
                  _stream(dev))
    return out


def gemv_forward_cuda_new(in_feats: torch.Tensor, kernel: torch.Tensor,
                          scaling_factors: torch.Tensor, zeros: torch.Tensor, m: int, n: int,
                          k: int, group_size: int) -> torch.Tensor:
    """Skinny-M W4A16 product for m in 1..7 (gemv_cuda.cu:197-281).

    Same errors as the reference: group_size != 128 -> "Unsupported group
    size", m outside 1..7 -> "Unsupported batch size".
    """
    what = "gemv_forward_cuda_new"
    dt = _dtype_code(in_feats, what)
    if group_size != GROUP_SIZE:
        _fail("Unsupported group size for gemv kernel.")
    if not 1 <= m <= 7:
        _fail("Unsupported batch size for gemv kernel.")
    if in_feats.numel() != m * k:
        _fail(f"{what}: in_feats has {in_feats.numel()} elements, expected m*k = {m * k}")
    _check_w4_tables(kernel, scaling_factors, zeros, n, k, in_feats.dtype, what)
    dev = _on_gpu(in_feats, kernel, scaling_factors, zeros, what=what)
    x = _contig(in_feats)
    out = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    with _device(dev):
        _lib.call("qv_w4a16_gemv", _ptr(x), _ptr(_contig(kernel)), _ptr(_contig(scaling_factors)),
                  _ptr(_contig(zeros)), C.c_void_p(0), _ptr(out), m, n, k, group_size, dt,
                  QV_EPI_NONE, _stream(dev))
    return out


def w4a16_dequantize(kernel: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                     in_features: int) -> torch.Tensor:
    """Dense (N, K) weights w = fp16_rn(q*s + sz) (dequantize.cuh:8-51 + hfma2)."""
    what = "w4a16_dequantize"
    dev = _on_gpu(kernel, scales, zeros, what=what)
    dt = _dtype_code(scales, what)
    K = in_features
    N = kernel.shape[0] * 4
    _check_w4_tables(kernel, scales, zeros, N, K, scales.dtype, what)
    out = torch.empty(N, K, dtype=scales.dtype, device=dev)
    with _device(dev):
        _lib.call("qv_w4a16_dequant", _ptr(_contig(kernel)), _ptr(_contig(scales)),
                  _ptr(_contig(zeros)), _ptr(out), N, K, dt, _stream(dev))
    return out


# ------------------------------------------------------ ops with no source
def gemm_forward_cuda(*args, **kwargs):
    """Legacy AWQ-v1 GEMM (pybind.cpp:19).  Its source (quantization/gemm_cuda_gen.cu)
    is absent from the reference, so there is nothing to reproduce."""
    raise NotImplementedError("gemm_forward_cuda: legacy AWQ-v1 op; its source is not part of "
                              "the reference extension. Use gemm_forward_cuda_new.")


def gemv_forward_cuda(*args, **kwargs):
    """Legacy AWQ-v1 GEMV (pybind.cpp:20); source absent from the reference."""
    raise NotImplementedError("gemv_forward_cuda: legacy AWQ-v1 op; its source is not part of "
                              "the reference extension. Use gemv_forward_cuda_new.")


def single_query_attention(*args, **kwargs):
    """FasterTransformer decode attention (pybind.cpp:24-27): an LLM KV-cache op
    outside the VGGT path (VGGT attention is bidirectional, no cache)."""
    raise NotImplementedError("single_query_attention: LLM decode attention is out of scope for "
                              "the VGGT path; use qvggt_amd.attention.attention_forward.")


def rotary_embedding_neox(*args, **kwargs):
    raise NotImplementedError("rotary_embedding_neox: not built yet")


def fused_rope_with_pos_forward_func(*args, **kwargs):
    raise NotImplementedError("fused_rope_with_pos_forward_func: not built yet")


def w8a8_gemm_forward_cuda(*args, **kwargs):
    raise NotImplementedError("w8a8_gemm_forward_cuda: not built yet")


def w8a8_gemm_fuse_bias_forward_cuda(*args, **kwargs):
    raise NotImplementedError("w8a8_gemm_fuse_bias_forward_cuda: not built yet")


def invoke_quant(*args, **kwargs):
    raise NotImplementedError("invoke_quant: not built yet")


def rms_norm_general(*args, **kwargs):
    raise NotImplementedError("rms_norm_general: not built yet")


def gelu_and_quant(*args, **kwargs):
    raise NotImplementedError("gelu_and_quant: not built yet")


def silu_and_mul(*args, **kwargs):
    raise NotImplementedError("silu_and_mul: not built yet")


def layernorm_forward_cuda(*args, **kwargs):
    raise NotImplementedError("layernorm_forward_cuda: not built yet")
