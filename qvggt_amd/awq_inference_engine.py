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
    """Contiguous view or copy.  A copy must be bound to a name that lives until
    the native call returns: passing ``_ptr(_contig(t))`` would hand the kernel
    the address of a temporary that the caching allocator may already have
    given to the next argument's copy."""
    return t if t.is_contiguous() else t.contiguous()


def _contig_opt(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else _contig(t)


def _check_out(out: torch.Tensor, M: int, N: int, dtype, what: str):
    """A caller-provided GEMM output: (..., N) with M*N elements, the input's
    dtype, contiguous, 16-byte aligned (the epilogue stores 16-byte rows)."""
    if not isinstance(out, torch.Tensor) or out.dtype != dtype:
        _fail(f"{what}: out must be a {dtype} tensor")
    if out.dim() < 1 or out.shape[-1] != N or out.numel() != M * N or not out.is_contiguous():
        _fail(f"{what}: out must be a contiguous (..., {N}) tensor of {M} x {N} elements, "
              f"got {tuple(out.shape)}")
    if out.data_ptr() % 16:
        _fail(f"{what}: out must be 16-byte aligned")


def _check_rope_tables(cos_table: torch.Tensor, sin_table: torch.Tensor, what: str):
    """2-D RoPE tables: contiguous float32 (P, 16), both the same shape (the
    kernels read row p at p*16, p clamped to P-1)."""
    for t in (cos_table, sin_table):
        if (not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or t.dim() != 2
                or t.shape[1] != 16 or t.shape[0] < 1 or not t.is_contiguous()):
            _fail(f"{what}: tables must be contiguous float32 (P, 16)")
    if cos_table.shape != sin_table.shape:
        _fail(f"{what}: cos and sin tables differ in shape")


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

    Routes M <= 16 to the GEMV entry and larger M to the GEMM entry; both run
    every M <= 64 on the skinny-M MFMA kernel.  Used by ``WQLinear`` to fuse
    qmodule.py:367's bias add.  ``out``, when given, must be a contiguous,
    16-byte aligned (..., N) tensor of the input's dtype.
    """
    what = "w4a16_linear"
    dt = _dtype_code(x, what)
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = qweight.shape[0] * 4
    _check_w4_tables(qweight, scales, scaled_zeros, N, K, x.dtype, what)
    if bias is not None and (bias.dtype != x.dtype or bias.numel() != N):
        _fail(f"{what}: bias must be ({N},) {x.dtype}")
    if out is not None:
        _check_out(out, M, N, x.dtype, what)
    dev = _on_gpu(x, qweight, scales, scaled_zeros, bias, out, what=what)
    x = _contig(x)
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
    # contiguous copies bound to names: they must outlive the native call
    qw, sc, sz, bb = _contig(qweight), _contig(scales), _contig(scaled_zeros), _contig_opt(bias)
    with _device(dev):
        args = (_ptr(x), _ptr(qw), _ptr(sc), _ptr(sz), _ptr(bb), _ptr(out))
        if 1 <= M <= 16:
            _lib.call("qv_w4a16_gemv", *args, M, N, K, GROUP_SIZE, dt, epilogue, _stream(dev))
        else:
            _lib.call("qv_w4a16_gemm", *args, M, N, K, dt, epilogue, _stream(dev))
    return out


def w4a16_linear_qkrope(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                        scaled_zeros: torch.Tensor, bias: torch.Tensor, positions: torch.Tensor,
                        cos_table: torch.Tensor, sin_table: torch.Tensor, heads: int,
                        q_gamma: torch.Tensor, q_beta: torch.Tensor, k_gamma: torch.Tensor,
                        k_beta: torch.Tensor, eps: float = 1e-6, out: torch.Tensor | None = None) -> torch.Tensor:
    """A VGGT block's qkv projection with its q/k LayerNorm and 2-D RoPE fused
    into the GEMM epilogue (fp16): the result of ``w4a16_linear(..., bias,
    QV_EPI_BIAS)`` followed by ``qknorm_rope2d`` in one kernel for M > 64 (the
    two calls themselves for smaller M).  Returns out (..., 3*heads*64)."""
    what = "w4a16_linear_qkrope"
    if x.dtype != torch.float16:
        _fail(f"{what}: x must be float16")
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = qweight.shape[0] * 4
    if N != 3 * heads * 64:
        _fail(f"{what}: the projection must have 3*heads*64 = {3 * heads * 64} outputs, got {N}")
    _check_w4_tables(qweight, scales, scaled_zeros, N, K, x.dtype, what)
    if bias is None or bias.dtype != x.dtype or bias.numel() != N:
        _fail(f"{what}: bias must be ({N},) {x.dtype}")
    for name, t in (("q_gamma", q_gamma), ("q_beta", q_beta), ("k_gamma", k_gamma), ("k_beta", k_beta)):
        if t.dtype != torch.float16 or t.numel() != 64:
            _fail(f"{what}: {name} must be float16 (64,)")
    if positions.dtype != torch.int32 or positions.numel() != 2 * M:
        _fail(f"{what}: positions must be int32 (M, 2)")
    _check_rope_tables(cos_table, sin_table, what)
    if out is not None:
        _check_out(out, M, N, x.dtype, what)
    dev = _on_gpu(x, qweight, scales, scaled_zeros, bias, positions, cos_table, sin_table, q_gamma, q_beta,
                  k_gamma, k_beta, out, what=what)
    x = _contig(x)
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=dev)
    # contiguous copies bound to names: they must outlive the native call
    qw, sc, sz, bb = _contig(qweight), _contig(scales), _contig(scaled_zeros), _contig(bias)
    pos = _contig(positions)
    qg, qb, kg, kb = _contig(q_gamma), _contig(q_beta), _contig(k_gamma), _contig(k_beta)
    with _device(dev):
        _lib.call("qv_w4a16_gemm_qkrope", _ptr(x), _ptr(qw), _ptr(sc), _ptr(sz), _ptr(bb), _ptr(out), M, N, K,
                  _ptr(pos), _ptr(cos_table), _ptr(sin_table), cos_table.shape[0], _ptr(qg), _ptr(qb), _ptr(kg),
                  _ptr(kb), C.c_float(eps), heads, _stream(dev))
    return out


def w4a16_linear_residual(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                          scaled_zeros: torch.Tensor, bias: torch.Tensor, gamma: torch.Tensor,
                          residual: torch.Tensor) -> torch.Tensor:
    """residual += gamma * fp16(x @ dequant(W)^T + bias), in place: a VGGT block's
    proj / fc2 linear fused with its LayerScale residual update
    (``x.addcmul_(linear(h), gamma)``).  Returns ``residual``."""
    what = "w4a16_linear_residual"
    dev = _on_gpu(x, qweight, scales, scaled_zeros, bias, gamma, residual, what=what)
    dt = _dtype_code(x, what)
    x = _contig(x)
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = qweight.shape[0] * 4
    _check_w4_tables(qweight, scales, scaled_zeros, N, K, x.dtype, what)
    for name, t in (("bias", bias), ("gamma", gamma)):
        if t.dtype != x.dtype or t.numel() != N:
            _fail(f"{what}: {name} must be ({N},) {x.dtype}")
    if residual.dtype != x.dtype or residual.numel() != M * N or not residual.is_contiguous():
        _fail(f"{what}: residual must be a contiguous {x.dtype} tensor of {M} x {N} elements")
    qw, sc, sz = _contig(qweight), _contig(scales), _contig(scaled_zeros)
    bb, gg = _contig(bias), _contig(gamma)
    with _device(dev):
        _lib.call("qv_w4a16_gemm_residual", _ptr(x), _ptr(qw), _ptr(sc), _ptr(sz), _ptr(bb), _ptr(gg),
                  _ptr(residual), M, N, K, dt, _stream(dev))
    return residual


def w4a16_plan(M: int, N: int, K: int, epilogue: int = _lib.QV_EPI_NONE) -> dict:
    """The launch plan of an M x K -> N W4A16 linear (no device work):
    ``kernel`` "skinny", "stream", "stream_ksplit" (K summed in two halves
    by two wave groups of one workgroup) or "stream_k128" (128-k pipeline
    stages; same sums as "stream"), ``tile`` rows of the first range,
    ``rows`` the rows it covers, ``tile2`` the second range's tile height
    (0: one range)."""
    plan = (C.c_int32 * 4)()
    _lib.call("qv_w4a16_plan", int(M), int(N), int(K), int(epilogue), C.cast(plan, C.c_void_p))
    kind = {0: "skinny", 1: "stream", 2: "stream_ksplit", 3: "stream_k128"}[plan[0]]
    return {"kernel": kind, "tile": plan[1], "rows": plan[2], "tile2": plan[3]}


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
    qw, sc, sz = _contig(kernel), _contig(scales), _contig(zeros)
    with _device(dev):
        _lib.call("qv_w4a16_gemm", _ptr(x), _ptr(qw), _ptr(sc), _ptr(sz), C.c_void_p(0), _ptr(out),
                  M, N, K, dt, QV_EPI_NONE, _stream(dev))
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
    if in_feats.dim() < 1 or in_feats.shape[-1] != k or in_feats.numel() != m * k:
        _fail(f"{what}: in_feats must be (..., k = {k}) with m*k = {m * k} elements, "
              f"got {tuple(in_feats.shape)}")
    if kernel.dim() != 2 or kernel.shape[0] * 4 != n:
        _fail(f"{what}: kernel must be (n/4, k) = ({n // 4}, {k}), got {tuple(kernel.shape)}")
    _check_w4_tables(kernel, scaling_factors, zeros, n, k, in_feats.dtype, what)
    dev = _on_gpu(in_feats, kernel, scaling_factors, zeros, what=what)
    x = _contig(in_feats)
    out = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=dev)
    qw, sc, sz = _contig(kernel), _contig(scaling_factors), _contig(zeros)
    with _device(dev):
        _lib.call("qv_w4a16_gemv", _ptr(x), _ptr(qw), _ptr(sc), _ptr(sz), C.c_void_p(0), _ptr(out),
                  m, n, k, group_size, dt, QV_EPI_NONE, _stream(dev))
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
    qw, sc, sz = _contig(kernel), _contig(scales), _contig(zeros)
    with _device(dev):
        _lib.call("qv_w4a16_dequant", _ptr(qw), _ptr(sc), _ptr(sz), _ptr(out), N, K, dt, _stream(dev))
    return out


def w4a16_pack(weight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
               group_size: int = 128):
    """Quantise and pack fp16 / bf16 weights into the WQLinear buffers on the GPU.

    weight (N, K), scales and zeros (N, K / group) in the weight's dtype (zeros
    integer-valued).  Returns (qweight int16 (N/4, K), scales (rows, N),
    scaled_zeros (rows, N)), element for element what ``WQLinear.from_linear``
    (qmodule.py:225-329) stores: q = round((W + z*s) / s) in the model dtype,
    AWQ-v2 packing, zero-padded transposed tables, scaled_zeros = -(s * z).
    """
    what = "w4a16_pack"
    dev = _on_gpu(weight, scales, zeros, what=what)
    dt = _dtype_code(weight, what)
    if weight.dim() != 2:
        _fail(f"{what}: weight must be (N, K)")
    N, K = weight.shape
    gs = K if group_size == -1 else group_size
    if gs <= 0 or K % gs:
        _fail(f"{what}: group size {group_size} does not divide K={K}")
    for name, t in (("scales", scales), ("zeros", zeros)):
        if t.dtype != weight.dtype or tuple(t.shape) != (N, K // gs):
            _fail(f"{what}: {name} must be ({N}, {K // gs}) {weight.dtype}")
    mult = 1 if group_size == -1 else {64: 2, 32: 4}.get(gs, 1)
    rows = (-(-(-(-(K // gs) // 8)) // mult)) * mult * 8   # calculate_zeros_width(K, gs) * 8 (qmodule.py:13-41)
    qweight = torch.empty(N // 4, K, dtype=torch.int16, device=dev)
    s_out = torch.empty(rows, N, dtype=weight.dtype, device=dev)
    sz_out = torch.empty(rows, N, dtype=weight.dtype, device=dev)
    w, s, z = _contig(weight), _contig(scales), _contig(zeros)
    with _device(dev):
        _lib.call("qv_w4a16_pack", _ptr(w), _ptr(s), _ptr(z), _ptr(qweight), _ptr(s_out), _ptr(sz_out),
                  N, K, group_size, dt, _stream(dev))
    return qweight, s_out, sz_out


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
    """1-D NeoX RoPE from a cos/sin cache (position_embedding/pos_encoding_kernels.cu:5-79):
    an LLM op outside the VGGT path (VGGT uses 2-D RoPE, see ``rope2d``)."""
    raise NotImplementedError("rotary_embedding_neox: LLM 1-D RoPE is out of scope for the VGGT path; "
                              "use fused_rope_with_pos_forward_func or rope2d.")


def silu_and_mul(*args, **kwargs):
    """SwiGLU activation (w8a8/act.cu:94-131): an LLM op; the VGGT MLP uses GELU."""
    raise NotImplementedError("silu_and_mul: SwiGLU is out of scope for the VGGT path (its MLP uses GELU).")


# -------------------------------------------------------------- W8A8 ops
_DT_ANY = {torch.float16: QV_F16, torch.bfloat16: QV_BF16, torch.float32: 2}


def _dtype_any(t: torch.Tensor, what: str) -> int:
    if t.dtype not in _DT_ANY:
        _fail(f"{what}: unsupported dtype {t.dtype} (expected float32, float16 or bfloat16)")
    return _DT_ANY[t.dtype]


def _need(t: torch.Tensor, dtype, what: str, name: str):
    if t.dtype != dtype:
        _fail(f"{what}: {name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        _fail(f"{what}: {name} must be contiguous (it is written in place)")


def _w8a8(in_feats, kernel, wscales, ascales, out_feats, bias, what, gamma=None, packed_n=None):
    for name, t, dt in (("in_feats", in_feats, torch.int8), ("kernel", kernel, torch.int8),
                        ("wscales", wscales, torch.float16), ("ascales", ascales, torch.float16),
                        ("out_feats", out_feats, torch.float16)):
        _need(t, dt, what, name)
    if in_feats.dim() != 2 or (packed_n is None and kernel.dim() != 2):
        _fail(f"{what}: in_feats and kernel must be 2-D (M,K) and (N,K)")
    M, K = in_feats.shape
    if packed_n is None:
        N = kernel.shape[0]
        if kernel.shape[1] != K:
            _fail(f"{what}: K mismatch {K} vs {kernel.shape[1]}")
    else:
        N = int(packed_n)
        if kernel.dim() != 1 or kernel.numel() != w8a8_packed_bytes(N, K):
            _fail(f"{what}: packed weight must be 1-D with {w8a8_packed_bytes(N, K)} bytes for N={N} K={K}, "
                  f"got shape {tuple(kernel.shape)}")
    if out_feats.shape[-2:] != (M, N):
        _fail(f"{what}: out_feats must be (M, N) = ({M}, {N}), got {tuple(out_feats.shape)}")
    if wscales.numel() != N or ascales.numel() != M:
        _fail(f"{what}: wscales must have N={N} and ascales M={M} elements")
    if bias is not None:
        _need(bias, torch.float16, what, "bias")
        if bias.numel() != N:
            _fail(f"{what}: bias must have N={N} elements")
    if gamma is not None:
        _need(gamma, torch.float16, what, "gamma")
        if gamma.numel() != N:
            _fail(f"{what}: gamma must have N={N} elements")
        if bias is None:
            _fail(f"{what}: the residual form needs the bias")
    dev = _on_gpu(in_feats, kernel, wscales, ascales, out_feats, bias, gamma, what=what)
    with _device(dev):
        if packed_n is not None:
            _lib.call("qv_w8a8_gemm_packed", _ptr(in_feats), _ptr(kernel), _ptr(wscales), _ptr(ascales),
                      _ptr(bias), _ptr(gamma), _ptr(out_feats), M, N, K, _stream(dev))
        elif gamma is None:
            _lib.call("qv_w8a8_gemm", _ptr(in_feats), _ptr(kernel), _ptr(wscales), _ptr(ascales), _ptr(bias),
                      _ptr(out_feats), M, N, K, _stream(dev))
        else:
            _lib.call("qv_w8a8_gemm_residual", _ptr(in_feats), _ptr(kernel), _ptr(wscales), _ptr(ascales),
                      _ptr(bias), _ptr(gamma), _ptr(out_feats), M, N, K, _stream(dev))


def w8a8_gemm_forward_cuda(in_feats, kernel, wscales, ascales, out_feats) -> None:
    """out_feats[M,N] = fp16((float(int8 A . int8 B^T) * ws[n]) * as[m]), written in place
    (w8a8/w8a8_gemm_cuda.cu:881-922)."""
    _w8a8(in_feats, kernel, wscales, ascales, out_feats, None, "w8a8_gemm_forward_cuda")


def w8a8_gemm_fuse_bias_forward_cuda(in_feats, kernel, wscales, ascales, out_feats, bias) -> None:
    """As ``w8a8_gemm_forward_cuda`` plus bias[n] (w8a8/w8a8_gemm_cuda.cu:564-607)."""
    _w8a8(in_feats, kernel, wscales, ascales, out_feats, bias, "w8a8_gemm_fuse_bias_forward_cuda")


def w8a8_linear_residual(in_feats, kernel, wscales, ascales, bias, gamma, residual) -> torch.Tensor:
    """residual += gamma * fp16(W8A8 GEMM + bias), in place (one rounding of
    residual + gamma * o in fp32): a VGGT block's W8A8 proj / fc2 fused with its
    LayerScale residual update (``x.addcmul_(o, gamma)``).  Returns ``residual``."""
    what = "w8a8_linear_residual"
    if not residual.is_contiguous():
        _fail(f"{what}: residual must be contiguous")
    _w8a8(in_feats, kernel, wscales, ascales, residual, bias, what, gamma=gamma)
    return residual


def w8a8_packed_bytes(N: int, K: int) -> int:
    """Size in bytes of an (N, K) int8 weight in the packed layout (N rounded up to 32)."""
    return (N + 31) // 32 * 32 * K


def w8a8_pack_weight(kernel: torch.Tensor) -> torch.Tensor:
    """One-time re-layout of an (N, K) int8 weight for ``w8a8_gemm_packed``: a
    1-D int8 tensor of ``w8a8_packed_bytes(N, K)`` bytes.  No reference
    counterpart (the reference's GEMM reads the (N, K) weight as stored); the
    packed GEMM loads each wave's weight fragments with one contiguous 1 KB
    load per instruction instead of staging them through LDS."""
    what = "w8a8_pack_weight"
    _need(kernel, torch.int8, what, "kernel")
    if kernel.dim() != 2:
        _fail(f"{what}: kernel must be 2-D (N, K)")
    N, K = kernel.shape
    dev = _on_gpu(kernel, what=what)
    packed = torch.empty(w8a8_packed_bytes(N, K), dtype=torch.int8, device=dev)
    with _device(dev):
        _lib.call("qv_w8a8_pack_weight", _ptr(kernel), _ptr(packed), N, K, _stream(dev))
    return packed


def w8a8_gemm_packed(in_feats, packed, N: int, wscales, ascales, out_feats, bias=None, gamma=None) -> None:
    """``w8a8_gemm_forward_cuda`` / ``w8a8_gemm_fuse_bias_forward_cuda`` (gamma None)
    or ``w8a8_linear_residual`` (gamma given, bias required, ``out_feats`` the
    residual, updated in place) from a ``w8a8_pack_weight`` weight of N output
    channels: the same results bit for bit."""
    what = "w8a8_gemm_packed"
    if gamma is not None and not out_feats.is_contiguous():
        _fail(f"{what}: residual must be contiguous")
    _w8a8(in_feats, packed, wscales, ascales, out_feats, bias, what, gamma=gamma, packed_n=N)


def w8a8_gemm_int32(in_feats: torch.Tensor, kernel: torch.Tensor) -> torch.Tensor:
    """Raw int32 accumulators in_feats (M,K) int8 . kernel (N,K)^T (bit-exact check)."""
    what = "w8a8_gemm_int32"
    _need(in_feats, torch.int8, what, "in_feats")
    _need(kernel, torch.int8, what, "kernel")
    M, K = in_feats.shape
    N = kernel.shape[0]
    dev = _on_gpu(in_feats, kernel, what=what)
    out = torch.empty(M, N, dtype=torch.int32, device=dev)
    with _device(dev):
        _lib.call("qv_w8a8_gemm_i32", _ptr(in_feats), _ptr(kernel), _ptr(out), M, N, K, _stream(dev))
    return out


def invoke_quant(out: torch.Tensor, input: torch.Tensor, scale: torch.Tensor) -> None:
    """Per-token int8 quantisation (w8a8/quantization.cu:81-96): out int8 like input,
    scale fp16 (tokens,) = amax/127."""
    what = "invoke_quant"
    dt = _dtype_any(input, what)
    _need(out, torch.int8, what, "out")
    _need(scale, torch.float16, what, "scale")
    D = input.shape[-1]
    M = input.numel() // D if D else 0
    if out.numel() != input.numel() or scale.numel() < M:
        _fail(f"{what}: out must match input and scale hold {M} tokens")
    dev = _on_gpu(out, input, scale, what=what)
    x = _contig(input)
    with _device(dev):
        _lib.call("qv_quant_per_token", _ptr(x), dt, _ptr(out), _ptr(scale), M, D, _stream(dev))


def rms_norm_general(out: torch.Tensor, input: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                     scaling: torch.Tensor, epsilon: float, use_per_token_quant: bool = True) -> None:
    """LayerNorm + int8 quantisation (w8a8/layernorm.cu:155-191; despite the name a full
    LayerNorm with mean and beta).  Per token: scaling (tokens,) fp16 is written; per
    tensor: scaling[0] fp16 is read and bias is not used."""
    what = "rms_norm_general"
    dt = _dtype_any(input, what)
    _need(out, torch.int8, what, "out")
    _need(scaling, torch.float16, what, "scaling")
    D = input.shape[-1]
    M = input.numel() // D if D else 0
    if weight.dtype != input.dtype or weight.numel() != D:
        _fail(f"{what}: weight must be ({D},) {input.dtype}")
    if use_per_token_quant and (bias is None or bias.dtype != input.dtype or bias.numel() != D):
        _fail(f"{what}: bias must be ({D},) {input.dtype}")
    if out.numel() != input.numel() or scaling.numel() < (M if use_per_token_quant else 1):
        _fail(f"{what}: out must match input; scaling too small")
    dev = _on_gpu(out, input, weight, bias if use_per_token_quant else None, scaling, what=what)
    x, w = _contig(input), _contig(weight)
    b = _contig(bias) if use_per_token_quant else None
    with _device(dev):
        _lib.call("qv_layernorm_quant", _ptr(x), dt, _ptr(w), _ptr(b), _ptr(out), _ptr(scaling),
                  C.c_float(epsilon), 1 if use_per_token_quant else 0, M, D, _stream(dev))


def gelu_and_quant(out: torch.Tensor, input: torch.Tensor, scale_out: torch.Tensor, tmp: torch.Tensor | None) -> None:
    """tanh-GELU (fp16 arithmetic) + per-token int8 (w8a8/act.cu:30-90); tmp gets the
    fp16 GELU values, scale_out the per-token fp16 scales.  ``tmp=None`` (an
    extension of the reference op, which always writes it) skips that store."""
    what = "gelu_and_quant"
    if input.dtype != torch.float16:
        _fail(f"{what}: input must be float16 (the reference kernel is half-only)")
    _need(out, torch.int8, what, "out")
    _need(scale_out, torch.float16, what, "scale_out")
    if tmp is not None:
        _need(tmp, torch.float16, what, "tmp")
    D = input.shape[-1]
    M = input.numel() // D if D else 0
    if out.numel() != input.numel() or (tmp is not None and tmp.numel() != input.numel()) or scale_out.numel() < M:
        _fail(f"{what}: out/tmp must match input, scale_out hold {M} tokens")
    dev = _on_gpu(out, input, scale_out, tmp, what=what)
    x = _contig(input)
    with _device(dev):
        _lib.call("qv_gelu_quant", _ptr(x), _ptr(out), _ptr(scale_out), _ptr(tmp), M, D, _stream(dev))


def layernorm_forward_cuda(_input: torch.Tensor, _gamma: torch.Tensor, _out: torch.Tensor, eps: float) -> None:
    """T5 RMSNorm (layernorm/layernorm.cu:98-116): input must be 3-D (m = size0*size1,
    n = size2), out written in place, fp16 outputs clamped to +-64504."""
    what = "layernorm_forward_cuda"
    if _input.dim() != 3:
        _fail(f"{what}: input must be 3-D (got {_input.dim()}-D)")
    dt = _dtype_code(_input, what)
    if _gamma.dtype != _input.dtype or _out.dtype != _input.dtype:
        _fail(f"{what}: gamma and out must have the input dtype {_input.dtype}")
    _need(_out, _input.dtype, what, "out")
    M = _input.shape[0] * _input.shape[1]
    D = _input.shape[2]
    if _gamma.numel() != D or _out.numel() != _input.numel():
        _fail(f"{what}: gamma must be ({D},) and out match input")
    dev = _on_gpu(_input, _gamma, _out, what=what)
    x, g = _contig(_input), _contig(_gamma)
    with _device(dev):
        _lib.call("qv_rmsnorm", _ptr(x), _ptr(g), _ptr(_out), C.c_float(eps), M, D, dt, _stream(dev))


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = 1e-6,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """torch.nn.LayerNorm semantics over the last dim (fp32 statistics): the VGGT
    blocks' norm1 / norm2.  No reference op (the model graph is external)."""
    what = "layer_norm"
    dt = _dtype_code(x, what)
    D = x.shape[-1]
    M = x.numel() // D if D else 0
    if weight.dtype != x.dtype or bias.dtype != x.dtype or weight.numel() != D or bias.numel() != D:
        _fail(f"{what}: weight/bias must be ({D},) {x.dtype}")
    dev = _on_gpu(x, weight, bias, out, what=what)
    x, w, b = _contig(x), _contig(weight), _contig(bias)
    if out is None:
        out = torch.empty_like(x)
    elif out.dtype != x.dtype or out.numel() != x.numel() or not out.is_contiguous():
        _fail(f"{what}: out must be a contiguous {x.dtype} tensor of {x.numel()} elements")
    with _device(dev):
        _lib.call("qv_layernorm", _ptr(x), _ptr(w), _ptr(b), _ptr(out), C.c_float(eps), M, D, dt,
                  _stream(dev))
    return out


# ----------------------------------------------------------------- RoPE
def fused_rope_with_pos_forward_func(input: torch.Tensor, freqs: torch.Tensor,
                                     transpose_output_memory: bool) -> torch.Tensor:
    """Rotate-half RoPE on input (s, b, h, d) (any strides) with fp32 angles freqs
    [b][s][d2] (rope_new/fused_rope_with_pos.cu:122-164).  Output (s, b, h, d), stored
    as (b, s, h, d) memory when transpose_output_memory."""
    what = "fused_rope_with_pos_forward_func"
    dt = _dtype_any(input, what)
    if input.dim() != 4:
        _fail(f"{what}: input must be 4-D (s, b, h, d)")
    if freqs.dtype != torch.float32:
        _fail(f"{what}: freqs must be float32")
    s, b, h, d = input.shape
    d2 = freqs.shape[-1]
    if freqs.numel() != b * s * d2 or d2 > d or d2 % 2:
        _fail(f"{what}: freqs must hold b*s*d2 = {b}*{s}*{d2} values, d2 even and <= d")
    dev = _on_gpu(input, freqs, what=what)
    if transpose_output_memory:
        out = torch.empty(b, s, h, d, dtype=input.dtype, device=dev).transpose(0, 1)
    else:
        out = torch.empty(s, b, h, d, dtype=input.dtype, device=dev)
    xs = (C.c_int64 * 4)(*input.stride())
    os_ = (C.c_int64 * 4)(*out.stride())
    fr = _contig(freqs)
    with _device(dev):
        _lib.call("qv_rope_with_pos", _ptr(input), _ptr(fr), _ptr(out), dt, s, b, h, d, d2, xs, os_,
                  _stream(dev))
    return out


def rope2d(qkv: torch.Tensor, positions: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
           heads: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """VGGT 2-D RoPE on the q and k parts of a fused qkv (T, 3*heads*64) fp16 tensor.

    positions int32 (T, 2) = (y, x) (0 = special token, unrotated), tables fp32 (P, 16)
    from ``rope2d_tables``.  Returns out (T, 2, heads, 64) (rotated q, k); pass
    ``out=qkv`` to rotate in place.
    """
    what = "rope2d"
    if qkv.dtype != torch.float16 or qkv.shape[-1] != 3 * heads * 64:
        _fail(f"{what}: qkv must be float16 (T, 3*heads*64)")
    T = qkv.numel() // qkv.shape[-1]
    if positions.dtype != torch.int32 or positions.numel() != 2 * T:
        _fail(f"{what}: positions must be int32 (T, 2)")
    _check_rope_tables(cos_table, sin_table, what)
    dev = _on_gpu(qkv, positions, cos_table, sin_table, out, what=what)
    if not qkv.is_contiguous():
        _fail(f"{what}: qkv must be contiguous")
    if out is None:
        out = torch.empty(T, 2, heads, 64, dtype=qkv.dtype, device=dev)
        dst_tok, dst_part = 2 * heads * 64, heads * 64
    elif out.data_ptr() == qkv.data_ptr():
        dst_tok, dst_part = 3 * heads * 64, heads * 64
    else:
        dst_tok, dst_part = out.stride(0), heads * 64
    pos = _contig(positions)
    with _device(dev):
        _lib.call("qv_rope2d", _ptr(qkv), _ptr(out), _ptr(pos), _ptr(cos_table), _ptr(sin_table),
                  cos_table.shape[0], T, heads, 3 * heads * 64, dst_tok, dst_part, _stream(dev))
    return out


def rope2d_tables(max_position: int, base: float = 100.0, device=None):
    """fp32 cos/sin tables (P, 16) for VGGT's 2-D RoPE: angle = p * base**(-i/16),
    i = 0..15, evaluated in float64 and rounded once."""
    import numpy as np
    p = np.arange(max_position, dtype=np.float64)[:, None]
    inv = base ** (-np.arange(16, dtype=np.float64) / 16.0)
    ang = p * inv[None, :].astype(np.float32).astype(np.float64)
    c = torch.from_numpy(np.cos(ang).astype(np.float32))
    s = torch.from_numpy(np.sin(ang).astype(np.float32))
    return (c.to(device), s.to(device)) if device is not None else (c, s)


# ------------------------------------------------------------- attention
def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_len: int, scale: float = 0.125,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """Flash attention over sequences of ``seq_len`` tokens (no mask).

    q, k, v: (T, H, 64) fp16 views with head stride 64 and unit dim stride (any
    token stride, e.g. ``qkv.view(T, 3, H, 64)[:, i]``); T = B * seq_len.
    Returns out (T, H, 64) contiguous.  VGGT frame attention: seq_len = 1374
    (one frame per sequence); global attention: seq_len = T.
    """
    what = "attention"
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.float16 or t.dim() != 3 or t.shape[-1] != 64:
            _fail(f"{what}: {name} must be float16 (T, H, 64)")
        if t.stride(-1) != 1 or t.stride(-2) != 64:
            _fail(f"{what}: {name} must have unit dim stride and head stride 64")
    T, H, _ = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        _fail(f"{what}: q, k, v shapes differ")
    if seq_len <= 0 or T % seq_len:
        _fail(f"{what}: T={T} is not a multiple of seq_len={seq_len}")
    dev = _on_gpu(q, k, v, out, what=what)
    if out is None:
        out = torch.empty(T, H, 64, dtype=torch.float16, device=dev)
    elif out.dtype != torch.float16 or out.shape != (T, H, 64) or out.stride(-1) != 1 or out.stride(-2) != 64:
        _fail(f"{what}: out must be float16 (T, H, 64) with head stride 64")
    with _device(dev):
        _lib.call("qv_attention_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(out), T // seq_len, seq_len, H, 64,
                  q.stride(0), k.stride(0), v.stride(0), out.stride(0), C.c_float(scale), _stream(dev))
    return out


def qknorm_rope2d(qkv: torch.Tensor, positions: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                  heads: int, q_gamma: torch.Tensor, q_beta: torch.Tensor, k_gamma: torch.Tensor,
                  k_beta: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """In place on qkv (T, 3*heads*64) fp16: per-head LayerNorm of q and k, then
    VGGT 2-D RoPE (see ``rope2d``).  Returns qkv."""
    what = "qknorm_rope2d"
    if qkv.dtype != torch.float16 or qkv.shape[-1] != 3 * heads * 64 or not qkv.is_contiguous():
        _fail(f"{what}: qkv must be contiguous float16 (T, 3*heads*64)")
    T = qkv.numel() // qkv.shape[-1]
    for name, t in (("q_gamma", q_gamma), ("q_beta", q_beta), ("k_gamma", k_gamma), ("k_beta", k_beta)):
        if t.dtype != torch.float16 or t.numel() != 64:
            _fail(f"{what}: {name} must be float16 (64,)")
    if positions.dtype != torch.int32 or positions.numel() != 2 * T:
        _fail(f"{what}: positions must be int32 (T, 2)")
    _check_rope_tables(cos_table, sin_table, what)
    dev = _on_gpu(qkv, positions, cos_table, sin_table, q_gamma, q_beta, k_gamma, k_beta, what=what)
    pos = _contig(positions)
    qg, qb, kg, kb = _contig(q_gamma), _contig(q_beta), _contig(k_gamma), _contig(k_beta)
    with _device(dev):
        _lib.call("qv_qknorm_rope2d", _ptr(qkv), _ptr(pos), _ptr(cos_table), _ptr(sin_table),
                  cos_table.shape[0], _ptr(qg), _ptr(qb), _ptr(kg), _ptr(kb), C.c_float(eps), T, heads,
                  3 * heads * 64, _stream(dev))
    return qkv
