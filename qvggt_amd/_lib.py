"""ctypes binding of libqvggt_hip.so (the C ABI in include/qvggt_hip.h).

The library is loaded from ``qvggt_amd/lib/`` (built in-tree by
``python -m qvggt_amd.build``).  There is no fallback: if the library is
missing or a symbol is absent, every op raises.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libqvggt_hip.so"

QV_OK = 0
QV_F16 = 0
QV_BF16 = 1
QV_EPI_NONE = 0
QV_EPI_BIAS = 1
QV_EPI_BIAS_GELU = 2
QV_EPI_GELU = 3

_vp = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int
_f32 = C.c_float

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "qv_last_error": [],
    "qv_version": [],
    "qv_w4a16_gemm": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp],
    "qv_w4a16_gemv": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp],
    "qv_w4a16_dequant": [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "qv_w4a16_pack": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp],
    "qv_w4a16_gemm_residual": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    "qv_w4a16_plan": [_i64, _i64, _i64, _i32, _vp],
    "qv_w4a16_gemm_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp],
    "qv_w4a16_gemm_qkrope": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64,
                             _vp, _vp, _vp, _vp, _f32, _i64, _vp],
    "qv_w8a8_gemm": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "qv_w8a8_gemm_residual": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "qv_w8a8_gemm_i32": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "qv_w8a8_packed_bytes": [_i64, _i64],
    "qv_w8a8_pack_weight": [_vp, _vp, _i64, _i64, _vp],
    "qv_w8a8_gemm_packed": [_vp] * 7 + [_i64] * 3 + [_vp],
    "qv_quant_per_token": [_vp, _i32, _vp, _vp, _i64, _i64, _vp],
    "qv_layernorm_quant": [_vp, _i32, _vp, _vp, _vp, _vp, _f32, _i32, _i64, _i64, _vp],
    "qv_gelu_quant": [_vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "qv_rmsnorm": [_vp, _vp, _vp, _f32, _i64, _i64, _i32, _vp],
    "qv_layernorm": [_vp, _vp, _vp, _vp, _f32, _i64, _i64, _i32, _vp],
    "qv_rope_with_pos": [_vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp],
    "qv_rope2d": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp],
    "qv_qknorm_rope2d": [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _f32, _i64, _i64, _i64, _vp],
    "qv_attention_fwd": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _vp],
}
_RESTYPES = {"qv_last_error": C.c_char_p, "qv_version": C.c_char_p, "qv_w8a8_packed_bytes": C.c_int64}

_lock = threading.Lock()
_lib = None


class NativeLibraryError(RuntimeError):
    pass


def load(path: Path | str | None = None):
    """Load (once) and return the ctypes handle; raise if unavailable."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise NativeLibraryError(
                f"{p} not found: build it with `python -m qvggt_amd.build` "
                "(no CPU fallback exists for these ops)")
        lib = C.CDLL(str(p))
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError -> missing export
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, C.c_int)
        if path is None:
            _lib = lib
        return lib


_fns: dict = {}


def call(name: str, *args) -> None:
    """Call an entry point; raise RuntimeError with the library's message on failure."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != QV_OK:
        msg = load().qv_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")
