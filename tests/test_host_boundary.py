"""CPU tests of the boundary: C-ABI exports, host-side validation and the
``WQLinear`` buffer contract.  No GPU compute is called here."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import awq as O
from qvggt_amd import _lib
from qvggt_amd import awq_inference_engine as E
from qvggt_amd.awq import WQLinear, calculate_zeros_width, pack_intweight

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(qv_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} missing: run `python -m qvggt_amd.build` first")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    declared = _declared_symbols()
    assert declared, "no qv_* declarations found in include/"
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # every declared symbol has a ctypes signature, and vice versa
    assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)
    _lib.load()
    assert b"gfx950" in _lib.load().qv_version()


def test_engine_exports_reference_op_names():
    # pybind.cpp:18-36
    ref_ops = ["layernorm_forward_cuda", "gemm_forward_cuda", "gemv_forward_cuda",
               "gemm_forward_cuda_new", "gemv_forward_cuda_new", "rotary_embedding_neox",
               "single_query_attention", "fused_rope_with_pos_forward_func",
               "w8a8_gemm_forward_cuda", "w8a8_gemm_fuse_bias_forward_cuda", "invoke_quant",
               "rms_norm_general", "silu_and_mul", "gelu_and_quant"]
    for name in ref_ops:
        assert callable(getattr(E, name)), name


def test_gemv_errors_match_reference_messages():
    x = torch.zeros(8, 256, dtype=torch.float16)
    qw = torch.zeros(64 // 4, 256, dtype=torch.int16)
    sc = torch.zeros(8, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Unsupported batch size"):
        E.gemv_forward_cuda_new(x, qw, sc, sc, 8, 64, 256, 128)
    with pytest.raises(RuntimeError, match="Unsupported group size"):
        E.gemv_forward_cuda_new(x[:2], qw, sc, sc, 2, 64, 256, 64)


def test_host_checks_reject_bad_shapes_before_any_launch():
    """Shapes that would make a kernel read or write out of bounds are refused
    on the host: an activation whose last dim is not k (the GEMV sizes its
    output from it), a caller-provided GEMM output of the wrong shape, dtype,
    layout or alignment, and RoPE tables narrower than (P, 16)."""
    m, n, k = 2, 64, 256
    qw = torch.zeros(n // 4, k, dtype=torch.int16)
    sc = torch.zeros(8, n, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="in_feats must be"):
        E.gemv_forward_cuda_new(torch.zeros(1, m * k, dtype=torch.float16), qw, sc, sc, m, n, k, 128)
    x = torch.zeros(m, k, dtype=torch.float16)
    for bad, msg in ((torch.zeros(m, n + 16, dtype=torch.float16), "out must be a contiguous"),
                     (torch.zeros(m, n, dtype=torch.float32), "out must be a torch.float16"),
                     (torch.zeros(n, m, dtype=torch.float16).t(), "out must be a contiguous"),
                     (torch.zeros(m * n + 4, dtype=torch.float16)[4:].view(m, n), "16-byte aligned")):
        with pytest.raises(RuntimeError, match=msg):
            E.w4a16_linear(x, qw, sc, sc, out=bad)
    T, H = 5, 16
    qkv = torch.zeros(T, 3 * H * 64, dtype=torch.float16)
    pos = torch.zeros(T, 2, dtype=torch.int32)
    g = torch.ones(64, dtype=torch.float16)
    for c, s_ in ((torch.zeros(38, 8), torch.zeros(38, 8)), (torch.zeros(38, 16, dtype=torch.float64),) * 2,
                  (torch.zeros(38, 16), torch.zeros(30, 16)), (torch.zeros(16, 38).t(), torch.zeros(38, 16))):
        with pytest.raises(RuntimeError, match="tables|differ"):
            E.qknorm_rope2d(qkv, pos, c, s_, H, g, g, g, g)
        with pytest.raises(RuntimeError, match="tables|differ"):
            E.rope2d(qkv, pos, c, s_, H)
    # a packed W8A8 weight whose size does not match (N, K)
    a8 = torch.zeros(m, 128, dtype=torch.int8)
    s8 = torch.zeros(m, dtype=torch.float16)
    ws = torch.zeros(n, dtype=torch.float16)
    o8 = torch.zeros(m, n, dtype=torch.float16)
    assert E.w8a8_packed_bytes(n, 128) == 64 * 128 and E.w8a8_packed_bytes(48, 128) == 64 * 128
    for bad in (torch.zeros(n * 128 - 16, dtype=torch.int8), torch.zeros(n, 128, dtype=torch.int8)):
        with pytest.raises(RuntimeError, match="packed weight must be"):
            E.w8a8_gemm_packed(a8, bad, n, ws, s8, o8)


def test_ops_refuse_cpu_tensors_and_bad_dtypes():
    x = torch.zeros(16, 256, dtype=torch.float16)
    qw = torch.zeros(16, 256, dtype=torch.int16)
    sc = torch.zeros(8, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU only"):
        E.gemm_forward_cuda_new(x, qw, sc, sc)
    with pytest.raises(RuntimeError):
        E.gemm_forward_cuda_new(x.float(), qw, sc, sc)


def test_legacy_and_llm_ops_raise_not_implemented():
    for name in ("gemm_forward_cuda", "gemv_forward_cuda", "single_query_attention"):
        with pytest.raises(NotImplementedError):
            getattr(E, name)()


def test_missing_library_raises(tmp_path):
    with pytest.raises(_lib.NativeLibraryError):
        _lib.load(tmp_path / "nope.so")


# ------------------------------------------------------------ WQLinear
@pytest.mark.parametrize("K,N", [(1024, 3072), (1024, 4096), (4096, 1024), (2048, 8192)])
def test_wqlinear_buffers_match_reference_shapes(K, N):
    m = WQLinear(4, 128, K, N, True, "cpu")
    rows = calculate_zeros_width(K, 128) * 8  # qmodule.py:169-189
    assert m.qweight.shape == (N // 4, K) and m.qweight.dtype == torch.int16
    assert m.scales.shape == (rows, N) and m.scales.dtype == torch.float16
    assert m.scaled_zeros.shape == (rows, N) and m.scaled_zeros.dtype == torch.float16
    assert m.bias.shape == (N,)
    assert set(dict(m.named_buffers())) == {"qweight", "scales", "scaled_zeros", "bias"}
    assert "w_bit=4" in m.extra_repr()


def test_wqlinear_rejects_other_bits():
    with pytest.raises(NotImplementedError):
        WQLinear(8, 128, 256, 64, False, "cpu")


@pytest.mark.parametrize("N,K", [(4, 64), (64, 256), (3072, 1024)])
def test_product_pack_matches_oracle(N, K):
    U = np.random.default_rng(N + K).integers(0, 16, size=(N, K))
    got = pack_intweight(torch.tensor(U), 4, 64).numpy()
    assert np.array_equal(got, O.pack_intweight(U))


def test_from_linear_recovers_integer_weights():
    N, K = 64, 256
    rng = np.random.default_rng(0)
    U = rng.integers(0, 16, size=(N, K))
    z = rng.integers(0, 16, size=(N, K // 128))
    s = (rng.integers(1, 64, size=(N, K // 128)) / 1024).astype(np.float16)  # exact in fp16
    W = (s.astype(np.float32).repeat(128, 1) * (U - z.repeat(128, 1))).astype(np.float16)
    lin = torch.nn.Linear(K, N, bias=True).half()
    lin.weight.data = torch.tensor(W)
    lin.bias.data = torch.arange(N, dtype=torch.float16)
    q = WQLinear.from_linear(lin, 4, 128, scales=torch.tensor(s), zeros=torch.tensor(z, dtype=torch.float16))
    assert np.array_equal(O.unpack_intweight(q.qweight.numpy(), N, K), U)
    sc, sz = O.build_tables(s, z, K)
    assert np.array_equal(q.scales.numpy(), sc)
    assert np.array_equal(q.scaled_zeros.numpy(), sz)
    assert torch.equal(q.bias, lin.bias.data)
    # init_only returns zero buffers of the right shapes (loader.py:450)
    e = WQLinear.from_linear(lin, 4, 128, init_only=True)
    assert e.qweight.shape == q.qweight.shape and not e.qweight.any()


def test_patch_projection_equals_the_convolution():
    """DinoPatchEmbed.project (patch unfold + one GEMM) is the 14x14 stride-14
    nn.Conv2d it replaces, on the same parameters (float64 on the CPU)."""
    from qvggt_amd import aggregator as AG
    torch.manual_seed(0)
    pe = AG.DinoPatchEmbed(torch.device("cpu"), depth=0).double()
    with torch.no_grad():
        pe.patch_embed.proj.weight.normal_()
        pe.patch_embed.proj.bias.normal_()
    img = torch.rand(2, 3, AG.IMG, AG.IMG, dtype=torch.float64)
    with torch.no_grad():
        ref = pe.patch_embed.proj(img).flatten(2).transpose(1, 2)
    got = pe.project(img)
    assert got.shape == (2, AG.GRID * AG.GRID, AG.DIM)
    assert torch.allclose(got, ref, rtol=1e-12, atol=1e-10)


def test_tanh_table_lookup_on_every_fp16_pattern():
    """The GELU+quant kernel's tanh step, restated on all 65536 fp16 patterns
    w: m = w & 0x7FFF, k = min(max(m - base, 0), last), t = min(m, table[k])
    | (w & 0x8000), against fp16(fp32(tanh)) of the float64 value (NaN
    patterns give +-1.0 by design: the GELU multiplies by its NaN input)."""
    from qvggt_amd import build

    base, last, table = build.tanh_f16_table()
    assert table.dtype == np.uint16 and len(table) % 8 == 0 and table[last] == 0x3C00
    w = np.arange(0x10000, dtype=np.uint32)
    m = (w & 0x7FFF).astype(np.int64)
    k = np.clip(m - base, 0, last)
    got = (np.minimum(m, table[k].astype(np.int64)) | (w & 0x8000)).astype(np.uint16)
    with np.errstate(invalid="ignore"):
        want = np.tanh(w.astype(np.uint16).view(np.float16).astype(np.float64)).astype(np.float32)
    want = want.astype(np.float16).view(np.uint16)
    nan = m > 0x7C00
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7FFF) == 0x3C00)


@pytest.mark.parametrize("M,N,K,epi,kind,tile,tile2", [
    (1, 3072, 1024, 1, "skinny", 0, 0),            # M <= 64: the skinny kernel
    (64, 1024, 4096, 1, "skinny", 0, 0),
    (1374, 3072, 1024, 1, "stream_k128", 96, 0),   # config 1: one round, 128-k stages
    (1000, 3072, 1024, 1, "stream_k128", 64, 0),
    (1374, 1024, 4096, 1, "stream_ksplit", 32, 0), # one round, K >= 2048: K split in the workgroup
    (2748, 1024, 4096, 1, "stream_ksplit", 64, 0),
    (1374, 1024, 1024, 1, "stream_ksplit", 32, 0), # one round of 32-row tiles
    (10992, 4096, 1024, 2, "stream", 128, 96),     # fc1 of the benchmark: two tile heights
    (10992, 1024, 4096, 1, "stream", 128, 64),     # fc2: one 128-row tile per CU, then 64-row tiles
])
def test_w4a16_plan_rules(M, N, K, epi, kind, tile, tile2):
    """The launch plan qv_w4a16_gemm picks (host-side planning, no device
    work): the kernel form per shape and the tile heights."""
    p = E.w4a16_plan(M, N, K, epi)
    assert p["kernel"] == kind and p["tile"] == tile and p["tile2"] == tile2, p
    if kind.startswith("stream"):
        assert 0 < p["rows"] <= M and (p["tile2"] or p["rows"] == M)


def test_w4a16_plan_rejects_bad_shapes():
    for args in [(0, 64, 128, 0), (8, 64, 100, 0), (8, 60, 128, 0), (8, 64, 128, 9)]:
        with pytest.raises(RuntimeError):
            E.w4a16_plan(*args)
