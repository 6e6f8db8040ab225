"""GPU quantise + pack (``w4a16_pack`` / ``WQLinear.from_linear`` on the GPU)
against the oracle (oracle/awq.py: quantize_intweight, pack_intweight,
build_tables): bit-exact for fp16 and bf16, group sizes 128 / 64 / 32 / -1,
and identical to the torch-op ``from_linear`` on the CPU."""
import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import awq as O

pytestmark = pytest.mark.gpu


def _minmax(W, gs):
    N, K = W.shape
    g = K if gs == -1 else gs
    Wg = W.float().view(N, K // g, g)
    lo, hi = Wg.amin(-1).clamp(max=0), Wg.amax(-1).clamp(min=0)
    # s over 14 steps, z rounded up, both from the 16-bit s: every q stays in
    # 0..15 despite the per-op roundings (the oracle's packer rejects others)
    s = ((hi - lo) / 14).clamp_min(1e-5).to(W.dtype).float()
    z = torch.ceil(-lo / s).clamp(0, 15)
    return s, z


@pytest.mark.parametrize("N,K,gs", [(64, 128, 128), (3072, 1024, 128), (48, 256, 64), (32, 512, 32),
                                    (16, 320, -1), (8, 1152, 128)])
def test_pack_fp16_bit_exact(gpu, N, K, gs):
    from qvggt_amd import awq_inference_engine as E
    g = torch.Generator().manual_seed(N + K)
    W = (0.05 * torch.randn(N, K, generator=g)).half()
    s, z = _minmax(W, gs)
    s, z = s.half(), z.half()
    qw, st, szt = E.w4a16_pack(W.to(gpu), s.to(gpu), z.to(gpu), gs)
    torch.cuda.synchronize()
    q = O.quantize_intweight(W.numpy(), s.numpy(), z.numpy(), gs)
    assert q.min() >= 0 and q.max() <= 15
    assert np.array_equal(qw.cpu().numpy(), O.pack_intweight(q))
    ref_s, ref_sz = O.build_tables(s.numpy(), z.numpy(), K, gs)
    assert np.array_equal(st.cpu().numpy().view(np.uint16), ref_s.view(np.uint16))
    assert np.array_equal(szt.cpu().numpy().view(np.uint16), ref_sz.view(np.uint16))


def test_pack_bf16_bit_exact(gpu):
    from qvggt_amd import awq_inference_engine as E
    N, K, gs = 96, 512, 128
    g = torch.Generator().manual_seed(3)
    W = (0.05 * torch.randn(N, K, generator=g)).bfloat16()
    s, z = _minmax(W, gs)
    s, z = s.bfloat16(), z.bfloat16()
    qw, st, szt = E.w4a16_pack(W.to(gpu), s.to(gpu), z.to(gpu), gs)
    torch.cuda.synchronize()
    q = O.quantize_intweight(W.float().numpy(), s.float().numpy(), z.float().numpy(), gs, dtype="bf16")
    assert np.array_equal(qw.cpu().numpy(), O.pack_intweight(q))
    sb = O.f64_to_bf16_bits(s.float().numpy().astype(np.float64))
    szb = O.f64_to_bf16_bits(-(s.float().numpy().astype(np.float64) * z.float().numpy()))
    rows = O.scale_rows(K, gs)
    ref_s = np.zeros((rows, N), np.uint16)
    ref_sz = np.zeros((rows, N), np.uint16)
    ref_s[: K // gs] = sb.T
    ref_sz[: K // gs] = szb.T
    assert np.array_equal(st.cpu().view(torch.int16).numpy().view(np.uint16), ref_s)
    assert np.array_equal(szt.cpu().view(torch.int16).numpy().view(np.uint16), ref_sz)


def test_from_linear_gpu_equals_cpu(gpu):
    """WQLinear.from_linear: the HIP pass on the GPU stores the same buffers as
    the torch-op recipe on the CPU, and the packed layer reproduces the
    dequantised product."""
    from qvggt_amd.awq.qmodule import WQLinear
    torch.manual_seed(0)
    lin = nn.Linear(1024, 768, dtype=torch.float16)
    lin.weight.data.normal_(0, 0.02)
    s, z = _minmax(lin.weight.data, 128)
    cpu = WQLinear.from_linear(lin, 4, 128, scales=s.half(), zeros=z.half())
    g = WQLinear.from_linear(lin.to(gpu), 4, 128, scales=s.half().to(gpu), zeros=z.half().to(gpu))
    for name in ("qweight", "scales", "scaled_zeros", "bias"):
        assert torch.equal(getattr(g, name).cpu(), getattr(cpu, name)), name
    x = torch.randn(5, 1024, device=gpu).half()
    W = O.dequantize(cpu.qweight.numpy(), cpu.scales.numpy(), cpu.scaled_zeros.numpy(), 768, 1024)
    ref = x.float().cpu().numpy() @ W.astype(np.float32).T + lin.bias.detach().float().cpu().numpy()
    assert O.rel_err(g(x).float().cpu().numpy(), ref) <= 1e-2


def test_pack_rejects_bad_shapes(gpu):
    from qvggt_amd import awq_inference_engine as E
    W = torch.zeros(8, 96, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError):
        E.w4a16_pack(W, torch.ones(8, 1, dtype=torch.float16, device=gpu),
                     torch.zeros(8, 1, dtype=torch.float16, device=gpu), 96)
