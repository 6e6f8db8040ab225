"""VGGT camera head with a W4A16 trunk on the GPU against the float64 oracle
(oracle/camera_head.py).

S pose tokens make the trunk linears run at M = S: S = 1 and 4 go through
the GEMV entry, S = 24 through the GEMM entry, and all three run on the
skinny-M MFMA kernel.  Every iteration's activated pose encoding
is compared; tolerance max|out - ref| / max|ref| <= 1e-2 (fp16 residual stream
and activations vs the float64 reference with the same dequantised weights).
"""
import numpy as np
import pytest
import torch

from oracle import camera_head as OC

pytestmark = pytest.mark.gpu


def _params(mod):
    return {k: v.detach().cpu().numpy() for k, v in mod.state_dict().items()}


@pytest.mark.parametrize("S", [1, 4, 24])
def test_camera_head_w4_matches_oracle(gpu, S):
    from qvggt_amd.camera_head import CameraHead
    head = CameraHead.random(seed=S, device=gpu)
    t = np.random.default_rng(S).standard_normal((S, OC.DIM)).astype(np.float16)
    outs = head(torch.from_numpy(t).to(gpu))
    torch.cuda.synchronize()
    p = _params(head)
    ref = OC.camera_head(t.astype(np.float64), p)
    assert len(outs) == len(ref) == 4
    for i, (o, r) in enumerate(zip(outs, ref)):
        got = o.cpu().numpy()
        err = np.abs(got - r).max() / np.abs(r).max()
        assert got.shape == (S, 9) and np.isfinite(got).all() and err <= 1e-2, (i, err)


def test_camera_head_takes_camera_tokens_of_the_aggregator_output(gpu):
    """The head reads the camera token (token 0) of each frame of the last
    [frame | global] aggregator layer; frames stay independent of their order."""
    from qvggt_amd.camera_head import CameraHead
    head = CameraHead.random(seed=5, device=gpu)
    layer = torch.randn(3, 20, OC.DIM, device=gpu).half()
    a = head(CameraHead.pose_tokens(layer))[-1]
    b = head(CameraHead.pose_tokens(layer[[2, 0, 1]]))[-1]
    torch.cuda.synchronize()
    assert (a[[2, 0, 1]] - b).abs().max().item() <= 1e-2 * a.abs().max().item()


def test_graphed_camera_head_replays_match_eager(gpu):
    """HIP-graph replay of the head: three replays on different inputs, with
    eager work and synchronisation between them, each equal to the eager
    forward on the same input; a repeated input replays bit for bit."""
    from qvggt_amd.camera_head import CameraHead, GraphedCameraHead
    head = CameraHead.random(seed=9, device=gpu)
    S = 8
    g = GraphedCameraHead(head, S)
    gen = torch.Generator(device=gpu).manual_seed(0)
    inputs = [torch.randn(S, OC.DIM, generator=gen, device=gpu).half() for _ in range(3)]
    first = None
    for i, t in enumerate(inputs):
        want = [o.clone() for o in head(t)]
        torch.cuda.synchronize()
        got = [o.clone() for o in g(t)]
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert (a - b).abs().max().item() <= 1e-3 * b.abs().max().item(), i
        if i == 0:
            first = got
    again = g(inputs[0])
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(again, first))
    with pytest.raises(ValueError):
        g(inputs[0][:4])
