"""Config 5 on the GPU: the full VGGT-1B aggregator (DINOv2-L/14-reg patch
embed, 24 frame + 24 global AA blocks, LayerScale 0.01) on S = 32 frames of
518 x 518 U[0, 1] images, with W4A16 g128 and with W8A8 AA linears -- the
forward the reference runs at qvggt/inference/cli.py:99 ->
FP16InferenceWrapper.forward (loader.py:68-76).

The whole-model reference is the composition of block references, so the
forward is checked block by block, teacher-forced: the input and output of
frame / global blocks 0, 11 and 23 are captured during the real forward and
each block is compared with oracle/aggregator.py:aa_block_delta from its
captured input (sampled rows; a frame block's keys are its own frame, a
global block's all 43968 tokens):

* in the forward itself (LayerScale 0.01): the fp16 block output against
  x_in + delta_ref.  The residual stream is fp16, so besides the tolerance on
  the update (tol * max|delta_ref|) each element may carry the two roundings
  of the stream (after the attention and after the MLP update), 1.5 fp16 ulp
  of its magnitude;
* the same block re-run on the captured input with LayerScale 1, so the
  attention and MLP outputs dominate: max|d - d_ref| / max|d_ref| <= tol.

tol = 1e-2 for W4A16 (fp32-dequantised reference).  W8A8 blocks are checked
against the reference's W8A8 op chain (each quantiser fed the fp16 tensor the
previous op stores) in stages: the attention output (its one op that is not
bit-exact) within 1e-2, the rest of the chain teacher-forced from the GPU's
own fp16 attention output bit for bit, and end to end within tol = 2e-2 (an
fp16 attention value one rounding off can move an int8 code of invoke_quant
by one step).  The W4A16 blocks' attention output is checked within 1e-2
too.  Size-independent invariants at full size: every output finite,
a re-run bitwise identical, and permuting frames 1..31 (frame 0 keeps token
set 0) permutes the outputs -- within 1e-2 of max|out| rather than bit for bit,
because global attention then sums its 43968 keys in another order.
"""
import numpy as np
import pytest
import torch

from oracle import aggregator as OA
from oracle import rope as R

pytestmark = pytest.mark.gpu

S = 32
CHECK_BLOCKS = (0, 11, 23)


def _params(mod):
    """The block's tensors as stored (int16 / int8 weights, fp16 tables and
    norms), named like the module tree, as oracle/aggregator.py reads them."""
    return {k: v.detach().cpu().numpy() for k, v in mod.state_dict().items()}


def _ulp16(a):
    return np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)


@pytest.fixture(scope="module")
def images(gpu):
    from qvggt_amd import aggregator as AG
    g = torch.Generator().manual_seed(2024)
    return torch.rand(S, 3, AG.IMG, AG.IMG, generator=g).half().to(gpu)


def _capture(agg):
    """Hooks that keep the input and output of the checked blocks."""
    cap, handles = {}, []
    for kind, blocks in (("frame", agg.frame_blocks), ("global", agg.global_blocks)):
        for i in CHECK_BLOCKS:
            key = (kind, i)
            handles.append(blocks[i].register_forward_pre_hook(
                lambda m, a, key=key: cap.__setitem__(key, [a[0].clone()])))
            handles.append(blocks[i].register_forward_hook(
                lambda m, a, out, key=key: cap[key].append(out.clone())))
    return cap, handles


@pytest.mark.parametrize("w8a8", [False, True], ids=["w4a16", "w8a8"])
def test_config5_full_aggregator_s32(gpu, images, w8a8):
    from qvggt_amd import aggregator as AG
    from qvggt_amd import awq_inference_engine as E
    tol = 2e-2 if w8a8 else 1e-2
    agg = AG.Aggregator.random(w8a8=w8a8, seed=5, device=gpu)
    assert len(agg.frame_blocks) == len(agg.global_blocks) == 24 and len(agg.patch_embed.blocks) == 24
    M = S * AG.TOKENS
    cap, handles = _capture(agg)
    out, layers = agg(images)
    torch.cuda.synchronize()
    print(f"[config5] {'w8a8' if w8a8 else 'w4a16'}: S = {S} forward done", flush=True)
    for h in handles:
        h.remove()
    assert out.shape == (M, AG.DIM) and torch.isfinite(out.float()).all()
    assert all(torch.isfinite(v.float()).all() for v in layers.values())

    # re-run: bitwise identical
    out2, _ = agg(images)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "re-run of the S = 32 forward is not bitwise identical"

    # teacher-forced block parity
    pos_all = AG.vggt_positions(S, gpu)
    pos_np = pos_all.cpu().numpy()
    tables = E.rope2d_tables(AG.GRID + 1, device=gpu)
    c, s_ = R.rope2d_tables(AG.GRID + 1)
    ws = agg._workspace(M, gpu)
    rng = np.random.default_rng(7)
    report = []
    for (kind, i), (x_in, x_out) in sorted(cap.items()):
        blk = (agg.frame_blocks if kind == "frame" else agg.global_blocks)[i]
        xi = x_in.float().cpu().numpy()
        xo = x_out.float().cpu().numpy()
        if kind == "frame":
            f = int(rng.integers(0, S))
            lo = f * AG.TOKENS
            sl = slice(lo, lo + AG.TOKENS)
            rows = np.sort(rng.choice(AG.TOKENS, 48, replace=False))
            xk, seq, posk, grow = xi[sl], AG.TOKENS, pos_np[sl], lo + rows
        else:
            rows = np.sort(rng.choice(M, 24, replace=False))
            xk, seq, posk, grow = xi, M, pos_np, rows
        # (1) in the forward, LayerScale 0.01 (the attention half is shared with (2))
        prm = _params(blk)
        att = {}
        o_ref = OA.aa_block_attention(xk, prm, seq, posk, c, s_, rows, w8a8=w8a8, eps=blk.eps, att_out=att)
        d_ref = OA.aa_block_finish(xk[rows], o_ref, prm, w8a8=w8a8, eps=blk.eps)
        ref_out = xi[grow].astype(np.float64) + d_ref
        slack = 1.5 * _ulp16(np.maximum(np.abs(xi[grow]), np.abs(ref_out))) + tol * np.abs(d_ref).max()
        excess = np.abs(xo[grow] - ref_out) - slack
        assert (excess <= 0).all(), f"{kind} block {i}: in-forward output off by {excess.max():.3e} past the bound"
        lit = np.abs(xo[grow] - ref_out).max() / np.abs(ref_out).max()
        assert lit <= 1e-2, f"{kind} block {i}: fp16 output rel err {lit:.3e}"
        # (2) re-run with LayerScale 1 on the captured input
        g1, g2 = blk.ls1.gamma.clone(), blk.ls2.gamma.clone()
        try:
            blk.ls1.gamma.fill_(1.0)
            blk.ls2.gamma.fill_(1.0)
            xr = x_in.clone()
            blk(xr, seq if kind == "frame" else M, pos_all, tables, ws)
            torch.cuda.synchronize()
        finally:
            blk.ls1.gamma.copy_(g1)
            blk.ls2.gamma.copy_(g2)
        d_got = xr.float().cpu().numpy()[grow].astype(np.float64) - xi[grow].astype(np.float64)   # exact
        att_gpu = ws["att"].cpu().numpy()[grow]      # this block's attention output (fp16)
        err_att = np.abs(att_gpu.astype(np.float64) - att["att"]).max() / np.abs(att["att"]).max()
        one = np.ones(AG.DIM)
        d1 = OA.aa_block_finish(xk[rows], o_ref, prm, w8a8=w8a8, eps=blk.eps, ls1=one, ls2=one)
        err = np.abs(d_got - d1).max() / np.abs(d1).max()
        line = f"{kind}{i}: attention {err_att:.2e}, delta {err:.2e}"
        if w8a8:
            tf = OA.w8a8_block_from_attention(xk[rows], att_gpu, prm, eps=blk.eps, ls1=one, ls2=one)
            err_tf = np.abs(d_got - tf).max() / np.abs(tf).max()
            line += f", from the GPU attention on {err_tf:.2e}"
            assert np.array_equal(d_got, tf), line    # bit-exact ops from here on
        report.append(line)
        print(f"[config5] {'w8a8' if w8a8 else 'w4a16'} {kind} block {i}: fp16 out rel err {lit:.2e}, "
              f"LayerScale 1: {line}", flush=True)
        assert err_att <= 1e-2, line
        assert np.isfinite(d_got).all() and err <= tol, f"{kind} block {i} (LayerScale 1): {line}"
    print("[config5]", "w8a8" if w8a8 else "w4a16", "block errors:", ", ".join(report), flush=True)

    # frame permutation (frame 0 fixed)
    perm = np.concatenate([[0], 1 + np.random.default_rng(3).permutation(S - 1)])
    outp, _ = agg(images[torch.from_numpy(perm).to(gpu)])
    torch.cuda.synchronize()
    want = out.view(S, AG.TOKENS, AG.DIM)[torch.from_numpy(perm).to(gpu)]
    diff = (outp.view(S, AG.TOKENS, AG.DIM).float() - want.float()).abs().max().item()
    assert diff <= 1e-2 * want.float().abs().max().item(), f"frame permutation: max diff {diff}"


def test_config5_dino_patch_embed_s32(gpu, images):
    """The fp16 DINOv2-L/14-reg patch embed inside the S = 32 forward, checked
    teacher-forced against oracle/aggregator.py's float64 restatement:

    * token assembly: the first block's input (patch projection of the
      normalised images + position embedding, cls + position 0, the four
      registers) against dino_tokens(dino_patch_project(...)) on three frames;
    * blocks 0 and 23 re-run on their captured input with LayerScale 1 (at the
      model's 1e-5 the update is below the fp16 stream's rounding): the
      residual update of 48 rows of one frame against dino_block_delta;
    * the final LayerNorm (specials dropped) from the last block's captured
      output against dino_final;
    * the aggregator's own token assembly (camera and register token sets,
      set 0 for frame 0 only) from the patch embed's output: bit for bit.
    Tolerance 1e-2 of the reference's max |value| (fp16 linears on
    hipBLASLt, fp16 storage between ops)."""
    from qvggt_amd import aggregator as AG
    agg = AG.Aggregator.random(w8a8=False, seed=5, device=gpu)
    pe = agg.patch_embed
    cap = {}
    hooks = [pe.register_forward_pre_hook(lambda m, a: cap.__setitem__("img", a[0].clone())),
             pe.register_forward_hook(lambda m, a, out: cap.__setitem__("pe_out", out.clone())),
             agg.frame_blocks[0].register_forward_pre_hook(lambda m, a: cap.__setitem__("agg_in", a[0].clone()))]
    for i in (0, len(pe.blocks) - 1):
        hooks.append(pe.blocks[i].register_forward_pre_hook(lambda m, a, i=i: cap.__setitem__(("in", i), a[0].clone())))
        hooks.append(pe.blocks[i].register_forward_hook(lambda m, a, out, i=i: cap.__setitem__(("out", i), out.clone())))
    agg(images)
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    T = AG.TOKENS
    prm = {k: v.detach().float().cpu().numpy() for k, v in pe.state_dict().items()}
    rng = np.random.default_rng(11)
    errs = []

    # token assembly from the normalised images
    frames = [0, 17, 31]
    img = cap["img"].float().cpu().numpy()[frames]
    proj = OA.dino_patch_project(img, prm["patch_embed.proj.weight"], prm["patch_embed.proj.bias"])
    tok_ref = OA.dino_tokens(proj, prm["cls_token"], prm["register_tokens"], prm["pos_embed"])
    tok = cap[("in", 0)].float().cpu().numpy().reshape(S, T, AG.DIM)[frames]
    e = np.abs(tok - tok_ref).max() / np.abs(tok_ref).max()
    errs.append(f"tokens {e:.2e}")
    assert e <= 1e-2, errs

    # blocks 0 and 23, LayerScale 1, on their captured input
    ws = agg._workspace(S * T, gpu)
    for i in (0, len(pe.blocks) - 1):
        blk = pe.blocks[i]
        xi = cap[("in", i)]
        f = int(rng.integers(0, S))
        rows = np.sort(rng.choice(T, 48, replace=False))
        g1, g2 = blk.ls1.gamma.clone(), blk.ls2.gamma.clone()
        try:
            blk.ls1.gamma.fill_(1.0)
            blk.ls2.gamma.fill_(1.0)
            xr = xi.clone()
            blk(xr, ws)
            torch.cuda.synchronize()
        finally:
            blk.ls1.gamma.copy_(g1)
            blk.ls2.gamma.copy_(g2)
        xf = xi.float().cpu().numpy()[f * T:(f + 1) * T]
        got = xr.float().cpu().numpy()[f * T + rows] - xf[rows]
        bp = {k[len(f"blocks.{i}."):]: v for k, v in prm.items() if k.startswith(f"blocks.{i}.")}
        one = np.ones(AG.DIM)
        ref = OA.dino_block_delta(xf, bp, rows, T, eps=blk.eps, ls1=one, ls2=one)
        e = np.abs(got - ref).max() / np.abs(ref).max()
        errs.append(f"block {i} {e:.2e}")
        assert np.isfinite(got).all() and e <= 1e-2, errs

    # final norm, teacher-forced from the last block's output
    last = cap[("out", len(pe.blocks) - 1)].float().cpu().numpy().reshape(S, T, AG.DIM)[frames]
    fin_ref = OA.dino_final(last.reshape(-1, AG.DIM), prm["norm.weight"], prm["norm.bias"], len(frames),
                            eps=pe.eps)
    fin = cap["pe_out"].float().cpu().numpy()[frames]
    e = np.abs(fin - fin_ref).max() / np.abs(fin_ref).max()
    errs.append(f"final norm {e:.2e}")
    assert e <= 1e-2, errs

    # the aggregator's token assembly, bit for bit
    want = OA.aggregator_tokens(cap["pe_out"].float().cpu().numpy(), agg.camera_token.float().cpu().numpy(),
                                agg.register_token.float().cpu().numpy()).astype(np.float16)
    assert np.array_equal(cap["agg_in"].cpu().numpy(), want)
    print("[config5] DINOv2 patch embed:", ", ".join(errs), flush=True)
