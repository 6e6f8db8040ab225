"""Host-side checkpoint loading (qvggt_amd/loader.py): the reference
loader's layout inference and layer selection (qvggt/inference/loader.py),
the WQLinear swap, the weight merge, safe file reading, and a full
save -> load round trip of a small quantised aggregator on the CPU."""
import pytest
import torch
import torch.nn as nn

from qvggt_amd import loader as LD
from qvggt_amd.aggregator import Aggregator
from qvggt_amd.awq.qmodule import WQLinear


def test_infer_quantization_layout():
    keys = ["aggregator.frame_blocks.3.attn.qkv.qweight", "aggregator.frame_blocks.0.mlp.fc1.qweight",
            "aggregator.global_blocks.7.attn.proj.qweight", "aggregator.global_blocks.7.attn.proj.scales",
            "camera_head.trunk.0.mlp.fc2.qweight", "aggregator.frame_blocks.5.attn.qkv.weight"]
    lay = LD.infer_quantization_layout({k: None for k in keys})
    assert lay == {"frame_blocks": [0, 3], "global_blocks": [7], "quantize_camera_head": True,
                   "layer_types": ["fc1", "fc2", "proj", "qkv"]}
    assert LD.infer_quantization_layout({"aggregator.camera_token": None}) == {
        "frame_blocks": None, "global_blocks": None, "quantize_camera_head": False, "layer_types": None}


def test_should_quantize_layer_truth_table():
    f = LD.should_quantize_layer
    assert f("aggregator.frame_blocks.2.attn.qkv", "specific_blocks", [2], None, None, False)
    assert not f("aggregator.frame_blocks.3.attn.qkv", "specific_blocks", [2], None, None, False)
    assert not f("aggregator.global_blocks.2.attn.qkv", "specific_blocks", [2], None, None, False)
    assert f("aggregator.global_blocks.9.mlp.fc2", "all", None, None, None, False)
    assert not f("aggregator.global_blocks.9.mlp.fc2", "all", None, None, ["qkv"], False)
    assert not f("aggregator.patch_embed.blocks.0.attn.qkv", "all", None, None, None, False)
    assert not f("camera_head.trunk.0.attn.qkv", "all", None, None, None, False)
    assert f("camera_head.trunk.0.attn.qkv", "all", None, None, None, True)
    assert not f("camera_head.trunk.0.norm1", "all", None, None, None, True)
    assert not f("camera_head.pose_branch.fc1", "all", None, None, None, True)
    assert not f("aggregator.frame_blocks.1.attn.qkv", "none", [1], [1], None, False)


def test_quantize_specified_blocks_swaps_only_the_selection():
    agg = Aggregator.empty(device="cpu", depth=2)
    names = LD.quantize_specified_blocks(agg, 4, 128, "specific_blocks", frame_blocks=[1], global_blocks=[0, 1],
                                         layer_types=["qkv", "fc2"])
    assert sorted(names) == sorted(["aggregator.frame_blocks.1.attn.qkv", "aggregator.frame_blocks.1.mlp.fc2",
                                    "aggregator.global_blocks.0.attn.qkv", "aggregator.global_blocks.0.mlp.fc2",
                                    "aggregator.global_blocks.1.attn.qkv", "aggregator.global_blocks.1.mlp.fc2"])
    assert isinstance(agg.frame_blocks[1].attn.qkv, WQLinear)
    assert isinstance(agg.frame_blocks[0].attn.qkv, nn.Linear)
    assert isinstance(agg.global_blocks[1].mlp.fc1, nn.Linear)
    q = agg.global_blocks[0].mlp.fc2
    assert q.qweight.shape == (1024 // 4, 4096) and q.qweight.dtype == torch.int16
    assert q.scales.shape == (32, 1024) and q.bias.shape == (1024,)
    assert all(isinstance(b.attn.qkv, nn.Linear) for b in agg.patch_embed.blocks)


def test_merge_state_dicts_overlays_and_drops_replaced_weights():
    base = {"aggregator.patch_embed.patch_embed.proj.weight": torch.zeros(1),
            "aggregator.camera_token": torch.zeros(1), "camera_head.pose_branch.fc1.weight": torch.zeros(1)}
    q = dict(base)
    q.update({"aggregator.frame_blocks.0.attn.qkv.qweight": torch.ones(2, dtype=torch.int16),
              "aggregator.frame_blocks.0.attn.qkv.scales": torch.ones(2),
              "aggregator.frame_blocks.0.attn.qkv.weight": torch.ones(3),
              "aggregator.frame_blocks.1.attn.qkv.weight": torch.ones(3),
              "cict_token": torch.arange(4.0)})
    merged, cict = LD.merge_state_dicts(q, None, "specific_blocks", [0], None, ["qkv"])
    assert torch.equal(cict, torch.arange(4.0)) and "cict_token" not in merged
    assert "aggregator.frame_blocks.0.attn.qkv.weight" not in merged
    assert "aggregator.frame_blocks.1.attn.qkv.weight" in merged
    assert torch.equal(merged["aggregator.frame_blocks.0.attn.qkv.qweight"], torch.ones(2, dtype=torch.int16))
    with pytest.raises(ValueError, match="not self-contained"):
        LD.merge_state_dicts({"aggregator.frame_blocks.0.attn.qkv.qweight": torch.ones(1)}, None)


def test_read_state_dict_refuses_pickled_objects(tmp_path):
    p = tmp_path / "bad.pt"
    torch.save({"w": torch.zeros(2), "obj": object()}, p)
    with pytest.raises(Exception):
        LD.read_state_dict(p)
    p2 = tmp_path / "good.pt"
    torch.save({"w": torch.arange(3)}, p2)
    assert torch.equal(LD.read_state_dict(p2)["w"], torch.arange(3))


def test_roundtrip_quantized_aggregator_checkpoint(tmp_path):
    """A seeded W4 aggregator saved under the checkpoint's key names loads back
    bit for bit, with the layout inferred from the .qweight keys."""
    from safetensors.torch import save_file
    src = Aggregator.random(w8a8=False, seed=7, device="cpu", depth=2)
    sd = {"aggregator." + k: v.contiguous() for k, v in src.state_dict().items() if not k.startswith("img_")}
    sd["camera_head.pose_branch.fc1.weight"] = torch.zeros(4, 4, dtype=torch.float16)
    sd["aggregator.patch_embed.mask_token"] = torch.zeros(1, 1024, dtype=torch.float16)
    path = tmp_path / "qvggt_w4.safetensors"
    save_file(sd, str(path))
    agg, rep = LD.load_quantized_aggregator(path, device="cpu", depth=2)
    assert len(rep["replaced"]) == 16 and not rep["missing"]
    assert set(rep["unused"]) == {"patch_embed.mask_token"}
    got, ref = agg.state_dict(), src.state_dict()
    assert got.keys() == ref.keys()
    for k in ref:
        assert got[k].dtype == ref[k].dtype and torch.equal(got[k], ref[k]), k


def test_roundtrip_quantized_camera_head_checkpoint(tmp_path):
    """A seeded camera head with a W4 trunk saved under ``camera_head.*`` loads
    back bit for bit: the 16 trunk linears become WQLinear (inferred from the
    ``camera_head.trunk.*.qweight`` keys), the rest stays fp16, and the CICT
    token is reported (the head has no use for it)."""
    from safetensors.torch import save_file
    from qvggt_amd.camera_head import CameraHead
    src = CameraHead.random(seed=3, device="cpu")
    sd = {"camera_head." + k: v.contiguous() for k, v in src.state_dict().items()}
    sd["aggregator.patch_embed.patch_embed.proj.weight"] = torch.zeros(2, dtype=torch.float16)
    sd["aggregator.camera_token"] = torch.zeros(2, dtype=torch.float16)
    sd["camera_head.cict_token"] = torch.arange(6, dtype=torch.float32)
    path = tmp_path / "qvggt_w4_head.safetensors"
    save_file(sd, str(path))
    head, rep = LD.load_quantized_camera_head(path, device="cpu")
    assert len(rep["replaced"]) == 16 and not rep["missing"]
    assert rep["unused"] == ["cict_token"]          # kept in the merge (loader.py:480 pops only top-level keys)
    assert all(n.startswith("camera_head.trunk.") for n in rep["replaced"])
    assert torch.equal(rep["cict_token"], torch.arange(6, dtype=torch.float32))
    assert isinstance(head.trunk[2].mlp.fc1, WQLinear) and isinstance(head.pose_branch.fc1, nn.Linear)
    got, ref = head.state_dict(), src.state_dict()
    assert got.keys() == ref.keys()
    for k in ref:
        assert got[k].dtype == ref[k].dtype and torch.equal(got[k], ref[k]), k


def test_model_config_is_read_like_the_reference(tmp_path):
    """The aggregator's eps / depth come from the checkpoint's config.json
    (loader.py:146-162 reads VGGTConfig from the fp16 model's directory): a
    config with LayerNorm eps 1e-5 and depth 2 builds blocks whose four norms
    use 1e-5; the fp16 model's directory wins over the checkpoint's; no
    config gives the defaults; unsupported dims are refused."""
    import json
    from safetensors.torch import save_file
    from qvggt_amd.aggregator import AggregatorConfig
    src = Aggregator.random(w8a8=False, seed=1, device="cpu", depth=2)
    sd = {"aggregator." + k: v.contiguous() for k, v in src.state_dict().items() if not k.startswith("img_")}
    sd["camera_head.pose_branch.fc1.weight"] = torch.zeros(4, 4, dtype=torch.float16)
    qdir, mdir = tmp_path / "q", tmp_path / "m"
    qdir.mkdir()
    mdir.mkdir()
    save_file(sd, str(qdir / "model.safetensors"))
    assert LD.load_model_config(qdir / "model.safetensors") == AggregatorConfig()
    (qdir / "config.json").write_text(json.dumps({"layer_norm_eps": 1e-5, "depth": 2, "patch_embed_depth": 2,
                                                  "rope_freq": 100}))
    agg, rep = LD.load_quantized_aggregator(qdir / "model.safetensors", device="cpu")
    assert rep["config"].block_ln_eps == 1e-5 and rep["config"].depth == 2 and len(agg.frame_blocks) == 2
    for blk in list(agg.frame_blocks) + list(agg.global_blocks):
        assert blk.eps == 1e-5
        assert {m.eps for m in (blk.norm1, blk.norm2, blk.attn.q_norm, blk.attn.k_norm)} == {1e-5}
    (mdir / "config.json").write_text(json.dumps({"aggregator": {"layer_norm_eps": 3e-6, "depth": 2}}))
    assert LD.load_model_config(qdir / "model.safetensors", mdir / "w.pt").block_ln_eps == 3e-6
    with pytest.raises(ValueError, match="unsupported"):
        AggregatorConfig.from_dict({"hidden_size": 768})


def test_model_config_sections_do_not_override_each_other():
    """A patch_embed_config section sets only the DINOv2 fields (its plain
    depth / layer_norm_eps included); the aggregator section's values set the
    AA blocks, whichever order the sections appear in."""
    from qvggt_amd.aggregator import AggregatorConfig
    d = {"aggregator_config": {"layer_norm_eps": 1e-5, "depth": 24},
         "patch_embed_config": {"layer_norm_eps": 1e-6, "depth": 12}}
    for cfg in (d, dict(reversed(list(d.items())))):
        c = AggregatorConfig.from_dict(cfg)
        assert (c.depth, c.block_ln_eps, c.dino_depth, c.dino_ln_eps) == (24, 1e-5, 12, 1e-6)
    c = AggregatorConfig.from_dict({"patch_embed_config": {"norm_eps": 1e-5}})
    assert (c.block_ln_eps, c.dino_ln_eps, c.depth) == (1e-6, 1e-5, 24)
    c = AggregatorConfig.from_dict({"aa_depth": 8, "patch_embed_depth": 6, "layer_norm_eps": 1e-5})
    assert (c.depth, c.dino_depth, c.block_ln_eps, c.dino_ln_eps) == (8, 6, 1e-5, 1e-6)
