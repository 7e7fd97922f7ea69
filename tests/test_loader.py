"""Checkpoint loader of the drop-in quantization module (CPU only).

A tiny Gemma-4 model is described by a synthetic compressed-tensors
(pack-quantized) checkpoint written here: per-expert ``gate_proj`` /
``up_proj`` / ``down_proj`` ``weight_packed`` + ``weight_scale`` tensors
(the layout the reference loader reads, quantization.py:383-421) plus one
ordinary tensor.  ``load_pack_quantized_backbone`` must swap in the 4-bit
experts module and stack the shards into its buffers with gate rows before up
rows; nothing here touches a GPU.
"""
import json

import pytest
import torch

pytest.importorskip("transformers.models.gemma4")
from safetensors.torch import save_file  # noqa: E402

from hybridagent_amd import quantization as q  # noqa: E402

H, I, E, LAYERS, G = 64, 32, 4, 2, 32


def _tiny_config():
    from transformers.models.gemma4 import configuration_gemma4 as c
    text = dict(hidden_size=H, intermediate_size=64, num_hidden_layers=LAYERS, num_attention_heads=2,
                num_key_value_heads=1, head_dim=32, vocab_size=128, vocab_size_per_layer_input=128,
                hidden_size_per_layer_input=16, enable_moe_block=True, num_experts=E, top_k_experts=2,
                moe_intermediate_size=I, sliding_window=16, max_position_embeddings=64,
                layer_types=["sliding_attention", "full_attention"])
    return c.Gemma4Config(text_config=text, vision_config=None, audio_config=None)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    cfg = _tiny_config().to_dict()
    cfg["quantization_config"] = {"quant_method": "compressed-tensors", "format": "pack-quantized",
                                  "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": G}}}}
    (d / "config.json").write_text(json.dumps(cfg))
    g = torch.Generator().manual_seed(5)
    rnd_i32 = lambda *s: torch.randint(-2**31, 2**31 - 1, s, generator=g, dtype=torch.int64).to(torch.int32)
    rnd_bf = lambda *s: (0.01 + 0.01 * torch.rand(*s, generator=g)).to(torch.bfloat16)
    sd, expect = {}, {}
    for ly in range(LAYERS):
        for e in range(E):
            pre = f"model.language_model.layers.{ly}.experts.{e}"
            t = {"gp": rnd_i32(I, H // 8), "gs": rnd_bf(I, H // G), "up": rnd_i32(I, H // 8), "us": rnd_bf(I, H // G),
                 "dp": rnd_i32(H, I // 8), "ds": rnd_bf(H, I // G)}
            for proj, (pk, sk) in {"gate_proj": ("gp", "gs"), "up_proj": ("up", "us"), "down_proj": ("dp", "ds")}.items():
                sd[f"{pre}.{proj}.weight_packed"] = t[pk]
                sd[f"{pre}.{proj}.weight_scale"] = t[sk]
                sd[f"{pre}.{proj}.weight_shape"] = torch.tensor(list(t[pk].shape[:1]) + [t[pk].shape[1] * 8])
            expect[(ly, e)] = t
        sd[f"model.language_model.layers.{ly}.router.proj.weight"] = rnd_bf(E, H)
        expect[(ly, "router")] = sd[f"model.language_model.layers.{ly}.router.proj.weight"]
    save_file(sd, str(d / "model.safetensors"))
    return d, expect


def test_is_pack_quantized_dir(checkpoint, tmp_path):
    d, _ = checkpoint
    assert q.is_pack_quantized_dir(d)
    assert not q.is_pack_quantized_dir(tmp_path)


def test_loader_stacks_expert_shards(checkpoint):
    d, expect = checkpoint
    model = q.load_pack_quantized_backbone(d, dtype=torch.bfloat16)
    layers = model.model.language_model.layers
    assert len(layers) == LAYERS
    for ly, layer in enumerate(layers):
        ex = layer.experts
        assert isinstance(ex, q.Gemma4TextExperts4Bit)
        assert ex.group_size == G
        assert ex.gate_up_packed.shape == (E, 2 * I, H // 8)
        assert ex.down_scale.shape == (E, H, I // G)
        for e in range(E):
            t = expect[(ly, e)]
            # gate rows first, then up rows (quantization.py:406-412)
            assert torch.equal(ex.gate_up_packed[e], torch.cat([t["gp"], t["up"]]))
            assert torch.equal(ex.gate_up_scale[e], torch.cat([t["gs"], t["us"]]))
            assert torch.equal(ex.down_packed[e], t["dp"])
            assert torch.equal(ex.down_scale[e], t["ds"])
        assert torch.equal(layer.router.proj.weight.data, expect[(ly, "router")])


def test_group_size_from_config():
    class C:
        quantization_config = {"config_groups": {"g": {"weights": {"group_size": 128}}}}
    assert q._group_size_from_config(C(), 32) == 128
    assert q._group_size_from_config(object(), 32) == 32


def test_parse_expert_key():
    assert q._parse_expert_key("model.language_model.layers.3.experts.17.up_proj.weight_scale") == (3, 17, "us")
    assert q._parse_expert_key("model.language_model.layers.3.mlp.up_proj.weight") is None
    assert q._parse_expert_key("model.language_model.layers.3.experts.1.up_proj.weight_shape") is None


def test_shard_reader_matches_safetensors(tmp_path):
    from hybridagent_amd import loader
    from safetensors.torch import load_file
    g = torch.Generator().manual_seed(9)
    sd = {
        "a.odd_bf16": torch.randn(3, generator=g).to(torch.bfloat16),   # 6 bytes: the next tensor starts unaligned
        "b.i32": torch.randint(-100, 100, (5, 7), generator=g, dtype=torch.int32),
        "c.f32": torch.randn(4, 2, generator=g),
        "d.i64": torch.arange(6, dtype=torch.int64).reshape(2, 3),
    }
    path = tmp_path / "x.safetensors"
    save_file(sd, str(path))
    ref = load_file(str(path))
    got = loader.ShardReader("cpu").open(path)
    assert set(got) == set(ref)
    for k in ref:
        assert got[k].dtype == ref[k].dtype and torch.equal(got[k], ref[k]), k


def test_placer_rejects_wrong_group_size_and_missing_experts():
    from hybridagent_amd import loader
    import types as _t
    cfg = _t.SimpleNamespace(num_experts=2, hidden_size=64, moe_intermediate_size=32,
                             hidden_activation="gelu_pytorch_tanh")
    m = q.Gemma4TextExperts4Bit(cfg, group_size=32)
    placer = loader.ExpertPlacer([m])
    with pytest.raises(ValueError, match="does not match"):
        placer.place(0, 0, "gs", torch.zeros(32, 4, dtype=torch.bfloat16))   # G = 16 scales
    placer.place(0, 0, "gp", torch.zeros(32, 8, dtype=torch.int32))
    with pytest.raises(ValueError, match="missing"):
        placer.check_complete()
    with pytest.raises(ValueError, match="outside"):
        placer.place(0, 5, "gp", torch.zeros(32, 8, dtype=torch.int32))
