"""Device-direct checkpoint loading (quantization.py:325-430) on the GPU: a
synthetic compressed-tensors checkpoint loaded with ``device="cuda:0"`` gives
the same tensors as the CPU load, and its experts run through the HIP
library against the oracle."""
import json

import numpy as np
import pytest
import torch

pytest.importorskip("transformers.models.gemma4")
from safetensors.torch import save_file  # noqa: E402

import oracle  # noqa: E402
from hybridagent_amd import _lib  # noqa: E402
from hybridagent_amd import quantization as q  # noqa: E402

pytestmark = pytest.mark.gpu

H, I, E, LAYERS, G = 64, 32, 4, 2, 32


def _write_checkpoint(d):
    from transformers.models.gemma4 import configuration_gemma4 as c
    text = dict(hidden_size=H, intermediate_size=64, num_hidden_layers=LAYERS, num_attention_heads=2,
                num_key_value_heads=1, head_dim=32, vocab_size=128, vocab_size_per_layer_input=128,
                hidden_size_per_layer_input=16, enable_moe_block=True, num_experts=E, top_k_experts=2,
                moe_intermediate_size=I, sliding_window=16, max_position_embeddings=64,
                layer_types=["sliding_attention", "full_attention"])
    cfg = c.Gemma4Config(text_config=text, vision_config=None, audio_config=None).to_dict()
    cfg["quantization_config"] = {"quant_method": "compressed-tensors", "format": "pack-quantized",
                                  "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": G}}}}
    (d / "config.json").write_text(json.dumps(cfg))
    g = torch.Generator().manual_seed(77)
    i32 = lambda *s: torch.randint(-2**31, 2**31 - 1, s, generator=g, dtype=torch.int64).to(torch.int32)
    bf = lambda *s: (0.01 + 0.01 * torch.rand(*s, generator=g)).to(torch.bfloat16)
    shards = [{}, {}]
    for ly in range(LAYERS):
        for e in range(E):
            pre = f"model.language_model.layers.{ly}.experts.{e}"
            sd = shards[(ly * E + e) % 2]          # experts of a layer spread over both shards
            for proj, (n, k) in {"gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}.items():
                sd[f"{pre}.{proj}.weight_packed"] = i32(n, k // 8)
                sd[f"{pre}.{proj}.weight_scale"] = bf(n, k // G)
        shards[ly % 2][f"model.language_model.layers.{ly}.router.proj.weight"] = bf(E, H)
    weight_map = {}
    for i, sd in enumerate(shards):
        name = f"model-{i:05d}-of-00002.safetensors"
        save_file(sd, str(d / name))
        weight_map.update({k: name for k in sd})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


def test_device_direct_load_matches_cpu_load(tmp_path):
    assert _lib.available(), "libw4a16moe.so must be built"
    dev = torch.device("cuda:0")
    _write_checkpoint(tmp_path)
    cpu = q.load_pack_quantized_backbone(tmp_path, dtype=torch.bfloat16)
    gpu = q.load_pack_quantized_backbone(tmp_path, dtype=torch.bfloat16, device=dev)
    lc, lg = cpu.model.language_model.layers, gpu.model.language_model.layers
    for ly in range(LAYERS):
        ec, eg = lc[ly].experts, lg[ly].experts
        assert eg.gate_up_packed.is_cuda and eg.group_size == G
        for name in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"):
            assert torch.equal(getattr(eg, name).cpu(), getattr(ec, name)), (ly, name)
        assert torch.equal(lg[ly].router.proj.weight.data.cpu(), lc[ly].router.proj.weight.data)
    # the loaded experts run on the device against the oracle
    ex = lg[1].experts
    M = 5
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(78)).to(torch.bfloat16)
    idx = torch.tensor([[0, 1], [2, 3], [1, 2], [3, 0], [2, 1]])
    w = torch.rand(M, 2, generator=torch.Generator().manual_seed(79)).float()
    y = ex(x.to(dev), idx.to(dev), w.to(dev))
    bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = oracle.moe_forward(x.float().numpy(), idx.numpy(), w.numpy(), ex.gate_up_packed.cpu().numpy(),
                             bits(ex.gate_up_scale), ex.down_packed.cpu().numpy(), bits(ex.down_scale), G)
    assert oracle.max_abs_rel(y.float().cpu().numpy(), ref) <= 1e-2
