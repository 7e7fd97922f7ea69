"""Drop-in replacement for HybridAgent's ``hybrid_agent/quantization.py``.

Same public names, constructor arguments, buffer names / shapes / dtypes and
``forward`` signatures as the reference module, so ``backends.py``,
``model.py`` and the compressed-tensors checkpoints work unchanged; every
computation runs in the gfx950 HIP library (``libw4a16moe.so``) through the
C ABI in ``include/w4a16moe.h``.  There is no Triton and no CPU path: calling
a forward on CPU tensors, or without the built library, raises.

Differences from the reference, all supersets:

* the group size is a parameter (``GROUP_SIZE`` = 32 stays the default, as
  in quantization.py:19); scale tensors have ``ceil(K / G)`` columns, so
  K = 704 with G = 128 (a partial last group) is expressible;
* ``_HAS_TRITON_W4A16`` keeps its name for ``backends.py`` but means "the HIP
  kernel library is available".
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Any
from unittest import mock

import torch
import torch.nn as nn

from . import _lib, loader

GROUP_SIZE = 32  # quantization.py:19 (the released 4-bit checkpoints)

# Name kept for backends.py:37-43,444; true when the HIP library loads.
_HAS_TRITON_W4A16 = _lib.available()
HIP_W4A16_AVAILABLE = _HAS_TRITON_W4A16


def _num_groups(K: int, G: int) -> int:
    return -(-K // G)


def _group_size_from_config(config: Any, default: int) -> int:
    """compressed-tensors ``quantization_config.config_groups.*.weights.group_size``."""
    q = getattr(config, "quantization_config", None)
    if isinstance(q, dict):
        for grp in (q.get("config_groups") or {}).values():
            g = (grp or {}).get("weights", {}).get("group_size")
            if g:
                return int(g)
    return default


def fused_triton_4bit_moe_forward(
    hidden_states: torch.Tensor,
    top_k_index: torch.Tensor,
    top_k_weights: torch.Tensor,
    gu_packed: torch.Tensor,
    gu_scale: torch.Tensor,
    dn_packed: torch.Tensor,
    dn_scale: torch.Tensor,
) -> torch.Tensor:
    """W4A16 MoE forward (quantization.py:88-129), same 7 arguments.

    Runs the gfx950 pipeline: expert sort -> grouped gate_up GEMM with the
    gated GELU fused -> grouped down GEMM -> weighted top-k combine, all on
    the current stream, no host synchronisation.  The name is kept so
    ``backends.fused_4bit_moe_op`` (backends.py:48-60) binds to it unchanged.
    """
    return _lib.moe_forward(hidden_states, top_k_index, top_k_weights, gu_packed, gu_scale,
                            dn_packed, dn_scale)


def dequantize_int4_packed(
    packed: torch.Tensor, scale: torch.Tensor, shifts: torch.Tensor | None = None,
    group_size: int | None = None,
) -> torch.Tensor:
    """Unpack int32-packed symmetric int4 (offset +8) times bf16 group scales
    (quantization.py:132-137), bit-identical to the reference's bf16 result.

    ``shifts`` is accepted for signature compatibility; the nibble order is
    fixed by the format (nibble i at bits 4i).  The group size is taken from
    the scale shape unless given.
    """
    if shifts is not None and shifts.numel() != 8:
        raise ValueError("shifts must be the 8 nibble shifts arange(0, 32, 4)")
    return _lib.dequantize(packed, scale, group_size)


class Linear4Bit(nn.Module):
    """4-bit pack-quantized W4A16 Linear (quantization.py:140-175)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bias: bool = False,
        dtype: torch.dtype = torch.bfloat16,
        group_size: int | None = None,
    ) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size or GROUP_SIZE
        self.register_buffer(
            "weight_packed", torch.empty((out_features, in_features // 8), dtype=torch.int32))
        self.register_buffer(
            "weight_scale",
            torch.empty((out_features, _num_groups(in_features, self.group_size)), dtype=dtype))
        self.register_buffer("_shifts", torch.arange(0, 32, 4, dtype=torch.int32), persistent=False)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _lib.linear(x, self.weight_packed, self.weight_scale,
                           None if self.bias is None else self.bias.detach(), self.group_size)


class Gemma4TextExperts4Bit(nn.Module):
    """4-bit pack-quantized W4A16 experts for Gemma 4 (quantization.py:178-294).

    Buffers (the checkpoint contract, quantization.py:191-223):
    ``gate_up_packed`` int32 [E, 2I, H/8] (gate rows first), ``gate_up_scale``
    [E, 2I, ceil(H/G)], ``down_packed`` int32 [E, H, I/8], ``down_scale``
    [E, H, ceil(I/G)], ``_shifts`` (non-persistent).
    """

    def __init__(self, config, dtype: torch.dtype = torch.bfloat16, group_size: int | None = None) -> None:
        super().__init__()
        self.num_experts = config.num_experts
        self.hidden_dim = config.hidden_size
        self.intermediate_dim = config.moe_intermediate_size
        act = getattr(config, "hidden_activation", "gelu_pytorch_tanh")
        if act != "gelu_pytorch_tanh":
            raise ValueError(f"the fused kernel implements gelu_pytorch_tanh, config asks for {act!r}")
        self.group_size = group_size or _group_size_from_config(config, GROUP_SIZE)
        E, H, I, G = self.num_experts, self.hidden_dim, self.intermediate_dim, self.group_size
        self.register_buffer("gate_up_packed", torch.empty((E, 2 * I, H // 8), dtype=torch.int32))
        self.register_buffer("gate_up_scale", torch.empty((E, 2 * I, _num_groups(H, G)), dtype=dtype))
        self.register_buffer("down_packed", torch.empty((E, H, I // 8), dtype=torch.int32))
        self.register_buffer("down_scale", torch.empty((E, H, _num_groups(I, G)), dtype=dtype))
        self.register_buffer("_shifts", torch.arange(0, 32, 4, dtype=torch.int32), persistent=False)

    def forward(
        self,
        hidden_states: torch.Tensor,
        top_k_index: torch.Tensor,
        top_k_weights: torch.Tensor,
    ) -> torch.Tensor:
        """[T, H] bf16 -> [T, H] bf16 (quantization.py:225-240); GPU only, zero-sync.
        Reads the tiled weight copies when ``tile_weights`` made them."""
        return fused_triton_4bit_moe_forward(
            hidden_states, top_k_index, top_k_weights,
            self.gate_up_packed, self.gate_up_scale, self.down_packed, self.down_scale)

    def tile_weights(self, decode: bool = True, prefill: bool = True) -> None:
        """Build the kernels' tiled copies of the loaded expert weights (no counterpart
        in the reference): the decode streamers read them as contiguous KiBs (group
        size 128, 32 or 64) and the prefill GEMMs as 8 KiB blocks.  Every forward on
        these buffers then uses them -- this module's, ``fused_triton_4bit_moe_forward``,
        the ``hybrid_agent::fused_4bit_moe`` op and ``ffn_moe_4bit_step`` -- with
        bit-identical results.  They take about
        one more copy of the experts' memory per kind; the buffers and the state dict
        are unchanged.  Call after the weights are loaded, on their device; when the
        buffers are changed in place (a reload) or replaced (moved), the copies are
        dropped at the next forward and the packed weights serve until this is called
        again."""
        tw = _lib.tile_experts(self.gate_up_packed, self.gate_up_scale, self.down_packed, self.down_scale,
                               self.group_size, decode=decode, prefill=prefill)
        _lib.register_tiles(self.gate_up_packed, self.gate_up_scale, self.down_packed, self.down_scale, tw)
        self._tiles = tw

    def untile_weights(self) -> None:
        """Drop the tiled copies made by ``tile_weights``."""
        _lib.unregister_tiles(self.gate_up_packed)
        self._tiles = None

    @property
    def tiles(self) -> "_lib.TiledWeights | None":
        """The tiled copies in use for the current buffers, or None."""
        return _lib.lookup_tiles(self.gate_up_packed, self.gate_up_scale, self.down_packed, self.down_scale)


def is_pack_quantized_dir(model_dir: Path) -> bool:
    """config.json declares compressed-tensors / pack-quantized (quantization.py:297-306)."""
    cfg_file = Path(model_dir) / "config.json"
    if not cfg_file.is_file():
        return False
    try:
        cfg = json.loads(cfg_file.read_text(encoding="utf-8"))
    except (OSError, ValueError):
        return False
    q = cfg.get("quantization_config") or {}
    return q.get("format") == "pack-quantized" or q.get("quant_method") == "compressed-tensors"


def _parse_expert_key(key: str):
    """model.language_model.layers.{l}.experts.{e}.{proj}.{kind} -> (l, e, tag) or None."""
    return loader.parse_expert_key(key)


def load_pack_quantized_backbone(
    model_dir: Path,
    *,
    dtype: torch.dtype = torch.bfloat16,
    trust_remote_code: bool = False,
    device: str | torch.device | None = None,
    tile: bool = False,
) -> nn.Module:
    """Instantiate Gemma4ForConditionalGeneration with 4-bit experts and stream the
    compressed-tensors shards into it (quantization.py:325-430).

    The group size comes from ``quantization_config`` (default ``GROUP_SIZE``).
    With ``device`` (e.g. ``"cuda:0"``) the model is built on that device and
    each shard is read into pinned host memory, copied to the device whole and
    written from there into the module tensors (experts straight into their
    slices of the stacked buffers); without it everything stays on the CPU,
    as in the reference.  ``tile`` (with a GPU ``device``) also builds every
    experts module's tiled weight copies (``Gemma4TextExperts4Bit.tile_weights``),
    so the decode and prefill kernels read them from the first forward on.
    """
    from transformers import AutoConfig, AutoModelForCausalLM
    from transformers.models.gemma4 import modeling_gemma4

    model_dir = Path(model_dir)
    config = AutoConfig.from_pretrained(str(model_dir), trust_remote_code=trust_remote_code)
    group_size = _group_size_from_config(config, GROUP_SIZE)
    if hasattr(config, "quantization_config"):
        delattr(config, "quantization_config")

    class _ExpertsCls(Gemma4TextExperts4Bit):
        def __init__(self, cfg):
            super().__init__(cfg, dtype=dtype, group_size=group_size)

    orig_init_weights = modeling_gemma4.Gemma4PreTrainedModel._init_weights

    def _skip_init(self, module):
        if isinstance(module, (Gemma4TextExperts4Bit, nn.Linear, nn.Embedding)):
            return
        orig_init_weights(self, module)

    dev = torch.device(device) if device is not None else torch.device("cpu")
    with mock.patch.object(modeling_gemma4, "Gemma4TextExperts", _ExpertsCls), \
            mock.patch.object(modeling_gemma4.Gemma4PreTrainedModel, "_init_weights", _skip_init), \
            torch.device(dev):
        backbone = AutoModelForCausalLM.from_config(config, dtype=dtype, trust_remote_code=trust_remote_code)

    layers = backbone.model.language_model.layers
    placer = loader.ExpertPlacer([ly.experts for ly in layers])
    targets = dict(backbone.named_parameters())
    targets.update(dict(backbone.named_buffers()))
    loader.stream_shards(loader.shard_files(model_dir), placer, targets, dev)
    if getattr(config, "tie_word_embeddings", True):
        backbone.tie_weights()
    if tile:
        if dev.type != "cuda":
            raise ValueError("tile=True needs a GPU device: the tiled copies live next to the weights")
        for ly in layers:
            ly.experts.tile_weights()
    return backbone
