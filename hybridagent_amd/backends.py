"""The hot-path part of HybridAgent's ``hybrid_agent/backends.py``, on HIP.

* ``fused_4bit_moe_op``: the ``hybrid_agent::fused_4bit_moe`` custom op with
  the reference's name, schema and fake (backends.py:48-65), so a
  ``torch.compile(fullgraph=True)`` caller such as ``_ffn_moe_4bit_step``
  (backends.py:77-126) traces it as one opaque node.  If the reference's
  ``backends.py`` is imported in the same process it registers the same op
  itself (bound to ``quantization.fused_triton_4bit_moe_forward``, i.e. to
  the HIP path when this package stands in for ``quantization.py``), and
  this module then reuses that registration instead of failing.
* ``moe_router``: the router lines of ``_ffn_moe_4bit_step``
  (backends.py:111-117) as one fused HIP pipeline, also as a custom op
  ``hybridagent_amd::moe_router``.
"""
from __future__ import annotations

import torch

from . import _lib
from .quantization import fused_triton_4bit_moe_forward


def _already_registered(qualname: str) -> bool:
    ns, name = qualname.split("::")
    try:
        return hasattr(getattr(torch.ops, ns), name)
    except (AttributeError, RuntimeError):
        return False


if _already_registered("hybrid_agent::fused_4bit_moe"):
    fused_4bit_moe_op = torch.ops.hybrid_agent.fused_4bit_moe
else:
    @torch.library.custom_op("hybrid_agent::fused_4bit_moe", mutates_args=())
    def fused_4bit_moe_op(
        hidden_states: torch.Tensor,
        top_k_index: torch.Tensor,
        top_k_weights: torch.Tensor,
        gu_packed: torch.Tensor,
        gu_scale: torch.Tensor,
        dn_packed: torch.Tensor,
        dn_scale: torch.Tensor,
    ) -> torch.Tensor:
        return fused_triton_4bit_moe_forward(
            hidden_states, top_k_index, top_k_weights, gu_packed, gu_scale, dn_packed, dn_scale)

    @fused_4bit_moe_op.register_fake
    def _(hidden_states, top_k_index, top_k_weights, gu_packed, gu_scale, dn_packed, dn_scale):
        return torch.empty_like(hidden_states)


@torch.library.custom_op("hybridagent_amd::moe_router", mutates_args=())
def _moe_router_op(
    residual: torch.Tensor,
    router_scale: torch.Tensor,
    scalar_root: float,
    proj_w: torch.Tensor,
    per_expert_scale: torch.Tensor,
    eps: float,
    top_k: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    return _lib.router_topk(residual, router_scale, scalar_root, proj_w, per_expert_scale, eps, top_k)


@_moe_router_op.register_fake
def _(residual, router_scale, scalar_root, proj_w, per_expert_scale, eps, top_k):
    M = residual.numel() // residual.shape[-1]
    return (residual.new_empty((M, top_k), dtype=torch.float32),
            residual.new_empty((M, top_k), dtype=torch.int64))


def moe_router(
    residual: torch.Tensor,
    router_scale: torch.Tensor,
    scalar_root: float,
    proj_w: torch.Tensor,
    per_expert_scale: torch.Tensor,
    eps: float,
    top_k: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(top_k_weights fp32 [M, k], top_k_index int64 [M, k]) of backends.py:111-117:
    ``softmax(F.linear(rms_norm(h) * scale * scalar_root, W_r))`` -> top-k ->
    renormalise -> ``* per_expert_scale[idx]``."""
    return _moe_router_op(residual, router_scale, float(scalar_root), proj_w, per_expert_scale,
                          float(eps), int(top_k))


def ffn_moe_4bit_step(
    residual: torch.Tensor,
    attn_out: torch.Tensor,
    post_attn_ln_w: torch.Tensor,
    pre_ff_ln_w: torch.Tensor,
    mlp_gate_w: torch.Tensor,
    mlp_up_w: torch.Tensor,
    mlp_down_w: torch.Tensor,
    post_ff_ln1_w: torch.Tensor,
    router_scale: torch.Tensor,
    router_scalar_root: float,
    router_proj_w: torch.Tensor,
    router_per_expert_scale: torch.Tensor,
    pre_ff_ln2_w: torch.Tensor,
    gu_packed: torch.Tensor,
    gu_scale: torch.Tensor,
    dn_packed: torch.Tensor,
    dn_scale: torch.Tensor,
    post_ff_ln2_w: torch.Tensor,
    post_ff_ln_w: torch.Tensor,
    layer_scalar: torch.Tensor,
    eps: float,
    top_k: int,
) -> torch.Tensor:
    """``_ffn_moe_4bit_step`` (backends.py:77-126) with the same 22 arguments: the
    post-attention RMSNorm and residual, the shared bf16 MLP, the router, the
    W4A16 experts, the four FFN RMSNorms and ``layer_scalar`` in one C-ABI call
    (``moe_ffn_block_forward``: two row kernels, two shared-MLP linears and the
    MoE layer's launches), no host synchronisation."""
    return _lib.ffn_block(residual, attn_out, post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w,
                          post_ff_ln1_w, router_scale, router_scalar_root, router_proj_w,
                          router_per_expert_scale, pre_ff_ln2_w, gu_packed, gu_scale, dn_packed, dn_scale,
                          post_ff_ln2_w, post_ff_ln_w, layer_scalar, eps, top_k)


def patch_ffn_4bit(backbone: torch.nn.Module) -> int:
    """Route every 4-bit MoE decoder layer's FFN block through ``ffn_moe_4bit_step``,
    the counterpart of ``patch_compiled_ffn_4bit`` (backends.py:132-201): the layer
    keeps its input RMSNorm and attention; everything after attention runs in
    the HIP library.  Returns the number of layers patched."""
    from .quantization import Gemma4TextExperts4Bit

    text_model = getattr(backbone.model, "language_model", backbone.model)
    patched = 0
    for layer in getattr(text_model, "layers", []):
        if not isinstance(getattr(layer, "experts", None), Gemma4TextExperts4Bit):
            continue
        eps = float(layer.input_layernorm.eps)
        top_k = int(layer.router.config.top_k_experts)
        scalar_root = float(layer.router.scalar_root_size)

        def _make_layer_fwd(lyr, _eps=eps, _top_k=top_k, _sr=scalar_root):
            def _fwd(hidden_states, per_layer_input=None, shared_kv_states=None, position_embeddings=None,
                     attention_mask=None, position_ids=None, past_key_values=None, **kwargs):
                residual = hidden_states
                hidden_states = lyr.input_layernorm(hidden_states)
                hidden_states, _ = lyr.self_attn(
                    hidden_states=hidden_states, position_embeddings=position_embeddings,
                    attention_mask=attention_mask, shared_kv_states=shared_kv_states,
                    position_ids=position_ids, past_key_values=past_key_values, **kwargs)
                return ffn_moe_4bit_step(
                    residual, hidden_states, lyr.post_attention_layernorm.weight,
                    lyr.pre_feedforward_layernorm.weight, lyr.mlp.gate_proj.weight, lyr.mlp.up_proj.weight,
                    lyr.mlp.down_proj.weight, lyr.post_feedforward_layernorm_1.weight, lyr.router.scale, _sr,
                    lyr.router.proj.weight, lyr.router.per_expert_scale, lyr.pre_feedforward_layernorm_2.weight,
                    lyr.experts.gate_up_packed, lyr.experts.gate_up_scale, lyr.experts.down_packed,
                    lyr.experts.down_scale, lyr.post_feedforward_layernorm_2.weight,
                    lyr.post_feedforward_layernorm.weight, lyr.layer_scalar, _eps, _top_k)
            return _fwd

        layer.forward = _make_layer_fwd(layer)
        patched += 1
    return patched


def bf16_experts_fast_forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                              top_k_weights: torch.Tensor) -> torch.Tensor:
    """``_bf16_experts_fast_forward`` (backends.py:209-283) for transformers'
    BF16 ``Gemma4TextExperts`` (parameters ``gate_up_proj`` [E, 2I, H] and
    ``down_proj`` [E, H, I]): the expert sort, the two grouped bf16 GEMMs (gated
    GELU fused) and the weighted top-k sum on the HIP library, at every batch
    size, with no host synchronisation."""
    out = _lib.bf16_experts_forward(hidden_states, top_k_index, top_k_weights, self.gate_up_proj,
                                    self.down_proj)
    return out.to(hidden_states.dtype)


def patch_bf16_experts_fastpath(backbone: torch.nn.Module) -> int:
    """Bind ``bf16_experts_fast_forward`` to every BF16 ``Gemma4TextExperts`` module
    (backends.py:286-298); returns the number of modules patched."""
    import types

    from .quantization import Gemma4TextExperts4Bit

    patched = 0
    for mod in backbone.modules():
        if mod.__class__.__name__ == "Gemma4TextExperts" and not isinstance(mod, Gemma4TextExperts4Bit):
            mod.forward = types.MethodType(bf16_experts_fast_forward, mod)
            patched += 1
    return patched


def moe_block(residual: torch.Tensor, h2_in: torch.Tensor, router, experts) -> torch.Tensor:
    """Router on ``residual`` + experts on ``h2_in`` (backends.py:111-122):
    ``router`` is a Gemma4TextRouter-like module (``scale``, ``proj``,
    ``per_expert_scale``, ``scalar_root_size``, ``eps``, ``config.top_k_experts``),
    ``experts`` a ``Gemma4TextExperts4Bit``."""
    D = residual.shape[-1]
    w, idx = moe_router(residual.reshape(-1, D), router.scale, router.scalar_root_size,
                        router.proj.weight, router.per_expert_scale, router.eps,
                        router.config.top_k_experts)
    out = fused_4bit_moe_op(h2_in.reshape(-1, D), idx, w, experts.gate_up_packed, experts.gate_up_scale,
                            experts.down_packed, experts.down_scale)
    return out.reshape(residual.shape)
