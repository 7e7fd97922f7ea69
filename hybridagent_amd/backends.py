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
