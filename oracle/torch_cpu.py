"""torch-CPU restatement of the reference's CPU W4A16 path -- TEST INFRASTRUCTURE ONLY.

The reference runs these torch ops whenever its Triton kernel is not used
(CPU tensors, ``quantization.py:231``); ``bench.py`` times this restatement
as the CPU baseline beside the GPU numbers (configs[0]: the dense
``Linear4Bit.forward``; configs[2]: one decode MoE layer with its router),
and ``tests/test_oracle.py`` pins it against the numpy oracle.  It is never
imported by the product path.

Restated from (``hybrid_agent/`` in the reference repository):

* ``dequantize``        quantization.py:132-137 (bf16 ``q * s``); the group
                         size is a parameter and the last group may be
                         partial (K zero-padded to ceil(K/G) * G);
* ``linear4bit``         quantization.py:171-175 (dequantise, then F.linear);
* ``experts_single``     quantization.py:241-263 (T == 1: the active experts'
                         weights dequantised at once, torch.mv for gate_up,
                         bmm for down, weighted sum);
* ``experts_loop``       quantization.py:265-294 (T > 1: one_hot expert mask,
                         per-expert torch.where in k-major order, F.linear,
                         bf16 index_add_);
* ``router``             backends.py:111-117 (RMSNorm * scale * scalar_root,
                         F.linear logits, fp32 softmax, top-k, renormalise,
                         per_expert_scale);
* ``ffn_block``          backends.py:101-126 (_ffn_moe_4bit_step in eager ops);
* ``bf16_experts``       backends.py:209-283 (the BF16 experts' three branches).

All tensors are CPU torch tensors in the reference's dtypes (bf16
activations and scales, int32 packed weights, fp32 routing weights).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

_SHIFTS = torch.arange(0, 32, 4, dtype=torch.int32)


def dequantize(packed: torch.Tensor, scale: torch.Tensor, G: int) -> torch.Tensor:
    """bf16 [..., N, K] = bf16(q) * s per group (quantization.py:132-137)."""
    q = ((packed.unsqueeze(-1) >> _SHIFTS) & 0xF) - 8
    q = q.flatten(-2).to(scale.dtype)                       # [..., N, K]
    K = q.shape[-1]
    ng = scale.shape[-1]
    if ng * G != K:                                         # partial last group
        q = F.pad(q, (0, ng * G - K))
    w = (q.view(*scale.shape, G) * scale.unsqueeze(-1)).flatten(-2)
    return w[..., :K]


def linear4bit(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, G: int,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    """Linear4Bit.forward (quantization.py:171-175)."""
    w = dequantize(packed, scale, G)
    if w.dtype != x.dtype:
        w = w.to(x.dtype)
    return F.linear(x, w, bias)


def _gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    return F.gelu(x, approximate="tanh")   # ACT2FN["gelu_pytorch_tanh"]


def experts_single(h: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, gu_p, gu_s, dn_p, dn_s,
                   G: int) -> torch.Tensor:
    """The T == 1 path (quantization.py:241-263)."""
    H = h.shape[-1]
    e = idx[0]
    h0 = h[0]
    w_gu = dequantize(gu_p[e], gu_s[e], G).to(h0.dtype)
    gu = torch.mv(w_gu.view(-1, H), h0).view(e.shape[0], -1)
    gate, up = gu.chunk(2, dim=-1)
    inter = _gelu_tanh(gate) * up
    w_dn = dequantize(dn_p[e], dn_s[e], G).to(inter.dtype)
    out = torch.bmm(w_dn, inter.unsqueeze(-1)).squeeze(-1)
    weights = w[0, :, None].to(out.dtype)
    return (out * weights).sum(dim=0, keepdim=True).to(h.dtype)


def experts_loop(h: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, gu_p, gu_s, dn_p, dn_s,
                 G: int) -> torch.Tensor:
    """The T > 1 path (quantization.py:265-294)."""
    E = gu_p.shape[0]
    final = torch.zeros_like(h)
    with torch.no_grad():
        mask = F.one_hot(idx, num_classes=E + 1).permute(2, 1, 0)
        hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for ex in hit:
        ex = ex[0]
        if ex == E:
            continue
        kpos, tok = torch.where(mask[ex])
        cur = h[tok]
        w_gu = dequantize(gu_p[ex], gu_s[ex], G).to(cur.dtype)
        gate, up = F.linear(cur, w_gu).chunk(2, dim=-1)
        a = _gelu_tanh(gate) * up
        w_dn = dequantize(dn_p[ex], dn_s[ex], G).to(cur.dtype)
        a = F.linear(a, w_dn)
        a = a * w[tok, kpos, None]
        final.index_add_(0, tok, a.to(final.dtype))
    return final


def experts(h, idx, w, gu_p, gu_s, dn_p, dn_s, G):
    """Gemma4TextExperts4Bit.forward on CPU tensors (quantization.py:237-294)."""
    if h.shape[0] == 1:
        return experts_single(h, idx, w, gu_p, gu_s, dn_p, dn_s, G)
    return experts_loop(h, idx, w, gu_p, gu_s, dn_p, dn_s, G)


def router(h: torch.Tensor, scale: torch.Tensor, scalar_root: float, proj_w: torch.Tensor,
           per_expert_scale: torch.Tensor, eps: float, top_k: int):
    """(top_k_weights fp32, top_k_index int64, logits bf16) of backends.py:111-117."""
    D = h.shape[-1]
    hf = h.reshape(-1, D)
    r = F.rms_norm(hf, (D,), None, eps) * scale * scalar_root
    scores = F.linear(r, proj_w)
    probs = F.softmax(scores, dim=-1, dtype=torch.float32)
    tw, ti = torch.topk(probs, k=top_k, dim=-1)
    tw = tw / tw.sum(dim=-1, keepdim=True)
    tw = tw * per_expert_scale[ti]
    return tw, ti, scores


def ffn_block(residual, attn_out, post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w,
              post_ff_ln1_w, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale,
              pre_ff_ln2_w, gu_packed, gu_scale, dn_packed, dn_scale, post_ff_ln2_w, post_ff_ln_w,
              layer_scalar, eps, top_k, G):
    """_ffn_moe_4bit_step (backends.py:101-126) in eager torch CPU ops, the 4-bit
    experts on the reference CPU path (``experts`` above)."""
    D = residual.shape[-1]
    h = F.rms_norm(attn_out, (D,), post_attn_ln_w, eps)
    residual = residual + h
    h_ff = F.rms_norm(residual, (D,), pre_ff_ln_w, eps)
    gate = F.gelu(F.linear(h_ff, mlp_gate_w), approximate="tanh")
    up = F.linear(h_ff, mlp_up_w)
    h_mlp = F.linear(gate * up, mlp_down_w)
    h_1 = F.rms_norm(h_mlp, (D,), post_ff_ln1_w, eps)
    h_flat = residual.reshape(-1, D)
    tw, ti, _ = router(h_flat, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale, eps,
                       top_k)
    h_2_in = F.rms_norm(h_flat, (D,), pre_ff_ln2_w, eps)
    h_2 = experts(h_2_in, ti, tw, gu_packed, gu_scale, dn_packed, dn_scale, G).reshape(residual.shape)
    h_2 = F.rms_norm(h_2, (D,), post_ff_ln2_w, eps)
    h_comb = F.rms_norm(h_1 + h_2, (D,), post_ff_ln_w, eps)
    return (residual + h_comb) * layer_scalar


def bf16_experts(h: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, gate_up_proj: torch.Tensor,
                 down_proj: torch.Tensor) -> torch.Tensor:
    """_bf16_experts_fast_forward (backends.py:209-283) on CPU tensors: the
    T == 1 branch (index_select, mv, bmm), the T <= 8 branch (einsum) and the
    per-expert loop (F.linear, bf16 index_add_) above that."""
    T = h.shape[0]
    H = h.shape[-1]
    E, two_i, _ = gate_up_proj.shape
    if T == 1:
        e = idx[0]
        gu = torch.mv(gate_up_proj.index_select(0, e).view(-1, H), h[0]).view(e.shape[0], two_i)
        gate, up = gu.chunk(2, dim=-1)
        inter = _gelu_tanh(gate) * up
        out = torch.bmm(down_proj.index_select(0, e), inter.unsqueeze(-1)).squeeze(-1)
        return (out * w[0, :, None].to(out.dtype)).sum(dim=0, keepdim=True).to(h.dtype)
    if T <= 8:
        B, K = idx.shape
        flat = idx.reshape(-1)
        gu = torch.einsum("bkih,bh->bki", gate_up_proj.index_select(0, flat).view(B, K, two_i, H), h)
        gate, up = gu.chunk(2, dim=-1)
        inter = _gelu_tanh(gate) * up
        out = torch.einsum("bkhi,bki->bkh", down_proj.index_select(0, flat).view(B, K, H, two_i // 2), inter)
        return (out * w.unsqueeze(-1).to(out.dtype)).sum(dim=1).to(h.dtype)
    final = torch.zeros_like(h)
    with torch.no_grad():
        mask = F.one_hot(idx, num_classes=E + 1).permute(2, 1, 0)
        hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for ex in hit:
        ex = ex[0]
        if ex == E:
            continue
        kpos, tok = torch.where(mask[ex])
        gate, up = F.linear(h[tok], gate_up_proj[ex]).chunk(2, dim=-1)
        a = F.linear(_gelu_tanh(gate) * up, down_proj[ex]) * w[tok, kpos, None]
        final.index_add_(0, tok, a.to(final.dtype))
    return final
