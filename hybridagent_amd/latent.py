"""Latent-mode MoE stack (benchmark configs[4]): the decode step of the
HybridAgent latent loop reduced to its MoE layers.

Each layer: ``h <- h + MoE(RMSNorm(h))``, the router reading the residual
``h`` as in backends.py:111-122 (attention replaced by the identity, the
shared MLP and post-FFN norms left out, as the config states).  After the
last layer the HybridLink map R(h) = LN(h + proj2(GELU(proj1(LN(h)))))
(hybridlink.py:17-28) scaled by sqrt(hidden) gives the next step's input.

The MoE layers run through the HIP library (router + experts in one C-ABI
call per layer), and so do the residual add and RMSNorm in front of each
(inside the previous layer's combine launch, moe_layer_forward_add_norm; in
front of the first layer one w4a16_add_rms_norm launch), and so does the
HybridLink map
(w4a16_hybridlink: two LayerNorm launches and two bf16 weight-streaming
linear launches with the bias, GELU and residual fused).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib, synth


@dataclass
class _Layer:
    router: synth.RouterWeights
    experts: synth.MoEWeights
    pre_norm: torch.Tensor  # RMSNorm weight of the MoE input (bf16 [H])
    tiles: _lib.TiledWeights | None = None  # the decode streamers' tiled weight copies


class LatentStack:
    def __init__(self, n_layers: int, E: int, H: int, I: int, top_k: int, group_size: int, seed: int,
                 device, eps: float = 1e-6, tiled: bool = True):
        self.H, self.top_k, self.G, self.eps = H, top_k, group_size, eps
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)
        self.layers = []
        for i in range(n_layers):
            rw = synth.router_weights(E, H, seed=seed + 31 * i, device=dev)
            ew = synth.moe_weights(E, H, I, group_size, seed=seed + 31 * i + 7, device=dev)
            pre = (1.0 + 0.05 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
            ly = _Layer(rw, ew, pre)
            if tiled and dev.type == "cuda":
                ly.tiles = _lib.tile_experts(ew.gate_up_packed, ew.gate_up_scale, ew.down_packed, ew.down_scale,
                                             group_size, decode=True, prefill=False)
            self.layers.append(ly)
        std = 1.0 / math.sqrt(H)
        mk = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g, device=dev)).to(torch.bfloat16)
        self.hl = {
            "ln1w": (1.0 + 0.05 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16),
            "ln1b": mk(H, sc=0.02),
            "p1w": mk(H, H, sc=std), "p1b": mk(H, sc=0.02),
            "p2w": mk(H, H, sc=std), "p2b": mk(H, sc=0.02),
            "ln2w": (1.0 + 0.05 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16),
            "ln2b": mk(H, sc=0.02),
        }

    def rms_norm(self, h: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """fp32 x * rsqrt(mean(x^2) + eps) * w, back to bf16 (TF:modeling_gemma4.py:197-215)."""
        return _lib.add_rms_norm(h, w, self.eps)[1]

    def moe(self, h: torch.Tensor, i: int):
        """MoE block of layer i on residual h -> (out, top_k_index, top_k_weights)."""
        return self.moe_on(h, self.rms_norm(h, self.layers[i].pre_norm), i)

    def moe_on(self, h: torch.Tensor, xin: torch.Tensor, i: int):
        """MoE block of layer i: router on the residual h, experts on xin = RMSNorm(h)."""
        ly = self.layers[i]
        rw, ew = ly.router, ly.experts
        out, w, idx = _lib.moe_layer_forward(h, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale,
                                             rw.eps, self.top_k, xin, ew.gate_up_packed, ew.gate_up_scale,
                                             ew.down_packed, ew.down_scale, group_size=self.G, tiles=ly.tiles)
        return out, idx, w

    def layer(self, h: torch.Tensor, i: int):
        """One MoE layer; returns (new h, top_k_index, top_k_weights)."""
        out, idx, w = self.moe(h, i)
        return h + out, idx, w

    def hybridlink(self, h: torch.Tensor) -> torch.Tensor:
        p = self.hl
        return _lib.hybridlink(h, p["ln1w"], p["ln1b"], p["p1w"], p["p1b"], p["p2w"], p["p2b"],
                               p["ln2w"], p["ln2b"])

    def step(self, h: torch.Tensor) -> torch.Tensor:
        """One latent step: all MoE layers, then HybridLink x sqrt(H).  The same
        arithmetic as calling layer() in turn: layer i's output is added to the
        residual, and layer i + 1's input normalised, inside layer i's combine
        launch (moe_layer_forward_add_norm)."""
        n = len(self.layers)
        if n == 0:
            return self.hybridlink(h) * math.sqrt(self.H)
        h, xin = _lib.add_rms_norm(h, self.layers[0].pre_norm, self.eps)
        for i in range(n - 1):
            h, xin = self.moe_add_norm(h, xin, i, self.layers[i + 1].pre_norm)
        out, _, _ = self.moe_on(h, xin, n - 1)
        return self.hybridlink(h + out) * math.sqrt(self.H)

    def moe_add_norm(self, h: torch.Tensor, xin: torch.Tensor, i: int, next_norm: torch.Tensor):
        """Layer i on (h, xin = RMSNorm(h)), then h + out and its RMSNorm with next_norm."""
        ly = self.layers[i]
        rw, ew = ly.router, ly.experts
        h_out, y, _, _, _ = _lib.moe_layer_forward_add_norm(
            h, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, rw.eps, self.top_k, xin,
            ew.gate_up_packed, ew.gate_up_scale, ew.down_packed, ew.down_scale, next_norm, self.eps,
            group_size=self.G, tiles=ly.tiles)
        return h_out, y
