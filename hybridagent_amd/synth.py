"""Seeded synthetic inputs in the compressed-tensors W4A16 layout.

Generates the value distributions the benchmark configurations name:
activations ~N(0,1) bf16, int4 weights uniform in [-8, 7] packed 8 per int32
along K (nibble i of word j = q[8j+i] + 8, ``quantization.py:136``), bf16 group
scales ~U(0.005, 0.02), router weights ~N(0, 0.02).  Uniform q makes every
nibble uniform on [0, 15], so a packed word is a uniform random 32-bit integer.

Works on any torch device; GPU generation keeps multi-GB weight sets fast.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


def num_groups(K: int, G: int) -> int:
    return -(-K // G)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def packed_int4(shape_nk, seed: int, device="cpu") -> torch.Tensor:
    """int32 [..., N, K/8] of uniform random words (= uniform q in [-8,7])."""
    *lead, N, K = shape_nk
    g = _gen(seed, device)
    return torch.randint(-(2 ** 31), 2 ** 31, (*lead, N, K // 8), generator=g,
                         dtype=torch.int64, device=device).to(torch.int32)


def group_scales(shape_nk, G: int, seed: int, device="cpu", lo=0.005, hi=0.02,
                 dtype=torch.bfloat16) -> torch.Tensor:
    *lead, N, K = shape_nk
    g = _gen(seed, device)
    s = torch.rand((*lead, N, num_groups(K, G)), generator=g, device=device, dtype=torch.float32)
    return (lo + (hi - lo) * s).to(dtype)


def activations(M: int, K: int, seed: int, device="cpu") -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randn((M, K), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)


@dataclass
class MoEWeights:
    gate_up_packed: torch.Tensor   # int32 [E, 2I, H/8]
    gate_up_scale: torch.Tensor    # bf16  [E, 2I, ceil(H/G)]
    down_packed: torch.Tensor      # int32 [E, H, I/8]
    down_scale: torch.Tensor       # bf16  [E, H, ceil(I/G)]
    group_size: int


def moe_weights(E: int, H: int, I: int, G: int, seed: int, device="cpu") -> MoEWeights:
    return MoEWeights(
        gate_up_packed=packed_int4((E, 2 * I, H), seed + 1, device),
        gate_up_scale=group_scales((E, 2 * I, H), G, seed + 2, device),
        down_packed=packed_int4((E, H, I), seed + 3, device),
        down_scale=group_scales((E, H, I), G, seed + 4, device),
        group_size=G,
    )


@dataclass
class RouterWeights:
    proj: torch.Tensor              # bf16 [E, H]
    scale: torch.Tensor             # bf16 [H]  (HF init: ones)
    per_expert_scale: torch.Tensor  # bf16 [E] (HF init: ones)
    scalar_root: float              # H ** -0.5
    eps: float = 1e-6


def router_weights(E: int, H: int, seed: int, device="cpu", std=0.02) -> RouterWeights:
    g = _gen(seed, device)
    proj = (std * torch.randn((E, H), generator=g, device=device)).to(torch.bfloat16)
    return RouterWeights(
        proj=proj,
        scale=torch.ones(H, dtype=torch.bfloat16, device=device),
        per_expert_scale=torch.ones(E, dtype=torch.bfloat16, device=device),
        scalar_root=H ** -0.5,
    )


ZIPF_C = 8.0


def zipf_router_weights(E: int, H: int, seed: int, s: float = 1.1, beta: float = 1.0,
                        n_empty: int = 8, noise_std: float = 1.0, device="cpu"):
    """Router whose expert load is Zipf(s)-skewed, with ``n_empty`` experts never chosen.

    The skew is built into the router itself.  Hidden coordinate 0 of every
    token is the constant ``ZIPF_C`` (see ``zipf_activations``); after the
    router's RMSNorm and ``scalar_root = H^-0.5`` it reaches the projection as
    ``r0 ~= ZIPF_C * H^-0.5``, so ``W_r[e, 0] = beta * log p_e / r0`` adds the
    bias ``beta * log p_e`` to expert e's logit, with p ∝ rank^-s over a seeded
    permutation of the experts.  The other columns are N(0, noise_std): the
    normalised router input has unit norm, so each logit gets N(0, noise_std)
    per-token noise and the top-k draw spreads load along the Zipf profile
    instead of picking the same k experts for every token.
    """
    g = _gen(seed, "cpu")
    proj = noise_std * torch.randn((E, H), generator=g)
    perm = torch.randperm(E, generator=g)
    ranks = torch.empty(E)
    ranks[perm] = torch.arange(1, E + 1, dtype=torch.float32)
    logp = -s * torch.log(ranks)
    bias = beta * logp
    if n_empty > 0:
        bias[perm[E - n_empty:]] = -1000.0
    r0 = ZIPF_C * H ** -0.5
    proj[:, 0] = bias / r0
    return RouterWeights(
        proj=proj.to(torch.bfloat16).to(device),
        scale=torch.ones(H, dtype=torch.bfloat16, device=device),
        per_expert_scale=torch.ones(E, dtype=torch.bfloat16, device=device),
        scalar_root=H ** -0.5,
    )


def zipf_activations(M: int, H: int, seed: int, device="cpu") -> torch.Tensor:
    """x ~ N(0,1) with x[:, 0] = ZIPF_C, the routing-bias coordinate of ``zipf_router_weights``."""
    x = activations(M, H, seed, device).float()
    x[:, 0] = ZIPF_C
    return x.to(torch.bfloat16)
