"""Writes tests/golden/w4a16_golden.npz: small seeded inputs and the oracle's
outputs for every function of the W4A16 MoE path.

The reference ships no golden vectors for this path, so these fixtures come
from the oracle (oracle/w4a16_oracle.py), itself pinned by the known-answer,
brute-force and library checks of tests/test_oracle.py.  They anchor later
changes: tests/test_golden.py regenerates them on the CPU (bit-exact) and runs
the HIP library against them on the GPU.

    python tests/golden/make_golden.py      # rewrites the .npz
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "w4a16_golden.npz"


def _bf16_bits(a):
    return oracle.to_bf16_bits(np.asarray(a, np.float32))


def _rand_bf16(rng, shape, scale=1.0):
    return oracle.bf16_round(rng.standard_normal(shape).astype(np.float32) * scale)


def _packed(rng, rows, K):
    q = rng.integers(-8, 8, size=(rows, K))
    return oracle.pack_int4(q)


def _scales(rng, rows, K, G):
    return oracle.bf16_round(rng.uniform(0.005, 0.02, size=(rows, oracle.num_groups(K, G))).astype(np.float32))


def build() -> dict:
    rng = np.random.default_rng(20261201)
    g = {}
    # dequantize_int4_packed (quantization.py:132-137), G = 128 with a partial group
    K, G = 320, 128
    p = _packed(rng, 8, K)
    s = _scales(rng, 8, K, G)
    g["dq_packed"], g["dq_scale_bits"], g["dq_G"] = p, _bf16_bits(s), np.int64(G)
    g["dq_out_bits"] = _bf16_bits(oracle.dequantize(p, _bf16_bits(s), G))

    # Linear4Bit.forward (quantization.py:171-175)
    K, N, G = 256, 48, 64
    x = _rand_bf16(rng, (4, K))
    p = _packed(rng, N, K)
    s = _scales(rng, N, K, G)
    g["lin_x_bits"], g["lin_packed"], g["lin_scale_bits"], g["lin_G"] = _bf16_bits(x), p, _bf16_bits(s), np.int64(G)
    g["lin_y_bits"] = _bf16_bits(oracle.linear(x, p, _bf16_bits(s), G))

    # router (backends.py:111-117)
    M, H, E, k = 6, 256, 16, 4
    h = _rand_bf16(rng, (M, H))
    sc = oracle.bf16_round(1 + 0.05 * rng.standard_normal(H).astype(np.float32))
    proj = _rand_bf16(rng, (E, H), 0.02)
    pes = oracle.bf16_round(1 + 0.05 * rng.standard_normal(E).astype(np.float32))
    root, eps = np.float32(H ** -0.5), np.float32(1e-6)
    lg, idx, w = oracle.router(h, sc, float(root), proj, pes, float(eps), k)
    g.update(rt_h_bits=_bf16_bits(h), rt_scale_bits=_bf16_bits(sc), rt_proj_bits=_bf16_bits(proj),
             rt_pes_bits=_bf16_bits(pes), rt_root=root, rt_eps=eps, rt_k=np.int64(k),
             rt_logits_bits=_bf16_bits(lg), rt_idx=idx, rt_w=w)

    # token -> expert grouping (quantization.py:266-276), with "no expert" slots
    M, k, E = 10, 4, 16
    idx = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int64)
    idx[::3, 3] = E
    sp, off = oracle.sort_permute(idx, E)
    g.update(srt_idx=idx, srt_E=np.int64(E), srt_sorted_pos=np.asarray(sp, np.int32),
             srt_offsets=np.asarray(off, np.int32))

    # MoE layer (quantization.py:88-129): I = 64 < G = 128 (one partial group)
    M, H, I, E, k, G = 5, 128, 64, 8, 3, 128
    x = _rand_bf16(rng, (M, H))
    idx = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int64)
    w = rng.uniform(0.05, 1.0, size=(M, k)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    gu_p = np.stack([_packed(rng, 2 * I, H) for _ in range(E)])
    gu_s = np.stack([_scales(rng, 2 * I, H, G) for _ in range(E)])
    dn_p = np.stack([_packed(rng, H, I) for _ in range(E)])
    dn_s = np.stack([_scales(rng, H, I, G) for _ in range(E)])
    y = oracle.moe_forward(x, idx, w, gu_p, _bf16_bits(gu_s), dn_p, _bf16_bits(dn_s), G)
    g.update(moe_x_bits=_bf16_bits(x), moe_idx=idx, moe_w=w, moe_gu_packed=gu_p, moe_gu_scale_bits=_bf16_bits(gu_s),
             moe_dn_packed=dn_p, moe_dn_scale_bits=_bf16_bits(dn_s), moe_G=np.int64(G), moe_y_bits=_bf16_bits(y))
    return g


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
