"""GPU: every kernel instantiation of the library reached and checked.

The dispatchers pick a compiled kernel form from the shape (k tiles per
wavefront and K split from K, wide scale loads from the group count, the
long-K loop above 24 k tiles, top-k forms from the expert count and the
router's K splits, the BF16 experts' row chunk from the rows per expert).
The shape tests elsewhere use the Gemma shape and a few small ones; the cases
here reach the remaining forms, each named after the kernel it runs, against
the numpy oracle (max_abs_rel <= 1e-2; routing bit-exact against the kernel's
own logits).  A kernel trace of the GPU test run (rocprofv3 --kernel-trace)
lists every kernel the library compiles.
"""
import numpy as np
import pytest
import torch

import oracle
from checks import margin
from hybridagent_amd import _lib, synth

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def dev():
    assert _lib.available(), "libw4a16moe.so must be built"
    return torch.device("cuda:0")


# ------------------------------------------------------------------ dense
# (K, G) -> k_decode<0, TPW, KSPLIT, LONGK, WIDE>: TPW / KSPLIT from the k
# tiles of 128 (<= 2: 2/1, <= 4: 4/1, <= 6: 6/1, <= 8: 2/4, <= 16: 4/4,
# <= 24: 6/4, more: the long-K loop), WIDE with an even group count at G = 128
@pytest.mark.parametrize("K,G", [
    (256, 128),    # <0, 2, 1, wide>
    (1024, 128),   # <0, 2, 4, wide>
    (512, 32),     # <0, 4, 1>
    (2048, 64),    # <0, 4, 4>
    (2048, 128),   # <0, 4, 4, wide>
    (768, 32),     # <0, 6, 1>
    (2816, 32),    # <0, 6, 4>
    (4096, 128),   # <0, 6, 4, long K>
])
def test_dense_linear_shape_forms(dev, K, G):
    M, N = 4, 80
    x = synth.activations(M, K, seed=3000 + K)
    p = synth.packed_int4((N, K), seed=3001 + K)
    s = synth.group_scales((N, K), G, seed=3002 + K)
    y = _lib.linear(x.to(dev), p.to(dev), s.to(dev), group_size=G)
    ref = oracle.linear(_np(x), p.numpy(), _bits(s), G)
    assert margin(f"dense K={K} G={G} M={M}", oracle.max_abs_rel(_np(y), ref)) <= TOL


# ------------------------------------------------------------------ MoE decode
def _moe_case(dev, E, Hh, Ii, G, M, k, seed, tiled):
    wts = synth.moe_weights(E, Hh, Ii, G, seed=seed)
    gpu = [t.to(dev) for t in (wts.gate_up_packed, wts.gate_up_scale, wts.down_packed, wts.down_scale)]
    x = synth.activations(M, Hh, seed=seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)])
    w = torch.rand(M, k, generator=g).float() + 0.05
    w = w / w.sum(1, keepdim=True)
    tiles = _lib.tile_experts(*gpu, group_size=G, prefill=False) if tiled else None
    y = _lib.moe_forward(x.to(dev), idx.to(dev), w.to(dev), *gpu, group_size=G, tiles=tiles)
    ref = oracle.moe_forward(_np(x), idx.numpy(), w.numpy(), wts.gate_up_packed.numpy(), _bits(wts.gate_up_scale),
                             wts.down_packed.numpy(), _bits(wts.down_scale), G)
    return oracle.max_abs_rel(_np(y), ref)


# H = 768: gate_up k_decode<1, 6, 1, ...> (six k tiles, no K split), packed
# wide, tiled (group size 128) and tiled with the copy's lane scales (32)
@pytest.mark.parametrize("G,tiled", [(128, False), (128, True), (32, True)])
def test_moe_gate_up_six_tiles(dev, G, tiled):
    err = _moe_case(dev, 16, 768, 128, G, M=3, k=4, seed=3100 + G, tiled=tiled)
    assert margin(f"moe H=768 I=128 G={G}{' (tiled)' if tiled else ''}", err) <= TOL


# H = 4096: the gate_up streamer's long-K loop, k_decode<1, 6, 4, long K>
def test_moe_gate_up_long_k(dev):
    err = _moe_case(dev, 8, 4096, 64, 128, M=2, k=2, seed=3200, tiled=False)
    assert margin("moe H=4096 I=64 G=128 (long K)", err) <= TOL


# I above 768: the down streamer with a 4-way K split, k_decode<2, TPW, 4>
# (I = 1024: 2 tiles per wavefront, 2048: 4, 2816: 6), packed (G = 32 and
# wide at 128) and on the tiled copies (128, and 32 with lane scales); I =
# 4096 the down streamer's long-K loop
@pytest.mark.parametrize("Ii", [1024, 2048, 2816])
@pytest.mark.parametrize("G,tiled", [(32, False), (128, False), (128, True), (32, True)])
def test_moe_down_k_split(dev, Ii, G, tiled):
    err = _moe_case(dev, 8, 256, Ii, G, M=2, k=2, seed=3300 + Ii + G, tiled=tiled)
    assert margin(f"moe H=256 I={Ii} G={G}{' (tiled)' if tiled else ''}", err) <= TOL


def test_moe_down_long_k(dev):
    err = _moe_case(dev, 8, 256, 4096, 128, M=2, k=2, seed=3400, tiled=False)
    assert margin("moe H=256 I=4096 G=128 (long K)", err) <= TOL


# top_k above 8: the combine's any-k form, k_combine<0> (80 routed rows, past
# the fused down + combine)
def test_moe_top_k_ten(dev):
    err = _moe_case(dev, 32, 256, 128, 128, M=8, k=10, seed=3500, tiled=False)
    assert margin("moe top_k=10 M=8", err) <= TOL


# ------------------------------------------------------------------ BF16 experts
# more than 32 rows per expert on average: 64-row chunks, k_bf16_expert<*, 4, *>
def test_bf16_experts_64_row_chunks(dev):
    E, Hh, Ii, M, k = 8, 256, 128, 256, 2
    g = torch.Generator().manual_seed(3600)
    gu = (torch.randn(E, 2 * Ii, Hh, generator=g) / 16).to(torch.bfloat16)
    dn = (torch.randn(E, Hh, Ii, generator=g) / 11).to(torch.bfloat16)
    x = synth.activations(M, Hh, seed=3601)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)])
    w = torch.rand(M, k, generator=g).float() + 0.05
    y = _lib.bf16_experts_forward(x.to(dev), idx.to(dev), w.to(dev), gu.to(dev), dn.to(dev))
    ref = oracle.moe_forward_bf16(_np(x), idx.numpy(), w.numpy(), _np(gu), _np(dn))
    assert margin(f"bf16 experts M={M} E={E} (64-row chunks)", oracle.max_abs_rel(_np(y), ref)) <= TOL


# ------------------------------------------------------------------ routing
def _router(E, Hh, seed):
    rw = synth.router_weights(E, Hh, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    rw.scale = (1 + 0.05 * torch.randn(Hh, generator=g)).to(torch.bfloat16)
    rw.per_expert_scale = (1 + 0.05 * torch.randn(E, generator=g)).to(torch.bfloat16)
    return rw


# finished logits with more than 128 experts: k_router_topk<0, 4 / 8>
@pytest.mark.parametrize("E", [256, 512])
def test_topk_from_logits_many_experts(dev, E):
    M, k = 50, 8
    g = torch.Generator().manual_seed(3700 + E)
    lg = torch.randn(M, E, generator=g).to(torch.bfloat16)
    pes = (1 + 0.05 * torch.randn(E, generator=g)).to(torch.bfloat16)
    w, idx = _lib.topk_from_logits(lg.to(dev), pes.to(dev), k)
    ridx, rw_ = oracle.topk_from_logits(_np(lg), _np(pes), k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw_, rtol=2e-6, atol=1e-7)


# large batches: the router's K splits from the workgroup count (128 tokens x
# 128 experts each: >= 64 -> 4 splits, >= 32 -> 8), k_router_topk<4 / 8, PER>
# with PER = 1 (E = 64), 4 (256), 8 (512)
@pytest.mark.parametrize("M,E", [(4000, 64), (8200, 64), (2000, 256), (4000, 256), (1000, 512), (2000, 512)])
def test_router_large_batch_expert_counts(dev, M, E):
    Hh, k = 512, 8
    rw = _router(E, Hh, seed=3800 + E)
    h = synth.activations(M, Hh, seed=3801 + M)
    w, idx, lg = _lib.router_topk(h.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev),
                                  rw.per_expert_scale.to(dev), rw.eps, k, return_logits=True)
    ref_lg = oracle.router_logits(_np(h), _np(rw.scale), rw.scalar_root, _np(rw.proj), rw.eps)
    got_lg = _np(lg)
    scale = np.abs(ref_lg).max()
    assert np.abs(got_lg - ref_lg).max() <= 2.0 ** -8 * scale
    idx2, w2 = oracle.topk_from_logits(got_lg, _np(rw.per_expert_scale), k)
    assert np.array_equal(idx.cpu().numpy(), idx2)
    np.testing.assert_allclose(w.cpu().numpy(), w2, rtol=2e-6, atol=1e-7)


# router + experts in one call with at most 64 routed rows: top-k and sort in
# one workgroup, k_router_topk_sort_small<16, PER, ROUNDS>; PER from the
# expert count (64: 1, 128: 2, 256: 4, 512: 8), ROUNDS 1 up to 8 tokens, 8
# above
@pytest.mark.parametrize("E,M,k", [(64, 16, 4), (128, 16, 4), (256, 1, 8), (256, 16, 4), (512, 1, 8),
                                   (512, 16, 4)])
def test_layer_forward_small_sort_forms(dev, E, M, k):
    Hh, Ii, G = 256, 64, 128
    rw = _router(E, Hh, seed=3900 + E + M)
    wts = synth.moe_weights(E, Hh, Ii, G, seed=3901 + E)
    gpu = [t.to(dev) for t in (wts.gate_up_packed, wts.gate_up_scale, wts.down_packed, wts.down_scale)]
    h = synth.activations(M, Hh, seed=3902 + M)
    x = synth.activations(M, Hh, seed=3903 + M)
    args = (h.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev), rw.per_expert_scale.to(dev), rw.eps, k)
    y, w, idx = _lib.moe_layer_forward(*args, x.to(dev), *gpu, group_size=G)
    w2, idx2, lg = _lib.router_topk(*args, return_logits=True)
    assert torch.equal(idx.cpu(), idx2.cpu()) and torch.equal(w.cpu(), w2.cpu())
    ridx, rw_ = oracle.topk_from_logits(_np(lg), _np(rw.per_expert_scale), k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    ref = oracle.moe_forward(_np(x), idx.cpu().numpy(), w.cpu().numpy(), wts.gate_up_packed.numpy(),
                             _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), G)
    assert margin(f"router+experts E={E} M={M} k={k}", oracle.max_abs_rel(_np(y), ref)) <= TOL
