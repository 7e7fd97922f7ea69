"""GPU parity: the HIP kernels (through the C ABI) against the numpy oracle.

Bars: bit-exact for dequantised weights, routing indices (given identical
logits) and the token permutation; max_abs_rel <= 1e-2 for layer outputs
(``max|y - y_ref| / max|y_ref|``, the tolerance the north star states).
"""
import math

import numpy as np
import pytest
import torch

import oracle
from checks import bf16_ulp, check_bf16_close, check_routing_order, margin
from hybridagent_amd import _lib, synth

pytestmark = pytest.mark.gpu

TOL = 1e-2
E, H, I, K_TOP = 128, 2816, 704, 8


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def dev():
    assert _lib.available(), "libw4a16moe.so must be built"
    return torch.device("cuda:0")


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("N,K,G", [(64, 2816, 128), (48, 704, 128), (32, 704, 32), (16, 256, 64)])
def test_dequant_bit_exact(dev, N, K, G):
    p = synth.packed_int4((N, K), seed=1)
    s = synth.group_scales((N, K), G, seed=2)
    got = _lib.dequantize(p.to(dev), s.to(dev))
    torch.cuda.synchronize()
    ref = oracle.dequantize(p.numpy(), _bits(s), G)
    assert np.array_equal(_bits(got), oracle.to_bf16_bits(ref))


# ------------------------------------------------------------------ dense linear (config 1)

@pytest.mark.parametrize("M", [1, 4, 16, 64])
@pytest.mark.parametrize("K,N", [(2816, 2816), (2816, 1408), (704, 2816)])
def test_dense_linear_config1(dev, M, K, N):
    G = 128
    x = synth.activations(M, K, seed=10 + M)
    p = synth.packed_int4((N, K), seed=11)
    s = synth.group_scales((N, K), G, seed=12)
    y = _lib.linear(x.to(dev), p.to(dev), s.to(dev))
    ref = oracle.linear(_np(x), p.numpy(), _bits(s), G)
    assert margin(f"dense configs[1] K={K} N={N} M={M}", oracle.max_abs_rel(_np(y), ref)) <= TOL


@pytest.mark.parametrize("G", [32, 64, 256])
def test_dense_linear_other_groups_and_bias(dev, G):
    M, K, N = 5, 1024, 96
    x = synth.activations(M, K, seed=20)
    p = synth.packed_int4((N, K), seed=21)
    s = synth.group_scales((N, K), G, seed=22)
    b = synth.activations(1, N, seed=23)[0]
    y = _lib.linear(x.to(dev), p.to(dev), s.to(dev), b.to(dev), group_size=G)
    ref = oracle.linear(_np(x), p.numpy(), _bits(s), G, bias=_np(b))
    assert oracle.max_abs_rel(_np(y), ref) <= TOL


def test_dense_linear_many_rows(dev):
    # M > 64 exercises the row-chunk loop
    M, K, N, G = 150, 512, 80, 128
    x = synth.activations(M, K, seed=30)
    p = synth.packed_int4((N, K), seed=31)
    s = synth.group_scales((N, K), G, seed=32)
    y = _lib.linear(x.to(dev), p.to(dev), s.to(dev))
    assert oracle.max_abs_rel(_np(y), oracle.linear(_np(x), p.numpy(), _bits(s), G)) <= TOL


# ------------------------------------------------------------------ router

def _router_inputs(M, seed):
    rw = synth.router_weights(E, H, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    rw.scale = (1 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16)
    rw.per_expert_scale = (1 + 0.05 * torch.randn(E, generator=g)).to(torch.bfloat16)
    h = synth.activations(M, H, seed=seed + 2)
    return h, rw


@pytest.mark.parametrize("M", [1, 8, 64, 300])
def test_topk_from_identical_logits_bit_exact(dev, M):
    h, rw = _router_inputs(M, seed=40)
    logits = oracle.router_logits(_np(h), _np(rw.scale), rw.scalar_root, _np(rw.proj), rw.eps)
    lt = torch.from_numpy(logits).to(torch.bfloat16)
    w, idx = _lib.topk_from_logits(lt.to(dev), rw.per_expert_scale.to(dev), K_TOP)
    ridx, rw_ = oracle.topk_from_logits(logits, _np(rw.per_expert_scale), K_TOP)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw_, rtol=2e-6, atol=1e-7)


def test_topk_tie_rule(dev):
    lg = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0, -1.0, 0.5, 3.0]], dtype=torch.bfloat16)
    w, idx = _lib.topk_from_logits(lg.to(dev), torch.ones(8, dtype=torch.bfloat16, device=dev), 5)
    assert idx.cpu().tolist() == [[1, 2, 4, 7, 3]]


# M > 64 runs the large-batch router (128 tokens per workgroup): 257 and
# 1000 with 16 K splits, 4096 with 8, 8193 with 4 and a ragged last block
@pytest.mark.parametrize("M", [1, 32, 257, 1000, 4096, 8193])
def test_router_end_to_end(dev, M):
    h, rw = _router_inputs(M, seed=50)
    w, idx, lg = _lib.router_topk(h.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev),
                                  rw.per_expert_scale.to(dev), rw.eps, K_TOP, return_logits=True)
    ref_lg, ref_idx, ref_w = oracle.router(_np(h), _np(rw.scale), rw.scalar_root, _np(rw.proj),
                                           _np(rw.per_expert_scale), rw.eps, K_TOP)
    got_lg = _np(lg)
    # fp32 reduction order (sum of squares, dot products) may move a logit by
    # one bf16 ulp; near zero an ulp is tiny, so bound those absolutely
    ulp = np.abs(oracle.to_bf16_bits(got_lg).astype(np.int32) - oracle.to_bf16_bits(ref_lg).astype(np.int32))
    scale = np.abs(ref_lg).max()
    big = np.abs(ref_lg) > 0.25 * scale
    assert ulp[big].max() <= 1 and (ulp > 0).mean() < 0.05
    assert np.abs(got_lg - ref_lg).max() <= 2.0 ** -8 * scale
    got_idx = idx.cpu().numpy()
    check_routing_order(got_lg, got_idx, ref_lg, ref_idx, K_TOP, f"router M={M}")
    # the kernel is bit-exact against its own logits
    idx2, w2 = oracle.topk_from_logits(got_lg, _np(rw.per_expert_scale), K_TOP)
    assert np.array_equal(got_idx, idx2)
    np.testing.assert_allclose(w.cpu().numpy(), w2, rtol=2e-6, atol=1e-7)


# other router shapes: expert counts that are not a multiple of 16 or that
# need several 128-expert groups, rows too long for the fused decode-size
# kernel (H > 3072: normalisation pass + K-split logits), and the
# large-batch kernels at those shapes
@pytest.mark.parametrize("M,Hr,Er", [(8, 4096, 200), (300, 4096, 200), (300, 1056, 64), (70, 2816, 512)])
def test_router_other_shapes(dev, M, Hr, Er):
    rw = synth.router_weights(Er, Hr, seed=60 + Er)
    g = torch.Generator().manual_seed(61 + Hr)
    rw.scale = (1 + 0.05 * torch.randn(Hr, generator=g)).to(torch.bfloat16)
    rw.per_expert_scale = (1 + 0.05 * torch.randn(Er, generator=g)).to(torch.bfloat16)
    h = synth.activations(M, Hr, seed=62 + M)
    w, idx, lg = _lib.router_topk(h.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev),
                                  rw.per_expert_scale.to(dev), rw.eps, K_TOP, return_logits=True)
    ref_lg = oracle.router_logits(_np(h), _np(rw.scale), rw.scalar_root, _np(rw.proj), rw.eps)
    got_lg = _np(lg)
    ulp = np.abs(oracle.to_bf16_bits(got_lg).astype(np.int32) - oracle.to_bf16_bits(ref_lg).astype(np.int32))
    scale = np.abs(ref_lg).max()
    big = np.abs(ref_lg) > 0.25 * scale
    assert ulp[big].max() <= 1 and (ulp > 0).mean() < 0.05
    assert np.abs(got_lg - ref_lg).max() <= 2.0 ** -8 * scale
    # selection and weights are bit-exact against the kernel's own logits
    idx2, w2 = oracle.topk_from_logits(got_lg, _np(rw.per_expert_scale), K_TOP)
    assert np.array_equal(idx.cpu().numpy(), idx2)
    np.testing.assert_allclose(w.cpu().numpy(), w2, rtol=2e-6, atol=1e-7)


# ------------------------------------------------------------------ sort / permute

@pytest.mark.parametrize("M", [1, 8, 64, 777, 4096])
def test_sort_permute_bit_exact(dev, M):
    g = torch.Generator().manual_seed(60 + M)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP] for _ in range(M)])
    sp, off = _lib.sort_permute(idx.to(dev), E)
    ref_sp, ref_off = oracle.sort_permute(idx.numpy(), E)
    assert np.array_equal(off.cpu().numpy(), ref_off)
    assert np.array_equal(sp.cpu().numpy(), ref_sp)


def test_sort_permute_skewed_and_invalid(dev):
    # Zipf-skewed routing with empty experts, plus "no expert" slots (index E)
    rw = synth.zipf_router_weights(E, H, seed=70)
    x = synth.zipf_activations(2048, H, seed=71)
    lg = oracle.router_logits(_np(x), _np(rw.scale), rw.scalar_root, _np(rw.proj), rw.eps)
    idx, _ = oracle.topk_from_logits(lg, _np(rw.per_expert_scale), K_TOP)
    idx[::7, 3] = E
    sp, off = _lib.sort_permute(torch.from_numpy(idx).to(dev), E)
    flat = idx.T.reshape(-1)
    keep = flat < E
    order = np.argsort(np.where(keep, flat, E), kind="stable")[: keep.sum()]
    M = idx.shape[0]
    ref_sp = ((order % M) * K_TOP + order // M).astype(np.int32)
    n = int(keep.sum())
    assert off.cpu().numpy()[-1] == n
    assert np.array_equal(sp.cpu().numpy()[:n], ref_sp)
    assert (np.diff(off.cpu().numpy()) == 0).sum() >= 8


# ------------------------------------------------------------------ MoE layer

@pytest.fixture(scope="module")
def moe128(dev):
    wts = synth.moe_weights(E, H, I, 128, seed=100)
    gpu = {k: getattr(wts, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")}
    cpu = {k: getattr(wts, k) for k in gpu}
    return cpu, gpu


def _route(M, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP] for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    return idx, (w / w.sum(1, keepdim=True)).float()


# dequantised expert weights per weight set, made once: the oracle's MoE
# forward on them (moe_forward_bf16, bit-equal to moe_forward on the packed
# weights; moe_forward_fp32_dequantized) then costs only the matmuls
_DEQ = {}


def _deq(cpu, G, fp32=False):
    key = (id(cpu), G, fp32)
    if key not in _DEQ:
        f = oracle.dequantize_fp32 if fp32 else oracle.dequantize
        _DEQ[key] = (f(cpu["gate_up_packed"].numpy(), _bits(cpu["gate_up_scale"]), G),
                     f(cpu["down_packed"].numpy(), _bits(cpu["down_scale"]), G))
    return _DEQ[key]


def _moe_ref(x, idx, w, cpu, G, rows=None, path="fused"):
    rows = np.arange(x.shape[0]) if rows is None else rows
    gu, dn = _deq(cpu, G)
    return oracle.moe_forward_bf16(_np(x)[rows], idx.numpy()[rows], w.numpy()[rows], gu, dn, path=path)


def _moe_ref_fp32(x, idx, w, cpu, G):
    gu, dn = _deq(cpu, G, fp32=True)
    return oracle.moe_forward_fp32_dequantized(_np(x), idx.numpy(), w.numpy(), gu, dn)


def _moe_gpu(x, idx, w, gpu, dev):
    return _lib.moe_forward(x.to(dev), idx.to(dev), w.to(dev), gpu["gate_up_packed"], gpu["gate_up_scale"],
                            gpu["down_packed"], gpu["down_scale"])


@pytest.mark.parametrize("M", [1, 8, 32, 64])
def test_moe_decode_config2(dev, moe128, M):
    cpu, gpu = moe128
    x = synth.activations(M, H, seed=200 + M)
    idx, w = _route(M, seed=300 + M)
    y = _moe_gpu(x, idx, w, gpu, dev)
    ref = _moe_ref(x, idx, w, cpu, 128)
    assert margin(f"moe decode configs[2] G=128 M={M}", oracle.max_abs_rel(_np(y), ref)) <= TOL
    # distance to the unrounded fp32 arithmetic: the kernel's and the
    # reference rounding points' (reported; the bound is the same tolerance)
    ref32 = _moe_ref_fp32(x, idx, w, cpu, 128)
    margin(f"moe decode configs[2] G=128 M={M}", oracle.max_abs_rel(_np(y), ref32), measure="max_abs_rel vs fp32")
    margin(f"moe decode configs[2] G=128 M={M}", oracle.max_abs_rel(ref, ref32),
           measure="oracle bf16 vs fp32")


@pytest.fixture(scope="module")
def moe32(dev):
    # the released checkpoints' group size (quantization.py:19) at the Gemma
    # shape: 88 gate_up and 22 down scale groups per row
    wts = synth.moe_weights(E, H, I, 32, seed=150)
    gpu = {k: getattr(wts, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")}
    cpu = {k: getattr(wts, k) for k in gpu}
    return cpu, gpu


@pytest.mark.parametrize("M", [1, 8, 64, 4096])
def test_moe_g32_full_shape(dev, moe32, M):
    # decode sizes: the exact-form streamer; M = 4096: the exact-form prefill
    # GEMM with the Zipf-skewed routing of configs[3]
    cpu, gpu = moe32
    if M <= 64:
        x = synth.activations(M, H, seed=260 + M)
        idx, w = _route(M, seed=360 + M)
        rows = np.arange(M)
    else:
        x = synth.zipf_activations(M, H, seed=261)
        rw = synth.zipf_router_weights(E, H, seed=262)
        w_d, idx_d = _lib.router_topk(x.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev),
                                      rw.per_expert_scale.to(dev), rw.eps, K_TOP)
        idx, w = idx_d.cpu(), w_d.cpu()
        rows = np.arange(M)
    y = _moe_gpu(x, idx, w, gpu, dev)
    ref = _moe_ref(x, idx, w, cpu, 32, rows=rows)
    assert margin(f"moe G=32 full shape M={M} (all rows)", oracle.max_abs_rel(_np(y)[rows], ref)) <= TOL
    ref32 = _moe_ref_fp32(x, idx, w, cpu, 32)
    margin(f"moe G=32 full shape M={M} (all rows)", oracle.max_abs_rel(_np(y), ref32), measure="max_abs_rel vs fp32")
    margin(f"moe G=32 full shape M={M} (all rows)", oracle.max_abs_rel(ref, ref32), measure="oracle bf16 vs fp32")


def test_moe_matches_loop_path(dev, moe128):
    cpu, gpu = moe128
    M = 16
    x = synth.activations(M, H, seed=210)
    idx, w = _route(M, seed=310)
    y = _moe_gpu(x, idx, w, gpu, dev)
    assert margin("moe M=16 vs the per-expert loop path", oracle.max_abs_rel(
        _np(y), _moe_ref(x, idx, w, cpu, 128, path="loop"))) <= TOL


def test_moe_prefill_all_rows(dev, moe128):
    cpu, gpu = moe128
    M = 512
    x = synth.activations(M, H, seed=220)
    idx, w = _route(M, seed=320)
    y = _moe_gpu(x, idx, w, gpu, dev)
    assert margin(f"moe prefill uniform M={M} (all rows)", oracle.max_abs_rel(
        _np(y), _moe_ref(x, idx, w, cpu, 128))) <= TOL


def test_moe_invalid_slots_contribute_nothing(dev, moe128):
    cpu, gpu = moe128
    M = 6
    x = synth.activations(M, H, seed=230)
    idx, w = _route(M, seed=330)
    idx_bad = idx.clone()
    idx_bad[:, 5:] = E        # the reference's "no expert" index
    w_cut = w.clone()
    w_cut[:, 5:] = 0.0
    y_bad = _moe_gpu(x, idx_bad, w, gpu, dev)
    y_cut = _moe_gpu(x, idx, w_cut, gpu, dev)
    assert torch.equal(y_bad.cpu(), y_cut.cpu())


@pytest.mark.parametrize("G", [32, 64])
def test_moe_small_groups(dev, G):
    e, h, i = 16, 512, 192
    wts = synth.moe_weights(e, h, i, G, seed=400 + G)
    M = 24
    x = synth.activations(M, h, seed=401)
    g = torch.Generator().manual_seed(402)
    idx = torch.stack([torch.randperm(e, generator=g)[:4] for _ in range(M)])
    w = torch.rand(M, 4, generator=g).float()
    y = _lib.moe_forward(x.to(dev), idx.to(dev), w.to(dev), wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev),
                         wts.down_packed.to(dev), wts.down_scale.to(dev))
    ref = oracle.moe_forward(_np(x), idx.numpy(), w.numpy(), wts.gate_up_packed.numpy(), _bits(wts.gate_up_scale),
                             wts.down_packed.numpy(), _bits(wts.down_scale), G)
    assert margin(f"moe small shape G={G} M={M}", oracle.max_abs_rel(_np(y), ref)) <= TOL


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 9, 24, 64, 100])
def test_layer_forward_router_plus_experts(dev, moe128, M):
    # router + experts in one call: routing equals the standalone router's,
    # output equals moe_forward on that routing and the oracle within tolerance
    # (M = 1: the gate_up launch routes; 2 <= M <= 8: the top-k + sort launch;
    # larger: the gate_up launch sorts the top-k itself where its wide form
    # runs, else the sort launch does)
    cpu, gpu = moe128
    h, rw = _router_inputs(M, seed=500 + M)
    x = synth.activations(M, H, seed=600 + M)
    args = (h.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev), rw.per_expert_scale.to(dev), rw.eps, K_TOP)
    y, w, idx = _lib.moe_layer_forward(*args, x.to(dev), gpu["gate_up_packed"], gpu["gate_up_scale"],
                                       gpu["down_packed"], gpu["down_scale"])
    w2, idx2 = _lib.router_topk(*args)
    assert torch.equal(idx.cpu(), idx2.cpu())
    assert torch.equal(w.cpu(), w2.cpu())
    y2 = _moe_gpu(x, idx2.cpu(), w2.cpu(), gpu, dev)
    assert torch.equal(y.cpu(), y2.cpu())
    ref = _moe_ref(x, idx.cpu(), w.cpu(), cpu, 128)
    assert margin(f"router+experts one call M={M}", oracle.max_abs_rel(_np(y), ref)) <= TOL


# ------------------------------------------------------ prefill grouped GEMM
# Batches above the decode threshold run the LDS-tiled grouped GEMM.

def _skewed_route(M, seed, hot=8):
    # every token routed to the same `hot` experts (in a per-token order):
    # segments of M rows, i.e. several m-tiles per expert plus a partial one
    g = torch.Generator().manual_seed(seed)
    hot_ids = torch.randperm(E, generator=g)[:hot]
    idx = torch.stack([hot_ids[torch.randperm(hot, generator=g)][:K_TOP] for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    return idx, (w / w.sum(1, keepdim=True)).float()


@pytest.mark.parametrize("M", [48, 200])
def test_moe_decode_experts_over_16_rows(dev, moe128, M):
    # decode sizes with every token on the same 8 experts: each expert has M
    # rows, more than one staging pass (16 rows) of the streaming kernels
    cpu, gpu = moe128
    x = synth.activations(M, H, seed=240 + M)
    idx, w = _skewed_route(M, seed=340 + M)
    y = _moe_gpu(x, idx, w, gpu, dev)
    assert margin(f"moe decode skewed M={M} (all rows)", oracle.max_abs_rel(
        _np(y), _moe_ref(x, idx, w, cpu, 128))) <= TOL


@pytest.mark.parametrize("M", [257, 300])
def test_moe_prefill_skewed_segments(dev, moe128, M):
    cpu, gpu = moe128
    x = synth.activations(M, H, seed=700 + M)
    idx, w = _skewed_route(M, seed=710 + M)
    y = _moe_gpu(x, idx, w, gpu, dev)
    assert margin(f"moe prefill skewed M={M} (all rows)", oracle.max_abs_rel(
        _np(y), _moe_ref(x, idx, w, cpu, 128))) <= TOL


def _paired_route(M, seed):
    # slots 2i and 2i + 1 of every token on one expert: the reference handles
    # each (token, slot) row on its own (quantization.py:112-129), so an expert
    # holds two rows of such a token
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP // 2].repeat_interleave(2) for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    return idx, (w / w.sum(1, keepdim=True)).float()


# decode streamers with the separate down + combine (M = 40: 320 rows), and
# the prefill GEMM (M = 300)
@pytest.mark.parametrize("M", [40, 300])
def test_moe_repeated_experts_per_token(dev, moe128, M):
    cpu, gpu = moe128
    x = synth.activations(M, H, seed=770 + M)
    idx, w = _paired_route(M, seed=771 + M)
    y = _moe_gpu(x, idx, w, gpu, dev)
    assert margin(f"moe repeated experts per token M={M} (all rows)", oracle.max_abs_rel(
        _np(y), _moe_ref(x, idx, w, cpu, 128))) <= TOL


def test_moe_prefill_invalid_slots(dev, moe128):
    cpu, gpu = moe128
    M = 400
    x = synth.activations(M, H, seed=720)
    idx, w = _route(M, seed=721)
    idx_bad = idx.clone()
    idx_bad[::3, 6:] = E
    idx_bad[1::7, 0] = -1
    w_cut = w.clone()
    w_cut[::3, 6:] = 0.0
    w_cut[1::7, 0] = 0.0
    assert torch.equal(_moe_gpu(x, idx_bad, w, gpu, dev).cpu(), _moe_gpu(x, idx, w_cut, gpu, dev).cpu())


@pytest.mark.parametrize("G", [32, 64, 128])
def test_moe_prefill_groups(dev, G):
    e, h, i, k = 16, 512, 192, 4
    wts = synth.moe_weights(e, h, i, G, seed=730 + G)
    M = 320
    x = synth.activations(M, h, seed=731)
    g = torch.Generator().manual_seed(732)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(M)])
    w = torch.rand(M, k, generator=g).float()
    y = _lib.moe_forward(x.to(dev), idx.to(dev), w.to(dev), wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev),
                         wts.down_packed.to(dev), wts.down_scale.to(dev))
    ref = oracle.moe_forward(_np(x), idx.numpy(), w.numpy(), wts.gate_up_packed.numpy(),
                             _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), G)
    assert margin(f"moe prefill small shape G={G} M={M} (all rows)", oracle.max_abs_rel(_np(y), ref)) <= TOL


# (640, 320, 128): odd group counts per row -> the fallback exact-form GEMM
# (k_prefill); (896, 960, 256) and (1024, 704, 128): k_prefill_x with partial
# last groups and half-width last n-tiles (gate_up when I % 128 == 64, down
# when H % 256 == 128)
@pytest.mark.parametrize("h,i,G", [(640, 320, 128), (896, 960, 256), (1024, 704, 128)])
def test_moe_prefill_half_items(dev, h, i, G):
    # items of at most 64 rows and half-width last n-tiles run with all eight
    # wavefronts on half the tile; segment sizes chosen to give tails of 122,
    # 2, 64, 40, 33, 20, 1 and 62 rows
    e, k = 8, 2
    wts = synth.moe_weights(e, h, i, G, seed=760)
    counts = [250, 130, 64, 40, 33, 20, 1, 62]
    M = sum(counts) // k
    x = synth.activations(M, h, seed=761)
    slots = np.repeat(np.arange(e), counts)
    idx = np.stack([slots[:M], slots[M:]], 1)
    assert (idx[:, 0] != idx[:, 1]).all()
    idx = torch.from_numpy(idx[np.random.default_rng(762).permutation(M)]).long()
    w = torch.rand(M, k, generator=torch.Generator().manual_seed(763)).float()
    y = _lib.moe_forward(x.to(dev), idx.to(dev), w.to(dev), wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev),
                         wts.down_packed.to(dev), wts.down_scale.to(dev))
    ref = oracle.moe_forward(_np(x), idx.numpy(), w.numpy(), wts.gate_up_packed.numpy(),
                             _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), G)
    assert margin(f"moe prefill h={h} i={i} G={G} M={M} (all rows)", oracle.max_abs_rel(_np(y), ref)) <= TOL
    # a token's output does not depend on the tile shape its rows land in
    # (270 tokens: still above the decode threshold, other segment tails)
    sub = torch.tensor([t for t in range(M) if t % 10 != 0])
    y_sub = _lib.moe_forward(x[sub].to(dev), idx[sub].to(dev), w[sub].to(dev), wts.gate_up_packed.to(dev),
                             wts.gate_up_scale.to(dev), wts.down_packed.to(dev), wts.down_scale.to(dev))
    assert torch.equal(y_sub.cpu(), y.cpu()[sub])


@pytest.mark.parametrize("h,i,G", [(1024, 704, 128), (896, 960, 256)])
def test_moe_prefill_wide_items_bit_identical(dev, h, i, G):
    # an expert's tail of at most 32 rows runs as a wide item (three n-tiles
    # per workgroup item), of more rows as a one-n-tile item: the same token
    # rows give the same bits either way.  Batch A: expert 0 holds 20 rows
    # (wide); batch B = A + 20 tokens on experts 0 and 7: expert 0 holds 40
    # rows (one-n-tile item of two m-blocks)
    e, k = 8, 2
    wts = synth.moe_weights(e, h, i, G, seed=790)
    counts = [20, 180, 100, 60, 33, 30, 97, 80]
    M = sum(counts) // k
    slots = np.repeat(np.arange(e), counts)
    idx = np.stack([slots[:M], slots[M:]], 1)
    assert (idx[:, 0] != idx[:, 1]).all()
    idx = idx[np.random.default_rng(791).permutation(M)]
    extra = np.tile(np.array([[0, 7]]), (20, 1))
    idx_b = torch.from_numpy(np.concatenate([idx, extra])).long()
    x_b = synth.activations(M + 20, h, seed=792)
    w_b = torch.rand(M + 20, k, generator=torch.Generator().manual_seed(793)).float()
    gpu = [wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev), wts.down_packed.to(dev), wts.down_scale.to(dev)]
    print(f"prefill wide items h={h} i={i} G={G} M={M} / {M + 20}", flush=True)
    y_a = _lib.moe_forward(x_b[:M].to(dev), idx_b[:M].to(dev), w_b[:M].to(dev), *gpu).cpu()
    y_b = _lib.moe_forward(x_b.to(dev), idx_b.to(dev), w_b.to(dev), *gpu).cpu()
    assert torch.equal(y_a, y_b[:M])
    ref = oracle.moe_forward(_np(x_b), idx_b.numpy(), w_b.numpy(), wts.gate_up_packed.numpy(),
                             _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), G)
    assert margin(f"moe prefill wide items h={h} i={i} G={G} M={M + 20} (all rows)",
                  oracle.max_abs_rel(_np(y_b), ref)) <= TOL


def test_moe_large_batch_untiled_shape(dev):
    # H not a multiple of 128 / I not a multiple of 64: large batches stay on
    # the streaming kernels and must still match
    e, h, i, k, G = 8, 544, 160, 2, 32
    wts = synth.moe_weights(e, h, i, G, seed=740)
    M = 300
    x = synth.activations(M, h, seed=741)
    g = torch.Generator().manual_seed(742)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(M)])
    w = torch.rand(M, k, generator=g).float()
    y = _lib.moe_forward(x.to(dev), idx.to(dev), w.to(dev), wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev),
                         wts.down_packed.to(dev), wts.down_scale.to(dev))
    ref = oracle.moe_forward(_np(x), idx.numpy(), w.numpy(), wts.gate_up_packed.numpy(),
                             _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), G)
    assert margin(f"moe streaming shape h={h} i={i} M={M} (all rows)", oracle.max_abs_rel(_np(y), ref)) <= TOL


def test_moe_prefill_config3_zipf(dev, moe128):
    # benchmark configs[3]: M=4096 with Zipf routing, every row against the
    # oracle (and the distances to the unrounded fp32 arithmetic reported),
    # plus two size-independent properties of the tiled GEMM:
    #  * batch invariance: a token's output does not depend on which other
    #    tokens share its tiles (same row in a different batch -> same bits);
    #  * permutation equivariance: permuting tokens permutes the output.
    cpu, gpu = moe128
    M = 4096
    x = synth.zipf_activations(M, H, seed=750)
    rw = synth.zipf_router_weights(E, H, seed=751)
    w_full, idx_full = _lib.router_topk(x.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev),
                                        rw.per_expert_scale.to(dev), rw.eps, K_TOP)
    idx, w = idx_full.cpu(), w_full.cpu()
    y = _moe_gpu(x, idx, w, gpu, dev).cpu()
    ref = _moe_ref(x, idx, w, cpu, 128)
    assert margin(f"moe prefill configs[3] G=128 M={M} (all rows)", oracle.max_abs_rel(_np(y), ref)) <= TOL
    ref32 = _moe_ref_fp32(x, idx, w, cpu, 128)
    margin(f"moe prefill configs[3] G=128 M={M} (all rows)", oracle.max_abs_rel(_np(y), ref32),
           measure="max_abs_rel vs fp32")
    margin(f"moe prefill configs[3] G=128 M={M} (all rows)", oracle.max_abs_rel(ref, ref32),
           measure="oracle bf16 vs fp32")
    sub = torch.arange(0, M, 13)        # 316 tokens: still above the decode threshold
    y_sub = _moe_gpu(x[sub], idx[sub], w[sub], gpu, dev).cpu()
    assert torch.equal(y_sub, y[sub])
    perm = torch.randperm(M, generator=torch.Generator().manual_seed(752))
    y_perm = _moe_gpu(x[perm], idx[perm], w[perm], gpu, dev).cpu()
    assert torch.equal(y_perm, y[perm])


# ------------------------------------------- latent stack (benchmark configs[4])

def test_latent_stack_layers_and_hybridlink(dev):
    # a small latent stack: every MoE layer against the oracle on the layer's
    # own input and routing, the routing against the oracle router, and the
    # HybridLink map against the oracle's fp32 formula
    from hybridagent_amd.latent import LatentStack
    e, h_, i_, k, G = 16, 256, 128, 4, 128
    st = LatentStack(3, e, h_, i_, k, G, seed=900, device=dev)
    h = synth.activations(6, h_, seed=901, device=dev)
    for li, ly in enumerate(st.layers):
        xin = st.rms_norm(h, ly.pre_norm)
        ref_x = oracle.rms_norm(_np(h), _np(ly.pre_norm), st.eps)
        assert np.abs(oracle.to_bf16_bits(_np(xin)).astype(np.int32) - oracle.to_bf16_bits(ref_x).astype(np.int32)).max() <= 1
        out, idx, w = st.moe(h, li)
        rw, ew = ly.router, ly.experts
        ref_lg, ref_idx, _ = oracle.router(_np(h), _np(rw.scale), rw.scalar_root, _np(rw.proj),
                                           _np(rw.per_expert_scale), rw.eps, k)
        srt = -np.sort(-ref_lg, axis=1)
        safe = srt[:, k - 1] - srt[:, k] > 2 * np.abs(srt[:, k - 1]) * 2.0 ** -7
        assert np.array_equal(np.sort(idx.cpu().numpy()[safe], 1), np.sort(ref_idx[safe], 1))
        ref_out = oracle.moe_forward(_np(xin), idx.cpu().numpy(), w.cpu().numpy(), ew.gate_up_packed.cpu().numpy(),
                                     _bits(ew.gate_up_scale.cpu()), ew.down_packed.cpu().numpy(),
                                     _bits(ew.down_scale.cpu()), G)
        assert oracle.max_abs_rel(_np(out), ref_out) <= TOL
        h = h + out
    p = {key: _np(v) for key, v in st.hl.items()}
    ref = oracle.hybridlink(_np(h), p["p1w"], p["p1b"], p["p2w"], p["p2b"], p["ln1w"], p["ln1b"], p["ln2w"], p["ln2b"])
    assert oracle.max_abs_rel(_np(st.hybridlink(h)), ref) <= 2 * TOL
    h0 = synth.activations(6, h_, seed=902, device=dev)
    out = st.step(h0)
    assert out.shape == (6, h_) and torch.isfinite(out.float()).all()
    # step() adds each layer's output inside the next layer's norm launch:
    # bit-identical to the layers one after the other
    hs = h0
    for li in range(len(st.layers)):
        hs, _, _ = st.layer(hs, li)
    assert torch.equal(out, st.hybridlink(hs) * math.sqrt(h_))


@pytest.mark.parametrize("M,H", [(1, 2816), (32, 2816), (5, 8), (3, 8192), (7, 1000)])
def test_add_rms_norm(dev, M, H):
    # x = bf16(h + delta) bit-exact against torch's bf16 add; y within one
    # bf16 ulp of the oracle's RMSNorm (fp32 reduction order)
    g = torch.Generator().manual_seed(M * 7 + H)
    h = torch.randn(M, H, generator=g).to(torch.bfloat16)
    d = (0.5 * torch.randn(M, H, generator=g)).to(torch.bfloat16)
    w = (1.0 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16)
    x, y = _lib.add_rms_norm(h.to(dev), w.to(dev), 1e-6, delta=d.to(dev))
    assert torch.equal(x.cpu(), h + d)
    ref = oracle.rms_norm(_np(h + d), _np(w), 1e-6)
    ulp = np.abs(oracle.to_bf16_bits(_np(y)).astype(np.int32) - oracle.to_bf16_bits(ref).astype(np.int32))
    assert ulp.max() <= 1
    x2, y2 = _lib.add_rms_norm(h.to(dev), w.to(dev), 1e-6)
    assert torch.equal(x2.cpu(), h)
    ref2 = oracle.rms_norm(_np(h), _np(w), 1e-6)
    assert np.abs(oracle.to_bf16_bits(_np(y2)).astype(np.int32) - oracle.to_bf16_bits(ref2).astype(np.int32)).max() <= 1


# ------------------------------------------------------------ HIP graph replay
# The layer is captured once and replayed several times with other eager work
# (another batch size through the same kernels) and synchronisations in
# between; every replay must reproduce the eager result bit for bit.  This
# covers state that lives across launches: the prefill work queues (zeroed by
# the expert sort, reset by the last workgroup of each launch) and the plan.

def _replays_match(capture, eager, disturb, n=3):
    ref = eager()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        capture()  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = capture()
    for i in range(n):
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r), f"replay {i} differs from the eager result"
        disturb()
        torch.cuda.synchronize()


@pytest.mark.parametrize("M", [512, 4096])
def test_graph_replay_prefill_experts(dev, moe128, M):
    cpu, gpu = moe128
    x = synth.activations(M, H, seed=800 + M).to(dev)
    idx, w = _route(M, seed=801 + M)
    idx, w = idx.to(dev), w.to(dev)
    args = (gpu["gate_up_packed"], gpu["gate_up_scale"], gpu["down_packed"], gpu["down_scale"])
    fwd = lambda: (_lib.moe_forward(x, idx, w, *args),)
    x2 = synth.activations(300, H, seed=802).to(dev)
    i2, w2 = _route(300, seed=803)
    i2, w2 = i2.to(dev), w2.to(dev)
    _replays_match(fwd, fwd, lambda: _lib.moe_forward(x2, i2, w2, *args))


@pytest.mark.parametrize("M", [1, 8, 64])
def test_graph_replay_decode_layer(dev, moe128, M):
    cpu, gpu = moe128
    h, rw = _router_inputs(M, seed=810 + M)
    x = synth.activations(M, H, seed=811 + M).to(dev)
    rargs = (h.to(dev), rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev), rw.per_expert_scale.to(dev),
             rw.eps, K_TOP)
    eargs = (gpu["gate_up_packed"], gpu["gate_up_scale"], gpu["down_packed"], gpu["down_scale"])
    fwd = lambda: _lib.moe_layer_forward(*rargs, x, *eargs)
    h2, _ = _router_inputs(33, seed=812)
    x2 = synth.activations(33, H, seed=813).to(dev)
    rargs2 = (h2.to(dev),) + rargs[1:]
    _replays_match(fwd, fwd, lambda: _lib.moe_layer_forward(*rargs2, x2, *eargs))


# ---------------------------------------------------- HybridLink (hybridlink.py)

def _hybridlink_params(H, seed, dev):
    g = torch.Generator().manual_seed(seed)
    std = 1.0 / math.sqrt(H)
    mk = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g)).to(torch.bfloat16).to(dev)
    return {"ln1w": (1.0 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev), "ln1b": mk(H, sc=0.02),
            "p1w": mk(H, H, sc=std), "p1b": mk(H, sc=0.02), "p2w": mk(H, H, sc=std), "p2b": mk(H, sc=0.02),
            "ln2w": (1.0 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev), "ln2b": mk(H, sc=0.02)}


# batch 32 at H = 2816 is the latent loop's shape; 1 / 17 / 100 cover one,
# two and several row tiles (ragged); H = 32 leaves seven of the eight
# K-split wavefronts without k steps; H = 4096 the LayerNorm's long-row form
# (more than 3072 values per row)
@pytest.mark.parametrize("B,Hh", [(32, 2816), (1, 2816), (17, 256), (100, 1024), (5, 32), (3, 4096)])
def test_hybridlink(dev, B, Hh):
    p = _hybridlink_params(Hh, seed=900 + Hh, dev=dev)
    h = synth.activations(B, Hh, seed=901 + B, device=dev)
    got = _lib.hybridlink(h, p["ln1w"], p["ln1b"], p["p1w"], p["p1b"], p["p2w"], p["p2b"], p["ln2w"], p["ln2b"])
    q = {key: _np(v) for key, v in p.items()}
    ref = oracle.hybridlink(_np(h), q["p1w"], q["p1b"], q["p2w"], q["p2b"], q["ln1w"], q["ln1b"], q["ln2w"], q["ln2b"])
    err = oracle.max_abs_rel(_np(got), ref)
    print(f"hybridlink B={B} H={Hh} max_abs_rel={err:.2e}")
    assert err <= 2 * TOL
    # the torch bf16 module (the reference's own arithmetic, torch CPU in fp32
    # per op with bf16 rounding between the ops) agrees as closely
    hc = h.cpu().float()
    pc = {key: v.cpu().float() for key, v in p.items()}
    rb = lambda t: t.to(torch.bfloat16).float()
    a = rb(torch.nn.functional.layer_norm(hc, (Hh,), pc["ln1w"], pc["ln1b"]))
    a = rb(torch.nn.functional.gelu(rb(a @ pc["p1w"].T + pc["p1b"])))
    p2 = rb(a @ pc["p2w"].T + pc["p2b"])
    r = rb(hc + p2)
    tref = rb(torch.nn.functional.layer_norm(r, (Hh,), pc["ln2w"], pc["ln2b"]))
    # same rounding points: per element in bf16 ulps (max_abs_rel, which
    # divides by the largest output, would let every element be off by ~6 ulps).
    # Beyond two ulps an element may differ by what rounding flips on its
    # path become through the LayerNorm: r = bf16(h + p2) moves by an ulp of
    # its larger operand per flip of p2 (many ulps of r when h and p2
    # cancel), times rstd * |w|; flips of upstream intermediates can stack in
    # p2, so up to four are allowed, on top of the output's own two ulps.  (A
    # CPU emulation with float64 instead of float32 accumulation shows up to
    # two stacked flips at B = 64, H = 2816.)
    rstd = 1.0 / torch.sqrt(r.var(-1, unbiased=False, keepdim=True) + 1e-5)
    big = np.maximum(np.abs(hc.numpy()), np.abs(p2.numpy()))
    slack = 4 * bf16_ulp(big) * rstd.numpy() * np.abs(pc["ln2w"].numpy()) + 2 * bf16_ulp(tref.numpy())
    check_bf16_close(_np(got), tref.numpy(), f"hybridlink B={B} H={Hh} vs torch bf16", slack=slack)
    # rows are independent: a sub-batch gives the same bits
    got_sub = _lib.hybridlink(h[: max(1, B // 2)], p["ln1w"], p["ln1b"], p["p1w"], p["p1b"], p["p2w"], p["p2b"],
                              p["ln2w"], p["ln2b"])
    assert torch.equal(got_sub, got[: max(1, B // 2)])
