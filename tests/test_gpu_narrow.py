"""GPU: the decode streamers' narrow and wide workgroup forms agree bit for bit.

With fewer work items than CUs the streamers run narrow workgroups (one
column group of 16 weight rows each, four times as many workgroups); larger
batches run the wide form (four column groups sharing one activation stage).
Both sum every output over the same K split in the same wavefront order, so a
row's result does not depend on the form: a token alone (narrow) equals the
same token inside a batch that runs wide, bit for bit -- on the dense linear
(configs[1] shapes) and on the MoE layer (gate_up narrow at M = 1 and 2, wide
at M = 8), packed and tiled, at group size 128 and 32.  The batch results
themselves are checked against the numpy oracle (max_abs_rel <= 1e-2).
"""
import numpy as np
import pytest
import torch

import oracle
from checks import margin
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


# dense: M = 1 and 4 run narrow, M = 64 wide (its narrow form would stage 8
# rows in each of 8 x 176 workgroups)
@pytest.mark.parametrize("K,N", [(2816, 2816), (2816, 1408), (704, 2816)])
def test_dense_narrow_equals_wide(dev, K, N):
    G = 128
    x = synth.activations(64, K, seed=5000 + K + N)
    p = synth.packed_int4((N, K), seed=5001 + K + N)
    s = synth.group_scales((N, K), G, seed=5002 + K + N)
    xd, pd, sd = x.to(dev), p.to(dev), s.to(dev)
    y64 = _lib.linear(xd, pd, sd, group_size=G)
    ref = oracle.linear(_np(x), p.numpy(), _bits(s), G)
    assert margin(f"dense K={K} N={N} M=64 (wide)", oracle.max_abs_rel(_np(y64), ref)) <= TOL
    for r in (0, 17, 63):
        y1 = _lib.linear(xd[r:r + 1], pd, sd, group_size=G)
        assert torch.equal(y1.cpu(), y64[r:r + 1].cpu()), f"row {r}: M=1 differs from M=64"
    y4 = _lib.linear(xd[20:24], pd, sd, group_size=G)
    assert torch.equal(y4.cpu(), y64[20:24].cpu())


@pytest.fixture(scope="module", params=[128, 32])
def stack(request, dev):
    G = request.param
    wts = synth.moe_weights(E, H, I, G, seed=5100 + G)
    gpu = [t.to(dev) for t in (wts.gate_up_packed, wts.gate_up_scale, wts.down_packed, wts.down_scale)]
    tiles = _lib.tile_experts(*gpu, group_size=G, prefill=False)
    return G, wts, gpu, tiles


def _route(M, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP] for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    return idx, (w / w.sum(1, keepdim=True)).float()


@pytest.mark.parametrize("tiled", [False, True])
def test_moe_narrow_equals_wide(dev, stack, tiled):
    G, wts, gpu, tiles = stack
    M = 8
    x = synth.activations(M, H, seed=5200 + G)
    idx, w = _route(M, seed=5201 + G)
    t = tiles if tiled else None
    xd, idd, wd = x.to(dev), idx.to(dev), w.to(dev)
    y8 = _lib.moe_forward(xd, idd, wd, *gpu, group_size=G, tiles=t)
    ref = oracle.moe_forward(_np(x), idx.numpy(), w.numpy(), wts.gate_up_packed.numpy(), _bits(wts.gate_up_scale),
                             wts.down_packed.numpy(), _bits(wts.down_scale), G)
    name = f"moe G={G} M=8{' (tiled)' if tiled else ''}"
    assert margin(name, oracle.max_abs_rel(_np(y8), ref)) <= TOL
    for r in range(0, M, 3):
        y1 = _lib.moe_forward(xd[r:r + 1], idd[r:r + 1], wd[r:r + 1], *gpu, group_size=G, tiles=t)
        assert torch.equal(y1.cpu(), y8[r:r + 1].cpu()), f"token {r}: M=1 differs from M=8"
    y2 = _lib.moe_forward(xd[4:6], idd[4:6], wd[4:6], *gpu, group_size=G, tiles=t)
    assert torch.equal(y2.cpu(), y8[4:6].cpu()), "M=2 differs from M=8"
