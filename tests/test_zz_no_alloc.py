"""moe_forward_static (the entry point that allocates nothing) against
moe_forward, through the C ABI: two calls in a row, the second with a smaller
batch, each bit-identical to moe_forward on the same inputs (the same kernels
on a different scratch buffer); sizes beyond the scratch are rejected before
any launch."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from hybridagent_amd import _lib, synth

pytestmark = pytest.mark.gpu

E, H, I, K_TOP, G = 128, 2816, 704, 8, 128
ERR_SHAPE = 2


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def setup():
    assert _lib.available(), "libw4a16moe.so must be built"
    dev = torch.device("cuda:0")
    wts = synth.moe_weights(E, H, I, G, seed=1500)
    gpu = [getattr(wts, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")]
    return dev, wts, gpu


def _inputs(M, seed, dev):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP] for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    w = (w / w.sum(1, keepdim=True)).float()
    x = synth.activations(M, H, seed=seed + 1)
    return x.to(dev), idx.to(dev), w.to(dev)


def _static(lib, x, idx, w, gpu, out):
    M = x.shape[0]
    stream = torch.cuda.current_stream(x.device).cuda_stream
    return lib.moe_forward_static(x.data_ptr(), idx.data_ptr(), w.data_ptr(), *[t.data_ptr() for t in gpu],
                                  out.data_ptr(), M, K_TOP, E, H, I, G, stream)


def test_static_matches_moe_forward_twice(setup):
    dev, wts, gpu = setup
    lib = _lib.load()
    for M, seed in ((64, 1510), (8, 1520), (257, 1530), (1, 1540)):
        print(f"moe_forward_static M={M}", flush=True)
        x, idx, w = _inputs(M, seed, dev)
        out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
        assert _static(lib, x, idx, w, gpu, out) == 0
        ref = _lib.moe_forward(x, idx, w, *gpu)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"M={M}: static scratch result differs from moe_forward"
        rows = np.arange(0, M, max(1, M // 8))
        err = oracle.max_abs_rel(_np(out)[rows], oracle.moe_forward(
            _np(x)[rows], idx.cpu().numpy()[rows], w.cpu().numpy()[rows], wts.gate_up_packed.numpy(),
            _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), G))
        assert err <= 1e-2


def test_static_rejects_sizes_beyond_the_scratch(setup):
    dev, _, gpu = setup
    lib = _lib.load()
    M = 4096  # needs ~267 MB of scratch: rejected on the host, nothing launched
    assert lib.moe_workspace_bytes(M, K_TOP, E, H, I) > 16 << 20
    fake = ctypes.c_void_p(4096)
    st = lib.moe_forward_static(fake, fake, fake, *[t.data_ptr() for t in gpu], fake, M, K_TOP, E, H, I, G,
                                torch.cuda.current_stream(dev).cuda_stream)
    assert st == ERR_SHAPE
