"""The post-attention FFN block (backends.py:77-126, installed per layer by
backends.py:132-201) on the GPU: ``moe_ffn_block_forward`` through the C ABI
against the oracle, and the installer against transformers' own
``Gemma4TextDecoderLayer.forward`` (the layer whose FFN half the reference's
compiled step replaces).

Every output row is checked against the oracle fed the routing the block's
own router took (read back from its workspace); the routing itself is
checked separately against the oracle's router: ordered equality on every
row whose 8th / 9th logits are clearly apart, and on the others any swap
must be between experts whose logits lie within two bf16 ulps (one ulp of
fp32 reduction order can flip such a near-tie).
"""
import math
import types
from unittest import mock

import numpy as np
import pytest
import torch

import oracle
from checks import margin
from hybridagent_amd import _lib, synth
from hybridagent_amd import backends
from hybridagent_amd import quantization as q

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


def _block_inputs(M, H, I, Im, E, G, seed, dev, layer_scalar=1.0):
    g = torch.Generator().manual_seed(seed)
    nrm = lambda: (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    lin = lambda o, i: (torch.randn(o, i, generator=g) / math.sqrt(i)).to(torch.bfloat16).to(dev)
    w = synth.moe_weights(E, H, I, G, seed=seed + 1, device=dev)
    rw = synth.router_weights(E, H, seed=seed + 2, device=dev)
    return dict(
        residual=synth.activations(M, H, seed=seed + 3, device=dev),
        attn_out=synth.activations(M, H, seed=seed + 4, device=dev),
        post_attn_ln_w=nrm(), pre_ff_ln_w=nrm(), mlp_gate_w=lin(Im, H), mlp_up_w=lin(Im, H),
        mlp_down_w=lin(H, Im), post_ff_ln1_w=nrm(), router_scale=nrm(), router_scalar_root=H ** -0.5,
        router_proj_w=rw.proj, router_per_expert_scale=rw.per_expert_scale, pre_ff_ln2_w=nrm(),
        gu_packed=w.gate_up_packed, gu_scale=w.gate_up_scale, dn_packed=w.down_packed, dn_scale=w.down_scale,
        post_ff_ln2_w=nrm(), post_ff_ln_w=nrm(),
        layer_scalar=torch.tensor([layer_scalar], dtype=torch.bfloat16, device=dev), eps=1e-6)


def _np_args(a):
    conv = {}
    for k, v in a.items():
        if isinstance(v, torch.Tensor):
            if v.dtype == torch.int32:
                conv[k] = v.cpu().numpy()
            elif k in ("gu_scale", "dn_scale"):
                conv[k] = _bits(v)
            else:
                conv[k] = _np(v)
        else:
            conv[k] = v
    conv["layer_scalar"] = float(conv["layer_scalar"].reshape(-1)[0])
    return conv


def _check(a, top_k, G, what):
    """The block through the C ABI (and through backends.ffn_moe_4bit_step, which
    must give the same bits); every row against the oracle on the kernel's
    routing; the routing against the oracle router."""
    out, idx, w = _lib.ffn_block(**a, top_k=top_k, group_size=G, return_routing=True)
    step = backends.ffn_moe_4bit_step(**a, top_k=top_k)
    torch.cuda.synchronize()
    assert torch.equal(out, step)
    conv = _np_args(a)
    ref, ref_idx, _ = oracle.ffn_block(**conv, top_k=top_k, G=G, return_routing=True)
    got_idx = idx.cpu().numpy()
    ref_on_kernel_routing = oracle.ffn_block(**conv, top_k=top_k, G=G, routing=(got_idx, w.cpu().numpy()))
    g = _np(out)
    assert np.isfinite(g).all()
    assert margin(what + " (all rows, kernel routing)", oracle.max_abs_rel(g, ref_on_kernel_routing)) <= TOL
    # routing: the oracle router's logits on the residual as the oracle forms it
    res = oracle.bf16_round(conv["residual"] + oracle.rms_norm(conv["attn_out"], conv["post_attn_ln_w"], conv["eps"]))
    lg = oracle.router_logits(res, conv["router_scale"], conv["router_scalar_root"], conv["router_proj_w"],
                              conv["eps"])
    srt = -np.sort(-lg, axis=1)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(srt[:, top_k - 1]), 1e-30))) - 7)
    clear = srt[:, top_k - 1] - srt[:, top_k] > 2 * ulp
    assert np.array_equal(got_idx[clear], ref_idx[clear]), f"{what}: routing differs on a clear-margin row"
    ulp_all = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(lg), 1e-30))) - 7)
    flips = np.nonzero((got_idx != ref_idx).any(1))[0]
    for r in flips:
        c = int(np.nonzero(got_idx[r] != ref_idx[r])[0][0])
        ea, eb = ref_idx[r, c], got_idx[r, c]
        assert abs(lg[r, ea] - lg[r, eb]) <= 2 * max(ulp_all[r, ea], ulp_all[r, eb]), \
            f"{what}: row {r} swaps experts {ea}/{eb} that are not near-tied"
    print(f"{what}: {len(flips)} of {len(got_idx)} rows route differently from the oracle (near-ties)")
    return out


# Gemma-4-26B-A4B shape; the shared MLP's intermediate size (2112) is an
# assumption: the checkpoint's config.json is not available here.  M = 1 and
# 8: the shared MLP's gate/up in the router's launch, its down in the
# top-k's; M = 32: down on its own; M = 300: both on their own
@pytest.mark.parametrize("M", [1, 8, 32, 300])
def test_ffn_block_gemma_shape(dev, M):
    H, I, Im, E, K, G = 2816, 704, 2112, 128, 8, 128
    a = _block_inputs(M, H, I, Im, E, G, seed=2000 + M, dev=dev)
    out = _check(a, K, G, f"ffn block M={M}")
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (M, H)


@pytest.mark.parametrize("G,ls", [(32, 0.5), (128, 2.0)])
def test_ffn_block_small_shapes(dev, G, ls):
    H, I, Im, E, K, M = 512, 192, 384, 16, 4, 5
    a = _block_inputs(M, H, I, Im, E, G, seed=2100 + G, dev=dev, layer_scalar=ls)
    out = _check(a, K, G, f"ffn block G={G} layer_scalar={ls}")
    # the block is row-independent: a sub-batch gives the same bits
    sub = dict(a, residual=a["residual"][1:4], attn_out=a["attn_out"][1:4])
    assert torch.equal(backends.ffn_moe_4bit_step(**sub, top_k=K), out[1:4])


# Where the router's launches cannot take the shared MLP's linears they run as
# launches of their own (k_linear_bf16): more than 64 routed rows (M = 12,
# top-8: the down linear), rows longer than the fused router takes (H = 4096:
# the gate/up linear, 16 and 32 rows per workgroup)
# (and M = 8, top-8 over 16 experts: down with the one-round top-k of few
# experts)
@pytest.mark.parametrize("M,K,H", [(12, 8, 512), (4, 4, 4096), (20, 4, 4096), (8, 8, 512)])
def test_ffn_block_separate_mlp_launches(dev, M, K, H):
    I, Im, E, G = 192, 384, 16, 128
    a = _block_inputs(M, H, I, Im, E, G, seed=2400 + M + H, dev=dev)
    _check(a, K, G, f"ffn block M={M} top_k={K} H={H} (separate linears)")


class _AttnStub(torch.nn.Module):
    """Stands in for self-attention (attention is outside this path): a fixed
    elementwise map of the normalised input."""

    def forward(self, hidden_states, **kwargs):
        return hidden_states * 0.5 + 0.25, None


def test_patch_ffn_4bit_matches_hf_decoder_layer(dev):
    pytest.importorskip("transformers.models.gemma4")
    from transformers.models.gemma4 import configuration_gemma4 as c, modeling_gemma4 as mg
    H, Im, E, I, K, G, M = 256, 320, 16, 128, 4, 32, 6
    cfg = c.Gemma4TextConfig(hidden_size=H, intermediate_size=Im, num_hidden_layers=1, num_attention_heads=2,
                             num_key_value_heads=1, head_dim=64, vocab_size=128, hidden_size_per_layer_input=0,
                             enable_moe_block=True, num_experts=E, top_k_experts=K, moe_intermediate_size=I,
                             layer_types=["full_attention"], max_position_embeddings=64)

    class _Experts(q.Gemma4TextExperts4Bit):
        def __init__(self, config):
            super().__init__(config, group_size=G)

    with mock.patch.object(mg, "Gemma4TextExperts", _Experts):
        layer = mg.Gemma4TextDecoderLayer(cfg, 0)
    assert isinstance(layer.experts, q.Gemma4TextExperts4Bit)
    layer.self_attn = _AttnStub()
    gen = torch.Generator().manual_seed(2200)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if p.dim() == 1:
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=gen))
            else:
                p.copy_(torch.randn(p.shape, generator=gen) / math.sqrt(p.shape[-1]))
        w = synth.moe_weights(E, H, I, G, seed=2201)
        for name in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"):
            getattr(layer.experts, name).copy_(getattr(w, name))
        layer.layer_scalar.fill_(0.75)
    layer = layer.to(device=dev, dtype=torch.bfloat16)
    x = synth.activations(M, H, seed=2202, device=dev).reshape(1, M, H)
    with torch.no_grad():
        ref = layer(x)                      # transformers' decoder layer, our experts module inside
        ref = ref[0] if isinstance(ref, tuple) else ref
        backbone = types.SimpleNamespace(model=types.SimpleNamespace(language_model=types.SimpleNamespace(
            layers=[layer])))
        assert backends.patch_ffn_4bit(backbone) == 1
        got = layer(x)
        # the router's margin on the residual the layer routes on (rows whose
        # k-th and (k+1)-th probabilities lie within two bf16 ulps may pick
        # the other expert under either router)
        res = x + layer.post_attention_layernorm(layer.self_attn(layer.input_layernorm(x))[0])
        rt = layer.router
        lg = rt.proj(rt.norm(res.reshape(-1, H)) * rt.scale * rt.scalar_root_size)
    srt = -np.sort(-_np(lg), axis=1)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(srt[:, K - 1]), 1e-30))) - 7)
    clear = srt[:, K - 1] - srt[:, K] > 2 * ulp
    assert got.shape == ref.shape and got.dtype == torch.bfloat16
    g, r = _np(got).reshape(M, H), _np(ref).reshape(M, H)
    assert np.isfinite(g).all() and clear.sum() >= M // 2
    err = oracle.max_abs_rel(g[clear], r[clear])
    print(f"patched layer vs transformers' Gemma4TextDecoderLayer: max_abs_rel={err:.2e} "
          f"on {clear.sum()}/{M} rows with a clear routing margin")
    assert err <= TOL


# The shared MLP runs on a second stream beside the routed experts (forked
# after the pre-norms, joined before the post-norm).  Captured into a graph,
# the fork and join become parallel branches: every replay, with eager calls
# and synchronisations between replays, gives the eager result bit for bit.
@pytest.mark.parametrize("M", [1, 32])
def test_ffn_block_graph_replay(dev, M):
    H, I, Im, E, K, G = 2816, 704, 2112, 128, 8, 128
    a = _block_inputs(M, H, I, Im, E, G, seed=2300 + M, dev=dev)
    other = dict(a, residual=synth.activations(M, H, seed=2310 + M, device=dev))
    eager = backends.ffn_moe_4bit_step(**a, top_k=K).clone()
    eager_other = backends.ffn_moe_4bit_step(**other, top_k=K).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        backends.ffn_moe_4bit_step(**a, top_k=K)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = backends.ffn_moe_4bit_step(**a, top_k=K)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager result"
        assert torch.equal(backends.ffn_moe_4bit_step(**other, top_k=K), eager_other)
        torch.cuda.synchronize()
