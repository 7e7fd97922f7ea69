"""The reference's own Python API on the GPU, against the oracle.

These are the names HybridAgent's callers use (quantization.py:88-240,
backends.py:48-65,111-129): ``Gemma4TextExperts4Bit`` built from a config
whose ``quantization_config`` names the group size, its ``forward``,
``Linear4Bit.forward``, the module-level ``dequantize_int4_packed``,
``fused_triton_4bit_moe_forward`` and the ``hybrid_agent::fused_4bit_moe``
custom op, eagerly and inside ``torch.compile(fullgraph=True, dynamic=True)``
in a function shaped like the MoE half of ``_ffn_moe_4bit_step``.  Every call
runs the HIP library (there is no other path).
"""
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from checks import check_routing_order
from hybridagent_amd import _lib, synth
from hybridagent_amd import backends
from hybridagent_amd import quantization as q

pytestmark = pytest.mark.gpu

TOL = 1e-2
E, H, I, K_TOP = 128, 2816, 704, 8


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _config(G):
    """The fields Gemma4TextExperts4Bit reads (quantization.py:184-190), with the
    group size in a compressed-tensors quantization_config."""
    return types.SimpleNamespace(
        num_experts=E, hidden_size=H, moe_intermediate_size=I, hidden_activation="gelu_pytorch_tanh",
        quantization_config={"quant_method": "compressed-tensors", "format": "pack-quantized",
                             "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": G}}}})


@pytest.fixture(scope="module")
def dev():
    assert _lib.available(), "libw4a16moe.so must be built"
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def experts(dev):
    """Gemma4TextExperts4Bit at the Gemma-4-26B-A4B shape, G = 128 from the
    config, buffers filled the way the loader fills them (copy_)."""
    mod = q.Gemma4TextExperts4Bit(_config(128))
    assert mod.group_size == 128
    assert tuple(mod.gate_up_scale.shape) == (E, 2 * I, 22) and tuple(mod.down_scale.shape) == (E, H, 6)
    w = synth.moe_weights(E, H, I, 128, seed=1200)
    for name in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"):
        getattr(mod, name).copy_(getattr(w, name))
    return mod.to(dev), w


def _route(M, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP] for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    return idx, (w / w.sum(1, keepdim=True)).float()


def _oracle_rows(x, idx, w, wts, rows):
    return oracle.moe_forward(_np(x)[rows], idx.numpy()[rows], w.numpy()[rows], wts.gate_up_packed.numpy(),
                              _bits(wts.gate_up_scale), wts.down_packed.numpy(), _bits(wts.down_scale), 128)


@pytest.mark.parametrize("M", [1, 64, 4096])
def test_experts_module_forward(dev, experts, M):
    mod, wts = experts
    x = synth.activations(M, H, seed=1210 + M)
    idx, w = _route(M, seed=1220 + M)
    y = mod(x.to(dev), idx.to(dev), w.to(dev))
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (M, H)
    rows = np.arange(M) if M <= 64 else np.r_[0:4, 1234, 2048, 3001, M - 4:M]
    err = oracle.max_abs_rel(_np(y)[rows], _oracle_rows(x, idx, w, wts, rows))
    print(f"Gemma4TextExperts4Bit.forward M={M} max_abs_rel={err:.2e}")
    assert err <= TOL
    # the reference's functional entry point gives the same bits
    y2 = q.fused_triton_4bit_moe_forward(x.to(dev), idx.to(dev), w.to(dev), mod.gate_up_packed,
                                         mod.gate_up_scale, mod.down_packed, mod.down_scale)
    assert torch.equal(y, y2)


def test_experts_module_empty_batch(dev, experts):
    mod, _ = experts
    x = torch.empty(0, H, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(0, K_TOP, dtype=torch.int64, device=dev)
    w = torch.empty(0, K_TOP, dtype=torch.float32, device=dev)
    y = mod(x, idx, w)
    assert tuple(y.shape) == (0, H)
    y2 = torch.ops.hybrid_agent.fused_4bit_moe(x, idx, w, mod.gate_up_packed, mod.gate_up_scale,
                                               mod.down_packed, mod.down_scale)
    assert tuple(y2.shape) == (0, H)


def test_experts_module_g32_from_config(dev):
    # the released checkpoints' group size (quantization.py:19) read from the config
    mod = q.Gemma4TextExperts4Bit(_config(32))
    assert mod.group_size == 32 and mod.gate_up_scale.shape[-1] == 88 and mod.down_scale.shape[-1] == 22
    mod = mod.to(dev)
    w = synth.moe_weights(E, H, I, 32, seed=1230)
    for name in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"):
        getattr(mod, name).copy_(getattr(w, name).to(dev))
    M = 8
    x = synth.activations(M, H, seed=1231)
    idx, rw = _route(M, seed=1232)
    y = mod(x.to(dev), idx.to(dev), rw.to(dev))
    ref = oracle.moe_forward(_np(x), idx.numpy(), rw.numpy(), w.gate_up_packed.numpy(), _bits(w.gate_up_scale),
                             w.down_packed.numpy(), _bits(w.down_scale), 32)
    assert oracle.max_abs_rel(_np(y), ref) <= TOL


@pytest.mark.parametrize("M", [1, 16])
def test_linear4bit_forward(dev, M):
    # Linear4Bit at configs[0]'s layer shape (K = N = 2816, G = 128), with bias
    lin = q.Linear4Bit(2816, 2816, bias=True, group_size=128)
    p = synth.packed_int4((2816, 2816), seed=1240)
    s = synth.group_scales((2816, 2816), 128, seed=1241)
    b = synth.activations(1, 2816, seed=1242)[0]
    lin.weight_packed.copy_(p)
    lin.weight_scale.copy_(s)
    with torch.no_grad():
        lin.bias.copy_(b)
    lin = lin.to(dev)
    x = synth.activations(M, 2816, seed=1243 + M)
    y = lin(x.to(dev))
    ref = oracle.linear(_np(x), p.numpy(), _bits(s), 128, bias=_np(b))
    err = oracle.max_abs_rel(_np(y), ref)
    print(f"Linear4Bit.forward M={M} max_abs_rel={err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("G", [32, 128])
def test_module_dequantize_int4_packed(dev, G):
    p = synth.packed_int4((3, 64, 704), seed=1250)
    s = synth.group_scales((3, 64, 704), G, seed=1251)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=dev)
    got = q.dequantize_int4_packed(p.to(dev), s.to(dev), shifts)
    assert tuple(got.shape) == (3, 64, 704) and got.dtype == torch.bfloat16
    assert np.array_equal(_bits(got), oracle.to_bf16_bits(oracle.dequantize(p.numpy(), _bits(s), G)))


def _moe_half(residual, router_scale, scalar_root: float, router_proj_w, router_per_expert_scale,
              pre_ff_ln2_w, post_ff_ln2_w, gu_packed, gu_scale, dn_packed, dn_scale, eps: float, top_k: int):
    """The MoE half of _ffn_moe_4bit_step (backends.py:110-122), verbatim in its
    torch ops, calling the custom op by its registered name."""
    D = residual.shape[-1]
    h_flat = residual.reshape(-1, D)
    r_norm = F.rms_norm(h_flat, (D,), None, eps) * router_scale * scalar_root
    scores = F.linear(r_norm, router_proj_w)
    probs = F.softmax(scores, dim=-1, dtype=torch.float32)
    top_k_weights, top_k_index = torch.topk(probs, k=top_k, dim=-1)
    top_k_weights = top_k_weights / top_k_weights.sum(dim=-1, keepdim=True)
    top_k_weights = top_k_weights * router_per_expert_scale[top_k_index]
    h_2_in = F.rms_norm(h_flat, (D,), pre_ff_ln2_w, eps)
    h_2 = torch.ops.hybrid_agent.fused_4bit_moe(
        h_2_in, top_k_index, top_k_weights, gu_packed, gu_scale, dn_packed, dn_scale).reshape(residual.shape)
    return F.rms_norm(h_2, (D,), post_ff_ln2_w, eps), top_k_index, top_k_weights, h_2_in


def test_custom_op_eager_and_compiled(dev, experts):
    mod, wts = experts
    assert backends.fused_4bit_moe_op is not None
    rw = synth.router_weights(E, H, seed=1260, device=dev)
    g = torch.Generator().manual_seed(1261)
    ln2 = (1 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    pln2 = (1 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    args = lambda res: (res, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, ln2, pln2,
                        mod.gate_up_packed, mod.gate_up_scale, mod.down_packed, mod.down_scale, 1e-6, K_TOP)
    # Inductor would generate Triton kernels for the torch glue around the op;
    # the "eager" backend runs the same dynamo trace (fake tensors, one graph:
    # the op must be one opaque node with a working fake) with eager kernels.
    # (aot_eager in this torch build passes F.rms_norm a corrupt symbolic
    # normalized_shape once the hidden size is dynamic, independent of the op.)
    compiled = torch.compile(_moe_half, fullgraph=True, dynamic=True, backend="eager")
    for M in (8, 24, 300):  # two decode sizes and one prefill size through one dynamic graph
        res = synth.activations(M, H, seed=1262 + M, device=dev)
        out_e, idx_e, w_e, h2in = _moe_half(*args(res))
        out_c, idx_c, w_c, _ = compiled(*args(res))
        torch.cuda.synchronize()
        assert torch.equal(idx_c, idx_e) and torch.equal(w_c, w_e)
        assert torch.equal(out_c, out_e), f"compiled and eager differ at M={M}"
        # the op returns what the library returns for the same routing
        direct = _lib.moe_forward(h2in, idx_e, w_e, mod.gate_up_packed, mod.gate_up_scale,
                                  mod.down_packed, mod.down_scale)
        op = torch.ops.hybrid_agent.fused_4bit_moe(h2in, idx_e, w_e, mod.gate_up_packed, mod.gate_up_scale,
                                                   mod.down_packed, mod.down_scale)
        assert torch.equal(op, direct)
        rows = np.arange(0, M, max(1, M // 8))
        err = oracle.max_abs_rel(_np(op)[rows], _oracle_rows(h2in.cpu(), idx_e.cpu(), w_e.cpu(), wts, rows))
        print(f"custom op M={M} max_abs_rel={err:.2e}")
        assert err <= TOL
    # the library router (the same router lines, backends.py:111-117) against the oracle
    res = synth.activations(64, H, seed=1299, device=dev)
    w_h, idx_h, lg_h = _lib.router_topk(res, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, 1e-6,
                                         K_TOP, return_logits=True)
    ref_lg, ref_idx, ref_w = oracle.router(_np(res), _np(rw.scale), rw.scalar_root, _np(rw.proj),
                                           _np(rw.per_expert_scale), 1e-6, K_TOP)
    check_routing_order(_np(lg_h), idx_h.cpu().numpy(), ref_lg, ref_idx, K_TOP, "library router M=64")


# The Inductor backend (torch.compile's default, what backends.py:129 builds):
# the torch glue around the op becomes generated kernels, the op stays one
# opaque node that runs the HIP library.  Static shapes (the dynamic-shape
# trace trips over F.rms_norm's symbolic normalized_shape in this torch
# build, as noted above).  The generated norm / softmax kernels may round
# differently from eager, so the op's output is checked against the library
# on the compiled graph's own routing and input, bit for bit, and the routing
# against eager's on all but near-tie rows.
def test_custom_op_inductor(dev, experts):
    mod, wts = experts
    rw = synth.router_weights(E, H, seed=1270, device=dev)
    g = torch.Generator().manual_seed(1271)
    ln2 = (1 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    pln2 = (1 + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    M = 8
    res = synth.activations(M, H, seed=1272, device=dev)
    args = (res, rw.scale, rw.scalar_root, rw.proj, rw.per_expert_scale, ln2, pln2,
            mod.gate_up_packed, mod.gate_up_scale, mod.down_packed, mod.down_scale, 1e-6, K_TOP)
    compiled = torch.compile(_moe_half, fullgraph=True, dynamic=False)
    out_c, idx_c, w_c, h2in_c = compiled(*args)
    out_e, idx_e, w_e, _ = _moe_half(*args)
    torch.cuda.synchronize()
    h2 = _lib.moe_forward(h2in_c, idx_c, w_c, mod.gate_up_packed, mod.gate_up_scale, mod.down_packed,
                          mod.down_scale)
    ref = torch.nn.functional.rms_norm(h2, (H,), pln2, 1e-6)
    assert torch.isfinite(out_c.float()).all()
    assert oracle.max_abs_rel(out_c.float().cpu().numpy(), ref.float().cpu().numpy()) <= 1e-2
    same = (idx_c == idx_e).all(dim=1).float().mean().item()
    print(f"inductor: {same * 100:.0f} % of rows route exactly as eager")
    # every expert the compiled graph picks is a top-k expert of eager's
    # probabilities or within 2 % of its k-th (a near-tie the generated
    # kernels' rounding can flip)
    r_norm = F.rms_norm(res.reshape(-1, H), (H,), None, 1e-6) * rw.scale * rw.scalar_root
    probs = F.softmax(F.linear(r_norm, rw.proj), dim=-1, dtype=torch.float32)
    kth = torch.topk(probs, K_TOP, dim=-1).values[:, -1:]
    picked = torch.gather(probs, 1, idx_c)
    assert (picked >= kth * (1 - 2e-2)).all(), "the compiled graph picked an expert far below eager's top-k"
    op = torch.ops.hybrid_agent.fused_4bit_moe(h2in_c, idx_c, w_c, mod.gate_up_packed, mod.gate_up_scale,
                                               mod.down_packed, mod.down_scale)
    assert torch.equal(op, h2)
