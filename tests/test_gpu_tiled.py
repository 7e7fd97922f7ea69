"""GPU: the tiled weight copies -- the decode streamers' (w4a16_tile kinds
GATE_UP_DECODE / DOWN_DECODE, group size 128, and 32 / 64 with the scales
inside) and the prefill GEMMs' -- and the kernels reading them.

* Each copy is checked byte for byte against a numpy restatement of its
  documented layout, at the Gemma shape and at the streamer shapes of other
  reduction lengths (2 / 4 / 6 tiles per wavefront, with and without the
  4-way K split).
* The layer, stage and FFN-block outputs on the copies equal the packed
  path bit for bit at group sizes 128 and 32 (same operands, same fold
  order); the fused down + combine on the copy equals the separate stages on
  it.
* The registry: Gemma4TextExperts4Bit.tile_weights() makes the reference's
  own entry points (the module forward, fused_triton_4bit_moe_forward, the
  hybrid_agent::fused_4bit_moe op, ffn_moe_4bit_step) read the copies --
  shown by zeroing the copies afterwards, which changes every output --
  and an in-place reload drops them.
"""
import types
import warnings

import numpy as np
import pytest
import torch

import oracle
from checks import margin
from hybridagent_amd import _lib, synth

pytestmark = pytest.mark.gpu

E, H, I, K_TOP = 128, 2816, 704, 8
TOL = 1e-2
GU_DEC, DN_DEC = _lib.TILED_GATE_UP_DECODE, _lib.TILED_DOWN_DECODE


@pytest.fixture(scope="module")
def dev():
    assert _lib.available(), "libw4a16moe.so must be built"
    return torch.device("cuda:0")


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy()


def _u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------ layout restatements

def _decode_shape(K):
    """The streamer's (tiles per wavefront, K-split wavefronts) for a reduction length."""
    nt = ((K >> 5) + 3) >> 2
    for lim, sh in ((2, (2, 1)), (4, (4, 1)), (6, (6, 1)), (8, (2, 4)), (16, (4, 4))):
        if nt <= lim:
            return sh
    return (6, 4)


def _decode_tiled_reference(which, packed, scale_bits, Hh, Ii, G):
    """The decode copy restated from its definition: block (e, ct, w) of TPW KiB
    tiles, lane l's 16 bytes of tile i = words 16 t + 4 (l / 16) + s, s = 0..3,
    of row r, t = ks TPW + i, with w = KSPLIT cg + ks, colblk = CG ct + cg,
    r = 8 colblk + j % 8 (+ I for j >= 8) for gate_up and 16 colblk + j for down
    (j = l % 16); zero past the row or matrix.  G = 32 / 64: then lane l's TPW
    scales (bf16), tile i's the scale of its chunk 4 t + l / 16, zero past K or
    the matrix."""
    Ex = packed.shape[0]
    N, K = (2 * Ii, Hh) if which == "gate_up" else (Hh, Ii)
    tpw, ks_n = _decode_shape(K)
    nw = 16 if ks_n == 4 else 4
    cg_n = nw // ks_n
    ncolblk = Ii // 8 if which == "gate_up" else (Hh + 15) // 16
    n_ct = (ncolblk + cg_n - 1) // cg_n
    lscale = G in (32, 64)
    K8 = K // 8
    # one zero word past every row, and one zero row past the matrix, for
    # the entries the layout leaves zero
    words = np.zeros((Ex, N + 1, K8 + 1), np.uint32)
    words[:, :N, :K8] = packed.view(np.uint32).reshape(Ex, N, K8)
    ng = scale_bits.shape[-1]
    sc = np.zeros((Ex, N + 1, ng + 1), np.uint16)
    sc[:, :N, :ng] = scale_bits.reshape(Ex, N, ng)
    blk_bytes = tpw * (1152 if lscale else 1024)
    out = np.zeros((Ex, n_ct, nw, blk_bytes), np.uint8)
    j = np.arange(16)
    l = np.arange(64)
    lj, lkb = l & 15, l >> 4
    for ct in range(n_ct):
        for w in range(nw):
            cg, ks = w // ks_n, w % ks_n
            colblk = cg_n * ct + cg
            if which == "gate_up":
                rows = 8 * colblk + (j & 7) + np.where(j >= 8, Ii, 0)
                rows = rows if 8 * colblk + 8 <= Ii else np.full(16, N)
            else:
                rows = np.where(16 * colblk + j < N, 16 * colblk + j, N)
            b32 = out[:, ct, w, :tpw * 1024].view(np.uint32).reshape(Ex, tpw, 64, 4)
            for i in range(tpw):
                t = ks * tpw + i
                for s_ in range(4):
                    wd = 16 * t + 4 * lkb + s_
                    wd = np.where(wd < K8, wd, K8)
                    b32[:, i, :, s_] = words[:, rows[lj], wd]
            if lscale:
                b16 = out[:, ct, w, tpw * 1024:].view(np.uint16).reshape(Ex, 64, tpw)
                for i in range(tpw):
                    c = 4 * (ks * tpw + i) + lkb
                    g = np.where(c < K // 32, (c * 32) // G, ng)
                    b16[:, :, i] = sc[:, rows[lj], g]
    return out.reshape(-1)


# the Gemma shape at both group sizes, and (H, I) whose reduction lengths give
# every streamer shape: K = 256 (2 tiles), 512 (4), 1024 (2, K split), 2048
# (4, K split), 2816 (6, K split), 704 (6)
LAYOUT_CASES = [("gate_up", H, I, 128), ("down", H, I, 128), ("gate_up", H, I, 32), ("down", H, I, 32),
                ("gate_up", 256, 512, 32), ("down", 256, 512, 64), ("gate_up", 512, 256, 128),
                ("gate_up", 1024, 256, 32), ("gate_up", 2048, 512, 128), ("down", 1024, 256, 128)]


@pytest.mark.parametrize("which,Hh,Ii,G", LAYOUT_CASES)
def test_decode_tile_layout(dev, which, Hh, Ii, G):
    Ex = 2
    wts = synth.moe_weights(Ex, Hh, Ii, G, seed=7100 + Hh + G)
    tw = _lib.tile_experts(wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev), wts.down_packed.to(dev),
                           wts.down_scale.to(dev), G, decode=True, prefill=False)
    tiled = tw.gu_decode if which == "gate_up" else tw.dn_decode
    assert tiled is not None
    packed = (wts.gate_up_packed if which == "gate_up" else wts.down_packed).numpy()
    scale = _u16(wts.gate_up_scale if which == "gate_up" else wts.down_scale)
    ref = _decode_tiled_reference(which, packed, scale, Hh, Ii, G)
    got = tiled.cpu().numpy().view(np.uint8)
    assert got.shape == ref.shape
    assert np.array_equal(got, ref)


def _prefill_rows(which: str, nt: int, tr: np.ndarray, I: int, N: int) -> np.ndarray:
    """Weight row of tile row tr of n-tile nt (gate_up: 32-row groups of 16 gate
    rows then their 16 up rows, 128 gate columns per n-tile; down: 256 rows per
    n-tile; rows past the matrix repeat its last row)."""
    if which == "gate_up":
        g, cc = tr >> 5, tr & 31
        col = np.minimum(128 * nt + 16 * g + (cc & 15), I - 1)
        return np.where(cc < 16, col, I + col)
    return np.minimum(256 * nt + tr, N - 1)


@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_tile_prefill_layout(dev, which):
    Ex = 2
    wts = synth.moe_weights(Ex, H, I, 128, seed=7150)
    tw = _lib.tile_experts(wts.gate_up_packed.to(dev), wts.gate_up_scale.to(dev), wts.down_packed.to(dev),
                           wts.down_scale.to(dev), 128, decode=False, prefill=True)
    tiled = tw.gu_prefill if which == "gate_up" else tw.dn_prefill
    assert tiled is not None and tw.gu_decode is None
    packed = (wts.gate_up_packed if which == "gate_up" else wts.down_packed).numpy()
    N, K = (2 * I, H) if which == "gate_up" else (H, I)
    n_nt = (I + 127) // 128 if which == "gate_up" else (H + 255) // 256
    nkt = K // 64
    rows = packed.view(np.uint8).reshape(Ex, N, K // 2)
    ref = np.empty((Ex, n_nt, nkt, 256, 32), np.uint8)
    tr = np.arange(256)
    for nt in range(n_nt):
        r = _prefill_rows(which, nt, tr, I, N)
        for kt in range(nkt):
            ref[:, nt, kt] = rows[:, r, 32 * kt:32 * kt + 32]
    got = tiled.cpu().numpy().view(np.uint8)
    assert np.array_equal(got, ref.reshape(-1))


def test_tile_unsupported_shapes(dev):
    # K = 8192 takes the streamer's long-K loop; G = 256 has no tiled decode form
    wts = synth.moe_weights(2, 8192, 64, 128, seed=7101)
    tw = _lib.tile_experts(*(getattr(wts, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed",
                                                               "down_scale")), 128, prefill=False)
    assert tw.gu_decode is None
    wts = synth.moe_weights(2, 1024, 256, 256, seed=7102)
    tw = _lib.tile_experts(*(getattr(wts, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed",
                                                               "down_scale")), 256, prefill=False)
    assert tw.gu_decode is None and tw.dn_decode is None


# ------------------------------------------------------------ kernels on the copies

@pytest.fixture(scope="module", params=[128, 32])
def layer(request, dev):
    G = request.param
    w = synth.moe_weights(E, H, I, G, seed=7200 + G)
    gpu = [getattr(w, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")]
    cpu = {k: getattr(w, k) for k in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")}
    rw = synth.router_weights(E, H, seed=7300)
    r = (rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev), rw.per_expert_scale.to(dev), 1e-6, K_TOP)
    tw = _lib.tile_experts(*gpu, G)
    return G, gpu, cpu, r, tw


_DEQ = {}


def _oracle(x, idx, w, cpu, G):
    key = (id(cpu), G)
    if key not in _DEQ:
        _DEQ[key] = (oracle.dequantize(cpu["gate_up_packed"].numpy(), _u16(cpu["gate_up_scale"]), G),
                     oracle.dequantize(cpu["down_packed"].numpy(), _u16(cpu["down_scale"]), G))
    gu, dn = _DEQ[key]
    return oracle.moe_forward_bf16(x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), gu, dn)


def _same_or_close(G, y_tiled, y_packed, ref_fn, what):
    """The copies hold the same operands for the same fold order: the output
    equals the packed path's bit for bit; the oracle margin is recorded."""
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y_tiled), _bits(y_packed)), f"{what}: tiled output differs"
    margin(f"{what} (tiled)", oracle.max_abs_rel(y_tiled.float().cpu().numpy(), ref_fn()))


@pytest.mark.parametrize("M", [1, 8, 32, 64, 300, 2048])
def test_layer_tiled(dev, layer, M):
    G, gpu, cpu, r, tw = layer
    print(f"tiled layer G={G} M={M}", flush=True)
    x = synth.activations(M, H, seed=7400 + M).to(dev)
    y0, w0, i0 = _lib.moe_layer_forward(x, *r, x, *gpu, tiles=None)
    y1, w1, i1 = _lib.moe_layer_forward(x, *r, x, *gpu, tiles=tw)
    torch.cuda.synchronize()
    assert torch.equal(i0, i1) and torch.equal(w0, w1)
    _same_or_close(G, y1, y0, lambda: _oracle(x, i1, w1, cpu, G), f"layer G={G} M={M}")


@pytest.mark.parametrize("M", [4, 64, 512])
def test_stage_api_tiled(dev, layer, M):
    """The stage API on the copies (gate_up and down both tiled, and gate_up
    tiled with the packed down) against the packed stages / the oracle."""
    G, gpu, cpu, r, tw = layer
    x = synth.activations(M, H, seed=7500 + M).to(dev)
    w, idx = _lib.router_topk(x, *r)
    outs = []
    for tg, td in ((None, None), (tw, tw), (tw, None)):
        st = _lib.MoEStages(M, K_TOP, E, H, I, G, dev)
        st.plan(x, idx)
        st.gate_up(x, gpu[0], gpu[1], tiles=tg)
        st.down(gpu[2], gpu[3], tiles=td)
        outs.append(st.combine(idx, w).clone())
    for k, o in enumerate(outs[1:]):
        _same_or_close(G, o, outs[0], lambda: _oracle(x, idx, w, cpu, G), f"stages G={G} M={M} variant {k}")


@pytest.mark.parametrize("M,k", [(1, 8), (2, 8), (4, 8), (3, 5)])
def test_fused_down_combine_on_copy(dev, layer, M, k):
    """At most 32 routed rows the one-call forward fuses down and combine: on
    the tiled down copy it equals the separate stages on the same copies bit
    for bit."""
    G, gpu, cpu, r, tw = layer
    x = synth.activations(M, H, seed=7550 + M).to(dev)
    g = torch.Generator().manual_seed(7551 + M)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(M)]).to(dev)
    w = (torch.rand(M, k, generator=g) + 0.05).float().to(dev)
    y = _lib.moe_forward(x, idx, w, *gpu, tiles=tw)
    st = _lib.MoEStages(M, k, E, H, I, G, dev)
    st.plan(x, idx)
    st.gate_up(x, gpu[0], gpu[1], tiles=tw)
    st.down(gpu[2], gpu[3], tiles=tw)
    ref = st.combine(idx, w).clone()
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y), _bits(ref)), f"G={G} M={M} k={k}"


@pytest.mark.parametrize("M", [32, 300])
def test_layer_tiled_graph_replay(dev, layer, M):
    """Captured in a HIP graph and replayed with eager work in between: every
    replay equals the eager result (decode and prefill sizes)."""
    G, gpu, cpu, r, tw = layer
    x = synth.activations(M, H, seed=7600).to(dev)
    fwd = lambda xx: _lib.moe_layer_forward(xx, *r, xx, *gpu, tiles=tw)
    eager = fwd(x)[0].clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        fwd(x)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fwd(x)[0]
    x2 = synth.activations(M, H, seed=7601).to(dev)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), _bits(eager)), f"replay {rep}"
        fwd(x2)
        torch.cuda.synchronize()


def _route(M, seed, dev, e=E, k=K_TOP):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(M)])
    w = torch.rand(M, k, generator=g) + 0.05
    return idx.to(dev), (w / w.sum(1, keepdim=True)).float().to(dev)


@pytest.mark.parametrize("M", [1, 8, 64, 2048])
def test_moe_forward_tiled(dev, layer, M):
    """The one-call experts forward (fused_triton_4bit_moe_forward) on all four
    copies against the packed path."""
    G, gpu, cpu, r, tw = layer
    x = synth.activations(M, H, seed=7700 + M).to(dev)
    idx, w = _route(M, 7701 + M, dev)
    y0 = _lib.moe_forward(x, idx, w, *gpu, tiles=None)
    y1 = _lib.moe_forward(x, idx, w, *gpu, tiles=tw)
    _same_or_close(G, y1, y0, lambda: _oracle(x, idx, w, cpu, G), f"moe_forward G={G} M={M}")


# every streamer shape on its copy: (H, I) = (256, 512) gate_up 2 tiles, down
# 4; (512, 256) 4 / 2; (1024, 256) 2 with the K split / 2; (2048, 512) 4 with
# the K split / 4
@pytest.mark.parametrize("Hh,Ii", [(256, 512), (512, 256), (1024, 256), (2048, 512)])
@pytest.mark.parametrize("G", [128, 32])
@pytest.mark.parametrize("M", [1, 8, 40])
def test_small_shapes_tiled(dev, Hh, Ii, G, M):
    e, k = 16, 4
    wts = synth.moe_weights(e, Hh, Ii, G, seed=7750 + Hh + Ii)
    gpu = [getattr(wts, n).to(dev) for n in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")]
    tw = _lib.tile_experts(*gpu, G, prefill=False)
    assert tw.gu_decode is not None and tw.dn_decode is not None
    x = synth.activations(M, Hh, seed=7751 + M).to(dev)
    idx, w = _route(M, 7752 + M, dev, e, k)
    y0 = _lib.moe_forward(x, idx, w, *gpu, tiles=None)
    y1 = _lib.moe_forward(x, idx, w, *gpu, tiles=tw)

    def ref():
        return oracle.moe_forward(x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(),
                                  wts.gate_up_packed.numpy(), _u16(wts.gate_up_scale), wts.down_packed.numpy(),
                                  _u16(wts.down_scale), G)

    _same_or_close(G, y1, y0, ref, f"small shape H={Hh} I={Ii} G={G} M={M}")


@pytest.mark.parametrize("M", [1, 32, 300])
def test_ffn_block_tiled(dev, layer, M):
    """The FFN block on the experts' tiled copies against the packed path (the
    block's other weights random, the experts from the layer fixture)."""
    G, gpu, cpu, r, tw = layer
    Im = 2112
    g = torch.Generator(device=dev).manual_seed(7900 + M)
    nrm = lambda: (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    lin = lambda o, i: (torch.randn(o, i, generator=g, device=dev) / i ** 0.5).to(torch.bfloat16)
    args = dict(post_attn_ln_w=nrm(), pre_ff_ln_w=nrm(), mlp_gate_w=lin(Im, H), mlp_up_w=lin(Im, H),
                mlp_down_w=lin(H, Im), post_ff_ln1_w=nrm(), router_scale=r[0], router_scalar_root=r[1],
                router_proj_w=r[2], router_per_expert_scale=r[3], pre_ff_ln2_w=nrm(), gu_packed=gpu[0],
                gu_scale=gpu[1], dn_packed=gpu[2], dn_scale=gpu[3], post_ff_ln2_w=nrm(), post_ff_ln_w=nrm(),
                layer_scalar=torch.ones(1, dtype=torch.bfloat16, device=dev), eps=1e-6, top_k=K_TOP)
    res = synth.activations(M, H, seed=7901 + M).to(dev)
    att = synth.activations(M, H, seed=7902 + M).to(dev)
    y0, i0, w0 = _lib.ffn_block(res, att, **args, group_size=G, tiles=None, return_routing=True)
    y1, i1, w1 = _lib.ffn_block(res, att, **args, group_size=G, tiles=tw, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(i0, i1) and torch.equal(w0, w1)
    assert np.array_equal(_bits(y0), _bits(y1)), f"G={G} M={M}"


# ------------------------------------------------------------ the registry

def _module(G, seed, dev):
    from hybridagent_amd import quantization as q
    cfg = types.SimpleNamespace(
        num_experts=E, hidden_size=H, moe_intermediate_size=I, hidden_activation="gelu_pytorch_tanh",
        quantization_config={"quant_method": "compressed-tensors", "format": "pack-quantized",
                             "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": G}}}})
    mod = q.Gemma4TextExperts4Bit(cfg)
    wts = synth.moe_weights(E, H, I, G, seed=seed)
    for name in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"):
        getattr(mod, name).copy_(getattr(wts, name))
    return mod.to(dev), wts


@pytest.mark.parametrize("G", [128, 32])
def test_module_tile_weights_reach_reference_entry_points(dev, G):
    """After tile_weights(): the module forward, fused_triton_4bit_moe_forward and
    the hybrid_agent::fused_4bit_moe op (eager and compiled) all equal an explicit
    forward on the copies; the state dict is unchanged; untile_weights() returns
    to the packed path."""
    from hybridagent_amd import backends
    from hybridagent_amd import quantization as q
    mod, _ = _module(G, 7800 + G, dev)
    keys = sorted(mod.state_dict())
    bufs = (mod.gate_up_packed, mod.gate_up_scale, mod.down_packed, mod.down_scale)
    mod.tile_weights()
    tw = mod.tiles
    assert tw is not None and tw.group_size == G
    assert _lib.lookup_tiles(*bufs) is tw
    compiled = torch.compile(lambda *a: torch.ops.hybrid_agent.fused_4bit_moe(*a), fullgraph=True, dynamic=True,
                             backend="eager")
    for M in (1, 64, 512):
        x = synth.activations(M, H, seed=7801 + M).to(dev)
        idx, w = _route(M, 7802 + M, dev)
        want = _lib.moe_forward(x, idx, w, *bufs, tiles=tw)
        packed = _lib.moe_forward(x, idx, w, *bufs, tiles=None)
        for got in (mod(x, idx, w), q.fused_triton_4bit_moe_forward(x, idx, w, *bufs),
                    backends.fused_4bit_moe_op(x, idx, w, *bufs), compiled(x, idx, w, *bufs)):
            torch.cuda.synchronize()
            assert np.array_equal(_bits(got), _bits(want)), f"G={G} M={M}"
        assert np.array_equal(_bits(want), _bits(packed))
    # the entry points read the registered copies: zeroed, every output changes
    # (decode sizes read the decode copies, M = 512 the prefill ones)
    for t in (tw.gu_decode, tw.dn_decode, tw.gu_prefill, tw.dn_prefill):
        t.zero_()
    for M in (1, 64, 512):
        x = synth.activations(M, H, seed=7801 + M).to(dev)
        idx, w = _route(M, 7802 + M, dev)
        packed = _lib.moe_forward(x, idx, w, *bufs, tiles=None)
        for got in (mod(x, idx, w), q.fused_triton_4bit_moe_forward(x, idx, w, *bufs),
                    backends.fused_4bit_moe_op(x, idx, w, *bufs), compiled(x, idx, w, *bufs)):
            torch.cuda.synchronize()
            assert not np.array_equal(_bits(got), _bits(packed)), f"G={G} M={M}: copies not read"
    mod.untile_weights()
    assert mod.tiles is None
    x = synth.activations(8, H, seed=7803).to(dev)
    idx, w = _route(8, 7804, dev)
    assert np.array_equal(_bits(mod(x, idx, w)), _bits(_lib.moe_forward(x, idx, w, *bufs, tiles=None)))
    assert sorted(mod.state_dict()) == keys


def test_registry_drops_stale_copies(dev):
    """An in-place reload of the weights (copy_, as load_state_dict does) makes
    the copies stale: the next forward warns, drops them and reads the new
    packed weights."""
    mod, _ = _module(128, 7810, dev)
    mod.tile_weights()
    new = synth.moe_weights(E, H, I, 128, seed=7811)
    mod.gate_up_packed.copy_(new.gate_up_packed.to(dev))
    x = synth.activations(4, H, seed=7812).to(dev)
    idx, w = _route(4, 7813, dev)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        y = mod(x, idx, w)
    assert any("tiled copies" in str(c.message) for c in caught)
    assert mod.tiles is None
    bufs = (mod.gate_up_packed, mod.gate_up_scale, mod.down_packed, mod.down_scale)
    assert np.array_equal(_bits(y), _bits(_lib.moe_forward(x, idx, w, *bufs, tiles=None)))


def test_ffn_step_reads_registered_copies(dev):
    """ffn_moe_4bit_step (the reference's 22-argument block) finds the copies
    registered for its expert tensors: its output equals the block on the
    explicit copies, and changes when they are zeroed."""
    from hybridagent_amd import backends
    mod, _ = _module(32, 7820, dev)
    rw = synth.router_weights(E, H, seed=7821, device=dev)
    Im = 2112
    g = torch.Generator(device=dev).manual_seed(7822)
    nrm = lambda: (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    lin = lambda o, i: (torch.randn(o, i, generator=g, device=dev) / i ** 0.5).to(torch.bfloat16)
    args = dict(post_attn_ln_w=nrm(), pre_ff_ln_w=nrm(), mlp_gate_w=lin(Im, H), mlp_up_w=lin(Im, H),
                mlp_down_w=lin(H, Im), post_ff_ln1_w=nrm(), router_scale=rw.scale, router_scalar_root=rw.scalar_root,
                router_proj_w=rw.proj, router_per_expert_scale=rw.per_expert_scale, pre_ff_ln2_w=nrm(),
                gu_packed=mod.gate_up_packed, gu_scale=mod.gate_up_scale, dn_packed=mod.down_packed,
                dn_scale=mod.down_scale, post_ff_ln2_w=nrm(), post_ff_ln_w=nrm(),
                layer_scalar=torch.ones(1, dtype=torch.bfloat16, device=dev), eps=1e-6, top_k=K_TOP)
    res = synth.activations(4, H, seed=7823).to(dev)
    att = synth.activations(4, H, seed=7824).to(dev)
    packed = backends.ffn_moe_4bit_step(res, att, **args)
    mod.tile_weights()
    got = backends.ffn_moe_4bit_step(res, att, **args)
    want = _lib.ffn_block(res, att, **args, tiles=mod.tiles)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(got), _bits(want)) and np.array_equal(_bits(got), _bits(packed))
    mod.tiles.gu_decode.zero_()
    assert not np.array_equal(_bits(backends.ffn_moe_4bit_step(res, att, **args)), _bits(packed))
