"""GPU: the tiled weight copies -- the decode gate_up streamer's
(w4a16_tile_gate_up) and the prefill GEMMs' (w4a16_tile_prefill) -- and the
kernels reading them.  Each copy is checked piece by piece against a numpy
restatement of its documented layout; the layer and stage outputs on the
tiled copies are compared bit for bit with the untiled path (same operands,
same fold order), at sizes where each copy is used and where it is not."""
import numpy as np
import pytest
import torch

from hybridagent_amd import _lib, synth

pytestmark = pytest.mark.gpu

E, H, I, K_TOP = 128, 2816, 704, 8


@pytest.fixture(scope="module")
def dev():
    assert _lib.available(), "libw4a16moe.so must be built"
    return torch.device("cuda:0")


def _tiled_reference(packed: np.ndarray, I: int, H: int, tpw: int) -> np.ndarray:
    """The tiled layout restated from its definition: piece (e, ct, w, i, l) =
    16 bytes of packed row r at byte 64 (ks tpw + i) + 16 (l / 16), w = 4 cg + ks,
    colblk = 4 ct + cg, r = 8 colblk + (l % 16) % 8 (+ I for l % 16 >= 8);
    zero past the row or for column blocks past I."""
    Ex = packed.shape[0]
    rowbytes = H // 2
    rows = packed.view(np.uint8).reshape(Ex, 2 * I, rowbytes)
    n_ct = (I // 8 + 3) // 4
    out = np.zeros((Ex, n_ct, 16, tpw, 64, 16), np.uint8)
    for ct in range(n_ct):
        for w in range(16):
            cg, ks = w >> 2, w & 3
            colblk = 4 * ct + cg
            if 8 * colblk + 8 > I:
                continue
            for i in range(tpw):
                for l in range(64):
                    j, kb = l & 15, l >> 4
                    r = 8 * colblk + (j & 7) + (I if j >= 8 else 0)
                    b = 64 * (ks * tpw + i) + 16 * kb
                    if b + 16 <= rowbytes:
                        out[:, ct, w, i, l] = rows[:, r, b:b + 16]
    return out.reshape(-1)


def test_tile_layout(dev):
    Ex = 3
    wts = synth.moe_weights(Ex, H, I, 128, seed=7100)
    tiled = _lib.tile_gate_up(wts.gate_up_packed.to(dev))
    assert tiled is not None
    got = tiled.cpu().numpy().view(np.uint8)
    ref = _tiled_reference(wts.gate_up_packed.numpy(), I, H, tpw=6)
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
    packed = (wts.gate_up_packed if which == "gate_up" else wts.down_packed).numpy()
    tiled = _lib.tile_prefill(torch.from_numpy(packed).to(dev), which)
    assert tiled is not None
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


def test_tile_down_layout(dev):
    """The decode down copy: 4 wavefronts (no K split), 6 k tiles each, column
    block 4 ct + w of 16 rows; piece (e, ct, w, i, l) = row 16 colblk + l % 16
    at byte 64 i + 16 (l / 16), zero past the 352-byte row."""
    Ex = 2
    wts = synth.moe_weights(Ex, H, I, 128, seed=7160)
    tiled = _lib.tile_down(wts.down_packed.to(dev))
    assert tiled is not None
    rowbytes = I // 2
    rows = wts.down_packed.numpy().view(np.uint8).reshape(Ex, H, rowbytes)
    n_ct, tpw = (H // 16 + 3) // 4, 6
    ref = np.zeros((Ex, n_ct, 4, tpw, 64, 16), np.uint8)
    for ct in range(n_ct):
        for w in range(4):
            for i in range(tpw):
                for l in range(64):
                    r, b = 16 * (4 * ct + w) + (l & 15), 64 * i + 16 * (l >> 4)
                    if r < H and b + 16 <= rowbytes:
                        ref[:, ct, w, i, l] = rows[:, r, b:b + 16]
    assert np.array_equal(tiled.cpu().numpy().view(np.uint8), ref.reshape(-1))


def test_tile_unsupported_shape(dev):
    # K = 8192 takes the streamer's long-K loop: no tiled form
    wts = synth.moe_weights(2, 8192, 64, 128, seed=7101)
    assert _lib.tile_gate_up(wts.gate_up_packed.to(dev)) is None


@pytest.fixture(scope="module", params=[128, 32])
def layer(request, dev):
    G = request.param
    w = synth.moe_weights(E, H, I, G, seed=7200 + G)
    gpu = [getattr(w, k).to(dev) for k in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale")]
    rw = synth.router_weights(E, H, seed=7300)
    r = (rw.scale.to(dev), rw.scalar_root, rw.proj.to(dev), rw.per_expert_scale.to(dev), 1e-6, K_TOP)
    tiles = (_lib.tile_gate_up(gpu[0]), _lib.tile_prefill(gpu[0], "gate_up"), _lib.tile_down(gpu[2]),
             _lib.tile_prefill(gpu[2], "down"))
    return (G, gpu, r) + tiles


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy()


# decode sizes (the tiled streamer at G = 128; G = 32 keeps the packed path)
# and prefill sizes (the prefill copies)
@pytest.mark.parametrize("M", [1, 8, 32, 64, 300, 2048])
def test_layer_tiled_equals_untiled(dev, layer, M):
    G, gpu, r, tiled, gpt, dt, dpt = layer
    print(f"tiled layer G={G} M={M}", flush=True)
    x = synth.activations(M, H, seed=7400 + M).to(dev)
    y0, w0, i0 = _lib.moe_layer_forward(x, r[0], r[1], r[2], r[3], r[4], r[5], x, gpu[0], gpu[1], gpu[2], gpu[3])
    y1, w1, i1 = _lib.moe_layer_forward(x, r[0], r[1], r[2], r[3], r[4], r[5], x, gpu[0], gpu[1], gpu[2], gpu[3],
                                        gu_tiled=tiled, gu_ptiled=gpt, dn_tiled=dt, dn_ptiled=dpt)
    torch.cuda.synchronize()
    assert torch.equal(i0, i1) and torch.equal(w0, w1)
    assert np.array_equal(_bits(y0), _bits(y1)), f"G={G} M={M}: tiled layer output differs"


@pytest.mark.parametrize("M", [4, 64, 512])
def test_stage_gate_up_tiled(dev, layer, M):
    """The stage API: gate_up on the tiled copy, then down and combine, equals
    the untiled stages bit for bit."""
    G, gpu, r, tiled, gpt, dt, dpt = layer
    x = synth.activations(M, H, seed=7500 + M).to(dev)
    w, idx = _lib.router_topk(x, *r)
    outs = []
    for t in (None, tiled):
        st = _lib.MoEStages(M, K_TOP, E, H, I, G, dev)
        st.plan(x, idx)
        st.gate_up(x, gpu[0], gpu[1], gu_tiled=t, gu_ptiled=None if t is None else gpt)
        st.down(gpu[2], gpu[3], dn_ptiled=None if t is None else dpt, dn_tiled=None if t is None else dt)
        outs.append(st.combine(idx, w).clone())
    torch.cuda.synchronize()
    assert np.array_equal(_bits(outs[0]), _bits(outs[1]))


@pytest.mark.parametrize("M", [32, 300])
def test_layer_tiled_graph_replay(dev, layer, M):
    """Captured in a HIP graph and replayed with eager work in between: every
    replay equals the eager result (decode and prefill sizes)."""
    G, gpu, r, tiled, gpt, dt, dpt = layer
    x = synth.activations(M, H, seed=7600).to(dev)
    fwd = lambda xx: _lib.moe_layer_forward(xx, r[0], r[1], r[2], r[3], r[4], r[5], xx, gpu[0], gpu[1], gpu[2],
                                            gpu[3], gu_tiled=tiled, gu_ptiled=gpt, dn_tiled=dt, dn_ptiled=dpt)
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


def _route(M, seed, dev):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:K_TOP] for _ in range(M)])
    w = torch.rand(M, K_TOP, generator=g) + 0.05
    return idx.to(dev), (w / w.sum(1, keepdim=True)).float().to(dev)


@pytest.mark.parametrize("M", [1, 8, 64, 2048])
def test_moe_forward_tiled(dev, layer, M):
    """The one-call experts forward (fused_triton_4bit_moe_forward) on all four
    copies equals the packed path bit for bit."""
    G, gpu, r, tiled, gpt, dt, dpt = layer
    x = synth.activations(M, H, seed=7700 + M).to(dev)
    idx, w = _route(M, 7701 + M, dev)
    y0 = _lib.moe_forward(x, idx, w, *gpu)
    y1 = _lib.moe_forward(x, idx, w, *gpu, gu_tiled=tiled, gu_ptiled=gpt, dn_tiled=dt, dn_ptiled=dpt)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y0), _bits(y1)), f"G={G} M={M}"


def test_module_tile_weights(dev):
    """Gemma4TextExperts4Bit.tile_weights: forward with the copies equals forward
    without them; the state dict is unchanged."""
    import types
    from hybridagent_amd import quantization as q
    cfg = types.SimpleNamespace(
        num_experts=E, hidden_size=H, moe_intermediate_size=I, hidden_activation="gelu_pytorch_tanh",
        quantization_config={"quant_method": "compressed-tensors", "format": "pack-quantized",
                             "config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": 128}}}})
    mod = q.Gemma4TextExperts4Bit(cfg)
    wts = synth.moe_weights(E, H, I, 128, seed=7800)
    for name in ("gate_up_packed", "gate_up_scale", "down_packed", "down_scale"):
        getattr(mod, name).copy_(getattr(wts, name))
    mod = mod.to(dev)
    keys = sorted(mod.state_dict())
    for M in (1, 64, 512):
        x = synth.activations(M, H, seed=7801 + M).to(dev)
        idx, w = _route(M, 7802 + M, dev)
        mod.untile_weights()
        y0 = mod(x, idx, w)
        mod.tile_weights()
        y1 = mod(x, idx, w)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y0), _bits(y1)), f"M={M}"
    assert sorted(mod.state_dict()) == keys


@pytest.mark.parametrize("M", [1, 32, 300])
def test_ffn_block_tiled(dev, layer, M):
    """The FFN block on the experts' tiled copies equals the packed path bit for
    bit (the block's other weights random, the experts from the layer fixture)."""
    G, gpu, r, tiled, gpt, dt, dpt = layer
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
    y0 = _lib.ffn_block(res, att, **args, group_size=G)
    y1 = _lib.ffn_block(res, att, **args, group_size=G, gu_tiled=tiled, gu_ptiled=gpt, dn_tiled=dt, dn_ptiled=dpt)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y0), _bits(y1)), f"G={G} M={M}"
