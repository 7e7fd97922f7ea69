"""numpy restatement of the reference W4A16 MoE path -- TEST INFRASTRUCTURE ONLY.

Used by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg as the checker; never by the product path.

Reference citations are ``path:line`` under the HybridAgent repository
(``hybrid_agent/...``) or ``TF:`` = ``transformers/`` 5.15 source.

Arithmetic contract restated here (bf16 = bfloat16, RNE = round to nearest even):

* packed int4 word ``p[n, j]`` (int32) holds ``w[n, 8j+i]`` for i = 0..7 in bits
  ``4i..4i+3`` as offset binary ``q + 8``  (``quantization.py:136``);
* ``dequant(p, s)[n, k] = bf16_RNE(q[n, k] * s[n, k // G])``
  (``quantization.py:132-137``).  The reference hard-codes ``G = 32``
  (``quantization.py:19``); here ``G`` is a parameter and the scale tensor has
  ``ceil(K / G)`` columns, the last group covering ``K - (ceil(K/G)-1)*G``
  columns (equal to zero-padding K to a multiple of G);
* bf16 matmuls accumulate in fp32 and round the result to bf16 once
  (``F.linear`` / ``torch.mv`` / ``torch.bmm`` on bf16 tensors,
  ``quantization.py:175,250,261,281,286``);
* the fused MoE forward rounds to bf16 at: gate_up output, GELU output,
  ``gelu * up``, down output, the top-k weight, and ``down * weight``; the
  final sum over the k slots accumulates in fp32 (``quantization.py:119-129``,
  identical rounding points on the single-token path ``:241-263``);
* the per-expert loop path (``quantization.py:265-294``) instead adds each
  expert's bf16 contribution into a bf16 accumulator (``index_add_``).

Pinning (what checks this restatement, see ``tests/test_oracle.py``):

* ``pack_int4`` / ``unpack_int4`` / ``dequantize``: exhaustive 16-nibble known
  answers, hand-computed words (0x76543210, 0xFEDCBA98, 0x88888888, 0),
  pack/unpack round trip, partial-group == zero-pad equivalence.
* ``linear``: brute-force float64 triple loop at tiny shapes, and torch CPU
  ``F.linear`` on identical bf16 operands (library routine).
* ``gelu_tanh``: torch ``F.gelu(approximate="tanh")``.
* ``rms_norm`` / ``router_logits`` / ``topk_from_logits``: torch ``F.rms_norm``,
  ``F.linear``, ``softmax`` + ``torch.topk`` on identical inputs; invariants
  (distinct indices, descending logits, weights sum to 1, tie rule).
* ``sort_permute``: ``torch.argsort(stable=True)`` of the k-major flattening,
  brute force over ``torch.where`` on tiny inputs, bijection / offset checks.
* ``moe_forward``: the "fused" and "loop" rounding paths agree within
  tolerance; a top-1 routing reduces to ``linear`` (down of gelu(gate)*up);
  linearity of the combine in the routing weights.
* ``hybridlink`` / ``rms_norm`` (config-4 harness only): torch ``nn.LayerNorm``,
  ``nn.GELU``, ``nn.Linear`` on identical inputs.
* ``moe_forward_bf16``: with the dequantised 4-bit weights as its bf16
  weights it equals ``moe_forward`` bit for bit (the dequantise-then-matmul
  identity); the torch CPU restatement of ``_bf16_experts_fast_forward``
  (``oracle/torch_cpu.py``) on identical inputs.
* ``moe_forward_fp32`` (every intermediate unrounded): a float64 brute-force
  loop over (token, slot, output) on tiny shapes; it stays within the
  tolerance of ``moe_forward`` (the two differ only by bf16 roundings);
  ``moe_forward_fp32_dequantized`` equals it bit for bit on the
  ``dequantize_fp32`` weights.
* ``ffn_block``: the same lines of ``_ffn_moe_4bit_step`` written with torch CPU
  ``F.rms_norm`` / ``F.linear`` / ``F.gelu`` / ``softmax`` + ``topk`` and the
  torch-CPU experts (``oracle/torch_cpu.py``) on identical inputs; a
  ``layer_scalar`` of 2 doubles the output exactly.

The reference ships no golden vectors or known-answer tests for this path, so
no reference-produced fixture pins any function; the checks above are the
pins.  Tie rule for top-k (value descending, then index ascending) is this
build's contract: ``torch.topk``'s tie order is implementation-defined.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = [
    "bf16_round", "to_bf16_bits", "from_bf16_bits", "num_groups",
    "pack_int4", "unpack_int4", "dequantize", "linear", "gelu_tanh",
    "rms_norm", "router_logits", "topk_from_logits", "router",
    "sort_permute", "moe_forward", "max_abs_rel", "hybridlink",
    "layer_norm", "gelu_erf", "ffn_block", "moe_forward_bf16",
    "dequantize_fp32", "gelu_tanh_fp32", "moe_forward_fp32", "moe_forward_fp32_dequantized",
]


# ---------------------------------------------------------------------------
# bfloat16 emulation
# ---------------------------------------------------------------------------

def to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round to nearest even; NaN kept quiet."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    b = f.view(np.uint32)
    rounded = (b + (np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)
    out = rounded.astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        out = np.where(nan, ((b >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), out)
    return out


def from_bf16_bits(b) -> np.ndarray:
    """bf16 bit pattern (uint16) -> float32 (exact)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (RNE), returned as float32."""
    return from_bf16_bits(to_bf16_bits(x))


def max_abs_rel(y, y_ref) -> float:
    """max|y - y_ref| / max|y_ref| -- the layer-output tolerance metric."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    den = np.max(np.abs(y_ref))
    if den == 0.0:
        return float(np.max(np.abs(y - y_ref)))
    return float(np.max(np.abs(y - y_ref)) / den)


# ---------------------------------------------------------------------------
# packed int4 layout  (quantization.py:1-5, 132-137, 153-159, 191-218)
# ---------------------------------------------------------------------------

def num_groups(K: int, G: int) -> int:
    """Scale columns per row: ceil(K / G) (the reference's K // 32 when 32 | K)."""
    return -(-K // G)


def pack_int4(q) -> np.ndarray:
    """q int in [-8, 7], shape [..., K] (K % 8 == 0) -> int32 [..., K // 8].

    Nibble i of word j stores q[8j + i] + 8 -- the inverse of the unpack at
    quantization.py:136 (``((p >> 4i) & 0xF) - 8``).
    """
    q = np.asarray(q)
    if q.shape[-1] % 8:
        raise ValueError("K must be a multiple of 8")
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("q out of [-8, 7]")
    u = (q.astype(np.int64) + 8).astype(np.uint32)
    u = u.reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    words = np.bitwise_or.reduce(u << shifts, axis=-1).astype(np.uint32)
    return words.view(np.int32)


def unpack_int4(packed) -> np.ndarray:
    """int32 [..., K/8] -> int8 q [..., K]  (quantization.py:136)."""
    p = np.ascontiguousarray(packed, dtype=np.int32).view(np.uint32)
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    q = ((p[..., None] >> shifts) & np.uint32(0xF)).astype(np.int8) - np.int8(8)
    return q.reshape(*p.shape[:-1], p.shape[-1] * 8)


def dequantize(packed, scale_bits, G: int) -> np.ndarray:
    """bf16 weights (as float32 values) [..., N, K]  (quantization.py:132-137).

    ``scale_bits`` are bf16 bit patterns [..., N, ceil(K/G)].  The product
    ``q * s`` is exact in fp32 (|q| <= 8, s has 8 significant bits) and is then
    rounded once to bf16, as the reference's bf16 ``q.to(bf16) * scale`` does.
    """
    q = unpack_int4(packed)
    K = q.shape[-1]
    s = from_bf16_bits(scale_bits)
    ng = num_groups(K, G)
    if s.shape[-1] != ng:
        raise ValueError(f"scale has {s.shape[-1]} groups, expected ceil({K}/{G})={ng}")
    s_full = np.repeat(s, G, axis=-1)[..., :K]
    return bf16_round(q.astype(np.float32) * s_full)


# ---------------------------------------------------------------------------
# dense W4A16 linear  (quantization.py:171-175)
# ---------------------------------------------------------------------------

def _matmul_bf16(x, w) -> np.ndarray:
    """bf16 x [M,K] @ bf16 w [N,K]^T with fp32 accumulation, rounded to bf16."""
    return bf16_round(np.matmul(np.asarray(x, np.float32), np.asarray(w, np.float32).T))


def linear(x, packed, scale_bits, G: int, bias=None) -> np.ndarray:
    """``Linear4Bit.forward``: F.linear(x, dequant(W), bias) in bf16 (quantization.py:171-175).

    ``x`` holds bf16 values as float32 [M, K]; returns bf16 values [M, N].
    A bias (bf16) is added to the fp32 accumulator before the final rounding,
    as a fused addmm does.
    """
    w = dequantize(packed, scale_bits, G)
    acc = np.matmul(np.asarray(x, np.float32), w.T)
    if bias is not None:
        acc = acc + np.asarray(bias, np.float32)
    return bf16_round(acc)


# ---------------------------------------------------------------------------
# activations / norms
# ---------------------------------------------------------------------------

def gelu_tanh(x) -> np.ndarray:
    """``gelu_pytorch_tanh`` = F.gelu(x, approximate="tanh") on bf16 input
    (TF:activations.py:45-48, 330; quantization.py:120, 254, 282): computed in
    fp32, rounded to bf16."""
    x = np.asarray(x, np.float32)
    c = np.float32(math.sqrt(2.0 / math.pi))
    inner = c * (x + np.float32(0.044715) * x * x * x)
    return bf16_round(np.float32(0.5) * x * (np.float32(1.0) + np.tanh(inner)))


def gelu_erf(x) -> np.ndarray:
    """nn.GELU() (exact erf form) in fp32 (hybridlink.py:21)."""
    from math import erf
    x = np.asarray(x, np.float64)
    v = np.vectorize(erf)(x / math.sqrt(2.0))
    return (0.5 * x * (1.0 + v)).astype(np.float32)


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """F.rms_norm on bf16 input: fp32 ``x * rsqrt(mean(x^2) + eps) [* w]`` -> bf16
    (backends.py:68-74, 112; TF:models/gemma4/modeling_gemma4.py:197-215)."""
    x = np.asarray(x, np.float32)
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32) + np.float32(eps)
    y = x * (np.float32(1.0) / np.sqrt(ms))
    if weight is not None:
        y = y * np.asarray(weight, np.float32)
    return bf16_round(y)


def layer_norm(x, weight, bias, eps: float = 1e-5) -> np.ndarray:
    """nn.LayerNorm in fp32 (hybridlink.py:23-24)."""
    x = np.asarray(x, np.float32)
    mu = x.mean(-1, keepdims=True, dtype=np.float32)
    var = ((x - mu) ** 2).mean(-1, keepdims=True, dtype=np.float32)
    return (x - mu) / np.sqrt(var + np.float32(eps)) * weight + bias


def ffn_block(residual, attn_out, post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w,
              post_ff_ln1_w, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale,
              pre_ff_ln2_w, gu_packed, gu_scale, dn_packed, dn_scale, post_ff_ln2_w, post_ff_ln_w,
              layer_scalar, eps, top_k, G, return_routing: bool = False, routing=None):
    """The post-attention FFN block ``_ffn_moe_4bit_step`` (backends.py:101-126), bf16
    rounding after every op as the eager torch ops round:

    * h = rms_norm(attn_out) * w; residual = bf16(residual + h)         (:102-103)
    * shared MLP: down(bf16(bf16(gelu_tanh(gate(h_ff))) * up(h_ff)))  (:105-108)
    * h_1 = rms_norm(h_mlp, post_ff_ln1)                                (:109)
    * router on the residual, MoE on rms_norm(residual, pre_ff_ln2)     (:111-122)
    * h_2 = rms_norm(moe_out, post_ff_ln2); h_comb = rms_norm(bf16(h_1 + h_2), post_ff_ln)
    * out = bf16(bf16(residual + h_comb) * layer_scalar)               (:123-126)

    Dense weights are bf16 values [out, in] (nn.Linear layout); ``layer_scalar``
    is one bf16 value.  Inputs/outputs are bf16 values held as float32.
    ``routing`` = (top_k_index, top_k_weights) replaces the router's decision
    (a row whose 8th and 9th logits are one rounding apart can go either way;
    with the routing a kernel took, every row is checkable).
    """
    h = rms_norm(attn_out, post_attn_ln_w, eps)
    res = bf16_round(np.asarray(residual, np.float32) + h)
    h_ff = rms_norm(res, pre_ff_ln_w, eps)
    gate = gelu_tanh(_matmul_bf16(h_ff, mlp_gate_w))
    up = _matmul_bf16(h_ff, mlp_up_w)
    h_mlp = _matmul_bf16(bf16_round(gate * up), mlp_down_w)
    h_1 = rms_norm(h_mlp, post_ff_ln1_w, eps)
    if routing is None:
        _, idx, w = router(res, router_scale, router_scalar_root, router_proj_w, router_per_expert_scale, eps,
                           top_k)
    else:
        idx, w = (np.asarray(routing[0], np.int64), np.asarray(routing[1], np.float32))
    h_2_in = rms_norm(res, pre_ff_ln2_w, eps)
    h_2 = moe_forward(h_2_in, idx, w, gu_packed, gu_scale, dn_packed, dn_scale, G)
    h_2 = rms_norm(h_2, post_ff_ln2_w, eps)
    h_comb = rms_norm(bf16_round(h_1 + h_2), post_ff_ln_w, eps)
    out = bf16_round(bf16_round(res + h_comb) * np.float32(layer_scalar))
    if return_routing:
        return out, idx, w
    return out


def hybridlink(h, p1w, p1b, p2w, p2b, ln1w, ln1b, ln2w, ln2b) -> np.ndarray:
    """HybridLink R(h) = post_ln(h + proj2(GELU(proj1(pre_ln(h))))) in fp32
    (hybridlink.py:17-28)."""
    h = np.asarray(h, np.float32)
    a = layer_norm(h, ln1w, ln1b) @ np.asarray(p1w, np.float32).T + p1b
    a = gelu_erf(a) @ np.asarray(p2w, np.float32).T + p2b
    return layer_norm(h + a, ln2w, ln2b)


# ---------------------------------------------------------------------------
# router  (backends.py:111-117; TF:models/gemma4/modeling_gemma4.py:1335-1356)
# ---------------------------------------------------------------------------

def router_logits(hidden, router_scale, scalar_root: float, proj_w, eps: float) -> np.ndarray:
    """bf16 expert scores [M, E] (backends.py:111-113).

    ``r = bf16(bf16(rms_norm(h) * scale) * scalar_root)`` then
    ``F.linear(r, W_r)`` with fp32 accumulation rounded to bf16.
    """
    r = rms_norm(hidden, None, eps)
    r = bf16_round(r * np.asarray(router_scale, np.float32))
    r = bf16_round(r * np.float32(scalar_root))
    return _matmul_bf16(r, proj_w)


def topk_from_logits(logits, per_expert_scale, k: int):
    """softmax(fp32) -> top-k -> renormalise -> * per_expert_scale[idx]
    (backends.py:114-117; TF:…/modeling_gemma4.py:1342-1354).

    Selection is done on the bf16 logits (softmax is strictly monotone, so
    the order of probabilities equals the order of logits); ties are broken by
    lower expert index first.  Returns (idx int64 [M, k], w float32 [M, k]).
    """
    lg = np.asarray(logits, np.float32)
    order = np.argsort(-lg, axis=-1, kind="stable")
    idx = order[:, :k].astype(np.int64)
    m = lg.max(axis=-1, keepdims=True)
    e = np.exp(lg - m, dtype=np.float32)
    p = e / e.sum(axis=-1, keepdims=True, dtype=np.float32)
    w = np.take_along_axis(p, idx, axis=-1).astype(np.float32)
    w = w / w.sum(axis=-1, keepdims=True, dtype=np.float32)
    w = w * np.asarray(per_expert_scale, np.float32)[idx]
    return idx, w.astype(np.float32)


def router(hidden, router_scale, scalar_root, proj_w, per_expert_scale, eps, k):
    """Full router: returns (bf16 logits, idx, weights)."""
    lg = router_logits(hidden, router_scale, scalar_root, proj_w, eps)
    idx, w = topk_from_logits(lg, per_expert_scale, k)
    return lg, idx, w


# ---------------------------------------------------------------------------
# token -> expert grouping  (quantization.py:266-276)
# ---------------------------------------------------------------------------

def sort_permute(idx, E: int):
    """Per-expert segments in the reference's implicit order.

    The reference visits experts in ascending order and, for expert e, takes
    ``torch.where(one_hot(idx).permute(2,1,0)[e])`` = (k-slot, token) pairs in
    k-slot-major, token-minor order (quantization.py:268-276).  That is a
    stable sort of the k-major flattening ``idx.T.flatten()`` by expert.

    Returns ``sorted_pos`` int32 [M*k] holding ``t*k + j`` (the row of the
    token-major flattening ``top_k_index.view(-1)``) and ``offsets`` int32
    [E+1] (exclusive prefix sum of per-expert counts).
    """
    idx = np.asarray(idx, np.int64)
    M, k = idx.shape
    kmajor = idx.T.reshape(-1)                       # p = j*M + t
    order = np.argsort(kmajor, kind="stable")
    j = order // M
    t = order % M
    sorted_pos = (t * k + j).astype(np.int32)
    counts = np.bincount(kmajor, minlength=E)[:E]
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    return sorted_pos, offsets


# ---------------------------------------------------------------------------
# MoE forward  (quantization.py:88-129, 241-263, 265-294)
# ---------------------------------------------------------------------------

def _moe_core(hidden, idx, weights, E, I, H, proj_gu, proj_dn, path, return_intermediates=False):
    """The routing, activation and combine of the MoE forward around two
    projections: ``proj_gu(e, x_rows)`` -> bf16 [rows, 2I] and
    ``proj_dn(e, a_rows)`` -> bf16 [rows, H] of expert e."""
    x = np.asarray(hidden, np.float32)
    idx = np.asarray(idx, np.int64)
    w = np.asarray(weights, np.float32)
    M, k = idx.shape
    if path == "fused":
        gu = np.zeros((M * k, 2 * I), np.float32)
        inter = np.zeros((M * k, I), np.float32)
        dn = np.zeros((M, k, H), np.float32)
        for e in np.unique(idx):
            rows = np.nonzero(idx.reshape(-1) == e)[0]          # t*k + j
            tok = rows // k
            g = proj_gu(e, x[tok])                              # :114-118
            gu[rows] = g
            a = bf16_round(gelu_tanh(g[:, :I]) * g[:, I:])     # :119-120
            inter[rows] = a
            dn[tok, rows % k] = proj_dn(e, a)                   # :123-127
        wb = bf16_round(w)                                       # :128
        prod = bf16_round(dn * wb[:, :, None])                   # :129
        y = bf16_round(prod.sum(axis=1, dtype=np.float32))
        if return_intermediates:
            return y, {"gu": gu, "inter": inter, "dn": dn}
        return y
    if path == "loop":
        final = np.zeros((M, H), np.float32)
        mask = np.zeros((E, k, M), bool)                          # :268-269
        for t in range(M):
            for j in range(k):
                mask[idx[t, j], j, t] = True
        for e in np.nonzero(mask.any(axis=(1, 2)))[0]:           # :270-275
            kpos, tok = np.nonzero(mask[e])                       # :276
            g = proj_gu(e, x[tok])                                # :278-281
            a = bf16_round(gelu_tanh(g[:, :I]) * g[:, I:])       # :281-282
            d = proj_dn(e, a)                                     # :283-286
            c = bf16_round(d * w[tok, kpos][:, None])            # :287-291
            final[tok] = bf16_round(final[tok] + c)              # :290-292
        return final
    raise ValueError(f"unknown path {path!r}")


def moe_forward(hidden, idx, weights, gu_packed, gu_scale, dn_packed, dn_scale, G: int,
                path: str = "fused", return_intermediates: bool = False):
    """W4A16 MoE layer output (bf16 values as float32) [M, H].

    ``path="fused"``: rounding points of ``fused_triton_4bit_moe_forward``
    (quantization.py:112-129) and of the single-token path (:241-263).
    ``path="loop"``: the per-expert loop (quantization.py:265-294), bf16
    ``index_add_`` accumulation in ascending expert order.
    """
    E, two_i, _ = gu_packed.shape
    return _moe_core(hidden, idx, weights, E, two_i // 2, dn_packed.shape[1],
                     lambda e, xr: linear(xr, gu_packed[e], gu_scale[e], G),
                     lambda e, ar: linear(ar, dn_packed[e], dn_scale[e], G), path, return_intermediates)


def dequantize_fp32(packed, scale_bits, G: int) -> np.ndarray:
    """q * s in fp32 without the bf16 rounding of the product (exact: |q| <= 8
    and s has 8 significant bits, so the product needs at most 12)."""
    q = unpack_int4(packed)
    K = q.shape[-1]
    s = from_bf16_bits(scale_bits)
    s_full = np.repeat(s, G, axis=-1)[..., :K]
    return q.astype(np.float32) * s_full


def gelu_tanh_fp32(x) -> np.ndarray:
    """F.gelu(x, approximate="tanh") in fp32, not rounded (TF:activations.py:45-48)."""
    x = np.asarray(x, np.float32)
    c = np.float32(math.sqrt(2.0 / math.pi))
    return np.float32(0.5) * x * (np.float32(1.0) + np.tanh(c * (x + np.float32(0.044715) * x * x * x)))


def _moe_fp32_core(hidden, idx, weights, E, I, H, gu_of, dn_of) -> np.ndarray:
    x = np.asarray(hidden, np.float32)
    idx = np.asarray(idx, np.int64)
    w = np.asarray(weights, np.float32)
    M, k = idx.shape
    y = np.zeros((M, H), np.float32)
    flat = idx.reshape(-1)
    for e in np.unique(flat):
        if e < 0 or e >= E:
            continue
        rows = np.nonzero(flat == e)[0]
        tok = rows // k
        g = x[tok] @ gu_of(e).T
        a = gelu_tanh_fp32(g[:, :I]) * g[:, I:]
        d = a @ dn_of(e).T
        np.add.at(y, tok, d * w[tok, rows % k][:, None])
    return y


def moe_forward_fp32(hidden, idx, weights, gu_packed, gu_scale, dn_packed, dn_scale, G: int) -> np.ndarray:
    """The MoE forward of quantization.py:88-129 with every intermediate kept in
    fp32: weights q * s unrounded, fp32 accumulation, no bf16 rounding of
    gate_up, GELU, ``gelu * up``, down, the routing weight or the products;
    output fp32.  The reference's bf16 rounding points (``moe_forward``) are
    the parity contract; this path measures how far they, and a kernel, sit
    from the unrounded arithmetic.  Slots whose expert is outside [0, E)
    contribute nothing."""
    E, two_i, _ = gu_packed.shape
    return _moe_fp32_core(hidden, idx, weights, E, two_i // 2, dn_packed.shape[1],
                          lambda e: dequantize_fp32(gu_packed[e], gu_scale[e], G),
                          lambda e: dequantize_fp32(dn_packed[e], dn_scale[e], G))


def moe_forward_fp32_dequantized(hidden, idx, weights, gu_w, dn_w) -> np.ndarray:
    """``moe_forward_fp32`` on weights already dequantised by ``dequantize_fp32``
    (gu_w [E, 2I, H], dn_w [E, H, I] float32), for callers that reuse them."""
    E, two_i, _ = gu_w.shape
    return _moe_fp32_core(hidden, idx, weights, E, two_i // 2, dn_w.shape[1], lambda e: gu_w[e],
                          lambda e: dn_w[e])


def moe_forward_bf16(hidden, idx, weights, gate_up_proj, down_proj, path: str = "fused"):
    """The BF16 experts (_bf16_experts_fast_forward, backends.py:209-283):
    the same forward with unquantised bf16 weights ``gate_up_proj`` [E, 2I, H]
    and ``down_proj`` [E, H, I] (bf16 values as float32).  ``path="fused"``:
    the T == 1 and T <= 8 branches (bmm / einsum, then a bf16 weighted sum);
    ``path="loop"``: the T > 8 per-expert loop with bf16 ``index_add_``."""
    gate_up_proj = np.asarray(gate_up_proj, np.float32)
    down_proj = np.asarray(down_proj, np.float32)
    E, two_i, _ = gate_up_proj.shape
    return _moe_core(hidden, idx, weights, E, two_i // 2, down_proj.shape[1],
                     lambda e, xr: _matmul_bf16(xr, gate_up_proj[e]),
                     lambda e, ar: _matmul_bf16(ar, down_proj[e]), path)
