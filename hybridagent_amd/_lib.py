"""ctypes binding of libw4a16moe.so (the C ABI declared in include/w4a16moe.h).

Tensors stay owned by PyTorch: this module checks device / dtype / shape /
contiguity, allocates outputs and workspaces through torch's caching
allocator, passes raw device pointers plus ``torch.cuda.current_stream()``,
and maps non-zero status codes to ``ValueError`` (bad arguments) or
``RuntimeError`` (launch failures).  There is no CPU fallback: every entry
point requires CUDA (HIP) tensors and the built library, and raises if
either is missing.
"""
from __future__ import annotations

import ctypes
import os
import threading
import warnings
import weakref
from dataclasses import dataclass
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libw4a16moe.so"

W4A16_OK = 0
_STATUS_EXC = {1: ValueError, 2: ValueError, 3: ValueError, 4: ValueError, 5: ValueError,
               6: RuntimeError}

# kinds of tiled weight copies (enum w4a16_tiled_kind)
TILED_GATE_UP_DECODE, TILED_DOWN_DECODE, TILED_GATE_UP_PREFILL, TILED_DOWN_PREFILL = 0, 1, 2, 3


class TiledExpertsC(ctypes.Structure):
    """struct w4a16_tiled_experts: the tiled copies of one expert stack and its shape."""
    _fields_ = [("E", ctypes.c_int64), ("H", ctypes.c_int64), ("I", ctypes.c_int64),
                ("group_size", ctypes.c_int64),
                ("gu_decode", ctypes.c_void_p), ("gu_decode_bytes", ctypes.c_size_t),
                ("dn_decode", ctypes.c_void_p), ("dn_decode_bytes", ctypes.c_size_t),
                ("gu_prefill", ctypes.c_void_p), ("gu_prefill_bytes", ctypes.c_size_t),
                ("dn_prefill", ctypes.c_void_p), ("dn_prefill_bytes", ctypes.c_size_t)]


# name -> (restype, argtypes); the exact set declared in include/w4a16moe.h
_VP, _I64, _SZ, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
_TP = ctypes.POINTER(TiledExpertsC)
SIGNATURES = {
    "w4a16moe_version": (ctypes.c_int, []),
    "w4a16moe_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "w4a16_dequantize": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I64, _I64, _VP]),
    "w4a16_linear_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "w4a16_add_rms_norm": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _F32, _VP]),
    "w4a16_linear": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "w4a16_hybridlink_workspace_bytes": (_SZ, [_I64, _I64]),
    "w4a16_hybridlink": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64,
                                        _F32, _VP, _SZ, _VP]),
    "moe_router_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "moe_router_topk": (ctypes.c_int, [_VP, _VP, _F32, _VP, _VP, _F32, _I64, _I64, _I64, _I64,
                                       _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_topk_from_logits": (ctypes.c_int, [_VP, _VP, _I64, _I64, _I64, _VP, _VP, _VP]),
    "moe_sort_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "moe_sort_permute": (ctypes.c_int, [_VP, _I64, _I64, _I64, _VP, _VP, _VP, _SZ, _VP]),
    "moe_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "moe_forward": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _VP, _SZ, _VP]),
    "moe_forward_static": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64,
                                          _I64, _I64, _VP]),
    "moe_plan": (ctypes.c_int, [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_gate_up": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_down": (ctypes.c_int, [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_combine": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_layer_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "moe_bf16_experts_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "moe_bf16_experts_forward": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64,
                                                _VP, _SZ, _VP]),
    "moe_ffn_block_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "moe_ffn_block_forward": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _F32, _VP, _VP, _VP,
                                             _VP, _VP, _VP, _VP, _VP, _VP, _VP, _F32, _VP, _I64, _I64, _I64,
                                             _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_layer_forward": (ctypes.c_int, [_VP, _VP, _F32, _VP, _VP, _F32, _VP, _VP, _VP, _VP, _VP, _VP,
                                         _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "w4a16_tiled_bytes": (_SZ, [ctypes.c_int, _I64, _I64, _I64, _I64]),
    "w4a16_tile": (ctypes.c_int, [ctypes.c_int, _VP, _VP, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_gate_up_tiled": (ctypes.c_int, [_VP, _VP, _VP, _TP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_down_tiled": (ctypes.c_int, [_VP, _VP, _TP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_forward_tiled": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _TP, _VP, _I64, _I64, _I64, _I64, _I64,
                                         _I64, _VP, _SZ, _VP]),
    "moe_layer_forward_tiled": (ctypes.c_int, [_VP, _VP, _F32, _VP, _VP, _F32, _VP, _VP, _VP, _VP, _VP, _TP,
                                               _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_layer_forward_add_norm": (ctypes.c_int, [_VP, _VP, _F32, _VP, _VP, _F32, _VP, _VP, _VP, _VP, _VP, _TP,
                                                  _VP, _VP, _VP, _VP, _F32, _VP, _VP, _I64, _I64, _I64, _I64, _I64,
                                                  _I64, _VP, _SZ, _VP]),
    "moe_ffn_block_forward_tiled": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _F32, _VP, _VP,
                                                   _VP, _VP, _VP, _VP, _VP, _TP, _VP, _VP, _VP, _F32, _VP, _I64,
                                                   _I64, _I64, _I64, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "moe_ffn_block_routing_offsets": (ctypes.c_int, [_I64, _I64, _I64, _I64, _I64, _I64,
                                                     ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
}

_lib = None


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raise if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} not found: the W4A16 MoE HIP library is not built "
            "(run `python -m hybridagent_amd.build`); there is no fallback path")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def available() -> bool:
    """True when the library file exists and loads."""
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def status_string(status: int) -> str:
    return load().w4a16moe_status_string(status).decode()


def _check(status: int, what: str) -> None:
    if status != W4A16_OK:
        exc = _STATUS_EXC.get(status, RuntimeError)
        raise exc(f"{what}: {status_string(status)} (status {status})")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "hybridagent_amd W4A16 kernels run on the GPU only (got a CPU tensor); "
                "there is no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    return t.contiguous()


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    return t.contiguous()


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def infer_group_size(K: int, n_groups: int) -> int:
    """Group size G (power of two >= 32) with ceil(K / G) == n_groups."""
    if n_groups <= 0:
        raise ValueError("scale has no groups")
    if n_groups == 1:
        g = 32
        while g < K:
            g *= 2
        return g
    g = 32
    while g <= K:
        if -(-K // g) == n_groups:
            return g
        g *= 2
    raise ValueError(f"no power-of-two group size gives ceil({K}/G) == {n_groups}")


# --------------------------------------------------------------------------- ops

def dequantize(packed: torch.Tensor, scale: torch.Tensor, group_size: int | None = None) -> torch.Tensor:
    """bf16 [..., N, K] = bf16_RNE(q * s)   (quantization.py:132-137)."""
    dev = _require_gpu(packed, scale)
    packed = _i32(packed, "packed")
    scale = _bf16(scale, "scale")
    K = packed.shape[-1] * 8
    if scale.shape[:-1] != packed.shape[:-1]:
        raise ValueError(f"scale leading shape {tuple(scale.shape)} does not match packed {tuple(packed.shape)}")
    G = group_size or infer_group_size(K, scale.shape[-1])
    if scale.shape[-1] != -(-K // G):
        raise ValueError(f"scale has {scale.shape[-1]} groups, expected ceil({K}/{G})")
    out = torch.empty((*packed.shape[:-1], K), dtype=torch.bfloat16, device=dev)
    rows = packed.numel() // max(1, packed.shape[-1])
    with torch.cuda.device(dev):
        _check(load().w4a16_dequantize(_ptr(packed), _ptr(scale), _ptr(out), rows, K, G, _stream(dev)),
               "w4a16_dequantize")
    return out


def add_rms_norm(h: torch.Tensor, weight: torch.Tensor, eps: float,
                 delta: torch.Tensor | None = None):
    """(x, y): x = bf16(h + delta) (h itself without delta), y = RMSNorm(x) * weight in fp32,
    rounded to bf16 (TF:modeling_gemma4.py:197-215); h, delta [..., H] bf16."""
    dev = _require_gpu(h, weight, delta)
    h = _bf16(h, "h")
    weight = _bf16(weight, "weight")
    H = h.shape[-1]
    if weight.shape != (H,):
        raise ValueError(f"weight must be [{H}]")
    h2 = h.reshape(-1, H)
    d2 = None
    if delta is not None:
        d2 = _bf16(delta, "delta").reshape(-1, H)
        if d2.shape != h2.shape:
            raise ValueError("delta must have the shape of h")
    M = h2.shape[0]
    y = torch.empty_like(h2)
    x = torch.empty_like(h2) if d2 is not None else h2
    lib = load()
    with torch.cuda.device(dev):
        _check(lib.w4a16_add_rms_norm(_ptr(h2), _ptr(d2), _ptr(weight), _ptr(x) if d2 is not None else None,
                                      _ptr(y), M, H, float(eps), _stream(dev)), "w4a16_add_rms_norm")
    return x.reshape(h.shape), y.reshape(h.shape)


def hybridlink(h: torch.Tensor, ln1_w: torch.Tensor, ln1_b: torch.Tensor, p1_w: torch.Tensor,
               p1_b: torch.Tensor, p2_w: torch.Tensor, p2_b: torch.Tensor, ln2_w: torch.Tensor,
               ln2_b: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """HybridLink R(h) = post_ln(h + proj2(GELU(proj1(pre_ln(h)))))  (hybridlink.py:17-28);
    h [..., H] bf16, LayerNorm/Linear parameters bf16 in the nn.Module layout."""
    params = (ln1_w, ln1_b, p1_w, p1_b, p2_w, p2_b, ln2_w, ln2_b)
    dev = _require_gpu(h, *params)
    h = _bf16(h, "h")
    H = h.shape[-1]
    names = ("pre_ln weight", "pre_ln bias", "proj1 weight", "proj1 bias", "proj2 weight",
             "proj2 bias", "post_ln weight", "post_ln bias")
    params = tuple(_bf16(p, n) for p, n in zip(params, names))
    for p, n in zip(params, names):
        want = (H, H) if n.endswith("weight") and n.startswith("proj") else (H,)
        if tuple(p.shape) != want:
            raise ValueError(f"{n} must be {list(want)}, got {list(p.shape)}")
    h2 = h.reshape(-1, H)
    B = h2.shape[0]
    out = torch.empty_like(h2)
    lib = load()
    ws = _workspace(lib.w4a16_hybridlink_workspace_bytes(B, H), dev)
    with torch.cuda.device(dev):
        _check(lib.w4a16_hybridlink(_ptr(h2), *[_ptr(p) for p in params], _ptr(out), B, H, float(eps),
                                    _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev)),
               "w4a16_hybridlink")
    return out.reshape(h.shape)


def linear(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
           bias: torch.Tensor | None = None, group_size: int | None = None) -> torch.Tensor:
    """y = x @ dequant(W)^T (+ bias)   (quantization.py:171-175); x [..., K] bf16."""
    dev = _require_gpu(x, w_packed, w_scale, bias)
    x = _bf16(x, "x")
    w_packed = _i32(w_packed, "weight_packed")
    w_scale = _bf16(w_scale, "weight_scale")
    if bias is not None:
        bias = _bf16(bias, "bias")
    N, K8 = w_packed.shape
    K = K8 * 8
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {K}")
    if w_scale.shape[0] != N:
        raise ValueError("weight_scale rows do not match weight_packed")
    G = group_size or infer_group_size(K, w_scale.shape[-1])
    if w_scale.shape[-1] != -(-K // G):
        raise ValueError(f"weight_scale has {w_scale.shape[-1]} groups, expected ceil({K}/{G})")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    lib = load()
    ws = _workspace(lib.w4a16_linear_workspace_bytes(M, K, G), dev)
    with torch.cuda.device(dev):
        _check(lib.w4a16_linear(_ptr(x2), _ptr(w_packed), _ptr(w_scale), _ptr(bias), _ptr(y), M, N, K, G,
                                _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev)),
               "w4a16_linear")
    return y.reshape(*lead, N)


def router_topk(hidden: torch.Tensor, router_scale: torch.Tensor, scalar_root: float,
                proj_w: torch.Tensor, per_expert_scale: torch.Tensor, eps: float, top_k: int,
                return_logits: bool = False):
    """Router of backends.py:111-117 -> (top_k_weights fp32, top_k_index int64[, logits bf16])."""
    dev = _require_gpu(hidden, router_scale, proj_w, per_expert_scale)
    H = hidden.shape[-1]
    h2 = _bf16(hidden, "hidden").reshape(-1, H)
    router_scale = _bf16(router_scale, "router scale")
    proj_w = _bf16(proj_w, "router proj weight")
    per_expert_scale = _bf16(per_expert_scale, "per_expert_scale")
    E = proj_w.shape[0]
    if proj_w.shape[1] != H or router_scale.numel() != H or per_expert_scale.numel() != E:
        raise ValueError("router parameter shapes do not match hidden size / expert count")
    M = h2.shape[0]
    idx = torch.empty((M, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((M, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((M, E), dtype=torch.bfloat16, device=dev) if return_logits else None
    lib = load()
    ws = _workspace(lib.moe_router_workspace_bytes(M, H, E), dev)
    with torch.cuda.device(dev):
        _check(lib.moe_router_topk(_ptr(h2), _ptr(router_scale), float(scalar_root), _ptr(proj_w),
                                   _ptr(per_expert_scale), float(eps), M, H, E, top_k, _ptr(logits),
                                   _ptr(idx), _ptr(w), _ptr(ws), 0 if ws is None else ws.numel(),
                                   _stream(dev)),
               "moe_router_topk")
    if return_logits:
        return w, idx, logits
    return w, idx


def topk_from_logits(logits: torch.Tensor, per_expert_scale: torch.Tensor, top_k: int):
    """softmax/top-k/renormalise/per-expert scale on given bf16 logits [M, E]."""
    dev = _require_gpu(logits, per_expert_scale)
    logits = _bf16(logits, "logits")
    per_expert_scale = _bf16(per_expert_scale, "per_expert_scale")
    M, E = logits.shape
    idx = torch.empty((M, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((M, top_k), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _check(load().moe_topk_from_logits(_ptr(logits), _ptr(per_expert_scale), M, E, top_k, _ptr(idx),
                                           _ptr(w), _stream(dev)),
               "moe_topk_from_logits")
    return w, idx


def sort_permute(top_k_index: torch.Tensor, num_experts: int):
    """(sorted_pos int32 [M*k], expert_offsets int32 [E+1])   (quantization.py:266-276)."""
    dev = _require_gpu(top_k_index)
    idx = top_k_index.to(torch.int64).contiguous()
    M, k = idx.shape
    sorted_pos = torch.empty(M * k, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    lib = load()
    ws = _workspace(lib.moe_sort_workspace_bytes(max(M, 1), k, num_experts), dev)
    with torch.cuda.device(dev):
        _check(lib.moe_sort_permute(_ptr(idx), M, k, num_experts, _ptr(sorted_pos), _ptr(offsets), _ptr(ws),
                                    0 if ws is None else ws.numel(), _stream(dev)),
               "moe_sort_permute")
    return sorted_pos, offsets


def moe_forward(hidden_states: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor,
                gu_packed: torch.Tensor, gu_scale: torch.Tensor, dn_packed: torch.Tensor,
                dn_scale: torch.Tensor, group_size: int | None = None, *, tiles="auto") -> torch.Tensor:
    """W4A16 MoE layer output [T, H] bf16  (quantization.py:88-129).  ``tiles``: the
    stack's tiled weight copies (a TiledWeights), None for none, or "auto" for the
    ones registered for these tensors (register_tiles)."""
    dev = _require_gpu(hidden_states, top_k_index, top_k_weights, gu_packed, gu_scale, dn_packed, dn_scale)
    H = hidden_states.shape[-1]
    x = _bf16(hidden_states, "hidden_states").reshape(-1, H)
    # explicit widths: reshape(0, -1) is ambiguous for an empty batch
    idx = top_k_index.reshape(x.shape[0], top_k_index.shape[-1]).to(torch.int64).contiguous()
    w = top_k_weights.reshape(x.shape[0], top_k_weights.shape[-1]).to(torch.float32).contiguous()
    gu_packed = _i32(gu_packed, "gate_up_packed")
    dn_packed = _i32(dn_packed, "down_packed")
    gu_scale = _bf16(gu_scale, "gate_up_scale")
    dn_scale = _bf16(dn_scale, "down_scale")
    if gu_packed.shape[-1] * 8 != H:
        raise ValueError(f"expert weight shape {tuple(gu_packed.shape)} does not match hidden size {H}")
    E, H, I, G = _expert_shape(gu_packed, gu_scale, dn_packed, dn_scale, group_size)
    if w.shape != idx.shape:
        raise ValueError("top_k_weights and top_k_index shapes differ")
    M, k = idx.shape
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    lib = load()
    ws = _workspace(lib.moe_workspace_bytes(max(M, 1), k, E, H, I), dev)
    st = _resolve_tiles(tiles, gu_packed, gu_scale, dn_packed, dn_scale, E, H, I, G)
    with torch.cuda.device(dev):
        if st is None:
            _check(lib.moe_forward(_ptr(x), _ptr(idx), _ptr(w), _ptr(gu_packed), _ptr(gu_scale), _ptr(dn_packed),
                                   _ptr(dn_scale), _ptr(out), M, k, E, H, I, G, _ptr(ws),
                                   0 if ws is None else ws.numel(), _stream(dev)),
                   "moe_forward")
        else:
            _check(lib.moe_forward_tiled(_ptr(x), _ptr(idx), _ptr(w), _ptr(gu_packed), _ptr(gu_scale),
                                         _ptr(dn_packed), _ptr(dn_scale), ctypes.byref(st), _ptr(out), M, k, E, H,
                                         I, G, _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev)),
                   "moe_forward_tiled")
    return out.reshape(*hidden_states.shape[:-1], H)


@dataclass
class TiledWeights:
    """Load-time tiled copies of one expert stack's packed weights (a re-layout
    beside quantization.py:325-430; the packed tensors stay as they are): the
    decode streamers' copies (group size 128, 32 or 64; at 32 and 64 they hold
    the group scales too) and the prefill GEMM's.  Any of them may be None:
    that kernel then reads the packed tensors."""
    E: int
    H: int
    I: int
    group_size: int
    gu_decode: torch.Tensor | None = None
    dn_decode: torch.Tensor | None = None
    gu_prefill: torch.Tensor | None = None
    dn_prefill: torch.Tensor | None = None

    def struct(self) -> TiledExpertsC:
        """The w4a16_tiled_experts the *_tiled entry points take."""
        nb = lambda t: 0 if t is None else t.numel() * t.element_size()
        return TiledExpertsC(self.E, self.H, self.I, self.group_size,
                             _ptr(self.gu_decode), nb(self.gu_decode), _ptr(self.dn_decode), nb(self.dn_decode),
                             _ptr(self.gu_prefill), nb(self.gu_prefill), _ptr(self.dn_prefill), nb(self.dn_prefill))

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.gu_decode, self.dn_decode, self.gu_prefill,
                                                          self.dn_prefill) if t is not None)


def tiled_bytes(kind: int, E: int, H: int, I: int, group_size: int) -> int:
    """Bytes of a tiled copy of ``kind`` (TILED_*) for the shape, 0 where none exists."""
    return load().w4a16_tiled_bytes(kind, E, H, I, group_size)


def _tile(kind: int, packed: torch.Tensor, scale: torch.Tensor | None, E: int, H: int, I: int, G: int):
    nbytes = tiled_bytes(kind, E, H, I, G)
    if nbytes == 0:
        return None
    dev = packed.device
    tiled = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _check(load().w4a16_tile(kind, _ptr(packed), _ptr(scale), E, H, I, G, _ptr(tiled), nbytes, _stream(dev)),
               "w4a16_tile")
    return tiled


def _expert_shape(gu_packed, gu_scale, dn_packed, dn_scale, group_size):
    E, two_i, h8 = gu_packed.shape
    H, I = h8 * 8, two_i // 2
    if dn_packed.shape != (E, H, I // 8) or two_i % 2:
        raise ValueError(f"expert weight shapes {tuple(gu_packed.shape)} / {tuple(dn_packed.shape)} do not match")
    G = group_size or infer_group_size(H, gu_scale.shape[-1])
    if gu_scale.shape != (E, two_i, -(-H // G)) or dn_scale.shape != (E, H, -(-I // G)):
        raise ValueError(f"scale shapes {tuple(gu_scale.shape)} / {tuple(dn_scale.shape)} "
                         f"do not match group size {G}")
    return E, H, I, G


def tile_experts(gu_packed: torch.Tensor, gu_scale: torch.Tensor, dn_packed: torch.Tensor,
                 dn_scale: torch.Tensor, group_size: int | None = None, decode: bool = True,
                 prefill: bool = True) -> TiledWeights:
    """The tiled copies of an expert stack (gate_up_packed [E, 2I, H/8], down_packed
    [E, H, I/8] and their scales): ``decode`` the decode streamers' (where they have
    a tiled form for the group size), ``prefill`` the prefill GEMM's.  About one more
    copy of the expert weights per kind asked for."""
    dev = _require_gpu(gu_packed, gu_scale, dn_packed, dn_scale)
    gu_packed, dn_packed = _i32(gu_packed, "gate_up_packed"), _i32(dn_packed, "down_packed")
    gu_scale, dn_scale = _bf16(gu_scale, "gate_up_scale"), _bf16(dn_scale, "down_scale")
    E, H, I, G = _expert_shape(gu_packed, gu_scale, dn_packed, dn_scale, group_size)
    tw = TiledWeights(E, H, I, G)
    if decode:
        tw.gu_decode = _tile(TILED_GATE_UP_DECODE, gu_packed, gu_scale, E, H, I, G)
        tw.dn_decode = _tile(TILED_DOWN_DECODE, dn_packed, dn_scale, E, H, I, G)
    if prefill:
        tw.gu_prefill = _tile(TILED_GATE_UP_PREFILL, gu_packed, None, E, H, I, G)
        tw.dn_prefill = _tile(TILED_DOWN_PREFILL, dn_packed, None, E, H, I, G)
    del dev
    return tw


# ------------------------------------------------------------ tiled-copy registry
# The reference's entry points pass only the packed tensors (the 7 arguments of
# fused_triton_4bit_moe_forward / hybrid_agent::fused_4bit_moe, quantization.py:88-96,
# backends.py:48-60, and the 22 of _ffn_moe_4bit_step).  Copies registered for a
# stack are found from those tensors: keyed by the packed gate_up buffer's address,
# valid while all four tensors are the ones tiled (same addresses, shapes and
# version counters -- an in-place reload through copy_ / load_state_dict bumps the
# counter).  A stale entry is dropped and the call reads the packed tensors.
_REGISTRY: dict[int, tuple] = {}
_REGISTRY_LOCK = threading.Lock()


def _version_of(t: torch.Tensor):
    # inference-mode tensors keep no version counter (and cannot be changed in
    # place outside inference mode)
    try:
        return t._version
    except RuntimeError:
        return None


def _signature(*ts: torch.Tensor) -> tuple:
    return tuple((t.data_ptr(), tuple(t.shape), _version_of(t)) for t in ts)


def register_tiles(gu_packed: torch.Tensor, gu_scale: torch.Tensor, dn_packed: torch.Tensor,
                   dn_scale: torch.Tensor, tiles: TiledWeights) -> None:
    """Make ``tiles`` the copies every forward finds for this expert stack."""
    key = gu_packed.data_ptr()
    entry = (_signature(gu_packed, gu_scale, dn_packed, dn_scale), tiles)
    with _REGISTRY_LOCK:
        _REGISTRY[key] = entry
    # the entry goes when the packed tensor does (its address may be reused)
    weakref.finalize(gu_packed, _drop_if_same, key, entry)


def _drop_if_same(key: int, entry) -> None:
    with _REGISTRY_LOCK:
        if _REGISTRY.get(key) is entry:
            del _REGISTRY[key]


def unregister_tiles(gu_packed: torch.Tensor) -> None:
    with _REGISTRY_LOCK:
        _REGISTRY.pop(gu_packed.data_ptr(), None)


def lookup_tiles(gu_packed: torch.Tensor, gu_scale: torch.Tensor, dn_packed: torch.Tensor,
                 dn_scale: torch.Tensor) -> TiledWeights | None:
    """The registered copies of this expert stack, or None (none, or stale: then dropped)."""
    if not _REGISTRY:
        return None
    key = gu_packed.data_ptr()
    with _REGISTRY_LOCK:
        entry = _REGISTRY.get(key)
        if entry is None:
            return None
        if entry[0] != _signature(gu_packed, gu_scale, dn_packed, dn_scale):
            del _REGISTRY[key]
            stale = True
        else:
            return entry[1]
    if stale:
        warnings.warn("the tiled copies of an expert stack were dropped: its weights changed after they were "
                      "made (tile them again to use them); this call reads the packed weights", RuntimeWarning,
                      stacklevel=3)
    return None


def _resolve_tiles(tiles, gu_packed, gu_scale, dn_packed, dn_scale, E, H, I, G):
    """``tiles`` "auto": the registry's (if made for this call's shape and group
    size); None: none; else the given TiledWeights, which must be for this shape
    (the C ABI checks it again)."""
    if isinstance(tiles, str):
        if tiles != "auto":
            raise ValueError("tiles must be 'auto', None or a TiledWeights")
        tiles = lookup_tiles(gu_packed, gu_scale, dn_packed, dn_scale)
        if tiles is not None and (tiles.E, tiles.H, tiles.I, tiles.group_size) != (E, H, I, G):
            tiles = None
    if tiles is None:
        return None
    if (tiles.E, tiles.H, tiles.I, tiles.group_size) != (E, H, I, G):
        raise ValueError(f"tiled copies are for (E, H, I, G) = {(tiles.E, tiles.H, tiles.I, tiles.group_size)}, "
                         f"the call is {(E, H, I, G)}")
    return tiles.struct()


def moe_layer_forward(router_in: torch.Tensor, router_scale: torch.Tensor, scalar_root: float,
                      proj_w: torch.Tensor, per_expert_scale: torch.Tensor, eps: float, top_k: int,
                      hidden_states: torch.Tensor, gu_packed: torch.Tensor, gu_scale: torch.Tensor,
                      dn_packed: torch.Tensor, dn_scale: torch.Tensor, group_size: int | None = None,
                      *, tiles="auto"):
    """Router (backends.py:111-117) on ``router_in`` + experts (quantization.py:88-129) on
    ``hidden_states`` in one call -> (out [T, H] bf16, top_k_weights fp32, top_k_index int64).
    ``tiles`` as for moe_forward."""
    dev = _require_gpu(router_in, router_scale, proj_w, per_expert_scale, hidden_states, gu_packed,
                       gu_scale, dn_packed, dn_scale)
    H = hidden_states.shape[-1]
    r2 = _bf16(router_in, "router_in").reshape(-1, H)
    x = _bf16(hidden_states, "hidden_states").reshape(-1, H)
    if r2.shape != x.shape:
        raise ValueError("router input and expert input must have the same shape")
    router_scale = _bf16(router_scale, "router scale")
    proj_w = _bf16(proj_w, "router proj weight")
    per_expert_scale = _bf16(per_expert_scale, "per_expert_scale")
    gu_packed, dn_packed = _i32(gu_packed, "gate_up_packed"), _i32(dn_packed, "down_packed")
    gu_scale, dn_scale = _bf16(gu_scale, "gate_up_scale"), _bf16(dn_scale, "down_scale")
    if gu_packed.shape[-1] * 8 != H:
        raise ValueError("expert weight shapes do not match the hidden size")
    E, H, I, G = _expert_shape(gu_packed, gu_scale, dn_packed, dn_scale, group_size)
    if proj_w.shape != (E, H):
        raise ValueError("router weight shape does not match the experts")
    M = x.shape[0]
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((M, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((M, top_k), dtype=torch.float32, device=dev)
    lib = load()
    ws = _workspace(lib.moe_layer_workspace_bytes(max(M, 1), top_k, E, H, I), dev)
    st = _resolve_tiles(tiles, gu_packed, gu_scale, dn_packed, dn_scale, E, H, I, G)
    common = (_ptr(r2), _ptr(router_scale), float(scalar_root), _ptr(proj_w), _ptr(per_expert_scale), float(eps),
              _ptr(x), _ptr(gu_packed), _ptr(gu_scale), _ptr(dn_packed), _ptr(dn_scale))
    tail = (_ptr(out), _ptr(idx), _ptr(w), M, top_k, E, H, I, G, _ptr(ws), 0 if ws is None else ws.numel(),
            _stream(dev))
    with torch.cuda.device(dev):
        if st is None:
            _check(lib.moe_layer_forward(*common, *tail), "moe_layer_forward")
        else:
            _check(lib.moe_layer_forward_tiled(*common, ctypes.byref(st), *tail), "moe_layer_forward_tiled")
    return out.reshape(*hidden_states.shape[:-1], H), w, idx


def moe_layer_forward_add_norm(router_in: torch.Tensor, router_scale: torch.Tensor, scalar_root: float,
                               proj_w: torch.Tensor, per_expert_scale: torch.Tensor, eps: float, top_k: int,
                               hidden_states: torch.Tensor, gu_packed: torch.Tensor, gu_scale: torch.Tensor,
                               dn_packed: torch.Tensor, dn_scale: torch.Tensor, norm_weight: torch.Tensor,
                               norm_eps: float, group_size: int | None = None, *, tiles="auto"):
    """moe_layer_forward on (router_in = h, hidden_states), then h_out = bf16(h + out) and
    y = RMSNorm(h_out) * norm_weight (add_rms_norm's arithmetic), the combine, the add and
    the norm in one launch where the layer has a combine launch of its own (the latent
    harness's step) -> (h_out, y, out, top_k_weights, top_k_index)."""
    dev = _require_gpu(router_in, router_scale, proj_w, per_expert_scale, hidden_states, gu_packed,
                       gu_scale, dn_packed, dn_scale, norm_weight)
    H = hidden_states.shape[-1]
    r2 = _bf16(router_in, "router_in").reshape(-1, H)
    x = _bf16(hidden_states, "hidden_states").reshape(-1, H)
    if r2.shape != x.shape:
        raise ValueError("router input and expert input must have the same shape")
    norm_weight = _bf16(norm_weight, "norm weight")
    if norm_weight.shape != (H,):
        raise ValueError(f"norm weight must be [{H}]")
    router_scale = _bf16(router_scale, "router scale")
    proj_w = _bf16(proj_w, "router proj weight")
    per_expert_scale = _bf16(per_expert_scale, "per_expert_scale")
    gu_packed, dn_packed = _i32(gu_packed, "gate_up_packed"), _i32(dn_packed, "down_packed")
    gu_scale, dn_scale = _bf16(gu_scale, "gate_up_scale"), _bf16(dn_scale, "down_scale")
    E, H, I, G = _expert_shape(gu_packed, gu_scale, dn_packed, dn_scale, group_size)
    if proj_w.shape != (E, H):
        raise ValueError("router weight shape does not match the experts")
    M = x.shape[0]
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    h_out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    y = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((M, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((M, top_k), dtype=torch.float32, device=dev)
    lib = load()
    ws = _workspace(lib.moe_layer_workspace_bytes(max(M, 1), top_k, E, H, I), dev)
    st = _resolve_tiles(tiles, gu_packed, gu_scale, dn_packed, dn_scale, E, H, I, G)
    with torch.cuda.device(dev):
        _check(lib.moe_layer_forward_add_norm(
            _ptr(r2), _ptr(router_scale), float(scalar_root), _ptr(proj_w), _ptr(per_expert_scale), float(eps),
            _ptr(x), _ptr(gu_packed), _ptr(gu_scale), _ptr(dn_packed), _ptr(dn_scale),
            None if st is None else ctypes.byref(st), _ptr(out), _ptr(idx), _ptr(w), _ptr(norm_weight),
            float(norm_eps), _ptr(h_out), _ptr(y), M, top_k, E, H, I, G, _ptr(ws),
            0 if ws is None else ws.numel(), _stream(dev)), "moe_layer_forward_add_norm")
    shape = hidden_states.shape
    return h_out.reshape(shape), y.reshape(shape), out.reshape(shape), w, idx


def bf16_experts_forward(hidden_states: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor,
                         gate_up_proj: torch.Tensor, down_proj: torch.Tensor) -> torch.Tensor:
    """MoE output [T, H] with unquantised bf16 experts (backends.py:209-283):
    gate_up_proj [E, 2I, H], down_proj [E, H, I] (Gemma4TextExperts parameters)."""
    dev = _require_gpu(hidden_states, top_k_index, top_k_weights, gate_up_proj, down_proj)
    H = hidden_states.shape[-1]
    x = _bf16(hidden_states, "hidden_states").reshape(-1, H)
    idx = top_k_index.reshape(x.shape[0], top_k_index.shape[-1]).to(torch.int64).contiguous()
    w = top_k_weights.reshape(x.shape[0], top_k_weights.shape[-1]).to(torch.float32).contiguous()
    gu = _bf16(gate_up_proj, "gate_up_proj")
    dn = _bf16(down_proj, "down_proj")
    E, two_i, h = gu.shape
    I = two_i // 2
    if h != H or two_i % 2 or dn.shape != (E, H, I):
        raise ValueError(f"expert weight shapes {tuple(gu.shape)} / {tuple(dn.shape)} do not match hidden size {H}")
    if w.shape != idx.shape:
        raise ValueError("top_k_weights and top_k_index shapes differ")
    M, k = idx.shape
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    lib = load()
    ws = _workspace(lib.moe_bf16_experts_workspace_bytes(max(M, 1), k, E, H, I), dev)
    with torch.cuda.device(dev):
        _check(lib.moe_bf16_experts_forward(_ptr(x), _ptr(idx), _ptr(w), _ptr(gu), _ptr(dn), _ptr(out), M, k, E,
                                            H, I, _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev)),
               "moe_bf16_experts_forward")
    return out.reshape(*hidden_states.shape[:-1], H)


def ffn_block(residual: torch.Tensor, attn_out: torch.Tensor, post_attn_ln_w: torch.Tensor,
              pre_ff_ln_w: torch.Tensor, mlp_gate_w: torch.Tensor, mlp_up_w: torch.Tensor,
              mlp_down_w: torch.Tensor, post_ff_ln1_w: torch.Tensor, router_scale: torch.Tensor,
              router_scalar_root: float, router_proj_w: torch.Tensor, router_per_expert_scale: torch.Tensor,
              pre_ff_ln2_w: torch.Tensor, gu_packed: torch.Tensor, gu_scale: torch.Tensor,
              dn_packed: torch.Tensor, dn_scale: torch.Tensor, post_ff_ln2_w: torch.Tensor,
              post_ff_ln_w: torch.Tensor, layer_scalar: torch.Tensor, eps: float, top_k: int,
              group_size: int | None = None, *, tiles="auto", return_routing: bool = False):
    """The post-attention FFN block ``_ffn_moe_4bit_step`` (backends.py:77-126), same
    arguments in the same order: residual / attn_out [..., H] bf16 -> [..., H] bf16.
    ``tiles`` as for moe_forward.  With ``return_routing`` also the routing the block's
    router step took: (out, top_k_index int64 [M, k], top_k_weights fp32 [M, k])."""
    dense = (post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w, post_ff_ln1_w, router_scale,
             router_proj_w, router_per_expert_scale, pre_ff_ln2_w, post_ff_ln2_w, post_ff_ln_w)
    dev = _require_gpu(residual, attn_out, *dense, gu_packed, gu_scale, dn_packed, dn_scale, layer_scalar)
    H = residual.shape[-1]
    res = _bf16(residual, "residual").reshape(-1, H)
    att = _bf16(attn_out, "attn_out").reshape(-1, H)
    if att.shape != res.shape:
        raise ValueError("attn_out must have the shape of residual")
    names = ("post_attention_layernorm", "pre_feedforward_layernorm", "mlp.gate_proj", "mlp.up_proj",
             "mlp.down_proj", "post_feedforward_layernorm_1", "router.scale", "router.proj",
             "router.per_expert_scale", "pre_feedforward_layernorm_2", "post_feedforward_layernorm_2",
             "post_feedforward_layernorm")
    dense = tuple(_bf16(t, n) for t, n in zip(dense, names))
    (post_attn_ln_w, pre_ff_ln_w, mlp_gate_w, mlp_up_w, mlp_down_w, post_ff_ln1_w, router_scale,
     router_proj_w, router_per_expert_scale, pre_ff_ln2_w, post_ff_ln2_w, post_ff_ln_w) = dense
    # layer_scalar is a bf16 buffer once the model is loaded in bf16; other
    # dtypes are rounded to it (the product is a bf16 tensor either way)
    ls = layer_scalar.reshape(-1)[:1].to(torch.bfloat16).contiguous()
    for t, n in ((post_attn_ln_w, names[0]), (pre_ff_ln_w, names[1]), (post_ff_ln1_w, names[5]),
                 (router_scale, names[6]), (pre_ff_ln2_w, names[9]), (post_ff_ln2_w, names[10]),
                 (post_ff_ln_w, names[11])):
        if tuple(t.shape) != (H,):
            raise ValueError(f"{n} weight must be [{H}]")
    Im = mlp_gate_w.shape[0]
    if tuple(mlp_gate_w.shape) != (Im, H) or tuple(mlp_up_w.shape) != (Im, H) or tuple(mlp_down_w.shape) != (H, Im):
        raise ValueError("shared MLP weights must be gate/up [Im, H] and down [H, Im]")
    gu_packed, dn_packed = _i32(gu_packed, "gate_up_packed"), _i32(dn_packed, "down_packed")
    gu_scale, dn_scale = _bf16(gu_scale, "gate_up_scale"), _bf16(dn_scale, "down_scale")
    if gu_packed.shape[-1] * 8 != H:
        raise ValueError("expert weight shapes do not match the hidden size")
    E, H, I, G = _expert_shape(gu_packed, gu_scale, dn_packed, dn_scale, group_size)
    if router_proj_w.shape != (E, H):
        raise ValueError("router weight shape does not match the experts")
    M = res.shape[0]
    out = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    lib = load()
    ws = _workspace(lib.moe_ffn_block_workspace_bytes(max(M, 1), top_k, E, H, I, Im), dev)
    st = _resolve_tiles(tiles, gu_packed, gu_scale, dn_packed, dn_scale, E, H, I, G)
    head = (_ptr(res), _ptr(att), _ptr(post_attn_ln_w), _ptr(pre_ff_ln_w), _ptr(mlp_gate_w), _ptr(mlp_up_w),
            _ptr(mlp_down_w), _ptr(post_ff_ln1_w), _ptr(router_scale), float(router_scalar_root),
            _ptr(router_proj_w), _ptr(router_per_expert_scale), _ptr(pre_ff_ln2_w), _ptr(gu_packed),
            _ptr(gu_scale), _ptr(dn_packed), _ptr(dn_scale))
    tail = (_ptr(post_ff_ln2_w), _ptr(post_ff_ln_w), _ptr(ls), float(eps), _ptr(out), M, int(top_k), E, H, I, Im,
            G, _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))
    with torch.cuda.device(dev):
        if st is None:
            _check(lib.moe_ffn_block_forward(*head, *tail), "moe_ffn_block_forward")
        else:
            _check(lib.moe_ffn_block_forward_tiled(*head, ctypes.byref(st), *tail), "moe_ffn_block_forward_tiled")
    out = out.reshape(residual.shape)
    if not return_routing:
        return out
    if M == 0:
        return out, torch.empty((0, top_k), dtype=torch.int64, device=dev), \
            torch.empty((0, top_k), dtype=torch.float32, device=dev)
    io, wo = ctypes.c_size_t(), ctypes.c_size_t()
    _check(lib.moe_ffn_block_routing_offsets(M, top_k, E, H, I, Im, ctypes.byref(io), ctypes.byref(wo)),
           "moe_ffn_block_routing_offsets")
    n = M * top_k
    idx = ws[io.value:io.value + 8 * n].view(torch.int64).reshape(M, top_k).clone()
    w = ws[wo.value:wo.value + 4 * n].view(torch.float32).reshape(M, top_k).clone()
    return out, idx, w


class MoEStages:
    """The four stages of ``moe_forward`` on one preallocated workspace.

    For callers that schedule or time the stages separately (the benchmark
    times ``gate_up`` alone); ``forward`` runs all four.  Sizes are fixed at
    construction; the workspace carries the routing plan and intermediates
    between stages, so calls must be made in order on one stream.
    """

    def __init__(self, M: int, top_k: int, E: int, H: int, I: int, group_size: int, device):
        self.M, self.k, self.E, self.H, self.I, self.G = M, top_k, E, H, I, group_size
        self.device = torch.device(device)
        self.lib = load()
        nbytes = self.lib.moe_workspace_bytes(max(M, 1), top_k, E, H, I)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.out = torch.empty((M, H), dtype=torch.bfloat16, device=self.device)

    def _dims(self):
        return self.M, self.k, self.E, self.H, self.I

    def plan(self, hidden: torch.Tensor, top_k_index: torch.Tensor) -> None:
        s = _stream(self.device)
        _check(self.lib.moe_plan(_ptr(hidden), _ptr(top_k_index), *self._dims(), self.G, _ptr(self.ws),
                                 self.ws.numel(), s), "moe_plan")

    def gate_up(self, hidden: torch.Tensor, gu_packed: torch.Tensor, gu_scale: torch.Tensor,
                tiles: TiledWeights | None = None) -> None:
        """Grouped gate_up GEMM; ``tiles`` (the stack's TiledWeights) serve the kernels
        that read them."""
        s = _stream(self.device)
        if tiles is None:
            _check(self.lib.moe_gate_up(_ptr(hidden), _ptr(gu_packed), _ptr(gu_scale), *self._dims(), self.G,
                                        _ptr(self.ws), self.ws.numel(), s), "moe_gate_up")
        else:
            st = tiles.struct()
            _check(self.lib.moe_gate_up_tiled(_ptr(hidden), _ptr(gu_packed), _ptr(gu_scale), ctypes.byref(st),
                                              *self._dims(), self.G, _ptr(self.ws), self.ws.numel(), s),
                   "moe_gate_up_tiled")

    def down(self, dn_packed: torch.Tensor, dn_scale: torch.Tensor, tiles: TiledWeights | None = None) -> None:
        """Grouped down GEMM; ``tiles`` serve the kernels that read them."""
        s = _stream(self.device)
        if tiles is None:
            _check(self.lib.moe_down(_ptr(dn_packed), _ptr(dn_scale), *self._dims(), self.G, _ptr(self.ws),
                                     self.ws.numel(), s), "moe_down")
        else:
            st = tiles.struct()
            _check(self.lib.moe_down_tiled(_ptr(dn_packed), _ptr(dn_scale), ctypes.byref(st), *self._dims(),
                                           self.G, _ptr(self.ws), self.ws.numel(), s), "moe_down_tiled")

    def combine(self, top_k_index: torch.Tensor, top_k_weights: torch.Tensor) -> torch.Tensor:
        s = _stream(self.device)
        _check(self.lib.moe_combine(_ptr(top_k_index), _ptr(top_k_weights), _ptr(self.out), *self._dims(),
                                    _ptr(self.ws), self.ws.numel(), s), "moe_combine")
        return self.out

    def forward(self, hidden, top_k_index, top_k_weights, gu_packed, gu_scale, dn_packed, dn_scale):
        for t in (hidden, top_k_index, top_k_weights, gu_packed, gu_scale, dn_packed, dn_scale):
            if not t.is_contiguous() or t.device != self.device:
                raise ValueError("MoEStages.forward expects contiguous tensors on its device")
        self.plan(hidden, top_k_index)
        self.gate_up(hidden, gu_packed, gu_scale)
        self.down(dn_packed, dn_scale)
        return self.combine(top_k_index, top_k_weights)
