"""C-ABI library checks that need no GPU: it loads, exports exactly what
include/w4a16moe.h declares, and rejects bad arguments on the host before any
HIP call (status codes -> Python exceptions)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from hybridagent_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "w4a16moe.h"


def header_functions():
    txt = HEADER.read_text()
    return set(re.findall(r"W4A16_API\s+[\w\s\*]+?\b(\w+)\s*\(", txt))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libw4a16moe.so not built")
    return _lib.load()


def test_header_matches_binding_table():
    assert header_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_header_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name


def test_version_and_status_strings(lib):
    assert lib.w4a16moe_version() >> 16 == 0
    for code in range(7):
        assert lib.w4a16moe_status_string(code)
    assert lib.w4a16moe_status_string(0).decode() == "ok"


NULL = None


def test_linear_host_validation(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    # K not a multiple of 32
    assert lib.w4a16_linear(fake, fake, fake, NULL, fake, 4, 16, 40, 32, NULL, 0, NULL) == 2
    # group size not a power of two / too small
    assert lib.w4a16_linear(fake, fake, fake, NULL, fake, 4, 16, 64, 48, NULL, 0, NULL) == 3
    assert lib.w4a16_linear(fake, fake, fake, NULL, fake, 4, 16, 64, 16, NULL, 0, NULL) == 3
    # null pointer
    assert lib.w4a16_linear(NULL, fake, fake, NULL, fake, 4, 16, 64, 32, NULL, 0, NULL) == 1
    # misaligned activation pointer
    assert lib.w4a16_linear(ctypes.c_void_p(4098), fake, fake, NULL, fake, 4, 16, 64, 32, NULL, 0, NULL) == 4
    # the dense path needs no scratch memory
    assert lib.w4a16_linear_workspace_bytes(4, 256, 128) == 0


def test_add_rms_norm_host_validation(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    f = lib.w4a16_add_rms_norm
    assert f(fake, NULL, fake, NULL, fake, 4, 12, 1e-6, NULL) == 2       # H % 8
    assert f(fake, NULL, fake, NULL, fake, 4, 8200, 1e-6, NULL) == 2     # H > 8192
    assert f(NULL, NULL, fake, NULL, fake, 4, 64, 1e-6, NULL) == 1       # h missing
    assert f(fake, fake, fake, NULL, fake, 4, 64, 1e-6, NULL) == 1       # delta without h_out
    assert f(ctypes.c_void_p(4098), NULL, fake, NULL, fake, 4, 64, 1e-6, NULL) == 4
    assert f(NULL, NULL, NULL, NULL, NULL, 0, 64, 1e-6, NULL) == 0       # nothing to do
    # K beyond what one LDS pass stages
    assert lib.w4a16_linear(fake, fake, fake, NULL, fake, 4, 16, 32768, 128, NULL, 0, NULL) == 2
    # M == 0 is a no-op
    assert lib.w4a16_linear(NULL, NULL, NULL, NULL, NULL, 0, 16, 64, 32, NULL, 0, NULL) == 0


def test_hybridlink_host_validation(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    p = [fake] * 9
    need = lib.w4a16_hybridlink_workspace_bytes(32, 2816)
    assert need >= 2 * 32 * 2816 * 2
    f = lib.w4a16_hybridlink
    assert f(*p, fake, 32, 2800, 1e-5, fake, need, NULL) == 2      # H % 32
    assert f(*p, fake, 32, 8224, 1e-5, fake, need, NULL) == 2      # H > 8192
    assert f(*p[:8], NULL, fake, 32, 2816, 1e-5, fake, need, NULL) == 1   # post_ln bias missing
    assert f(*p, fake, 32, 2816, 1e-5, fake, need - 1, NULL) == 5  # workspace too small
    assert f(ctypes.c_void_p(4098), *p[1:], fake, 32, 2816, 1e-5, fake, need, NULL) == 4
    assert f(*([NULL] * 10), 0, 2816, 1e-5, NULL, 0, NULL) == 0    # nothing to do
    # batch limit: the linears' grid.y = ceil(B / 64) must stay <= 65535
    big = 65535 * 64
    assert f(*p, fake, big + 1, 2816, 1e-5, fake, 1 << 62, NULL) == 2


def test_row_launch_limits(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    # one 256-thread workgroup per row: rows * 256 must stay below 2^32
    assert lib.w4a16_add_rms_norm(fake, NULL, fake, NULL, fake, 1 << 24, 64, 1e-6, NULL) == 2
    # dense weights whose packed bytes reach 2 GiB would overflow the 32-bit
    # buffer offsets: rejected instead of reading the wrong rows
    assert lib.w4a16_linear(fake, fake, fake, NULL, fake, 4, 1 << 20, 4096, 128, NULL, 0, NULL) == 2
    # just below the limit the shape passes (and the missing x is reported)
    assert lib.w4a16_linear(NULL, fake, fake, NULL, fake, 4, (1 << 20) - 8, 4096, 128, NULL, 0,
                            NULL) == 1


def test_moe_host_validation(lib):
    fake = ctypes.c_void_p(4096)
    args = [fake] * 8
    ws_need = lib.moe_workspace_bytes(8, 8, 128, 2816, 704)
    assert ws_need > 8 * 8 * (2816 + 704) * 2
    # E too large
    assert lib.moe_forward(*args, 8, 8, 1024, 2816, 704, 128, fake, ws_need, NULL) == 2
    # top_k > 32
    assert lib.moe_forward(*args, 8, 33, 128, 2816, 704, 128, fake, ws_need, NULL) == 2
    # I not a multiple of 32
    assert lib.moe_forward(*args, 8, 8, 128, 2816, 700, 128, fake, ws_need, NULL) == 2
    # bad group
    assert lib.moe_forward(*args, 8, 8, 128, 2816, 704, 96, fake, ws_need, NULL) == 3
    # workspace too small
    assert lib.moe_forward(*args, 8, 8, 128, 2816, 704, 128, fake, ws_need - 1, NULL) == 5
    # null weight pointer
    bad = list(args)
    bad[3] = NULL
    assert lib.moe_forward(*bad, 8, 8, 128, 2816, 704, 128, fake, ws_need, NULL) == 1
    # router: top_k > E
    assert lib.moe_router_topk(fake, fake, 0.1, fake, fake, 1e-6, 4, 2816, 4, 8, NULL, fake, fake,
                               fake, 1 << 20, NULL) == 2
    assert lib.moe_topk_from_logits(fake, fake, 4, 128, 0, fake, fake, NULL) == 2
    assert lib.moe_sort_permute(fake, 4, 8, 128, fake, fake, NULL, 0, NULL) == 5
    # fused layer: workspace too small, then a misaligned router scale
    lw = lib.moe_layer_workspace_bytes(8, 8, 128, 2816, 704)
    assert lw > ws_need
    largs = [fake, fake, 0.1, fake, fake, 1e-6, fake, fake, fake, fake, fake, fake, fake, fake]
    assert lib.moe_layer_forward(*largs, 8, 8, 128, 2816, 704, 128, fake, lw - 1, NULL) == 5
    largs[1] = ctypes.c_void_p(4098)
    assert lib.moe_layer_forward(*largs, 8, 8, 128, 2816, 704, 128, fake, lw, NULL) == 4


def test_moe_forward_static_host_validation(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    args = [fake] * 8
    f = lib.moe_forward_static
    # needs more scratch than the static array holds
    assert lib.moe_workspace_bytes(4096, 8, 128, 2816, 704) > (16 << 20)
    assert f(*args, 4096, 8, 128, 2816, 704, 128, NULL) == 2
    # the shape checks of moe_forward
    assert f(*args, 8, 8, 128, 2816, 700, 128, NULL) == 2
    assert f(*args, 8, 8, 128, 2816, 704, 96, NULL) == 3
    bad = list(args)
    bad[0] = NULL
    assert f(*bad, 8, 8, 128, 2816, 704, 128, NULL) == 1
    assert f(*([NULL] * 8), 0, 8, 128, 2816, 704, 128, NULL) == 0   # nothing to do


def test_dequant_host_validation(lib):
    fake = ctypes.c_void_p(4096)
    assert lib.w4a16_dequantize(fake, fake, fake, 4, 12, 32, NULL) == 2
    assert lib.w4a16_dequantize(fake, fake, fake, 4, 64, 24, NULL) == 3
    assert lib.w4a16_dequantize(fake, fake, ctypes.c_void_p(4097), 4, 64, 32, NULL) == 4


def test_infer_group_size():
    assert _lib.infer_group_size(2816, 22) == 128
    assert _lib.infer_group_size(2816, 88) == 32
    assert _lib.infer_group_size(704, 6) == 128   # partial last group
    assert _lib.infer_group_size(704, 22) == 32
    assert _lib.infer_group_size(704, 11) == 64
    assert _lib.infer_group_size(64, 1) == 64
    with pytest.raises(ValueError):
        _lib.infer_group_size(2816, 7)


def test_python_ops_refuse_cpu_tensors():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    wp = torch.zeros(16, 8, dtype=torch.int32)
    ws = torch.zeros(16, 2, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        _lib.linear(x, wp, ws)
    with pytest.raises(RuntimeError, match="GPU only"):
        _lib.dequantize(wp, ws)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(tmp_path / "libw4a16moe.so")


def test_ffn_block_and_bf16_experts_host_validation(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    # moe_bf16_experts_forward: hidden, idx, w, gate_up_proj, down_proj, out
    f = lib.moe_bf16_experts_forward
    need = lib.moe_bf16_experts_workspace_bytes(8, 8, 128, 2816, 704)
    assert need == lib.moe_workspace_bytes(8, 8, 128, 2816, 704)
    assert f(fake, fake, fake, fake, fake, fake, 8, 8, 128, 2816, 700, fake, need, NULL) == 2  # I % 32
    assert f(fake, fake, fake, fake, fake, fake, 8, 8, 128, 2816, 704, fake, need - 1, NULL) == 5
    assert f(fake, fake, fake, NULL, fake, fake, 8, 8, 128, 2816, 704, fake, need, NULL) == 1
    assert f(ctypes.c_void_p(4098), fake, fake, fake, fake, fake, 8, 8, 128, 2816, 704, fake, need, NULL) == 4
    assert f(*([NULL] * 6), 0, 8, 128, 2816, 704, NULL, 0, NULL) == 0
    # moe_ffn_block_forward: 9 pointers, root, 10 pointers, eps, out, sizes
    g = lib.moe_ffn_block_forward
    wsb = lib.moe_ffn_block_workspace_bytes(8, 8, 128, 2816, 704, 2112)
    assert wsb > lib.moe_layer_workspace_bytes(8, 8, 128, 2816, 704)
    p9, p10 = [fake] * 9, [fake] * 10
    ok = (8, 8, 128, 2816, 704, 2112, 128)
    assert g(*p9, 0.1, *p10, 1e-6, fake, 8, 8, 128, 2816, 704, 2100, 128, fake, wsb, NULL) == 2  # Im % 32
    assert g(*p9, 0.1, *p10, 1e-6, fake, 8, 8, 128, 8224, 704, 2112, 128, fake, wsb, NULL) == 2  # H > 8192
    assert g(*p9, 0.1, *p10, 1e-6, fake, *ok, fake, wsb - 1, NULL) == 5
    assert g(*p9, 0.1, *p10, 1e-6, fake, 8, 8, 128, 2816, 704, 2112, 96, fake, wsb, NULL) == 3
    bad = list(p10)
    bad[9] = NULL                       # layer_scalar
    assert g(*p9, 0.1, *bad, 1e-6, fake, *ok, fake, wsb, NULL) == 1
    assert g(*p9, 0.1, *p10, 1e-6, ctypes.c_void_p(4098), *ok, fake, wsb, NULL) == 4


GU_DEC, DN_DEC, GU_PRE, DN_PRE = 0, 1, 2, 3


def test_tiled_decode_sizes(lib):
    """Sizes of the decode streamers' tiled copies (no GPU needed)."""
    tb = lib.w4a16_tiled_bytes
    # Gemma shape, G = 128: gate_up 22 column-tile items of 16 wavefronts x 6
    # KiB tiles per expert; down 44 items of 4 wavefronts x 6 KiB
    assert tb(GU_DEC, 128, 2816, 704, 128) == 128 * 22 * 16 * 6 * 1024
    assert tb(GU_DEC, 1, 2816, 704, 128) == 22 * 16 * 6 * 1024
    assert tb(DN_DEC, 128, 2816, 704, 128) == 128 * 44 * 4 * 6 * 1024
    # G = 32 / 64: each block of 6 tiles also carries 64 lanes x 6 tile scales
    for g in (32, 64):
        assert tb(GU_DEC, 128, 2816, 704, g) == 128 * 22 * 16 * 6 * 1152
        assert tb(DN_DEC, 128, 2816, 704, g) == 128 * 44 * 4 * 6 * 1152
    # no tiled decode form: long-K loop, I not a multiple of 32, an odd group
    # count per row at G = 128, other group sizes, E out of range
    assert tb(GU_DEC, 8, 8192, 704, 128) == 0
    assert tb(GU_DEC, 8, 2816, 700, 128) == 0
    assert tb(GU_DEC, 8, 2816 + 128, 704, 128) == 0     # 23 groups
    assert tb(GU_DEC, 8, 2816, 704, 256) == 0
    assert tb(GU_DEC, 0, 2816, 704, 128) == 0
    assert tb(GU_DEC, 8, 2816, 704, 48) == 0            # not a group size
    assert tb(7, 8, 2816, 704, 128) == 0                # no such kind


def test_tile_host_validation(lib):
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    t = lib.w4a16_tile
    need = lib.w4a16_tiled_bytes(GU_DEC, 2, 2816, 704, 128)
    assert t(GU_DEC, fake, fake, 8, 8192, 704, 128, fake, 1 << 30, NULL) == 2    # no tiled form
    assert t(GU_DEC, NULL, fake, 2, 2816, 704, 128, fake, need, NULL) == 1
    assert t(GU_DEC, fake, fake, 2, 2816, 704, 128, ctypes.c_void_p(4100), need, NULL) == 4
    assert t(GU_DEC, fake, fake, 2, 2816, 704, 128, fake, need - 16, NULL) == 5
    assert t(GU_DEC, fake, fake, 2, 2816, 704, 96, fake, need, NULL) == 3        # bad group
    # G = 32 copies hold the scales: a NULL scale is refused
    need32 = lib.w4a16_tiled_bytes(DN_DEC, 2, 2816, 704, 32)
    assert t(DN_DEC, fake, NULL, 2, 2816, 704, 32, fake, need32, NULL) == 1


def test_tiled_prefill_host_side(lib):
    """Size of the prefill GEMMs' tiled copies and the validation that returns
    before any launch."""
    tb = lib.w4a16_tiled_bytes
    # gate_up: 6 n-tiles x 44 k stages x 8 KiB per expert; down: 11 x 11 x 8 KiB
    assert tb(GU_PRE, 128, 2816, 704, 128) == 128 * 6 * 44 * 8192
    assert tb(DN_PRE, 128, 2816, 704, 128) == 128 * 11 * 11 * 8192
    assert tb(DN_PRE, 128, 2816, 704, 32) == 128 * 11 * 11 * 8192     # any group size
    assert tb(GU_PRE, 128, 2816, 736, 128) == 0       # I not a multiple of 64
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    need = tb(DN_PRE, 2, 2816, 704, 128)
    assert lib.w4a16_tile(GU_PRE, fake, NULL, 2, 2816, 736, 128, fake, 1 << 30, NULL) == 2
    assert lib.w4a16_tile(DN_PRE, NULL, NULL, 2, 2816, 704, 128, fake, need, NULL) == 1
    assert lib.w4a16_tile(DN_PRE, fake, NULL, 2, 2816, 704, 128, ctypes.c_void_p(4100), need, NULL) == 4
    assert lib.w4a16_tile(DN_PRE, fake, NULL, 2, 2816, 704, 128, fake, need - 16, NULL) == 5


def test_tiled_experts_descriptor_checks(lib):
    """The *_tiled entry points check the w4a16_tiled_experts against the call
    before any launch: the shape tag, each copy's size and alignment."""
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    E, H, I, G, M, k = 8, 2816, 704, 128, 4, 8
    ws = lib.moe_workspace_bytes(M, k, E, H, I)
    need = lib.w4a16_tiled_bytes(GU_DEC, E, H, I, G)

    def call(t):
        return lib.moe_forward_tiled(fake, fake, fake, fake, fake, fake, fake, ctypes.byref(t), fake,
                                     M, k, E, H, I, G, fake, ws, NULL)

    def desc(**kw):
        t = _lib.TiledExpertsC(E, H, I, G)
        for name, v in kw.items():
            setattr(t, name, v)
        return t

    assert call(desc(E=E + 1, gu_decode=4096, gu_decode_bytes=need)) == 2       # made for another stack
    assert call(desc(group_size=32, gu_decode=4096, gu_decode_bytes=need)) == 2  # another group size
    assert call(desc(gu_decode=4096, gu_decode_bytes=need - 1)) == 5            # short copy
    assert call(desc(gu_decode=4100, gu_decode_bytes=need)) == 4                # misaligned
    # a copy the shape has no tiled form for
    t = _lib.TiledExpertsC(E, 8192, I, G, 4096, 1 << 30)
    assert lib.moe_forward_tiled(fake, fake, fake, fake, fake, fake, fake, ctypes.byref(t), fake,
                                 M, k, E, 8192, I, G, fake, lib.moe_workspace_bytes(M, k, E, 8192, I), NULL) == 2
    # the FFN block's routing lives at fixed workspace offsets
    io, wo = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.moe_ffn_block_routing_offsets(8, 8, 128, 2816, 704, 2112, ctypes.byref(io), ctypes.byref(wo)) == 0
    assert wo.value >= io.value + 8 * 8 * 8 and io.value % 256 == 0 and wo.value % 256 == 0
    assert wo.value + 4 * 64 <= lib.moe_ffn_block_workspace_bytes(8, 8, 128, 2816, 704, 2112)
    assert lib.moe_ffn_block_routing_offsets(0, 8, 128, 2816, 704, 2112, ctypes.byref(io), ctypes.byref(wo)) == 2
