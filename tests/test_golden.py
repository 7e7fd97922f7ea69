"""Committed golden fixtures (tests/golden/w4a16_golden.npz, written by
tests/golden/make_golden.py from the oracle).

CPU: the oracle still reproduces every fixture bit for bit.
GPU: the HIP library on the fixture inputs -- bit-exact for dequantisation,
routing indices and the expert permutation; max-abs-rel <= 1e-2 for the
linear and MoE outputs (fp32 accumulation order differs from numpy's).
"""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from hybridagent_amd import _lib

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 1e-2


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN / "w4a16_golden.npz", allow_pickle=False))


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def test_oracle_reproduces_fixtures(golden):
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.build()
    assert sorted(fresh) == sorted(golden)
    for k, v in fresh.items():
        assert np.array_equal(np.asarray(v), golden[k]), k


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


@pytest.mark.gpu
def test_golden_dequant(golden, dev):
    out = _lib.dequantize(torch.from_numpy(golden["dq_packed"]).to(dev), _bf16(golden["dq_scale_bits"]).to(dev),
                          int(golden["dq_G"]))
    assert np.array_equal(_bits(out), golden["dq_out_bits"])


@pytest.mark.gpu
def test_golden_linear(golden, dev):
    y = _lib.linear(_bf16(golden["lin_x_bits"]).to(dev), torch.from_numpy(golden["lin_packed"]).to(dev),
                    _bf16(golden["lin_scale_bits"]).to(dev), group_size=int(golden["lin_G"]))
    ref = oracle.from_bf16_bits(golden["lin_y_bits"])
    assert oracle.max_abs_rel(y.float().cpu().numpy(), ref) <= TOL


@pytest.mark.gpu
def test_golden_router(golden, dev):
    w, idx, lg = _lib.router_topk(_bf16(golden["rt_h_bits"]).to(dev), _bf16(golden["rt_scale_bits"]).to(dev),
                                  float(golden["rt_root"]), _bf16(golden["rt_proj_bits"]).to(dev),
                                  _bf16(golden["rt_pes_bits"]).to(dev), float(golden["rt_eps"]),
                                  int(golden["rt_k"]), return_logits=True)
    ulp = np.abs(_bits(lg).astype(np.int32) - golden["rt_logits_bits"].astype(np.int32))
    assert ulp.max() <= 1
    assert np.array_equal(idx.cpu().numpy(), golden["rt_idx"])
    np.testing.assert_allclose(w.cpu().numpy(), golden["rt_w"], rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
def test_golden_sort(golden, dev):
    sp, off = _lib.sort_permute(torch.from_numpy(golden["srt_idx"]).to(dev), int(golden["srt_E"]))
    assert np.array_equal(off.cpu().numpy(), golden["srt_offsets"])
    n = int(golden["srt_offsets"][-1])
    assert np.array_equal(sp.cpu().numpy()[:n], golden["srt_sorted_pos"][:n])


@pytest.mark.gpu
def test_golden_moe(golden, dev):
    y = _lib.moe_forward(_bf16(golden["moe_x_bits"]).to(dev), torch.from_numpy(golden["moe_idx"]).to(dev),
                         torch.from_numpy(golden["moe_w"]).to(dev), torch.from_numpy(golden["moe_gu_packed"]).to(dev),
                         _bf16(golden["moe_gu_scale_bits"]).to(dev), torch.from_numpy(golden["moe_dn_packed"]).to(dev),
                         _bf16(golden["moe_dn_scale_bits"]).to(dev), group_size=int(golden["moe_G"]))
    ref = oracle.from_bf16_bits(golden["moe_y_bits"])
    err = oracle.max_abs_rel(y.float().cpu().numpy(), ref)
    print(f"golden moe max_abs_rel={err:.2e}")
    assert err <= TOL
