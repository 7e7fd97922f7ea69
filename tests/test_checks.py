"""The shared routing check (tests/checks.py) on the CPU: it must accept what
a one-ulp logit disagreement can do and reject planted mistakes."""
import numpy as np
import pytest

import oracle
from checks import check_routing_order

K = 8


def _logits(M, E=128, seed=0):
    rng = np.random.default_rng(seed)
    return oracle.bf16_round(rng.standard_normal((M, E)).astype(np.float32) * 0.3)


def _nudge(lg, frac, seed):
    """Move a fraction of the logits by one bf16 ulp (what an fp32 reduction
    order difference can do)."""
    rng = np.random.default_rng(seed)
    bits = oracle.to_bf16_bits(lg).astype(np.int32)
    mask = rng.random(lg.shape) < frac
    step = rng.choice([-1, 1], size=lg.shape)
    return oracle.from_bf16_bits((bits + mask * step).astype(np.uint16))


def test_identical_logits_are_all_determined():
    lg = _logits(500)
    idx, _ = oracle.topk_from_logits(lg, np.ones(128, np.float32), K)
    det, flips = check_routing_order(lg, idx, lg, idx, K, "identical")
    assert det.all() and len(flips) == 0


def test_one_ulp_moves_pass_and_are_counted():
    ref = _logits(2000, seed=1)
    got = _nudge(ref, 0.03, seed=2)
    ridx, _ = oracle.topk_from_logits(ref, np.ones(128, np.float32), K)
    gidx, _ = oracle.topk_from_logits(got, np.ones(128, np.float32), K)
    det, flips = check_routing_order(got, gidx, ref, ridx, K, "nudged", max_flip_frac=0.2)
    assert 0 < det.mean() < 1


def test_planted_swap_on_a_determined_row_fails():
    lg = _logits(64, seed=3)
    idx, _ = oracle.topk_from_logits(lg, np.ones(128, np.float32), K)
    bad = idx.copy()
    bad[5, [0, 1]] = bad[5, [1, 0]]  # order swapped, same set
    with pytest.raises(AssertionError, match="determined rows differ"):
        check_routing_order(lg, bad, lg, idx, K, "planted")


def test_planted_far_swap_on_a_moved_row_fails():
    ref = _logits(64, seed=4)
    got = ref.copy()
    # move one logit far outside the top-9 so the row is not determined
    top = np.argsort(-ref[7])[:K + 1]
    got[7, top[0]] = oracle.bf16_round(np.float32(ref[7, top[0]] + 1.0))
    ridx, _ = oracle.topk_from_logits(ref, np.ones(128, np.float32), K)
    gidx = ridx.copy()
    far = np.argsort(-ref[7])[-1]          # the lowest-ranked expert
    gidx[7, 3] = far
    with pytest.raises(AssertionError, match="not near-tied"):
        check_routing_order(got, gidx, ref, ridx, K, "planted")
