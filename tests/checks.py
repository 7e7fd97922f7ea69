"""Shared checks of the test suite (no GPU needed to import)."""
import numpy as np

import oracle

# worst error seen per (config, measure) in this pytest run: the terminal
# summary (conftest.py) prints them, so a test log shows every margin
MARGINS = {}


def margin(config, err, bound=1e-2, measure="max_abs_rel vs oracle"):
    """Record ``err`` for ``config`` (the worst one is kept), print it, return it."""
    key = (config, measure)
    if key not in MARGINS or err > MARGINS[key][0]:
        MARGINS[key] = (float(err), bound)
    print(f"{config}: {measure} = {err:.3e} (bound {bound:g})", flush=True)
    return err


def check_routing_order(got_lg, got_idx, ref_lg, ref_idx, k, what, max_flip_frac=0.05):
    """End-to-end routing against the oracle, in order.

    A row is *determined* when the kernel's bf16 logits at the oracle's
    top-k experts are bit-identical to the oracle's and every other expert
    ranks after the k-th under the kernel's logits (value descending, lower
    index first): the kernel's top-k is then the oracle's, in the same
    order, so the ordered indices must be equal.  On the other rows a logit
    moved by the fp32 reduction order (at most one bf16 ulp) may reorder
    near-tied experts: such rows are counted ("flips"), and every flip must
    swap experts whose oracle logits lie within two bf16 ulps of each other.
    """
    M, E = ref_lg.shape
    top = np.argsort(-ref_lg, axis=1, kind="stable")[:, :k]
    g_at = np.take_along_axis(got_lg, top, 1)
    r_at = np.take_along_axis(ref_lg, top, 1)
    same_top = (oracle.to_bf16_bits(g_at) == oracle.to_bf16_bits(r_at)).all(1)
    # every other expert ranks after the k-th under the kernel's logits
    others = got_lg.copy()
    np.put_along_axis(others, top, -np.inf, 1)
    vk, ik = r_at[:, k - 1:k], top[:, k - 1:k]
    after = (others < vk) | ((others == vk) & (np.arange(E)[None, :] > ik))
    det = same_top & after.all(1)
    assert np.array_equal(got_idx[det], ref_idx[det]), f"{what}: determined rows differ in order"
    flips = np.nonzero((got_idx != ref_idx).any(1))[0]
    # bf16 ulp of each oracle logit; with each logit within one ulp of the
    # oracle's, two experts can trade places only if their oracle logits are
    # at most two ulps apart
    ulp_ref = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref_lg), 1e-30))) - 7)
    for r in flips:
        c = int(np.nonzero(got_idx[r] != ref_idx[r])[0][0])
        a, b = ref_idx[r, c], got_idx[r, c]
        assert abs(ref_lg[r, a] - ref_lg[r, b]) <= 2 * max(ulp_ref[r, a], ulp_ref[r, b]), \
            f"{what}: row {r} slot {c} swaps experts {a}/{b} that are not near-tied"
    print(f"{what}: {det.sum()}/{M} rows determined (ordered-equal), {len(flips)} near-tie flips "
          f"({len(flips) / M:.2%})")
    assert len(flips) <= max(1, max_flip_frac * M)
    return det, flips


def bf16_ulp_distance(a, b) -> np.ndarray:
    """Distance in bf16 ulps between the bf16 roundings of a and b (values
    of either sign; +0 and -0 are 0 apart)."""
    def ordered(x):
        bits = oracle.to_bf16_bits(np.asarray(x, np.float32)).astype(np.int32)
        mag = bits & 0x7FFF
        return np.where(bits & 0x8000, -mag, mag)
    return np.abs(ordered(a) - ordered(b))


def bf16_ulp(x) -> np.ndarray:
    """One bf16 ulp at |x| (the spacing of bf16 values around x)."""
    a = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def check_bf16_close(got, ref, what, exact_frac=0.999, slack=None):
    """Per-element bf16 agreement with a restatement that rounds at the same
    points: at least ``exact_frac`` of the elements within one ulp, and every
    element within two ulps or within ``slack`` (per element, absolute): an
    intermediate that rounded the other way in one of the two moves the
    output by what one ulp of that intermediate becomes downstream, which is
    many ulps of an output near zero.  Default slack: 2^-8 x the row's RMS."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    ulps = bf16_ulp_distance(got, ref)
    hist = {f"{u}": int((ulps == u).sum()) for u in range(3)}
    hist[">2"] = int((ulps > 2).sum())
    if slack is None:
        slack = 2.0 ** -8 * np.sqrt(np.mean(np.square(ref.astype(np.float64)), axis=-1, keepdims=True))
    d = np.abs(got.astype(np.float64) - ref)
    worst = float((d / slack)[ulps > 2].max()) if (ulps > 2).any() else 0.0
    print(f"{what}: bf16 ulp histogram {hist} of {ulps.size}; beyond 2 ulps the worst is {worst:.2f} x slack")
    assert (ulps <= 1).mean() >= exact_frac, f"{what}: only {(ulps <= 1).mean():.4%} within one ulp"
    far = (ulps > 2) & (d > slack)
    assert not far.any(), f"{what}: {far.sum()} elements beyond two ulps and the slack"
    return ulps
