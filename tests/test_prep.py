"""Scene input preparation (gsplat_tt_amd/prep.py): Morton order against a
bit-by-bit interleave, permutation and stability invariants; opacity prune
keeps exactly the Gaussians the projection's opacity test keeps, in order."""
import numpy as np

from gsplat_tt_amd import prep


def _interleave_ref(q):
    """30-bit Morton code by looping over the bits (x bit b -> 3b, y -> 3b+1, z -> 3b+2)."""
    out = np.zeros(q.shape[0], np.uint64)
    for b in range(10):
        for axis in range(3):
            bit = (q[:, axis].astype(np.uint64) >> np.uint64(b)) & np.uint64(1)
            out |= bit << np.uint64(3 * b + axis)
    return out


def test_morton_codes_match_bitwise_interleave():
    rng = np.random.default_rng(0)
    means = rng.normal(size=(5000, 3)) * np.array([3.0, 0.1, 2.0])
    lo = np.percentile(means, 0.5, axis=0)
    hi = np.percentile(means, 99.5, axis=0)
    q = (np.clip((means - lo) / (hi - lo), 0, 1) * 1023).astype(np.uint64)
    assert np.array_equal(prep.morton_codes(means), _interleave_ref(q))
    assert int(prep.morton_codes(means).max()) < (1 << 30)


def test_morton_order_is_a_stable_sorting_permutation():
    rng = np.random.default_rng(1)
    means = np.round(rng.uniform(-1, 1, (4000, 3)), 1)  # many equal codes
    order = prep.morton_order(means)
    assert np.array_equal(np.sort(order), np.arange(4000))
    codes = prep.morton_codes(means)[order]
    assert np.all(codes[1:] >= codes[:-1])
    ties = codes[1:] == codes[:-1]
    assert ties.any() and np.all(order[1:][ties] > order[:-1][ties])  # stable
    arrays = {"means": means, "op": np.arange(4000, dtype=np.float32)}
    out, perm = prep.morton_reorder(arrays)
    assert np.array_equal(perm, order) and np.array_equal(out["op"], arrays["op"][order])


def test_opacity_prune_keeps_order_and_nan():
    op = np.array([0.5, 1.0 / 255.0, 0.001, np.nan, 0.0039, 0.9], np.float32)
    keep = prep.opacity_keep_mask(op)
    # 1/255 itself is kept (not below), NaN is kept (passes the projection's test)
    assert keep.tolist() == [True, True, False, True, False, True]
    arrays = {"opacities": op, "id": np.arange(6)}
    out = prep.opacity_prune(arrays)
    assert out["id"].tolist() == [0, 1, 3, 5]
