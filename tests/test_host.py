"""Host-side logic without a GPU: scene generators, the bench contract, and
host models of two device algorithms whose correctness does not depend on the
hardware (the wave-wide 64-ary lower bound of the tile-range kernel and the
reciprocal-estimate division of the pair-emission kernel), checked against
exact references the way the reference checks its device logic on the host."""
import subprocess
import sys

import numpy as np
import pytest

from gsplat_tt_amd import scenes
from oracle import oracle as O


def test_scene_cov3d_matches_oracle_bitexact():
    scene, _ = scenes.config1(seed=4, n=5000)
    a = scenes.cov3d(scene.scales, scene.quats)
    b = O.cov3d(scene.scales, scene.quats)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_scene_generators_are_deterministic():
    a, _ = scenes.config1(seed=9, n=1000)
    b, _ = scenes.config1(seed=9, n=1000)
    assert np.array_equal(a.means, b.means) and np.array_equal(a.colors, b.colors)
    k1, v1 = scenes.config4_keys(n=10_000)
    k2, v2 = scenes.config4_keys(n=10_000)
    assert np.array_equal(k1, k2) and np.array_equal(v1, np.arange(10_000, dtype=np.uint32))
    tiles = (k1 >> np.uint64(32)).astype(np.int64)
    assert tiles.min() >= 0 and tiles.max() < 5000
    depth = (k1 & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    assert depth.min() >= 0.2 and depth.max() <= 100.0


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def wave_lower_bound(keys, p, t):
    """Host model of wave_lower_bound (gsplat_tt_amd/csrc/tiles.hip): 64 lanes
    probe evenly spaced keys, a ballot count narrows the range 64-fold."""
    lo, hi = 0, p
    while hi - lo > 64:
        step = (hi - lo + 63) // 64
        q = lo + (np.arange(64) + 1) * step - 1
        pred = (q < hi) & (keys[np.minimum(q, p - 1)] < t)
        c = int(pred.sum())
        assert pred[:c].all() and not pred[c:].any()  # the ballot is a prefix
        hi = min(hi, lo + (c + 1) * step - 1)
        lo += c * step
    q = lo + np.arange(64)
    return lo + int(((q < hi) & (keys[np.minimum(q, max(p - 1, 0))] < t)).sum()) if p else 0


@pytest.mark.parametrize("p", [0, 1, 63, 64, 65, 4097, 300_001])
def test_tile_bounds_search_model(p):
    rng = np.random.default_rng(p)
    keys = np.sort(rng.integers(0, 60, size=p)).astype(np.int64)
    for t in range(-1, 62):
        assert wave_lower_bound(keys, p, t) == np.searchsorted(keys, t, "left")


def test_divmod_small_model():
    """divmod_small: q = trunc(j * rcp(w)) with a reciprocal estimate within 1 ulp,
    then one correction step, is exact for j < 2^24, w < 2^16."""
    rng = np.random.default_rng(1)
    j = rng.integers(0, 1 << 24, size=400_000).astype(np.int64)
    w = rng.integers(1, 1 << 16, size=400_000).astype(np.int64)
    j[:1000] = (1 << 24) - 1
    w[:1000] = rng.integers(1, 64, size=1000)
    r32 = (np.float32(1.0) / w.astype(np.float32)).astype(np.float32)
    for rcp in (r32, np.nextafter(r32, np.float32(0)), np.nextafter(r32, np.float32(1))):
        qi = (j.astype(np.float32) * rcp).astype(np.float32).astype(np.int64)
        ri = j - qi * w
        qi = np.where(ri < 0, qi - 1, np.where(ri >= w, qi + 1, qi))
        ri = j - qi * w
        assert np.array_equal(qi, j // w) and np.array_equal(ri, j % w)
