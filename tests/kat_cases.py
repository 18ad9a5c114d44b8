"""Known-answer cases restated from the reference's own unit tests, run against
any implementation of the four stages (the CPU oracle and the HIP stage API).

Each case takes a backend `B` with
  B.project(means, cov3d9, w2c, K, colors, opac, H, W) -> dict(valid, means2d, covs2d,
                                                              depths, radii, ...)
  B.tile_assign(means2d, radii, H, W, tile_size, covs2d, opac, contrib_floor)
      -> (gaussian_ids, tile_ids, pairs_pre)
  B.sort_and_bin(gids, tids, depths, tiles_x, tiles_y) -> (sorted_ids, tile_ranges (T,2))
  B.blend(means2d, covs2d, colors, opac, sorted_ids, tile_ranges, tiles_x, tiles_y,
          tile_size, H, W) -> float32 image (H, W, 3)   [cull + blend, AVX2 rules]
"""
from __future__ import annotations

import math

import numpy as np

F = np.float32
EYE4 = np.eye(4, dtype=F)


def _intr(fx, cx=0.0, cy=0.0):
    return np.array([[fx, 0, cx], [0, fx, cy], [0, 0, 1]], F)


# ---------------------------------------------------------------- project
def kat_project_hand_computed(B):
    """tests/unit/test_project.cpp:166-196, 283-322: unit-scale Gaussian on the
    optical axis at z=2 with fx=2 -> cov2d = I + 0.3 = 1.3 I, r = ceil(3 sqrt(1.3))."""
    means = np.array([[0, 0, 2]], F)
    cov = np.eye(3, dtype=F).reshape(1, 9)
    o = B.project(means, cov, EYE4, _intr(2.0), np.ones((1, 3), F), np.ones(1, F), 512, 512)
    assert o["depths"].shape[0] == 1
    assert abs(float(o["means2d"][0, 0])) < 1e-5 and abs(float(o["means2d"][0, 1])) < 1e-5
    c = o["covs2d"][0]
    assert abs(c[0] - 1.3) < 1e-5 and abs(c[1]) < 1e-5 and abs(c[3] - 1.3) < 1e-5
    r = math.ceil(3.0 * math.sqrt(F(1.3)))
    assert r == 4
    assert float(o["radii"][0, 0]) == r and float(o["radii"][0, 1]) == r


def kat_project_near_plane(B):
    """tests/unit/test_project.cpp:260-281: z = 0.1 lies in front of the 0.2 near plane."""
    means = np.array([[0, 0, 0.1]], F)
    cov = (np.eye(3, dtype=F) * F(0.01)).reshape(1, 9)
    o = B.project(means, cov, EYE4, _intr(1.0), np.ones((1, 3), F), np.ones(1, F), 512, 512)
    assert not bool(o["valid"][0])
    assert o["depths"].shape[0] == 0


# ---------------------------------------------------------------- tile assign
def kat_tile_one_tile(B):
    """test_tile_assign.cpp:17-30: radius-8 Gaussian at (48,48) -> tile (1,1) only."""
    g, t, _ = B.tile_assign(np.array([[48, 48]], F), np.array([[8, 8]], F), 256, 256, 32,
                            None, None, F(15.0 / 255.0))
    assert list(g) == [0] and list(t) == [1 * 8 + 1]


def kat_tile_four_tiles(B):
    """test_tile_assign.cpp:32-43: (32,32) radius 16 straddles four tiles."""
    g, t, ppre = B.tile_assign(np.array([[32, 32]], F), np.array([[16, 16]], F), 256, 256, 32,
                               None, None, F(15.0 / 255.0))
    assert len(g) == 4 and ppre == 4
    assert sorted(int(x) for x in t) == [0, 1, 8, 9]


def kat_tile_cull_drops(B):
    """test_tile_assign.cpp:45-61: sharp Gaussians (cov 0.01) keep only their own tile."""
    m = np.array([[16, 16], [240, 240]], F)
    r = np.array([[20, 20], [20, 20]], F)
    cv = np.array([[0.01, 0, 0, 0.01], [0.01, 0, 0, 0.01]], F)
    op = np.array([0.5, 0.5], F)
    g0, _, p0 = B.tile_assign(m, r, 256, 256, 32, None, None, F(15.0 / 255.0))
    g1, t1, p1 = B.tile_assign(m, r, 256, 256, 32, cv, op, F(15.0 / 255.0))
    assert len(g1) < len(g0) and p1 == p0 == len(g0)
    assert list(t1) == [0, 7 * 8 + 7]


def kat_tile_sum_equals_pairs(B):
    """test_tile_assign.cpp:63-78: pairs are Gaussian-major and their count equals
    the rectangle areas minus the culled pairs."""
    m = np.array([[100, 50], [200, 150], [80, 120]], F)
    r = np.array([[24, 18], [30, 22], [12, 16]], F)
    cv = np.array([[1, 0, 0, 1], [2, 0, 0, 2], [0.5, 0, 0, 0.5]], F)
    op = np.array([0.9, 0.8, 0.7], F)
    g, t, ppre = B.tile_assign(m, r, 256, 256, 32, cv, op, F(15.0 / 255.0))
    assert np.all(np.diff(g) >= 0)            # Gaussian-major
    areas = 0
    for (px, py), (rx, ry) in zip(m, r):
        x0, x1 = int((px - rx) / 32), int((px + rx) / 32)
        y0, y1 = int((py - ry) / 32), int((py + ry) / 32)
        areas += (min(x1, 7) - max(x0, 0) + 1) * (min(y1, 7) - max(y0, 0) + 1)
    assert ppre == areas and len(g) <= areas


def kat_tile_empty(B):
    """test_tile_assign.cpp:80-87."""
    g, t, ppre = B.tile_assign(np.zeros((0, 2), F), np.zeros((0, 2), F), 256, 256, 32, None,
                               None, F(15.0 / 255.0))
    assert len(g) == 0 and len(t) == 0 and ppre == 0


# ---------------------------------------------------------------- sort
def kat_sort_depth_order(B):
    """test_sort.cpp:5-17."""
    s, _ = B.sort_and_bin([0, 1, 2], [5, 5, 5], np.array([0.5, 0.3, 0.7], F), 3, 3)
    assert list(s) == [1, 0, 2]


def kat_sort_ranges(B):
    """test_sort.cpp:19-35."""
    _, r = B.sort_and_bin([0, 1, 2, 3, 4], [2, 2, 7, 7, 10],
                          np.array([0.4, 0.6, 0.5, 0.8, 0.3, 0.9], F), 4, 3)
    assert tuple(r[2]) == (0, 2) and tuple(r[7]) == (2, 4) and tuple(r[10]) == (4, 5)


def kat_sort_empty_tiles_zero(B):
    """test_sort.cpp:37-51."""
    _, r = B.sort_and_bin([0], [3], np.array([1.0], F), 4, 4)
    assert tuple(r[0]) == (0, 0) and tuple(r[3]) == (0, 1) and tuple(r[5]) == (0, 0)


def kat_sort_by_depth_not_id(B):
    """test_sort.cpp:53-63: depths are indexed by Gaussian id."""
    s, _ = B.sort_and_bin([5, 1], [4, 4], np.array([0.2, 0.9, 0.4, 0.6, 0.1, 0.8], F), 4, 4)
    assert list(s) == [5, 1]


def kat_sort_ties_by_input_order(B):
    """Stable: equal (tile, depth) keys keep the emitted (Gaussian-major) order."""
    s, r = B.sort_and_bin([3, 1, 2, 0], [0, 0, 0, 0], np.array([0.5, 0.5, 0.5, 0.5], F), 1, 1)
    assert list(s) == [3, 1, 2, 0] and tuple(r[0]) == (0, 4)


def kat_sort_empty(B):
    """test_sort.cpp:65-75."""
    s, r = B.sort_and_bin([], [], np.array([1.0], F), 2, 2)
    assert len(s) == 0 and r.shape == (4, 2) and not r.any()


# ---------------------------------------------------------------- blend
def _one_tile_blend(B, means, covs, colors, opac, H=32, W=32, ts=32, tile=0):
    n = len(opac)
    tx, ty = (W + ts - 1) // ts, (H + ts - 1) // ts
    ranges = np.zeros((tx * ty, 2), np.int64)
    ranges[tile] = (0, n)
    return B.blend(np.array(means, F).reshape(n, 2), np.array(covs, F).reshape(n, 4),
                   np.array(colors, F).reshape(n, 3), np.array(opac, F), np.arange(n),
                   ranges, tx, ty, ts, H, W)


def kat_blend_center_red(B):
    """test_blend.cpp:28-50: at the centre the Gaussian is at full weight, so the
    pixel is alpha_max = 0.99 red (exactly: exp4(0) = 1)."""
    img = _one_tile_blend(B, [16.5, 16.5], [50, 0, 0, 50], [1, 0, 0], [1.0])
    assert float(img[16, 16, 0]) == F(0.99)
    assert img[16, 16, 1] == 0 and img[16, 16, 2] == 0


def kat_blend_second_dominates(B):
    """test_blend.cpp:52-72."""
    img = _one_tile_blend(B, [16.5, 16.5, 16.5, 16.5], [50, 0, 0, 50, 50, 0, 0, 50],
                          [1, 0, 0, 0, 1, 0], [0.01, 1.0])
    assert img[16, 16, 0] < 0.05 and img[16, 16, 1] > 0.95


def kat_blend_early_out(B):
    """test_blend.cpp:74-104: 100 stacked opaque red Gaussians saturate at <= 1."""
    n = 100
    img = _one_tile_blend(B, [16.5] * (2 * n), [0.01, 0, 0, 0.01] * n, [1, 0, 0] * n,
                          [1.0] * n)
    assert 0.99 < float(img[16, 16, 0]) <= 1.0


def kat_blend_empty_tile(B):
    """test_blend.cpp:106-123: a tile with an empty range stays black."""
    img = B.blend(np.array([[16.5, 16.5]], F), np.array([[1, 0, 0, 1]], F),
                  np.array([[1, 1, 1]], F), np.array([1.0], F), np.array([0]),
                  np.zeros((1, 2), np.int64), 1, 1, 32, 32, 32)
    assert not img.any()


def kat_blend_edge_tile(B):
    """test_blend.cpp:125-151: the corner tile of a 40x40 image (tile 32) is
    blended only inside the image."""
    img = _one_tile_blend(B, [35.5, 35.5], [20, 0, 0, 20], [0, 0, 1], [1.0], H=40, W=40,
                          tile=3)
    assert img[35, 35, 2] > 0.5 and img[0, 0, 0] == 0 and img[39, 39, 2] > 0.1


ALL = [v for k, v in sorted(globals().items()) if k.startswith("kat_")]
