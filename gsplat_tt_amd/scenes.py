"""Seeded synthetic scenes and cameras for the five benchmark workloads.

Conventions follow the reference (gsplat/utils.py:133-152, types.h:68-97):
world-to-camera 4x4 row-major with R | t in column 3, OpenCV camera (+z
forward, +y down), quaternions wxyz, intrinsics 3x3 with fx, fy, cx, cy.
Activations follow gsplat/loading_gaussians.py:7-30 (exp scales, normalised
quaternions, sigmoid opacity). Colour is RGB (N,3) or SH coefficients
(N, (d+1)^2, 3).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


@dataclass
class Scene:
    means: np.ndarray          # (N,3) f32
    scales: np.ndarray         # (N,3) f32 (activated)
    quats: np.ndarray          # (N,4) f32 wxyz, unit
    opacities: np.ndarray      # (N,) f32 (activated)
    colors: np.ndarray | None  # (N,3) f32 RGB, or None when sh is set
    sh: np.ndarray | None      # (N,K,3) f32
    sh_degree: int
    meta: dict = field(default_factory=dict)

    @property
    def n(self) -> int:
        return int(self.means.shape[0])


@dataclass
class Camera:
    w2c: np.ndarray   # (4,4) f32
    K: np.ndarray     # (3,3) f32
    height: int
    width: int


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _unit_quats(rng, n):
    q = rng.standard_normal((n, 4)).astype(np.float64)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q.astype(np.float32)


def intrinsics(fx, fy, cx, cy) -> np.ndarray:
    return np.array([[fx, 0, cx], [0, fy, cy], [0, 0, 1]], np.float32)


def look_at_w2c(eye, target, up=(0.0, -1.0, 0.0)) -> np.ndarray:
    """World-to-camera for an OpenCV camera at `eye` looking at `target`
    (+z forward, +y down; `up` is the world's up direction)."""
    eye = np.asarray(eye, np.float64)
    fwd = np.asarray(target, np.float64) - eye
    fwd /= np.linalg.norm(fwd)
    upv = np.asarray(up, np.float64)
    right = np.cross(fwd, upv)
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    R = np.stack([right, down, fwd], 0)  # rows: camera x, y, z axes in world
    t = -R @ eye
    w2c = np.eye(4)
    w2c[:3, :3] = R
    w2c[:3, 3] = t
    return w2c.astype(np.float32)


def config1(seed: int = 1, n: int = 100_000):
    """100K Gaussians, 640x480, pinhole fx=fy=500 at the image centre, camera at
    the origin looking +z, RGB colours."""
    rng = np.random.default_rng(seed)
    means = np.stack([rng.uniform(-2, 2, n), rng.uniform(-2, 2, n), rng.uniform(2, 8, n)],
                     1).astype(np.float32)
    scales = np.exp(rng.normal(-4.0, 0.5, (n, 3))).astype(np.float32)
    quats = _unit_quats(rng, n)
    opac = _sigmoid(rng.standard_normal(n)).astype(np.float32)
    rgb = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    scene = Scene(means, scales, quats, opac, rgb, None, 0,
                  dict(config=1, seed=seed, n=n))
    cam = Camera(np.eye(4, dtype=np.float32), intrinsics(500, 500, 320, 240), 480, 640)
    return scene, [cam]


def _sh_coeffs(rng, n, degree):
    K = (degree + 1) ** 2
    sh = np.empty((n, K, 3), np.float32)
    sh[:, 0, :] = rng.uniform(0, 1, (n, 3))
    if K > 1:
        sh[:, 1:, :] = rng.normal(0, 0.1, (n, K - 1, 3))
    return sh


def config2(seed: int = 2, n: int = 1_000_000, degree: int = 3):
    """1M Gaussians from a 64-component mixture in a 10 m cube, SH degree 3,
    1280x720, one camera 6 m from the centroid looking +z (fov 50 deg)."""
    rng = np.random.default_rng(seed)
    centers = rng.uniform(-5, 5, (64, 3))
    comp = rng.integers(0, 64, n)
    means = (centers[comp] + rng.normal(0, 0.5, (n, 3))).astype(np.float32)
    scales = np.exp(rng.normal(-4.5, 0.7, (n, 3))).astype(np.float32)
    quats = _unit_quats(rng, n)
    opac = _sigmoid(rng.normal(0, 1.5, n)).astype(np.float32)
    sh = _sh_coeffs(rng, n, degree)
    centroid = means.astype(np.float64).mean(0)
    eye = centroid + np.array([0.0, 0.0, -6.0])
    f = 0.5 * 1280 / math.tan(math.radians(25.0))
    w2c = look_at_w2c(eye, centroid)
    scene = Scene(means, scales, quats, opac, None, sh, degree,
                  dict(config=2, seed=seed, n=n, focal=f))
    return scene, [Camera(w2c, intrinsics(f, f, 640, 360), 720, 1280)]


def config3(seed: int = 3, n: int = 6_000_000, degree: int = 3, views: int = 64,
            slab_frac: float = 0.6):
    """Scene-scale cloud: a dense ground-plane slab plus a surrounding shell,
    heavy-tailed log-scales (98% N(-5,1), 2% N(-2,0.5)), SH degree 3, rendered
    at 1237x822 over a 64-view orbit (radius 4 m, 1 m above the centroid,
    fx=fy=1100). World up is -y (OpenCV-style world)."""
    rng = np.random.default_rng(seed)
    n_slab = int(n * slab_frac)
    n_shell = n - n_slab
    slab = np.stack([rng.uniform(-6, 6, n_slab), rng.normal(0.0, 0.05, n_slab),
                     rng.uniform(-6, 6, n_slab)], 1)
    d = rng.standard_normal((n_shell, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    d[:, 1] = -np.abs(d[:, 1])  # upper hemisphere (world up is -y)
    rad = rng.uniform(7.0, 9.0, n_shell)
    shell = d * rad[:, None]
    means = np.concatenate([slab, shell], 0).astype(np.float32)
    perm = rng.permutation(n)
    means = means[perm]
    ls = rng.normal(-5.0, 1.0, (n, 3))
    big = rng.uniform(0, 1, n) < 0.02
    ls[big] = rng.normal(-2.0, 0.5, (int(big.sum()), 3))
    scales = np.exp(ls).astype(np.float32)
    quats = _unit_quats(rng, n)
    opac = _sigmoid(rng.normal(0, 2.0, n)).astype(np.float32)
    sh = _sh_coeffs(rng, n, degree)
    centroid = np.zeros(3)
    cams = []
    for v in range(views):
        a = 2 * math.pi * v / views
        eye = centroid + np.array([4.0 * math.cos(a), -1.0, 4.0 * math.sin(a)])
        cams.append(Camera(look_at_w2c(eye, centroid), intrinsics(1100, 1100, 618.5, 411.0),
                           822, 1237))
    scene = Scene(means, scales, quats, opac, None, sh, degree,
                  dict(config=3, seed=seed, n=n, slab_frac=slab_frac,
                       slab="x,z~U[-6,6], y~N(0,0.05)", shell="r~U[7,9], upper hemisphere"))
    return scene, cams


def config4_keys(seed: int = 4, n: int = 50_000_000, tiles: int = 5000, s: float = 1.1):
    """Standalone tile/depth sort keys: hi32 = Zipf(s) tile id over `tiles`,
    lo32 = fp32 bits of a log-uniform depth in [0.2, 100]; payload = index."""
    rng = np.random.default_rng(seed)
    w = 1.0 / np.arange(1, tiles + 1, dtype=np.float64) ** s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    tile = np.searchsorted(cdf, rng.uniform(0, 1, n), side="right").astype(np.uint64)
    np.minimum(tile, tiles - 1, out=tile)
    depth = np.exp(rng.uniform(math.log(0.2), math.log(100.0), n)).astype(np.float32)
    keys = (tile << np.uint64(32)) | depth.view(np.uint32).astype(np.uint64)
    vals = np.arange(n, dtype=np.uint32)
    return keys, vals


def config5(seed: int = 5, n: int = 1_000_000, degree: int = 1):
    """Training workload: 1M Gaussians, SH degree 1, 1280x720; the target is a
    render of a perturbed copy (means + N(0,0.01), colours + N(0,0.05))."""
    scene, cams = config2(seed=seed, n=n, degree=degree)
    rng = np.random.default_rng(seed + 1000)
    tgt = Scene(scene.means + rng.normal(0, 0.01, scene.means.shape).astype(np.float32),
                scene.scales.copy(), scene.quats.copy(), scene.opacities.copy(), None,
                scene.sh.copy(), degree, dict(scene.meta, perturbed=True))
    tgt.sh[:, 0, :] += rng.normal(0, 0.05 / 0.28209479177387814, (n, 3)).astype(np.float32)
    scene.meta["config"] = 5
    return scene, tgt, cams
