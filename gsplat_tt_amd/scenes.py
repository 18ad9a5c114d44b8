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


def cov3d(scales: np.ndarray, quats: np.ndarray) -> np.ndarray:
    """Sigma = (R(q) diag(s)) (R(q) diag(s))^T, (N, 9) row-major float32, with the
    reference's operation order (types.h:68-97; quaternion wxyz used as given).
    numpy float32 ufuncs round every operation, so this equals the reference's
    -ffp-contract=off result bit for bit."""
    s = np.ascontiguousarray(scales, np.float32)
    q = np.ascontiguousarray(quats, np.float32)
    q0, q1, q2, q3 = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    two, one = np.float32(2.0), np.float32(1.0)
    r = np.empty((s.shape[0], 3, 3), np.float32)
    r[:, 0, 0] = one - two * (q2 * q2 + q3 * q3)
    r[:, 0, 1] = two * (q1 * q2 - q0 * q3)
    r[:, 0, 2] = two * (q1 * q3 + q0 * q2)
    r[:, 1, 0] = two * (q1 * q2 + q0 * q3)
    r[:, 1, 1] = one - two * (q1 * q1 + q3 * q3)
    r[:, 1, 2] = two * (q2 * q3 - q0 * q1)
    r[:, 2, 0] = two * (q1 * q3 - q0 * q2)
    r[:, 2, 1] = two * (q2 * q3 + q0 * q1)
    r[:, 2, 2] = one - two * (q1 * q1 + q2 * q2)
    r *= s[:, None, :]
    out = np.empty((s.shape[0], 3, 3), np.float32)
    for a in range(3):
        for b in range(3):
            out[:, a, b] = (r[:, a, 0] * r[:, b, 0] + r[:, a, 1] * r[:, b, 1]) + \
                r[:, a, 2] * r[:, b, 2]
    return out.reshape(-1, 9)


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
    dc = rng.random((n, 3), dtype=np.float32)
    sh = rng.standard_normal((n, K * 3), dtype=np.float32)  # one contiguous draw
    sh *= np.float32(0.1)
    sh[:, :3] = dc
    return sh.reshape(n, K, 3)


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
            slab_frac: float = 0.8, slab_half: float = 3.5, shell_r=(4.5, 6.5)):
    """Scene-scale cloud: a dense ground-plane slab plus a surrounding shell,
    heavy-tailed log-scales (98% N(-5,1), 2% N(-2,0.5)), SH degree 3, rendered
    at 1237x822 over a 64-view orbit (radius 4 m, 1 m above the centroid,
    fx=fy=1100). World up is -y (OpenCV-style world). The slab is
    x,z ~ U[-slab_half, slab_half], y ~ N(0, 0.05); the shell is the upper
    hemisphere at radius ~ U[shell_r]."""
    rng = np.random.default_rng(seed)
    f32 = np.float32
    n_slab = int(n * slab_frac)
    n_shell = n - n_slab
    means = np.empty((n, 3), f32)
    means[:n_slab, 0] = rng.uniform(-slab_half, slab_half, n_slab)
    means[:n_slab, 1] = rng.standard_normal(n_slab, dtype=f32) * f32(0.05)
    means[:n_slab, 2] = rng.uniform(-slab_half, slab_half, n_slab)
    d = rng.standard_normal((n_shell, 3), dtype=f32)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    d[:, 1] = -np.abs(d[:, 1])  # upper hemisphere (world up is -y)
    d *= rng.uniform(shell_r[0], shell_r[1], n_shell).astype(f32)[:, None]
    means[n_slab:] = d
    means = means[rng.permutation(n)]
    ls = rng.standard_normal((n, 3), dtype=f32) + f32(-5.0)
    big = rng.random(n, dtype=f32) < f32(0.02)
    ls[big] = rng.standard_normal((int(big.sum()), 3), dtype=f32) * f32(0.5) + f32(-2.0)
    scales = np.exp(ls)
    q = rng.standard_normal((n, 4), dtype=f32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    opac = (1.0 / (1.0 + np.exp(-2.0 * rng.standard_normal(n, dtype=f32)))).astype(f32)
    sh = _sh_coeffs(rng, n, degree)
    centroid = np.zeros(3)
    cams = []
    for v in range(views):
        a = 2 * math.pi * v / views
        eye = centroid + np.array([4.0 * math.cos(a), -1.0, 4.0 * math.sin(a)])
        cams.append(Camera(look_at_w2c(eye, centroid), intrinsics(1100, 1100, 618.5, 411.0),
                           822, 1237))
    scene = Scene(means, scales, q, opac, None, sh, degree,
                  dict(config=3, seed=seed, n=n, slab_frac=slab_frac,
                       slab=f"x,z~U[-{slab_half},{slab_half}], y~N(0,0.05)",
                       shell=f"r~U[{shell_r[0]},{shell_r[1]}], upper hemisphere"))
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


def train_params(scene: "Scene") -> dict:
    """Optimizer-space parameters of a scene (gsplat/train_oracle.py conventions):
    means, log_scales = log(scales), quats (w x y z), opacity_logits = logit(op), sh."""
    op = np.clip(scene.opacities.astype(np.float64), 1e-6, 1 - 1e-6)
    return {
        "means": scene.means.astype(np.float32),
        "log_scales": np.log(scene.scales).astype(np.float32),
        "quats": scene.quats.astype(np.float32),
        "opacity_logits": np.log(op / (1.0 - op)).astype(np.float32),
        "sh": scene.sh.astype(np.float32),
    }
