"""A scene loaded from a .ply file (gsplat_tt_amd.ply.load_ply, the reference's
gsplat/loading_gaussians.py:32-65 activations) rendered on the GPU through the
plugin backend's render_fused and through render_clean.render_view, against
the oracle on the same activated values: counts exact, f32 image <= 1e-5, and
the SH3 file rendered with its higher-order coefficients."""
import numpy as np
import pytest
import torch

import gsplat_tt_amd
from gsplat_tt_amd import backend as B
from gsplat_tt_amd import ply
from oracle import oracle as O
from tests import oracle_frames as F

pytestmark = pytest.mark.gpu


def _write_scene(path, n, rest, seed):
    """A trained-scene-like file: means in front of the first C1 camera, log
    scales, raw quaternions, SH DC (+ rest) and opacity logits."""
    rng = np.random.default_rng(seed)
    a = {"x": rng.uniform(-2.0, 2.0, n), "y": rng.uniform(-1.5, 1.5, n),
         "z": rng.uniform(2.0, 8.0, n), "nx": np.zeros(n), "ny": np.zeros(n), "nz": np.zeros(n)}
    for i in range(3):
        a[f"f_dc_{i}"] = rng.normal(0, 1.0, n)
    for i in range(rest):
        a[f"f_rest_{i}"] = rng.normal(0, 0.2, n)
    a["opacity"] = rng.normal(0, 2.0, n)
    for i in range(3):
        a[f"scale_{i}"] = rng.normal(-4.0, 0.7, n)
    for i in range(4):
        a[f"rot_{i}"] = rng.normal(size=n)
    ply.write_ply(path, {k: np.asarray(v, np.float32) for k, v in a.items()})


class _Cam:
    """Camera at the origin looking down +z (w2c = I), 640x480, f = 500."""
    height, width = 480, 640
    w2c = np.eye(4, dtype=np.float32)
    K = np.array([[500.0, 0.0, 320.0], [0.0, 500.0, 240.0], [0.0, 0.0, 1.0]], np.float32)


def _camera():
    return _Cam()


def test_ply_scene_through_backend_and_render_view(tmp_path):
    print("ply -> render_fused / render_view", flush=True)
    p = str(tmp_path / "scene.ply")
    _write_scene(p, 20_000, 0, seed=5)
    g = ply.load_ply(p)
    cam = _camera()
    cov = O.cov3d(g.scales, g.rotations)
    ref, st_o, _ = O.render_full(g.means, cov, g.opacities, g.colors, cam.w2c, cam.K,
                                 cam.height, cam.width, tile_size=32)
    assert st_o["num_visible"] > 1000
    b = B.get_backend("hip", cull_stats=True)
    try:
        img, st = b.render_fused(g, torch.from_numpy(cam.w2c), torch.from_numpy(cam.K),
                                 cam.height, cam.width)
    finally:
        b.close()
    for k in ("num_visible", "num_entries", "pairs_dropped", "pairs_kept_per_mb"):
        assert st[k] == st_o[k], (k, st[k], st_o[k])
    assert float(np.abs(img - ref).max()) <= 1e-5
    # render_clean.render_view on the same loaded scene (16-px tiles, f32 out)
    rc = gsplat_tt_amd.render_clean_module()
    ref16 = F.frame(g.means, cov, g.opacities, g.colors, cam, 16)
    img16, st16 = rc.render_view(g.means, cov.reshape(-1, 3, 3), g.opacities, g.colors,
                                 cam.w2c, cam.K, cam.height, cam.width, tile_size=16,
                                 min_opacity=1.0 / 255.0, contrib_floor=1.0 / 16384.0,
                                 mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                                 transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
                                 use_isoellipse=False, output="f32")
    assert st16["num_visible"] == ref16["M"] and st16["num_entries"] == ref16["P"]
    assert float(np.abs(np.array(img16) - ref16["image"]).max()) <= 1e-5


def test_ply_sh3_scene_renders_with_its_coefficients(tmp_path, gpu_ctx):
    print("ply SH3 -> frame", flush=True)
    p = str(tmp_path / "sh3.ply")
    _write_scene(p, 10_000, 45, seed=6)
    g = ply.load_ply(p)
    assert g.sh_degree == 3
    cam = _camera()
    cov = O.cov3d(g.scales, g.rotations)
    # the oracle's SH colour for this view, then the reference renderer
    rgb = O.sh_rgb(g.means, g.sh, 3, cam.w2c)
    ref = F.frame(g.means, cov, g.opacities, rgb, cam, 16)
    from gsplat_tt_amd import _lib as L
    gpu_ctx.set_scene(g.means, cov, g.opacities, g.sh, sh_degree=3)
    img, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16,
                                         output="f32"))
    assert st["num_visible"] == ref["M"] and st["num_entries"] == ref["P"]
    assert float(np.abs(img - ref["image"]).max()) <= 1e-5
