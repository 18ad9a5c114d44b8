"""The plugin backend (gsplat_tt_amd.backend.HipBackend) driven like the
reference's Pipeline (gsplat/pipeline.py:149-182): stage by stage and through
render_fused, both against the CPU oracle at the reference's 32-pixel tiles.
Integer outputs bit-exact, images <= 1e-5 (fp32)."""
import numpy as np
import pytest
import torch

from gsplat_tt_amd import backend as B
from gsplat_tt_amd import scenes
from oracle import oracle as O

pytestmark = pytest.mark.gpu


class _Gaussians:
    def __init__(self, scene):
        self.means = torch.from_numpy(scene.means)
        self.scales = torch.from_numpy(scene.scales)
        self.rotations = torch.from_numpy(scene.quats)
        self.opacities = torch.from_numpy(scene.opacities)
        self.colors = torch.from_numpy(scene.colors)


@pytest.fixture(scope="module")
def hip_backend():
    b = B.get_backend("hip")
    yield b
    b.close()


def test_backend_stages_match_oracle(hip_backend):
    print("backend stages", flush=True)
    scene, cams = scenes.config1(seed=61, n=25_000)
    cam = cams[0]
    H, W = cam.height, cam.width
    cov = O.cov3d(scene.scales, scene.quats)
    g = _Gaussians(scene)
    m2, c2, dp, rd, valid = hip_backend.project(g.means, g.scales, g.rotations,
                                                torch.from_numpy(cam.w2c),
                                                torch.from_numpy(cam.K), H, W, g.opacities)
    o = O.project(scene.means, cov, cam.w2c, cam.K, scene.colors, scene.opacities, H, W)
    assert np.array_equal(valid.numpy(), o["valid"])
    assert c2.shape == (len(o["depths"]), 2, 2) and m2.dtype == torch.float32
    assert np.array_equal(m2.numpy(), o["means2d"]) and np.array_equal(dp.numpy(), o["depths"])
    assert np.array_equal(rd.numpy(), o["radii"])
    assert np.array_equal(c2.numpy().reshape(-1, 4), o["covs2d"])
    op_v = scene.opacities[o["valid"]]
    gid, tid, tpg = hip_backend.tile_assign(m2, rd, H, W, 32, c2, torch.from_numpy(op_v))
    og, ot, _ = O.tile_assign(o["means2d"], o["radii"], H, W, 32, o["covs2d"], op_v)
    assert gid.dtype == torch.int64 and np.array_equal(gid.numpy(), og)
    assert np.array_equal(tid.numpy(), ot)
    assert int(tpg.sum()) == len(og) and tpg.shape[0] == len(o["depths"])
    tx, ty = (W + 31) // 32, (H + 31) // 32
    sid, rng = hip_backend.sort(gid, tid, dp, tx, ty)
    os_, orr = O.sort_and_bin(og, ot, o["depths"], tx, ty)
    assert np.array_equal(sid.numpy(), os_) and np.array_equal(rng.numpy(), orr)
    col_v = scene.colors[o["valid"]]
    img, sub = hip_backend.blend(m2, c2, torch.from_numpy(col_v), torch.from_numpy(op_v),
                                 sid, rng, H, W)
    ref_img, _ = O.cull_and_blend(o["means2d"], o["covs2d"], col_v, op_v, os_, orr, tx, ty,
                                  32, H, W)
    assert img.shape == (H, W, 3) and img.dtype == np.float32
    assert float(np.abs(img - ref_img).max()) <= 1e-5


def test_backend_render_fused_matches_oracle(hip_backend):
    print("backend render_fused", flush=True)
    scene, cams = scenes.config1(seed=62, n=30_000)
    cam = cams[0]
    assert hip_backend.has_render_fused()
    g, e, k = _Gaussians(scene), torch.from_numpy(cam.w2c), torch.from_numpy(cam.K)
    img0, st0 = hip_backend.render_fused(g, e, k, cam.height, cam.width)
    assert "pairs_dropped" not in st0 and "pairs_kept_per_mb" not in st0  # not asked for
    counted = B.get_backend("hip", cull_stats=True)
    try:
        img, st = counted.render_fused(g, e, k, cam.height, cam.width)
    finally:
        counted.close()
    assert np.array_equal(img, img0)
    cov = O.cov3d(scene.scales, scene.quats)
    ref, st_o, _ = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c,
                                 cam.K, cam.height, cam.width, tile_size=32)
    print(st)
    # the stats dict of render_full (pybind_module.cpp:1537-1542), counts exact
    for k in ("num_visible", "num_entries", "pairs_in", "pairs_dropped", "pairs_kept_per_mb"):
        assert st[k] == st_o[k], (k, st[k], st_o[k])
    for k in ("project_ms", "tile_assign_ms", "sort_ms", "cull_ms", "blend_ms", "total_ms"):
        assert st[k] >= 0.0, k
    assert float(np.abs(img - ref).max()) <= 1e-5
