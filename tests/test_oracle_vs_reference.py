"""The C oracle against the reference's own CPU module, compiled from its sources
into oracle/_ref (skipped where the reference checkout is absent): bit-exact
projection, tile assignment, sort, image and stats on seeded C1-shaped scenes."""
import numpy as np
import pytest

from gsplat_tt_amd import scenes
from oracle import oracle as O

R = O.ref_module()
pytestmark = pytest.mark.skipif(R is None, reason="oracle/_ref not built (no reference checkout)")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


@pytest.mark.parametrize("seed,ts,cull_disabled", [(7, 16, False), (8, 32, False), (9, 16, True)])
def test_render_full_bitexact(seed, ts, cull_disabled):
    scene, cams = scenes.config1(seed=seed, n=20_000)
    cam = cams[0]
    cov = O.cov3d(scene.scales, scene.quats)
    covr = np.asarray(R.compute_cov3d(scene.scales, scene.quats), np.float32).reshape(-1, 9)
    assert np.array_equal(_bits(cov), _bits(covr))
    img, st, inter = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c,
                                   cam.K, cam.height, cam.width, tile_size=ts,
                                   cull_disabled=cull_disabled)
    imgr, str_ = R.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c, cam.K,
                               cam.height, cam.width, tile_size=ts, cull_disabled=cull_disabled)
    assert np.array_equal(_bits(img), _bits(np.asarray(imgr)))
    for k in ("num_visible", "num_entries", "pairs_in", "pairs_dropped", "pairs_kept_per_mb"):
        assert st[k] == str_[k], k
    pr = inter["project"]
    m2, c2, d, r, v = R.project_full_with_cov3d(scene.means, cov, cam.w2c, cam.K, cam.height,
                                                cam.width, scene.opacities)
    assert np.array_equal(np.asarray(v).astype(bool), pr["valid"])
    for a, b in ((m2, pr["means2d"]), (c2, pr["covs2d"]), (d, pr["depths"]), (r, pr["radii"])):
        assert np.array_equal(_bits(np.asarray(a)), _bits(b))
    if not cull_disabled:
        g, t, _ = R.tile_assign(pr["means2d"], pr["radii"], cam.height, cam.width, ts,
                                pr["covs2d"], pr["opacities"], 1.0 / 16384.0)
        assert np.array_equal(np.asarray(g), inter["gids"])
        assert np.array_equal(np.asarray(t), inter["tids"])
        s, rr = R.sort(g, t, pr["depths"], (cam.width + ts - 1) // ts,
                       (cam.height + ts - 1) // ts)
        assert np.array_equal(np.asarray(s), inter["sorted_ids"])
        assert np.array_equal(np.asarray(rr).reshape(-1, 2), inter["tile_ranges"])


def test_sh_matches_reference_free_closed_form():
    """SH degree 3 colour of the oracle against a float64 evaluation of the same
    real-SH basis (gsplat/train_oracle.py:46-52,99-122)."""
    rng = np.random.default_rng(5)
    n = 256
    means = rng.normal(size=(n, 3)).astype(np.float32) * 3
    sh = rng.normal(size=(n, 16, 3)).astype(np.float32) * 0.3
    w2c = scenes.look_at_w2c(np.array([0.5, -1.0, -4.0]), np.zeros(3))
    rgb = O.sh_rgb(means, sh, 3, w2c, clamp_hi=False)
    R3, t = w2c[:3, :3].astype(np.float64), w2c[:3, 3].astype(np.float64)
    c = -R3.T @ t
    d = means.astype(np.float64) - c
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    x, y, z = d[:, 0], d[:, 1], d[:, 2]
    C0, C1 = 0.28209479177387814, 0.4886025119029199
    C2 = [1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
          0.5462742152960396]
    C3 = [-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
          -0.4570457994644658, 1.445305721320277, -0.5900435899266435]
    xx, yy, zz = x * x, y * y, z * z
    basis = [np.full(n, C0), -C1 * y, C1 * z, -C1 * x,
             C2[0] * x * y, C2[1] * y * z, C2[2] * (2 * zz - xx - yy), C2[3] * x * z,
             C2[4] * (xx - yy),
             C3[0] * y * (3 * xx - yy), C3[1] * x * y * z, C3[2] * y * (4 * zz - xx - yy),
             C3[3] * z * (2 * zz - 3 * xx - 3 * yy), C3[4] * x * (4 * zz - xx - yy),
             C3[5] * z * (xx - yy), C3[6] * x * (xx - 3 * yy)]
    want = sum(b[:, None] * sh[:, k, :].astype(np.float64) for k, b in enumerate(basis)) + 0.5
    assert np.allclose(rgb, np.maximum(want, 0.0), atol=2e-6)
