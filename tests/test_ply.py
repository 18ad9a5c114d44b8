"""PLY loading with the reference's activations (gsplat/loading_gaussians.py:7-65),
on files this test writes: binary little- and big-endian and ascii, with and
without the higher-order SH coefficients."""
import numpy as np
import pytest
import torch

from gsplat_tt_amd import ply


def _raw(n, rest=0, seed=3):
    rng = np.random.default_rng(seed)
    a = {"x": rng.normal(size=n), "y": rng.normal(size=n), "z": rng.uniform(2, 8, n),
         "nx": np.zeros(n), "ny": np.zeros(n), "nz": np.zeros(n)}
    for i in range(3):
        a[f"f_dc_{i}"] = rng.normal(0, 2, n)
    for i in range(rest):
        a[f"f_rest_{i}"] = rng.normal(0, 0.3, n)
    a["opacity"] = rng.normal(0, 3, n)
    for i in range(3):
        a[f"scale_{i}"] = rng.normal(-4, 1, n)
    for i in range(4):
        a[f"rot_{i}"] = rng.normal(size=n)
    return {k: np.asarray(v, np.float32) for k, v in a.items()}


@pytest.mark.parametrize("fmt", ["binary_little_endian", "binary_big_endian", "ascii"])
def test_load_ply_activations(tmp_path, fmt):
    raw = _raw(500)
    p = str(tmp_path / "s.ply")
    ply.write_ply(p, raw, fmt)
    g = ply.load_ply(p)
    assert g.num_gaussians == 500 and g.sh is None and g.sh_degree == -1
    t = {k: torch.from_numpy(v) for k, v in raw.items()}
    # the reference's torch expressions, fp32
    means = torch.stack([t["x"], t["y"], t["z"]], -1)
    scales = torch.exp(torch.stack([t[f"scale_{i}"] for i in range(3)], -1))
    q = torch.stack([t[f"rot_{i}"] for i in range(4)], -1)
    q = q / q.norm(dim=-1, keepdim=True)
    col = torch.clamp(0.5 + ply.SH_C0 * torch.stack([t[f"f_dc_{i}"] for i in range(3)], -1),
                      0.0, 1.0)
    op = torch.sigmoid(t["opacity"])
    for a, b in ((g.means, means), (g.scales, scales), (g.rotations, q), (g.colors, col),
                 (g.opacities, op)):
        assert np.array_equal(a, b.numpy())
    # closed forms, independent of torch: exp / sigmoid to 1 ulp in float64,
    # unit quaternions, colours and opacities in range
    ls = np.stack([raw[f"scale_{i}"] for i in range(3)], -1).astype(np.float64)
    np.testing.assert_allclose(g.scales, np.exp(ls), rtol=2.4e-7)
    np.testing.assert_allclose(g.opacities, 1.0 / (1.0 + np.exp(-raw["opacity"].astype(
        np.float64))), rtol=2.4e-7)
    np.testing.assert_allclose(np.linalg.norm(g.rotations.astype(np.float64), axis=1), 1.0,
                               atol=1e-6)
    assert g.colors.min() >= 0.0 and g.colors.max() <= 1.0
    assert g.opacities.min() > 0.0 and g.opacities.max() < 1.0
    for arr in (g.means, g.scales, g.rotations, g.colors, g.opacities):
        assert arr.dtype == np.float32


@pytest.mark.parametrize("deg", [1, 2, 3])
def test_load_ply_sh_rest_layout(tmp_path, deg):
    K = (deg + 1) ** 2
    raw = _raw(64, rest=3 * (K - 1))
    p = str(tmp_path / "sh.ply")
    ply.write_ply(p, raw)
    g = ply.load_ply(p)
    assert g.sh.shape == (64, K, 3) and g.sh_degree == deg
    for c in range(3):
        assert np.array_equal(g.sh[:, 0, c], raw[f"f_dc_{c}"])
        for k in range(1, K):
            # stored channel-major: f_rest_{c (K-1) + k - 1}
            assert np.array_equal(g.sh[:, k, c], raw[f"f_rest_{c * (K - 1) + k - 1}"])


def test_load_ply_errors(tmp_path):
    p = tmp_path / "bad.ply"
    p.write_bytes(b"not a ply\n")
    with pytest.raises(ValueError):
        ply.load_ply(str(p))
    raw = _raw(8)
    del raw["opacity"]
    ply.write_ply(str(p), raw)
    with pytest.raises(ValueError, match="opacity"):
        ply.load_ply(str(p))
    raw = _raw(8, rest=5)
    ply.write_ply(str(p), raw)
    with pytest.raises(ValueError):
        ply.load_ply(str(p))
