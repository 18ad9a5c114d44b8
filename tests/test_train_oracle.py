"""The training oracle (oracle/train_oracle.py) against the reference's own
training dumps (gsplat/train_oracle.py, fp64 torch autograd; tests/golden/t0_*)
and against central finite differences."""
import json

import numpy as np
import pytest

from oracle import train_oracle as TO
from tests import golden_io


def _case(name):
    g = golden_io.load(name)
    cfg_j = g["cfg_json"]
    cfg = TO.Cfg(sh_degree=g["sh_degree"], near=cfg_j["near"], lowpass=cfg_j["lowpass"],
                 alpha_max=cfg_j["alpha_max"], alpha_min=cfg_j["alpha_min"],
                 t_min=cfg_j["t_min"], background=tuple(cfg_j["background"]))
    params = {k: g["param_" + k] for k in TO.PARAM_NAMES}
    return g, cfg, params


def rel_err(a, ref, floor_frac=1e-4):
    """max |a - ref| / max(|ref|, floor_frac * max |ref|) (train_oracle.py:406-418)."""
    a, ref = np.asarray(a, np.float64).ravel(), np.asarray(ref, np.float64).ravel()
    scale = np.abs(ref).max() if ref.size else 0.0
    if scale == 0.0:
        return float(np.abs(a).max()) if a.size else 0.0
    return float((np.abs(a - ref) / np.maximum(np.abs(ref), floor_frac * scale)).max())


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_forward_matches_dump(name):
    g, cfg, params = _case(name)
    pr, image, final_T, order, live = TO.forward(params, g["w2c"], g["K"], g["H"], g["W"], cfg)
    assert np.array_equal(pr["valid"], g["valid"])
    assert np.array_equal(pr["visible"], g["visible"])
    assert np.array_equal(order, g["order"])
    for k, ref in (("means2d", g["means2d"]), ("conic", g["conic"]), ("colors", g["colors"]),
                   ("opacity", g["opacity"]), ("depth", g["depth"])):
        assert np.allclose(pr[k][pr["valid"]], ref[pr["valid"]], rtol=1e-12, atol=1e-12), k
    assert np.allclose(image, g["image"], atol=1e-12)
    assert np.allclose(final_T, g["final_T"], atol=1e-12)


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_blend_backward_matches_dump(name):
    g, cfg, params = _case(name)
    pr, image, final_T, order, live = TO.forward(params, g["w2c"], g["K"], g["H"], g["W"], cfg)
    gb = TO.blend_backward(pr, order, live, final_T, g["dL_dimage"], g["H"], g["W"], cfg)
    for k in ("dL_dmeans2d", "dL_dconic", "dL_dopacity", "dL_dcolors"):
        assert rel_err(gb[k], g[k]) < 1e-8, k


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_projection_backward_matches_dump(name):
    g, cfg, params = _case(name)
    pr = TO.project(params, g["w2c"], g["K"], g["H"], g["W"], cfg)
    g2 = {k: g[k] for k in ("dL_dmeans2d", "dL_dconic", "dL_dopacity", "dL_dcolors")}
    grads = TO.projection_backward(pr, g2, cfg)
    for k in TO.PARAM_NAMES:
        assert rel_err(grads[k], g["grad_" + k]) < 1e-8, k


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_sparse_adam_matches_dump(name):
    g, cfg, params = _case(name)
    grads = {k: g["grad_" + k] for k in TO.PARAM_NAMES}
    m = {k: g["adam_m_in_" + k] for k in TO.PARAM_NAMES}
    v = {k: g["adam_v_in_" + k] for k in TO.PARAM_NAMES}
    lr = g["adam_lr_json"]
    out = TO.sparse_adam(params, grads, m, v, g["adam_step_in"], g["visible"], lr,
                         tuple(g["adam_betas"]), float(g["adam_eps"]))
    for k in TO.PARAM_NAMES:
        p, mm, vv = out[k]
        assert np.array_equal(mm, g["adam_fp32_m_" + k]), k
        assert np.array_equal(vv, g["adam_fp32_v_" + k]), k
        assert np.allclose(p, g["adam_fp32_param_" + k], rtol=0, atol=1e-7), k
        # untouched rows stay bit-identical
        inv = ~g["visible"]
        assert np.array_equal(p[inv], np.asarray(params[k], np.float32)[inv])


def test_bf16_round_is_torch_rne():
    """bf16_round against torch's float -> bfloat16 conversion (round to nearest
    even) on edge patterns and random floats, and the tie cases by hand."""
    import torch
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)  # bf16 spacing at 1
    ties = np.array([one + ulp / 2, one + 3 * ulp / 2, -(one + ulp / 2)], np.float32)
    assert np.array_equal(TO.bf16_round(ties), np.array([one, one + 2 * ulp, -one], np.float32))
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(
        -30, 30, 100_000), np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-45, -1e-40],
                                    np.float32)]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(TO.bf16_round(x).view(np.uint32), ref.view(np.uint32))
    assert np.isnan(TO.bf16_round(np.array([np.nan], np.float32))).all()


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_sparse_adam_bf16_moments_matches_dump(name):
    """The reference's bf16-moment Adam (moment_dtype bfloat16): moments in
    from the dump's adam_bf16_*_in, moments out bit-exact, parameters 1e-7."""
    g, cfg, params = _case(name)
    grads = {k: g["grad_" + k] for k in TO.PARAM_NAMES}
    m = {k: g["adam_bf16_m_in_" + k] for k in TO.PARAM_NAMES}
    v = {k: g["adam_bf16_v_in_" + k] for k in TO.PARAM_NAMES}
    out = TO.sparse_adam(params, grads, m, v, g["adam_step_in"], g["visible"],
                         g["adam_lr_json"], tuple(g["adam_betas"]), float(g["adam_eps"]),
                         bf16_moments=True)
    for k in TO.PARAM_NAMES:
        p, mm, vv = out[k]
        assert np.array_equal(mm, g["adam_bf16_m_" + k]), k
        assert np.array_equal(vv, g["adam_bf16_v_" + k]), k
        assert not (mm.view(np.uint32) & 0xFFFF).any() and not (vv.view(np.uint32) & 0xFFFF).any()
        assert np.allclose(p, g["adam_bf16_param_" + k], rtol=0, atol=1e-7), k
        # the bf16 step differs from the fp32 one (the fixture pins a real change)
    assert any(not np.array_equal(out[k][1], g["adam_fp32_m_" + k]) for k in TO.PARAM_NAMES)


def test_l1_gradient():
    rng = np.random.default_rng(0)
    a = rng.uniform(size=(4, 5, 3))
    b = a.copy()
    b[0, 0, 0] += 0.5
    b[1, 1, 1] -= 0.25
    loss, grad = TO.l1_loss_grad(a, b)
    assert np.isclose(loss, 0.75 / a.size)
    assert grad[0, 0, 0] == -1.0 / a.size and grad[1, 1, 1] == 1.0 / a.size
    assert np.count_nonzero(grad) == 2   # sign(0) = 0


def _tiny_scene(seed, n=12, H=24, W=24, deg=1):
    rng = np.random.default_rng(seed)
    K = (deg + 1) ** 2
    params = {
        "means": np.column_stack([rng.uniform(-0.6, 0.6, n), rng.uniform(-0.6, 0.6, n),
                                  rng.uniform(2.5, 4.0, n)]),
        "log_scales": rng.normal(-2.3, 0.3, (n, 3)),
        "quats": rng.normal(size=(n, 4)),
        "opacity_logits": rng.normal(0.0, 1.0, n),
        "sh": np.concatenate([rng.uniform(0, 1, (n, 1, 3)),
                              rng.normal(0, 0.2, (n, K - 1, 3))], 1),
    }
    w2c = np.eye(4)
    w2c[:3, 3] = [0.05, -0.02, 0.1]
    Kc = np.array([[30.0, 0, W / 2], [0, 30.0, H / 2], [0, 0, 1]])
    return params, w2c, Kc, H, W


@pytest.mark.parametrize("deg", [1, 2])
def test_gradients_vs_finite_differences(deg):
    """Analytic blend + projection backward vs central differences of the L1 loss,
    with the forward's discrete decisions (live pairs, clamps, order) frozen by
    choosing a step (1e-6) far below any decision margin."""
    params, w2c, Kc, H, W = _tiny_scene(7 + deg, deg=deg)
    cfg = TO.Cfg(sh_degree=deg)
    rng = np.random.default_rng(1)
    target = rng.uniform(0, 1, (H, W, 3))
    pr, image, final_T, order, live = TO.forward(params, w2c, Kc, H, W, cfg)
    _, dimg = TO.l1_loss_grad(image, target)
    g2 = TO.blend_backward(pr, order, live, final_T, dimg, H, W, cfg)
    grads = TO.projection_backward(pr, g2, cfg)

    def loss_of(p):
        _, im, _, _, lv = TO.forward(p, w2c, Kc, H, W, cfg)
        if not np.array_equal(lv, live):
            return None
        return float(np.abs(im - target).sum() / im.size)

    eps = 1e-6
    checked = 0
    for name in TO.PARAM_NAMES:
        flat = params[name].reshape(-1)
        for idx in rng.choice(flat.size, size=min(12, flat.size), replace=False):
            pp = {k: v.copy() for k, v in params.items()}
            pp[name].reshape(-1)[idx] += eps
            lp = loss_of(pp)
            pm = {k: v.copy() for k, v in params.items()}
            pm[name].reshape(-1)[idx] -= eps
            lm = loss_of(pm)
            if lp is None or lm is None:
                continue
            fd = (lp - lm) / (2 * eps)
            an = grads[name].reshape(-1)[idx]
            scale = np.abs(grads[name]).max()
            assert abs(fd - an) <= 1e-5 * scale + 1e-9, (name, idx, fd, an)
            checked += 1
    assert checked > 40


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_ssim_loss_matches_dump(name):
    """The dumps' `loss` and `dL_dimage` are the reference's full 3DGS loss
    0.8 L1 + 0.2 (1 - SSIM) and its fp64 autograd image gradient."""
    g = golden_io.load(name)
    loss, l1, ssim, grad = TO.ssim_loss_grad(g["image"], g["target"], 0.2)
    assert abs(loss - float(g["loss"])) <= 1e-12
    assert rel_err(grad, g["dL_dimage"]) < 1e-10
    assert 0.0 < ssim < 1.0 and l1 > 0.0


def test_ssim_identity_and_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.uniform(0, 1, (9, 13, 3))
    # identical images: SSIM = 1 exactly at every pixel, a maximum (zero gradient)
    loss, l1, ssim, grad = TO.ssim_loss_grad(x, x, 0.2)
    assert abs(ssim - 1.0) < 1e-12 and l1 == 0.0 and abs(loss) < 1e-12
    assert np.abs(grad).max() < 1e-12
    # pure SSIM term (lambda = 1, no L1 kink) against central differences
    y = np.clip(x + rng.normal(0, 0.1, x.shape), 0, 1)
    _, _, _, g = TO.ssim_loss_grad(x, y, 1.0)
    eps = 1e-6
    for idx in rng.choice(x.size, 25, replace=False):
        xp = x.copy().reshape(-1)
        xp[idx] += eps
        xm = x.copy().reshape(-1)
        xm[idx] -= eps
        fd = (TO.ssim_loss_grad(xp.reshape(x.shape), y, 1.0)[0] -
              TO.ssim_loss_grad(xm.reshape(x.shape), y, 1.0)[0]) / (2 * eps)
        assert abs(fd - g.reshape(-1)[idx]) <= 1e-7 * np.abs(g).max() + 1e-12
    # the window is the reference's normalised 11-tap Gaussian (sigma 1.5)
    w = TO.gauss_window()
    assert w.shape == (11,) and abs(w.sum() - 1.0) < 1e-15 and np.argmax(w) == 5
