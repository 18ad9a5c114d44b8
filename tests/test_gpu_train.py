"""The HIP training path (gs_train_* entry points) against the reference's own
training dumps (tests/golden/t0_*: fp64 autograd of gsplat/train_oracle.py) and
against the training oracle (oracle/train_oracle.py) on a C5-shaped scene.
Bars: forward values 1e-5 relative, images 1e-4 absolute; gradients rel 1e-2 in
the reference's rel_error (its gate for the device backward); Adam moments
bit-exact, parameters within 1e-7."""
import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes
from oracle import train_oracle as TO
from tests import golden_io
from tests.test_train_oracle import rel_err

pytestmark = pytest.mark.gpu


def _fixture(name):
    g = golden_io.load(name)
    c = g["cfg_json"]
    cfg = L.make_train_cfg(near=c["near"], lowpass=c["lowpass"], alpha_max=c["alpha_max"],
                           alpha_min=c["alpha_min"], t_min=c["t_min"],
                           background=c["background"], lr=g["adam_lr_json"],
                           betas=tuple(g["adam_betas"]), eps=float(g["adam_eps"]))
    view = L.make_view(g["w2c"], g["K"], g["H"], g["W"], tile_size=16)
    params = {k: g["param_" + k].astype(np.float32) for k in TO.PARAM_NAMES}
    return g, cfg, view, params


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_train_forward_matches_dump(gpu_ctx, name):
    print("train forward", name, flush=True)
    g, cfg, view, params = _fixture(name)
    tr = L.Trainer(gpu_ctx, params, g["sh_degree"])
    img, T, pj, st = tr.forward(view, cfg, want_proj=True)
    assert np.array_equal(pj["valid"], g["valid"])
    assert np.array_equal(pj["visible"], g["visible"])
    v = g["valid"]
    for k in ("means2d", "conic", "colors", "opacity", "depth"):
        assert np.allclose(pj[k][v], g[k][v], rtol=2e-5, atol=1e-6), k
    assert float(np.abs(img - g["image"]).max()) < 1e-4
    assert float(np.abs(T - g["final_T"]).max()) < 1e-4


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_train_backward_matches_dump(gpu_ctx, name):
    print("train backward", name, flush=True)
    g, cfg, view, params = _fixture(name)
    tr = L.Trainer(gpu_ctx, params, g["sh_degree"])
    tr.forward(view, cfg)
    g2d, _ = tr.backward(cfg, dimage=g["dL_dimage"].astype(np.float32), want_g2d=True)
    ref = {"dL_dmeans2d": g2d[:, 0:2], "dL_dconic": g2d[:, 2:5], "dL_dopacity": g2d[:, 5],
           "dL_dcolors": g2d[:, 6:9]}
    for k, a in ref.items():
        e = rel_err(a, g[k])
        print(k, e)
        assert e < 1e-2, k
    grads = tr.read(3)
    for k in TO.PARAM_NAMES:
        e = rel_err(grads[k], g["grad_" + k])
        print("grad", k, e)
        assert e < 1e-2, k


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_train_adam_matches_dump(gpu_ctx, name):
    print("train adam", name, flush=True)
    g, cfg, view, params = _fixture(name)
    tr = L.Trainer(gpu_ctx, params, g["sh_degree"])
    tr.write(1, {k: g["adam_m_in_" + k] for k in TO.PARAM_NAMES})
    tr.write(2, {k: g["adam_v_in_" + k] for k in TO.PARAM_NAMES})
    tr.write(3, {k: g["grad_" + k].astype(np.float32) for k in TO.PARAM_NAMES})
    tr.set_visible(g["visible"])
    tr.set_step(int(g["adam_step_in"]))
    tr.adam(cfg)
    p, m, v = tr.read(0), tr.read(1), tr.read(2)
    for k in TO.PARAM_NAMES:
        assert np.array_equal(m[k], g["adam_fp32_m_" + k]), k
        assert np.array_equal(v[k], g["adam_fp32_v_" + k]), k
        assert np.allclose(p[k], g["adam_fp32_param_" + k], rtol=0, atol=1e-7), k



@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_train_adam_bf16_moments_matches_dump(gpu_ctx, name):
    """k_sparse_adam with bf16-stored moments against the reference's
    moment_dtype=bfloat16 step (train_oracle.py:434-470): moments bit-exact,
    parameters within 1e-7; switching the format carries the moments over."""
    print("train adam bf16 moments", name, flush=True)
    g, cfg, view, params = _fixture(name)
    tr = L.Trainer(gpu_ctx, params, g["sh_degree"])
    try:
        tr.write(1, {k: g["adam_m_in_" + k] for k in TO.PARAM_NAMES})
        tr.set_moments(True)  # fp32 moments carried over, rounded to nearest even
        m_b = tr.read(1)
        for k in TO.PARAM_NAMES:
            assert np.array_equal(m_b[k], TO.bf16_round(g["adam_m_in_" + k])), k
        tr.write(1, {k: g["adam_bf16_m_in_" + k] for k in TO.PARAM_NAMES})
        tr.write(2, {k: g["adam_bf16_v_in_" + k] for k in TO.PARAM_NAMES})
        tr.write(3, {k: g["grad_" + k].astype(np.float32) for k in TO.PARAM_NAMES})
        tr.set_visible(g["visible"])
        tr.set_step(int(g["adam_step_in"]))
        tr.adam(cfg)
        p, m, v = tr.read(0), tr.read(1), tr.read(2)
        for k in TO.PARAM_NAMES:
            assert np.array_equal(m[k], g["adam_bf16_m_" + k]), k
            assert np.array_equal(v[k], g["adam_bf16_v_" + k]), k
            assert np.allclose(p[k], g["adam_bf16_param_" + k], rtol=0, atol=1e-7), k
        tr.set_moments(False)  # back to fp32: the bf16 values exactly
        m32 = tr.read(1)
        for k in TO.PARAM_NAMES:
            assert np.array_equal(m32[k], g["adam_bf16_m_" + k]), k
    finally:
        tr.set_moments(False)

def _c5_small(n=1500, H=90, W=160, seed=55):
    scene, tgt_scene, cams = scenes.config5(seed=seed, n=n)
    K = scenes.intrinsics(0.5 * W / np.tan(np.deg2rad(25.0)), 0.5 * W / np.tan(np.deg2rad(25.0)),
                          W / 2, H / 2)
    return scenes.train_params(scene), scenes.train_params(tgt_scene), cams[0].w2c, K, H, W


def test_train_steps_match_oracle(gpu_ctx):
    """Three whole steps (forward + L1 + backward + sparse Adam) of a C5-shaped
    scene (SH degree 1) against the oracle's steps from the same parameters."""
    print("train steps c5-shaped", flush=True)
    params, tparams, w2c, K, H, W = _c5_small()
    cfg_o = TO.Cfg(sh_degree=1)
    cfg = L.make_train_cfg()
    view = L.make_view(w2c, K, H, W, tile_size=16)
    # target: the oracle's render of the perturbed copy
    _, target, _, _, _ = TO.forward(tparams, w2c, K, H, W, cfg_o)
    target = target.astype(np.float32)
    tr = L.Trainer(gpu_ctx, params, 1)
    p_o = {k: v.astype(np.float32) for k, v in params.items()}
    m_o = {k: np.zeros_like(v) for k, v in p_o.items()}
    v_o = {k: np.zeros_like(v) for k, v in p_o.items()}
    for step in range(3):
        st = tr.step(view, cfg, target)
        pr, img, fT, order, live = TO.forward(p_o, w2c, K, H, W, cfg_o)
        loss, dimg = TO.l1_loss_grad(img, target)
        g2 = TO.blend_backward(pr, order, live, fT, dimg, H, W, cfg_o)
        grads = TO.projection_backward(pr, g2, cfg_o)
        out = TO.sparse_adam(p_o, grads, m_o, v_o, step, pr["visible"])
        p_o = {k: out[k][0] for k in out}
        m_o = {k: out[k][1] for k in out}
        v_o = {k: out[k][2] for k in out}
        print(f"step {step}: loss gpu {st['loss']:.6f} oracle {loss:.6f}, M {st['num_blendable']}"
              f" P {st['num_entries']}")
        assert abs(st["loss"] - loss) <= 1e-4 * max(loss, 1e-6) + 1e-7
    p = tr.read(0)
    for k in TO.PARAM_NAMES:
        d = np.abs(p[k] - p_o[k]).max()
        moved = np.abs(p_o[k] - params[k]).max()
        print(k, "max diff", d, "moved", moved)
        assert d <= 1e-2 * max(moved, 1e-12) + 1e-6, k


@pytest.mark.parametrize("name", golden_io.TRAIN_CASES)
def test_train_loss_ssim_matches_dump(gpu_ctx, name):
    """gs_train_loss with lambda 0.2 is the reference's full loss: its value and
    dL/dimage against the dump (fp64 autograd of 0.8 L1 + 0.2 (1 - SSIM)), on the
    dump's image rounded to fp32 (the oracle re-evaluated on those inputs pins
    the rounding part)."""
    print("train loss ssim", name, flush=True)
    g = golden_io.load(name)
    img, tgt = g["image"].astype(np.float32), g["target"].astype(np.float32)
    loss, l1, ssim, grad = gpu_ctx.train_loss(img, tgt, 0.2)
    lo, l1o, so, go = TO.ssim_loss_grad(img, tgt, 0.2)
    print(f"loss gpu {loss:.9f} oracle {lo:.9f} dump {float(g['loss']):.9f}; "
          f"grad rel {rel_err(grad, go):.3g}")
    assert abs(loss - lo) <= 1e-6 * lo and abs(l1 - l1o) <= 1e-6 * l1o
    assert abs(ssim - so) <= 1e-6
    assert abs(lo - float(g["loss"])) <= 1e-6 * lo  # fp32 rounding of the inputs only
    assert rel_err(grad, go) < 1e-3
    assert rel_err(grad, g["dL_dimage"]) < 1e-2  # the reference's device-backward gate


def test_train_loss_ssim_full_size(gpu_ctx):
    """1280x720 image against a noisy, blurred-edge target: device loss terms and
    gradient against the fp64 oracle; lambda 0 gives the plain L1 gradient."""
    print("train loss ssim 1280x720", flush=True)
    rng = np.random.default_rng(9)
    H, W = 720, 1280
    tgt = rng.uniform(0, 1, (H, W, 3)).astype(np.float32)
    img = np.clip(tgt + rng.normal(0, 0.05, tgt.shape), 0, 1).astype(np.float32)
    img[100:300, 200:600] = 0.5  # a flat patch: low-variance SSIM terms
    loss, l1, ssim, grad = gpu_ctx.train_loss(img, tgt, 0.2)
    lo, l1o, so, go = TO.ssim_loss_grad(img, tgt, 0.2)
    e = rel_err(grad, go)
    print(f"loss gpu {loss:.9f} oracle {lo:.9f} ssim {ssim:.7f}/{so:.7f} grad rel {e:.3g}")
    assert abs(loss - lo) <= 1e-6 * lo and abs(ssim - so) <= 1e-6
    assert e < 1e-3
    l0, l10, s0, g0 = gpu_ctx.train_loss(img, tgt, 0.0, loss_scale=2.0)
    d = img.astype(np.float64) - tgt
    assert s0 == 0.0 and abs(l0 - 2.0 * np.abs(d).mean()) <= 1e-6 * l0
    assert np.array_equal(g0, (np.sign(d) * (2.0 / d.size)).astype(np.float32))


def test_train_step_ssim_loss_matches_oracle(gpu_ctx):
    """One whole step with the full 3DGS loss (lambda 0.2) of a C5-shaped scene
    against the oracle's forward, SSIM loss gradient, backward and Adam."""
    print("train step ssim c5-shaped", flush=True)
    params, tparams, w2c, K, H, W = _c5_small(seed=57)
    cfg_o = TO.Cfg(sh_degree=1)
    cfg = L.make_train_cfg(lambda_dssim=0.2)
    view = L.make_view(w2c, K, H, W, tile_size=16)
    _, target, _, _, _ = TO.forward(tparams, w2c, K, H, W, cfg_o)
    target = target.astype(np.float32)
    tr = L.Trainer(gpu_ctx, params, 1)
    st = tr.step(view, cfg, target)
    p_o = {k: v.astype(np.float32) for k, v in params.items()}
    pr, img, fT, order, live = TO.forward(p_o, w2c, K, H, W, cfg_o)
    loss, l1, ssim, dimg = TO.ssim_loss_grad(img, target, 0.2)
    g2 = TO.blend_backward(pr, order, live, fT, dimg, H, W, cfg_o)
    grads = TO.projection_backward(pr, g2, cfg_o)
    zeros = {k: np.zeros_like(v) for k, v in p_o.items()}
    out = TO.sparse_adam(p_o, grads, zeros, dict(zeros), 0, pr["visible"])
    print(f"loss gpu {st['loss']:.7f} oracle {loss:.7f}; ssim {st['ssim']:.7f}/{ssim:.7f}")
    assert abs(st["loss"] - loss) <= 1e-4 * loss
    assert abs(st["ssim"] - ssim) <= 1e-5 and abs(st["l1"] - l1) <= 1e-4 * l1
    p = tr.read(0)
    for k in TO.PARAM_NAMES:
        d = np.abs(p[k] - out[k][0]).max()
        moved = np.abs(out[k][0] - params[k]).max()
        print(k, "max diff", d, "moved", moved)
        assert d <= 1e-2 * max(moved, 1e-12) + 1e-6, k



def test_train_pair_capacity_retry():
    """A first training forward whose candidate pairs exceed the context's
    starting capacity (max(2^20, 8N)): 4000 large, faint Gaussians at 320x240
    (300 tiles) give about 1.19M candidates. The forward grows the capacity and
    re-runs: its image and loss equal the oracle's, and its backward equals the
    backward of the same forward run again at the grown capacity (no re-run).
    (The oracle blends every pixel for every Gaussian, so its cost is at least
    256 x 2^20 pixel evaluations: its backward is left to the smaller cases.)"""
    print("train pair-capacity retry", flush=True)
    rng = np.random.default_rng(61)
    n, H, W = 4000, 240, 320
    z = rng.uniform(4.0, 6.0, n)
    params = {
        "means": np.stack([rng.uniform(-1.2, 1.2, n) * z / 4.0,
                           rng.uniform(-0.9, 0.9, n) * z / 4.0, z], -1).astype(np.float32),
        "log_scales": rng.normal(np.log(2.2), 0.1, (n, 3)).astype(np.float32),
        "quats": rng.normal(0, 1, (n, 4)).astype(np.float32),
        "opacity_logits": rng.normal(-3.5, 0.3, n).astype(np.float32),
        "sh": rng.uniform(-0.5, 0.5, (n, 1, 3)).astype(np.float32),
    }
    target = rng.uniform(0.0, 1.0, (H, W, 3)).astype(np.float32)
    w2c = np.eye(4, dtype=np.float32)
    K = scenes.intrinsics(250.0, 250.0, W / 2, H / 2)
    cfg = L.make_train_cfg()
    view = L.make_view(w2c, K, H, W, tile_size=16)
    ctx = L.Context(0)  # a fresh context: the capacity starts at the default
    try:
        tr = L.Trainer(ctx, params, 0)
        img, T, _, st = tr.forward(view, cfg, target)
        print(f"pairs_pre {st['pairs_pre']} capacity {st['pair_capacity']} "
              f"P {st['num_entries']}", flush=True)
        assert st["pairs_pre"] > (1 << 20)
        assert st["pair_capacity"] >= st["pairs_pre"]
        tr.backward(cfg)
        g_retry = tr.read(3)
        cap = st["pair_capacity"]
        img2, _, _, st2 = tr.forward(view, cfg, target)
        assert st2["pair_capacity"] == cap and st2["pairs_pre"] == st["pairs_pre"]
        assert np.array_equal(img2, img) and st2["loss"] == st["loss"]
        tr.backward(cfg)
        g_direct = tr.read(3)
    finally:
        ctx.close()
    for k in TO.PARAM_NAMES:
        # atomics add in another order: equal up to fp32 summation order
        e = rel_err(g_retry[k], g_direct[k])
        d = float(np.abs(g_retry[k] - g_direct[k]).max() / np.abs(g_direct[k]).max())
        print("grad", k, "retry vs direct: rel", e, "max-normalised", d)
        assert e < 1e-2 and d < 1e-4, k
    cfg_o = TO.Cfg(sh_degree=0)
    _, img_o, T_o, _, _ = TO.forward(params, w2c, K, H, W, cfg_o)
    loss_o, _ = TO.l1_loss_grad(img_o, target)
    d = float(np.abs(img - img_o).max())
    print(f"image max_abs {d:.3g}; loss gpu {st['loss']:.7f} oracle {loss_o:.7f}", flush=True)
    assert d < 1e-4 and float(np.abs(T - T_o).max()) < 1e-4
    assert abs(st["loss"] - loss_o) <= 1e-4 * loss_o
