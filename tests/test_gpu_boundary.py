"""The drop-in boundary against the oracle, and the option paths of the frame.

  * render_clean.render_view (the reference's module surface, render/host/
    render.cpp:263-273) with its defaults: f32, bf16 and the default u8 output.
    The u8 image is the bf16 image packed as the reference's render_view does
    (img_pack_u8.h:9-14): bit-exact from the GPU's own bf16 image, and within
    one level of the oracle image packed by the same rule.
  * cull_disabled=True frames (no per-pair cull, every microblock the AABB
    touches) and use_isoellipse=True (eigen-decomposed AABB): ids and ranges
    against the oracle run with the same options.
  * the reference's microblock-cull statistics (pairs_dropped,
    pairs_kept_per_mb) at 16- and 32-pixel tiles.
  * a bounded look-back wait that gives up (a host-set spin limit of one round)
    makes the call fail with a device error instead of returning results; every
    kernel still exits, and the next call with the default limit is exact.
"""
import numpy as np
import pytest

import gsplat_tt_amd
from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes
from oracle import oracle as O
from tests import oracle_frames as F

pytestmark = pytest.mark.gpu

DEFAULTS = dict(tile_size=16, min_opacity=1.0 / 255.0, contrib_floor=1.0 / 16384.0,
                mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
                use_isoellipse=False)


@pytest.fixture(scope="module")
def c1():
    scene, cams = scenes.config1(seed=71, n=100_000)
    cam = cams[0]
    cov = O.cov3d(scene.scales, scene.quats)
    return scene, cam, cov


def test_render_view_outputs_match_oracle(c1):
    print("render_view f32/bf16/u8 vs oracle", flush=True)
    scene, cam, cov = c1
    rc = gsplat_tt_amd.render_clean_module()
    ref = F.frame(scene.means, cov, scene.opacities, scene.colors, cam, 16)
    args = (scene.means, cov.reshape(-1, 3, 3), scene.opacities, scene.colors, cam.w2c, cam.K,
            cam.height, cam.width)
    imgs = {}
    for out in ("f32", "bf16", "u8"):
        img, st = rc.render_view(*args, **DEFAULTS, output=out)
        assert st["num_visible"] == ref["M"] and st["num_entries"] == ref["P"]
        imgs[out] = np.array(img)
    d32 = float(np.abs(imgs["f32"] - ref["image"]).max())
    gb = F._bf16_to_f32(imgs["bf16"])
    dbf, p = float(np.abs(gb - ref["image"]).max()), F.psnr(gb, ref["image"])
    # the device's u8 is its own bf16 image packed by the reference's rule
    assert np.array_equal(imgs["u8"], O.pack_u8(gb))
    du8 = np.abs(imgs["u8"].astype(np.int16) - O.pack_u8(ref["image"]).astype(np.int16))
    print(f"render_view: f32 {d32:.3g}, bf16 {dbf:.3g} psnr {p:.1f}, u8 max {du8.max()} "
          f"exact {np.mean(du8 == 0):.6f}", flush=True)
    assert d32 <= 1e-5
    assert dbf <= 2e-3 and p >= 55.0
    assert du8.max() <= 1 and np.mean(du8 == 0) >= 0.995
    # render_view's positional call in the reference's argument order, default u8
    img, _ = rc.render_view(*args, 16, 1.0 / 255.0, 1.0 / 16384.0, 1.0 / 16384.0, False,
                            1.0 / 255.0, 0, 3.0, False)
    assert np.array(img).dtype == np.uint8 and np.array_equal(np.array(img), imgs["u8"])
    t = rc.stage_timings()
    for k in ("views", "head", "project", "tile_assign", "sort", "blend_setup", "mat", "cull",
              "blend", "d2h", "assemble", "tail", "xview", "xview_hits", "xview_misses",
              "view_total"):
        assert k in t, k


@pytest.mark.parametrize("ts", [16, 32])
def test_cull_disabled_frame(gpu_ctx, c1, ts):
    print(f"cull_disabled frame ts={ts}", flush=True)
    scene, cam, cov = c1
    ref = F.frame(scene.means, cov, scene.opacities, scene.colors, cam, ts, cull_disabled=True)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=ts, output="f32",
                       cull_disabled=True)
    img, st = gpu_ctx.render(view)
    assert ref["P"] == ref["pairs_pre"]  # no per-pair cull
    F.check_frame(gpu_ctx, view, ref, img, st, bf16=False, label=f"cull_disabled ts={ts}")


def test_isoellipse_frame(gpu_ctx, c1):
    """use_isoellipse: the AABB from the eigen-decomposition of the 2D covariance
    (types.h:154-171). The reference takes atan2/cos/sin from glibc's float
    functions, the GPU from the device library; they can differ in the last bit,
    which changes a radius only where k*sqrt(.) lands within an ulp of an
    integer. Measured here: the Gaussians whose radii differ, and the frame."""
    print("isoellipse frame", flush=True)
    scene, cam, cov = c1
    ref = F.frame(scene.means, cov, scene.opacities, scene.colors, cam, 16,
                  use_isoellipse=True)
    g = gpu_ctx.project(scene.means, cov, scene.opacities, scene.colors,
                        L.make_view(cam.w2c, cam.K, cam.height, cam.width, use_isoellipse=True))
    o = ref["project"]
    assert np.array_equal(g["valid"], o["valid"])
    diff = int(np.sum(np.any(g["radii"] != o["radii"], axis=1)))
    print(f"isoellipse: {diff} of {o['radii'].shape[0]} radii differ", flush=True)
    assert diff <= max(1, o["radii"].shape[0] // 10_000)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, output="f32",
                       use_isoellipse=True)
    img, st = gpu_ctx.render(view)
    if diff == 0:
        F.check_frame(gpu_ctx, view, ref, img, st, bf16=False, label="isoellipse")
    else:
        assert float(np.abs(img - ref["image"]).max()) <= 2e-3


@pytest.mark.parametrize("ts", [16, 32])
def test_cull_stats_match_reference(gpu_ctx, c1, ts):
    """pairs_dropped / pairs_kept_per_mb of render_full's stats
    (cull_and_blend.cpp:384-504,835-836), exact."""
    print(f"cull stats ts={ts}", flush=True)
    scene, cam, cov = c1
    _, st_o, _ = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c, cam.K,
                               cam.height, cam.width, tile_size=ts)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    gpu_ctx.set_cull_stats(True)
    try:
        _, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=ts))
    finally:
        gpu_ctx.set_cull_stats(False)
    print(f"ts={ts}: dropped {st['pairs_dropped_mb']} kept {st['pairs_kept_mb']} "
          f"(oracle {st_o['pairs_dropped']} {st_o['pairs_kept_per_mb']})", flush=True)
    assert st["pairs_dropped_mb"] == st_o["pairs_dropped"]
    assert st["pairs_kept_mb"] == st_o["pairs_kept_per_mb"]
    _, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=ts))
    assert st["pairs_dropped_mb"] == -1 and st["pairs_kept_mb"] == -1


def test_lookback_give_up_is_an_error(gpu_ctx):
    """With a spin limit of one round, waits on predecessors that have not
    published yet give up at once; the frame, the training forward and the sort
    then return GS_E_DEVICE instead of results (the kernels that would read the
    wrong prefixes return early), and with the default limit the same calls are
    exact again."""
    print("look-back give-up: frame / sort", flush=True)
    scene, cams = scenes.config2(seed=81, n=1_000_000)
    cam = cams[0]
    cov = scenes.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, output="f32")
    good, st_good = gpu_ctx.render(view)
    n = 8_000_000
    keys, vals = scenes.config4_keys(n=n)
    dk, dv, dr = gpu_ctx.dev_alloc(n * 8), gpu_ctx.dev_alloc(n * 4), gpu_ctx.dev_alloc(5000 * 8)
    try:
        gpu_ctx.set_spin_limit(1)
        with pytest.raises(L.GsError, match="look-back"):
            gpu_ctx.render(view)
        gpu_ctx.h2d(dk, keys)
        gpu_ctx.h2d(dv, vals)
        with pytest.raises(L.GsError, match="look-back"):
            gpu_ctx.sort_tile_depth_dev(dk, dv, n, 5000, dr)
        tscene, _, tcams = scenes.config5(seed=82, n=400_000)
        tc = tcams[0]
        tview = L.make_view(tc.w2c, tc.K, tc.height, tc.width, tile_size=16)
        tr = L.Trainer(gpu_ctx, scenes.train_params(tscene), 1)
        target = np.zeros((tc.height, tc.width, 3), np.float32)
        with pytest.raises(L.GsError, match="look-back"):
            tr.step(tview, L.make_train_cfg(), target)
        gpu_ctx.set_spin_limit(0)
        assert tr.step(tview, L.make_train_cfg(), target)["loss"] > 0.0
        again, st = gpu_ctx.render(view)
        assert st["num_entries"] == st_good["num_entries"]
        assert np.array_equal(again.view(np.uint32), good.view(np.uint32))
        gpu_ctx.h2d(dk, keys)
        gpu_ctx.h2d(dv, vals)
        gpu_ctx.sort_tile_depth_dev(dk, dv, n, 5000, dr)
        vo = np.empty(n, np.uint32)
        gpu_ctx.d2h(vo, dv)
        assert np.array_equal(vo, np.argsort(keys, kind="stable").astype(np.uint32))
    finally:
        gpu_ctx.set_spin_limit(0)
        for p in (dk, dv, dr):
            gpu_ctx.dev_free(p)
