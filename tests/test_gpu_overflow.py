"""The overflow floor ladder on the GPU: a frame whose candidate pairs exceed
the pair limit (gs_set_pair_limit) is rendered again at a coarser contribution
floor (render/host/overflow_retry.h:26-61, render/host/render.cpp:537-565), and
that frame is the reference's render at the floor it reports: M, candidate
pairs, P, tile-sorted ids and ranges bit-exact, the f32 image within 1e-5, on
the 100K-Gaussian view. After the limit is lifted the view renders at its own
floor again (the opacity terms of the coarser floor do not outlive the frame),
also in a gs_render_batch of frames in flight; with the cull disabled no floor
can help and the call fails with GS_E_CAPACITY."""
import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes
from oracle import oracle as O
from tests import oracle_frames as F

pytestmark = pytest.mark.gpu


def _oracle_frame(scene, cov, cam, floor):
    img, st, it = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c, cam.K,
                                cam.height, cam.width, tile_size=16, contrib_floor=floor,
                                mb_contrib_floor=floor)
    T = ((cam.width + 15) // 16) * ((cam.height + 15) // 16)
    return dict(M=st["num_visible"], pairs_pre=int(it["pairs_pre"]), P=st["num_entries"],
                sorted_ids=np.asarray(it["sorted_ids"], np.int64),
                tile_ranges=np.asarray(it["tile_ranges"], np.int64).reshape(T, 2), image=img)


def test_pair_limit_renders_the_view_at_a_coarser_floor(gpu_ctx):
    print("overflow ladder: 100K view", flush=True)
    scene, cams = scenes.config1()
    cam = cams[0]
    cov = O.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, output="f32")
    img0, st0 = gpu_ctx.render(view)
    assert st0["floor_retries"] == 0 and st0["contrib_floor"] == view.contrib_floor
    limit = int(st0["pairs_pre"] * 0.6)
    try:
        gpu_ctx.set_pair_limit(limit)
        img, st = gpu_ctx.render(view)
        f = st["contrib_floor"]
        print(f"limit {limit}: floor 1/{1 / f:.0f} after {st['floor_retries']} retries, "
              f"pairs {st['pairs_pre']} (at 1/16384: {st0['pairs_pre']})", flush=True)
        assert st["floor_retries"] >= 1 and view.contrib_floor < f <= 0.5
        assert st["pairs_pre"] <= limit
        F.check_frame(gpu_ctx, view, _oracle_frame(scene, cov, cam, f), img, st, bf16=False,
                      label="C1 at the ladder's floor")
    finally:
        gpu_ctx.set_pair_limit(0)
    img2, st2 = gpu_ctx.render(view)
    assert st2["floor_retries"] == 0 and st2["pairs_pre"] == st0["pairs_pre"]
    assert np.array_equal(img2, img0)


def test_pair_limit_in_a_batch_of_frames_in_flight(gpu_ctx):
    print("overflow ladder: batch of 6 views", flush=True)
    scene, cams = scenes.config1()
    cov = O.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    cam = cams[0]
    H, W = cam.height, cam.width
    # six poses: the view shifted sideways a little each time
    views = []
    for k in range(6):
        w2c = np.array(cam.w2c, np.float32).copy()
        w2c[0, 3] += 0.05 * k
        views.append(L.make_view(w2c, cam.K, H, W, tile_size=16, output="f32"))
    direct = [gpu_ctx.render(v) for v in views]
    limit = int(min(s["pairs_pre"] for _, s in direct) * 0.7)
    outs = [np.empty((H, W, 3), np.float32) for _ in views]
    try:
        gpu_ctx.set_pair_limit(limit)
        sts = gpu_ctx.render_batch(views, outs, out_on_device=False)
        singles = [gpu_ctx.render(v) for v in views]
    finally:
        gpu_ctx.set_pair_limit(0)
    for k, (st, (simg, sst)) in enumerate(zip(sts, singles)):
        assert st["floor_retries"] >= 1 and st["pairs_pre"] <= limit, k
        assert st["contrib_floor"] == sst["contrib_floor"] and st["pairs_pre"] == sst["pairs_pre"]
        assert np.array_equal(outs[k], simg), k
    # lifted: every view at its own floor again, equal to its first render
    sts2 = gpu_ctx.render_batch(views, outs, out_on_device=False)
    for k, st in enumerate(sts2):
        assert st["floor_retries"] == 0 and np.array_equal(outs[k], direct[k][0]), k


def test_pair_limit_with_the_cull_disabled_fails(gpu_ctx):
    scene, cams = scenes.config1()
    cam = cams[0]
    cov = O.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, output="f32",
                       cull_disabled=True)
    _, st0 = gpu_ctx.render(view)
    try:
        gpu_ctx.set_pair_limit(int(st0["pairs_pre"] // 2))
        with pytest.raises(L.GsError, match="pair limit"):
            gpu_ctx.render(view)
    finally:
        gpu_ctx.set_pair_limit(0)
    _, st1 = gpu_ctx.render(view)
    assert st1["pairs_pre"] == st0["pairs_pre"]


def test_failing_frame_in_a_batch_finishes_the_others(gpu_ctx):
    """A frame of a gs_render_batch that fails (the cull disabled, more
    candidates than the pair limit) fails the call only after every other
    frame still in flight has finished writing its output: the outputs do not
    change after the error returns, and the next batch renders every view."""
    print("overflow: failing frame in a batch of 6", flush=True)
    scene, cams = scenes.config1()
    cov = O.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    cam = cams[0]
    H, W = cam.height, cam.width
    views = []
    for k in range(6):
        w2c = np.array(cam.w2c, np.float32).copy()
        w2c[0, 3] += 0.05 * k
        views.append(L.make_view(w2c, cam.K, H, W, tile_size=16, output="f32",
                                 cull_disabled=(k == 2)))
    direct = [gpu_ctx.render(v) for v in views]
    outs = [np.zeros((H, W, 3), np.float32) for _ in views]
    try:
        gpu_ctx.set_pair_limit(int(direct[2][1]["pairs_pre"] // 2))
        with pytest.raises(L.GsError, match="pair limit"):
            gpu_ctx.render_batch(views, outs, out_on_device=False)
        snap = [o.copy() for o in outs]
    finally:
        gpu_ctx.set_pair_limit(0)
    gpu_ctx.render(views[0])
    for k in range(6):
        assert np.array_equal(outs[k], snap[k]), k
    sts = gpu_ctx.render_batch(views, outs, out_on_device=False)
    for k, st in enumerate(sts):
        assert st["floor_retries"] == 0 and np.array_equal(outs[k], direct[k][0]), k
