"""Chunk frustum skip (gs_set_chunk_cull; render/host/chunk_cull.h): on a
Morton-ordered scene, frames with the skip on equal the frames without it bit
for bit (images, visible count, pair counts) over orbit views, views from inside
and beside the cloud and a wide-angle lens, while partitions are actually
skipped; a scene in its generated (random) order skips nothing; views with
k_cap above 3 are never skipped; render_clean's GSPLAT_TT_CHUNK_CULL gives the
same images. A skipped partition holding a Gaussian that reaches the image
would change the visible count, so equal counts over these views are the
conservativeness check of the skip test."""
import math

import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import prep, scenes
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def morton_scene():
    scene, cams = scenes.config3(seed=91, n=400_000, views=8)
    cov = O.cov3d(scene.scales, scene.quats)
    arrays, _ = prep.morton_reorder({"means": scene.means, "cov": cov,
                                     "opacities": scene.opacities, "sh": scene.sh})
    return scene, cams, cov, arrays


def _views(cams):
    H, W = cams[0].height, cams[0].width
    rng = np.random.default_rng(5)
    views = [L.make_view(c.w2c, c.K, H, W, tile_size=16, output="f32") for c in cams]
    K = scenes.intrinsics(1100, 1100, 618.5, 411.0)
    wide = scenes.intrinsics(300, 300, 618.5, 411.0)
    for i in range(24):
        eye = rng.uniform(-7, 7, 3) * np.array([1.0, 0.3, 1.0]) - np.array([0, 0.5, 0])
        target = rng.uniform(-4, 4, 3) * np.array([1.0, 0.2, 1.0])
        if np.linalg.norm(target - eye) < 0.5:
            continue
        w2c = scenes.look_at_w2c(eye, target)
        views.append(L.make_view(w2c, wide if i % 4 == 0 else K, H, W, tile_size=16,
                                 output="f32"))
    return views


def _frames(ctx, views):
    out = []
    for v in views:
        img, st = ctx.render(v)
        out.append((img, st["num_visible"], st["pairs_pre"], st["num_entries"],
                    st["chunks_skipped"]))
    return out


def test_chunk_cull_is_exact_on_morton_scene(morton_scene):
    _, cams, _, a = morton_scene
    views = _views(cams)
    ctx = L.Context(0, timing=False)
    try:
        ctx.set_scene(a["means"], a["cov"], a["opacities"], a["sh"], sh_degree=3)
        ref = _frames(ctx, views)
        ctx.set_chunk_cull(True)
        got = _frames(ctx, views)
        skipped = [g[4] for g in got]
        print("partitions skipped per view:", skipped, flush=True)
        for i, (r, g) in enumerate(zip(ref, got)):
            assert r[4] == 0
            assert r[1:4] == g[1:4], i
            assert np.array_equal(r[0], g[0]), i
        assert sum(skipped) > 0
        ctx.set_chunk_cull(False)
        assert _frames(ctx, views[:2])[0][4] == 0
    finally:
        ctx.close()


def test_chunk_cull_random_order_and_kcap(morton_scene):
    scene, cams, cov, a = morton_scene
    ctx = L.Context(0, timing=False)
    try:
        ctx.set_chunk_cull(True, 1.5)
        ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
        c = cams[0]
        v = L.make_view(c.w2c, c.K, c.height, c.width, tile_size=16, output="f32")
        img, st = ctx.render(v)
        assert st["chunks_skipped"] == 0  # random order: every partition spans the scene
        ctx.set_scene(a["means"], a["cov"], a["opacities"], a["sh"], sh_degree=3)
        away = scenes.look_at_w2c(np.array([0.0, -1.0, 9.0]), np.array([0.0, -1.0, 20.0]))
        va = L.make_view(away, c.K, c.height, c.width, tile_size=16, output="f32")
        _, st_on = ctx.render(va)
        vk = L.make_view(away, c.K, c.height, c.width, tile_size=16, output="f32", k_cap=3.5)
        _, st_k = ctx.render(vk)
        ctx.set_chunk_cull(False)
        _, st_off = ctx.render(vk)
        nparts = -(-a["means"].shape[0] // L.PROJECT_PARTITION)
        assert st_on["chunks_skipped"] >= 0.9 * nparts  # the cloud is behind this camera
        assert st_on["num_visible"] == st_off["num_visible"]
        assert st_k["chunks_skipped"] == 0
        assert st_k["num_visible"] == st_off["num_visible"]
        with pytest.raises(ValueError):
            ctx.set_chunk_cull(True, float("nan"))
    finally:
        ctx.close()


def test_render_clean_chunk_cull_env(morton_scene, monkeypatch):
    import gsplat_tt_amd
    rc = gsplat_tt_amd.render_clean_module()
    _, cams, _, a = morton_scene
    args = dict(image_height=cams[0].height, image_width=cams[0].width, tile_size=16,
                min_opacity=1.0 / 255.0, contrib_floor=1.0 / 16384.0,
                mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
                use_isoellipse=False)
    monkeypatch.setenv("GSPLAT_TT_OUT_ZEROCOPY", "0")
    monkeypatch.setenv("GSPLAT_TT_CHUNK_CULL", "0")
    plain = [rc.render_view(a["means"], a["cov"], a["opacities"], a["sh"], c.w2c, c.K,
                            **args) for c in cams[:3]]
    monkeypatch.setenv("GSPLAT_TT_CHUNK_CULL", "1")
    for c, (img0, st0) in zip(cams[:3], plain):
        img, st = rc.render_view(a["means"], a["cov"], a["opacities"], a["sh"], c.w2c, c.K,
                                 **args)
        assert np.array_equal(img, img0) and st == st0
    monkeypatch.setenv("GSPLAT_TT_CHUNK_CULL", "0")
    rc.render_view(a["means"], a["cov"], a["opacities"], a["sh"], cams[0].w2c, cams[0].K, **args)
