"""Zero-copy output ring on the GPU (gs_render_out_ring, render/host/out_ring.h,
render/host/render.cpp:598-612): ring images equal gs_render's images; a held
image is never rewritten, also past the cap (slots replaced); freed slots are
reused; the announced-next-view pipelining gives the same frames; render_clean's
render_view returns the ring image by default and a fresh array with
GSPLAT_TT_OUT_ZEROCOPY=0, the two equal."""
import gc
import os

import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _data_ptr(a):
    return a.__array_interface__["data"][0]


@pytest.fixture(scope="module")
def orbit():
    scene, cams = scenes.config3(seed=81, n=50_000, views=6)
    return scene, cams, O.cov3d(scene.scales, scene.quats)


def _ctx(scene, cov):
    ctx = L.Context(0, timing=False)
    ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
    return ctx


@pytest.mark.parametrize("fmt", ["u8", "bf16"])
def test_ring_images_equal_render(orbit, fmt):
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    try:
        for c in cams[:3]:
            v = L.make_view(c.w2c, c.K, c.height, c.width, tile_size=16, output=fmt)
            ref, st = ctx.render(v)
            img, st2 = ctx.render_ring(v)
            assert img.shape == ref.shape and img.dtype == ref.dtype
            assert np.array_equal(img, ref)
            assert (st["num_visible"], st["num_entries"]) == (st2["num_visible"], st2["num_entries"])
            del img
        gc.collect()
        assert ctx.out_ring_info()[1] == 0  # every lease released
    finally:
        ctx.close()


def test_ring_held_images_survive(orbit):
    """Keep-previous cycles two slots; hoarding past a cap of 2 replaces slots
    and every held image keeps its frame; released slots come back."""
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    try:
        views = [L.make_view(c.w2c, c.K, c.height, c.width, tile_size=16, output="u8")
                 for c in cams]
        refs = [ctx.render(v)[0] for v in views]
        held, _ = ctx.render_ring(views[0])
        for i in range(1, len(views)):
            nxt, _ = ctx.render_ring(views[i])
            assert _data_ptr(nxt) != _data_ptr(held)
            assert np.array_equal(held, refs[i - 1])
            held = nxt
        size, nheld, grows, replaced = ctx.out_ring_info()
        assert (size, nheld, grows, replaced) == (2, 1, 2, 0)
        del held, nxt
        gc.collect()
        ctx.out_ring_config(2)
        kept = [ctx.render_ring(v)[0] for v in views[:5]]
        assert all(np.array_equal(k, r) for k, r in zip(kept, refs[:5]))
        size, nheld, grows, replaced = ctx.out_ring_info()
        assert size == 2 and nheld == 2 and replaced == 3
        ptrs = {_data_ptr(k) for k in kept}
        assert len(ptrs) == 5
        del kept
        gc.collect()
        assert ctx.out_ring_info()[1] == 0
        a, _ = ctx.render_ring(views[0])
        b, _ = ctx.render_ring(views[1])
        pa = _data_ptr(a)
        del a
        gc.collect()
        c, _ = ctx.render_ring(views[2])
        assert _data_ptr(c) == pa  # the freed slot after the last one written
        assert np.array_equal(b, refs[1]) and np.array_equal(c, refs[2])
        assert ctx.out_ring_info()[3] == 3  # no replacement while slots are free
    finally:
        ctx.close()


def test_ring_image_outlives_context(orbit):
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    c = cams[0]
    v = L.make_view(c.w2c, c.K, c.height, c.width, tile_size=16, output="bf16")
    ref, _ = ctx.render(v)
    img, _ = ctx.render_ring(v)
    ctx.close()
    assert np.array_equal(img, ref)  # pinned buffer kept alive by the lease
    del img
    gc.collect()


def test_ring_next_view_pipelined(orbit):
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    try:
        views = [L.make_view(c.w2c, c.K, c.height, c.width, tile_size=16, output="u8")
                 for c in cams]
        refs = [ctx.render(v)[0] for v in views]
        for i, v in enumerate(views):
            nxt = views[i + 1] if i + 1 < len(views) else None
            img, _ = ctx.render_ring(v, nxt)
            assert np.array_equal(img, refs[i]), i
    finally:
        ctx.close()


def test_render_clean_zero_copy(orbit, monkeypatch):
    import gsplat_tt_amd
    rc = gsplat_tt_amd.render_clean_module()
    scene, cams, cov = orbit
    args = dict(image_height=cams[0].height, image_width=cams[0].width, tile_size=16,
                min_opacity=1.0 / 255.0, contrib_floor=1.0 / 16384.0,
                mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
                use_isoellipse=False)

    def rv(c, **kw):
        return rc.render_view(scene.means, cov, scene.opacities, scene.sh, c.w2c, c.K,
                              **args, **kw)[0]

    monkeypatch.setenv("GSPLAT_TT_OUT_ZEROCOPY", "0")
    plain = [rv(c) for c in cams[:3]]
    assert all(p.flags.owndata for p in plain)
    monkeypatch.delenv("GSPLAT_TT_OUT_ZEROCOPY")
    monkeypatch.setenv("GSPLAT_TT_OUT_ZEROCOPY_SLOTS", "2")
    a = rv(cams[0])
    b = rv(cams[1])
    assert not a.flags.owndata and a.base is not None
    assert np.array_equal(a, plain[0]) and np.array_equal(b, plain[1])
    assert _data_ptr(a) != _data_ptr(b)
    pa = _data_ptr(a)
    view_of_a = a[10:20]
    del a
    gc.collect()
    c = rv(cams[2], next_extrinsics=cams[0].w2c)  # a's buffer is still held by its view
    assert _data_ptr(c) != pa and np.array_equal(c, plain[2])
    assert np.array_equal(view_of_a, plain[0][10:20])
    d = rv(cams[0])  # the announced view, completed from the second slot
    assert np.array_equal(d, plain[0])
    assert np.array_equal(view_of_a, plain[0][10:20]) and np.array_equal(b, plain[1])


def test_ring_announced_view_missed_and_dropped(orbit):
    """An announced view's frame writes into a ring image leased for it: when
    the next call asks for another view, that frame is completed and its image
    returns to the ring (no lease left behind), and the call's own image is
    right; a context closed with an announced frame pending releases it too."""
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    try:
        views = [L.make_view(c.w2c, c.K, c.height, c.width, tile_size=16, output="u8")
                 for c in cams]
        refs = [ctx.render(v)[0] for v in views]
        ctx.out_ring_config(3)
        a, _ = ctx.render_ring(views[0], views[1])   # views[1] announced
        assert np.array_equal(a, refs[0])
        b, _ = ctx.render_ring(views[2], views[3])   # a miss: views[1]'s frame is dropped
        assert np.array_equal(b, refs[2])
        c, _ = ctx.render_ring(views[3])             # the announced one, taken
        assert np.array_equal(c, refs[3])
        d = ctx.render(views[4])[0]                  # another entry point between
        assert np.array_equal(d, refs[4])
        del a, b, c
        gc.collect()
        assert ctx.out_ring_info()[1] == 0  # every lease released, the internal ones too
        e, _ = ctx.render_ring(views[5], views[0])   # left announced at close
        assert np.array_equal(e, refs[5])
    finally:
        ctx.close()
    assert np.array_equal(e, refs[5])  # the caller's image outlives the context
    del e
    gc.collect()


def test_ring_announced_view_that_fails(orbit):
    """An announced frame that fails when taken (the cull disabled, more
    candidates than the pair limit) raises in the call that takes it, and the
    ring image leased for it goes back to the ring; the context renders the
    view once the limit is lifted."""
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    try:
        va = L.make_view(cams[0].w2c, cams[0].K, cams[0].height, cams[0].width, tile_size=16,
                         output="u8")
        vb = L.make_view(cams[1].w2c, cams[1].K, cams[1].height, cams[1].width, tile_size=16,
                         output="u8", cull_disabled=True)
        ref_b, st_b = ctx.render(vb)
        try:
            ctx.set_pair_limit(int(st_b["pairs_pre"] // 2))
            a, _ = ctx.render_ring(va, vb)  # vb announced; va re-rendered at a coarser floor
            with pytest.raises(L.GsError, match="pair limit"):
                ctx.render_ring(vb)
            assert ctx.out_ring_info()[1] == 1  # only `a` is held
        finally:
            ctx.set_pair_limit(0)
        del a
        gc.collect()
        assert ctx.out_ring_info()[1] == 0
        b, _ = ctx.render_ring(vb)
        assert np.array_equal(b, ref_b)
        del b
        gc.collect()
    finally:
        ctx.close()
