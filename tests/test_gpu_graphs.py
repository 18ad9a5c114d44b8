"""gs_render_batch frames replayed from captured HIP graphs (gs_set_graphs, on
by default) equal frames whose kernels are enqueued directly, bit for bit, with
the same counts: every frame of several passes over an orbit, one frame per
call and four frames in flight, with directly enqueued frames, readbacks and
synchronisations between the replays, and across changes of the frame shape
(each a new capture). A capacity re-run is always enqueued directly (the
re-run itself is covered by test_gpu_parity.py::test_render_pair_capacity_retry);
the frame after it captures again."""
import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes
from oracle import oracle as O

pytestmark = pytest.mark.gpu

COUNTS = ("num_visible", "pairs_pre", "num_entries")


@pytest.fixture(scope="module")
def orbit():
    scene, cams = scenes.config3(seed=91, n=300_000, views=8)
    return scene, cams, O.cov3d(scene.scales, scene.quats)


def _ctx(scene, cov):
    ctx = L.Context(0, timing=False)
    ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
    return ctx


def _views(cams, fmt="bf16", ts=16):
    H, W = cams[0].height, cams[0].width
    return [L.make_view(c.w2c, c.K, H, W, tile_size=ts, output=fmt) for c in cams]


def _direct(ctx, views):
    """The frames with every kernel enqueued directly (host images, stats)."""
    ctx.set_graphs(False)
    try:
        return [ctx.render(v) for v in views]
    finally:
        ctx.set_graphs(True)


def _batch1(ctx, view, ref_img, out):
    """One frame through gs_render_batch (slot 0), read back to the host."""
    st = ctx.render_batch([view], [out])[0]
    img = np.empty_like(ref_img)
    ctx.d2h(img, out)
    return img, st


def _check(got, ref, label):
    (img, st), (img_r, st_r) = got, ref
    assert np.array_equal(img, img_r), label
    for k in COUNTS:
        assert st[k] == st_r[k], (label, k)


def test_graph_frames_equal_direct(orbit):
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    out = None
    try:
        views = _views(cams)
        ref = _direct(ctx, views)
        out = ctx.dev_alloc(ref[0][0].nbytes)
        for rep in range(3):
            for i, v in enumerate(views):
                _check(_batch1(ctx, v, ref[i][0], out), ref[i], f"replay {rep} view {i}")
                if i == 3:
                    # directly enqueued work between replays: a single frame
                    # and a timed batch frame (neither replays a graph), a
                    # readback of the frame buffers, then replays again
                    _check(ctx.render(views[5]), ref[5], f"direct {rep}")
                    L._check(ctx._L.gs_set_timing(ctx.handle, 1))
                    _check(_batch1(ctx, views[6], ref[6][0], out), ref[6], f"timed {rep}")
                    L._check(ctx._L.gs_set_timing(ctx.handle, 0))
                    counts = ctx.frame_readback(ids=False, ranges=False)
                    print("readback", rep, counts, flush=True)
        caps, reps = ctx.graph_counts()
        print("graphs captured", caps, "replayed", reps, flush=True)
        assert reps >= 2 * len(views), (caps, reps)  # the graph path itself was tested
    finally:
        if out is not None:
            ctx.dev_free(out)
        ctx.close()


def test_graph_readback_equal_direct(orbit):
    """The product frame's tile-sorted ids and tile ranges after a replayed
    frame equal those after the directly enqueued frame."""
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    out = None
    try:
        views = _views(cams[:3])
        ref = _direct(ctx, views[2:])
        rb_direct = ctx.frame_readback()
        out = ctx.dev_alloc(ref[0][0].nbytes)
        for v in views + views:  # a capture, then replays
            img, st = _batch1(ctx, v, ref[0][0], out)
        _check((img, st), ref[0], "last replay")
        rb = ctx.frame_readback()
        for k in ("M", "pairs_pre", "P"):
            assert rb[k] == rb_direct[k], k
        assert np.array_equal(rb["sorted_ids"], rb_direct["sorted_ids"])
        assert np.array_equal(rb["tile_ranges"], rb_direct["tile_ranges"])
    finally:
        if out is not None:
            ctx.dev_free(out)
        ctx.close()


def test_graph_batch_equal_direct(orbit):
    """Four frames in flight, one output buffer per frame slot (the slots'
    graphs are replayed from the second call on)."""
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    outs = []
    try:
        views = _views(cams)
        ref = _direct(ctx, views)
        nbytes = ref[0][0].nbytes
        outs = [ctx.dev_alloc(nbytes) for _ in range(4)]
        for rep in range(3):
            for j in range(0, len(views), 4):
                sts = ctx.render_batch(views[j:j + 4], outs)
                for k in range(4):
                    img = np.empty_like(ref[j + k][0])
                    ctx.d2h(img, outs[k])
                    _check((img, sts[k]), ref[j + k], f"batch {rep} view {j + k}")
        caps, reps = ctx.graph_counts()
        print("graphs captured", caps, "replayed", reps, flush=True)
        assert reps >= 12, (caps, reps)  # four slots, six calls
    finally:
        for o in outs:
            ctx.dev_free(o)
        ctx.close()


def test_graph_shape_changes(orbit):
    """Frames alternating between shapes (tile size, output format, image
    size): each change is a new capture, and each frame equals its direct
    one."""
    scene, cams, cov = orbit
    ctx = _ctx(scene, cov)
    out = None
    try:
        small = [scenes.Camera(c.w2c, scenes.intrinsics(550, 550, 309.0, 205.0), 411, 618)
                 for c in cams[:2]]
        seq = [_views(cams[:2])[0], _views(cams[:2], ts=32)[1], _views(cams[:2], fmt="f32")[0],
               _views(small)[1], _views(cams[:2])[1], _views(cams[:2], ts=32)[0]]
        ref = _direct(ctx, seq)
        out = ctx.dev_alloc(max(r[0].nbytes for r in ref))
        for rep in range(2):
            for i, v in enumerate(seq):
                _check(_batch1(ctx, v, ref[i][0], out), ref[i], f"shape {rep} frame {i}")
        caps, reps = ctx.graph_counts()
        print("graphs captured", caps, "replayed", reps, flush=True)
        assert caps >= len(seq)  # every change of shape captured anew
    finally:
        if out is not None:
            ctx.dev_free(out)
        ctx.close()


def test_graph_odd_pass_count_goes_direct():
    """A 4160x4200 frame of 68380 tiles sorts its tiles in three passes, so a
    frame flips the sort's look-back half and never leaves its state as it
    found it: after two captures that cannot be replayed its frames are
    enqueued directly, and every frame equals the direct one."""
    H, W = 4160, 4200
    scene, cams = scenes.config1(seed=31, n=4_000)
    K = scenes.intrinsics(500 * W / 640, 500 * W / 640, W / 2, H / 2)
    view = L.make_view(cams[0].w2c, K, H, W, tile_size=16, output="bf16")
    ctx = L.Context(0, timing=False)
    out = None
    try:
        ctx.set_scene(scene.means, O.cov3d(scene.scales, scene.quats), scene.opacities,
                      scene.colors)
        ref = _direct(ctx, [view])[0]
        out = ctx.dev_alloc(ref[0].nbytes)
        for f in range(5):
            _check(_batch1(ctx, view, ref[0], out), ref, f"frame {f}")
        caps, reps = ctx.graph_counts()
        print("graphs captured", caps, "replayed", reps, flush=True)
        assert caps == 2 and reps == 0, (caps, reps)
    finally:
        if out is not None:
            ctx.dev_free(out)
        ctx.close()
