"""GPU parity of every stage and the whole frame against the CPU oracle
(oracle/gs_oracle.c, itself pinned to the reference's own CPU module and
golden vectors). Integer/index outputs must be bit-exact; fp32 stage outputs
are bit-exact too (the kernels keep the reference's operation order with
-ffp-contract=off); images: max-abs <= 2e-3 with bf16 output and PSNR >= 55 dB
(the tolerance stated for this path)."""
import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def psnr(a, b):
    mse = float(np.mean((a.astype(np.float64) - b.astype(np.float64)) ** 2))
    return float("inf") if mse == 0 else 10 * np.log10(1.0 / mse)


def _scene(n, seed, H=480, W=640):
    scene, cams = scenes.config1(seed=seed, n=n)
    cam = cams[0]
    if (H, W) != (480, 640):
        K = scenes.intrinsics(500 * W / 640, 500 * W / 640, W / 2, H / 2)
        cam = scenes.Camera(cam.w2c, K, H, W)
    return scene, cam, O.cov3d(scene.scales, scene.quats)


@pytest.mark.parametrize("ts", [16, 32])
def test_project_bitexact(gpu_ctx, ts):
    scene, cam, cov = _scene(30_000, 21)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=ts)
    g = gpu_ctx.project(scene.means, cov, scene.opacities, scene.colors, view)
    o = O.project(scene.means, cov, cam.w2c, cam.K, scene.colors, scene.opacities,
                  cam.height, cam.width)
    print("project M", len(o["depths"]))
    assert np.array_equal(g["valid"], o["valid"])
    for k in ("means2d", "covs2d", "depths", "radii", "colors", "opacities"):
        assert np.array_equal(_bits(g[k]), _bits(o[k])), k


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
@pytest.mark.parametrize("clamp", [True, False])
def test_project_sh_colour_bitexact(gpu_ctx, deg, clamp):
    """Colour from SH of every degree inside the fused projection, bit-exact
    against the oracle's SH evaluation (train_oracle.py:99-122) of the visible
    Gaussians; the per-Gaussian records have odd lengths (3, 12, 27, 48 floats)."""
    scene, cam, cov = _scene(20_000, 40 + deg)
    rng = np.random.default_rng(deg)
    K = (deg + 1) ** 2
    sh = rng.standard_normal((scene.n, K, 3)).astype(np.float32) * np.float32(0.4)
    sh[:, 0, :] = rng.uniform(-0.5, 2.5, (scene.n, 3)).astype(np.float32)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, sh_clamp=clamp)
    g = gpu_ctx.project(scene.means, cov, scene.opacities, sh, view, sh_degree=deg)
    o = O.project(scene.means, cov, cam.w2c, cam.K, scene.colors, scene.opacities,
                  cam.height, cam.width)
    assert np.array_equal(g["valid"], o["valid"])
    ref = O.sh_rgb(scene.means, sh, deg, cam.w2c, clamp_hi=clamp)[o["valid"]]
    assert ref.shape[0] > 1000
    if not clamp:
        assert (ref > 1.0).any()
    assert np.array_equal(_bits(g["colors"]), _bits(ref))


@pytest.mark.parametrize("ts", [16, 32])
def test_tile_assign_bitexact(gpu_ctx, ts):
    scene, cam, cov = _scene(30_000, 22)
    o = O.project(scene.means, cov, cam.w2c, cam.K, scene.colors, scene.opacities,
                  cam.height, cam.width)
    gg, gt, gpre = gpu_ctx.tile_assign(o["means2d"], o["radii"], cam.height, cam.width, ts,
                                       o["covs2d"], o["opacities"])
    og, ot, opre = O.tile_assign(o["means2d"], o["radii"], cam.height, cam.width, ts,
                                 o["covs2d"], o["opacities"])
    print("pairs", len(og), "pre", opre)
    assert gpre == opre
    assert np.array_equal(gg, og) and np.array_equal(gt, ot)
    # no-cull variant
    gg, gt, _ = gpu_ctx.tile_assign(o["means2d"], o["radii"], cam.height, cam.width, ts)
    og, ot, _ = O.tile_assign(o["means2d"], o["radii"], cam.height, cam.width, ts)
    assert np.array_equal(gg, og) and np.array_equal(gt, ot)


def test_sort_and_bin_bitexact(gpu_ctx):
    scene, cam, cov = _scene(30_000, 23)
    o = O.project(scene.means, cov, cam.w2c, cam.K, scene.colors, scene.opacities,
                  cam.height, cam.width)
    og, ot, _ = O.tile_assign(o["means2d"], o["radii"], cam.height, cam.width, 16,
                              o["covs2d"], o["opacities"])
    tx, ty = 40, 30
    gs_, gr = gpu_ctx.sort_and_bin(og, ot, o["depths"], tx, ty)
    os_, orr = O.sort_and_bin(og, ot, o["depths"], tx, ty)
    assert np.array_equal(gs_, os_)
    assert np.array_equal(gr, orr)


@pytest.mark.parametrize("ts", [16, 32])
def test_cull_and_blend(gpu_ctx, ts):
    scene, cam, cov = _scene(30_000, 24)
    img_o, st, inter = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c,
                                     cam.K, cam.height, cam.width, tile_size=ts)
    pr = inter["project"]
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=ts, output="f32")
    img_g = gpu_ctx.cull_and_blend(pr["means2d"], pr["covs2d"], pr["colors"], pr["opacities"],
                                   inter["sorted_ids"], inter["tile_ranges"], view)
    d = np.abs(img_g - img_o)
    print("blend max abs f32", d.max(), "exact frac", np.mean(_bits(img_g) == _bits(img_o)))
    assert d.max() <= 1e-5


@pytest.mark.parametrize("ts,H,W", [(16, 480, 640), (32, 480, 640), (16, 237, 301),
                                    (32, 237, 301)])
def test_render_frame(gpu_ctx, ts, H, W):
    scene, cam, cov = _scene(40_000, 25, H, W)
    img_o, st_o, _ = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c,
                                   cam.K, H, W, tile_size=ts)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    img32, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, H, W, tile_size=ts, output="f32"))
    assert st["num_visible"] == st_o["num_visible"]
    assert st["num_entries"] == st_o["num_entries"]
    d32 = np.abs(img32 - img_o).max()
    imgbf, _ = gpu_ctx.render(L.make_view(cam.w2c, cam.K, H, W, tile_size=ts, output="bf16"))
    imgb = _bf16_to_f32(imgbf)
    dbf = np.abs(imgb - img_o).max()
    p = psnr(imgb, img_o)
    print(f"frame ts={ts} {H}x{W}: M={st['num_visible']} P={st['num_entries']} "
          f"f32 maxabs={d32:.3g} bf16 maxabs={dbf:.3g} psnr={p:.1f}")
    assert d32 <= 1e-5
    assert dbf <= 2e-3
    assert p >= 55.0


def test_render_frame_three_tile_digits(gpu_ctx):
    """A 4160x4200 frame has 260x263 = 68380 16-px tiles: 17 tile-id bits, so
    the tile sort runs three passes (digits of 6, 6 and 5 bits) and the pair
    emission produces three tile-digit histograms."""
    H, W = 4160, 4200
    scene, cam, cov = _scene(4_000, 31, H, W)
    img_o, st_o, _ = O.render_full(scene.means, cov, scene.opacities, scene.colors, cam.w2c,
                                   cam.K, H, W, tile_size=16)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    img, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, H, W, tile_size=16, output="f32"))
    print(f"three tile digits: M={st['num_visible']} P={st['num_entries']}", flush=True)
    assert st["num_visible"] == st_o["num_visible"]
    assert st["num_entries"] == st_o["num_entries"]
    assert np.abs(img - img_o).max() <= 1e-5


def test_render_pair_capacity_retry():
    """A fresh context starts with room for max(2^20, 8N) candidate pairs; 4200
    large Gaussians make 1.3M pairs, so the first frame overflows, is detected
    after the fact and re-run with a larger capacity. Both that frame and the
    next (no overflow) must equal the oracle's."""
    rng = np.random.default_rng(31)
    n = 4200
    means = np.stack([rng.uniform(-1.5, 1.5, n), rng.uniform(-1.1, 1.1, n),
                      rng.uniform(3.0, 6.0, n)], 1).astype(np.float32)
    scales = np.exp(rng.normal(np.log(0.4), 0.25, (n, 3))).astype(np.float32)
    q = rng.standard_normal((n, 4))
    quats = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    opac = rng.uniform(0.05, 0.35, n).astype(np.float32)
    rgb = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    cov = O.cov3d(scales, quats)
    K = scenes.intrinsics(500, 500, 320, 240)
    w2c = np.eye(4, dtype=np.float32)
    img_o, st_o, _ = O.render_full(means, cov, opac, rgb, w2c, K, 480, 640, tile_size=16)
    ctx = L.Context(0)
    try:
        ctx.set_scene(means, cov, opac, rgb)
        view = L.make_view(w2c, K, 480, 640, tile_size=16, output="f32")
        for frame in range(2):
            img, st = ctx.render(view)
            print("capacity frame", frame, st["num_entries"], st["pairs_pre"])
            assert st["pairs_pre"] > (1 << 20)
            assert st["num_visible"] == st_o["num_visible"]
            assert st["num_entries"] == st_o["num_entries"]
            assert np.abs(img - img_o).max() <= 1e-5
    finally:
        ctx.close()


def test_render_edge_cases(gpu_ctx):
    scene, cam, cov = _scene(2_000, 26)
    # everything behind the camera -> M == 0 -> black image
    w2c = cam.w2c.copy()
    w2c[2, 3] = -100.0
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.colors)
    img, st = gpu_ctx.render(L.make_view(w2c, cam.K, 64, 80, output="f32"))
    assert st["num_visible"] == 0 and not img.any()
    # a single Gaussian
    gpu_ctx.set_scene(scene.means[:1], cov[:1], scene.opacities[:1], scene.colors[:1])
    img, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, cam.height, cam.width, output="f32"))
    ref, st_o, _ = O.render_full(scene.means[:1], cov[:1], scene.opacities[:1],
                                 scene.colors[:1], cam.w2c, cam.K, cam.height, cam.width,
                                 tile_size=16)
    assert st["num_entries"] == st_o["num_entries"]
    assert np.abs(img - ref).max() <= 1e-5
    with pytest.raises(ValueError):
        gpu_ctx.render(L.make_view(cam.w2c, cam.K, 64, 80, tile_size=24))
    # a tile grid wider than 65535 tiles is refused before anything is launched
    with pytest.raises(ValueError):
        gpu_ctx.render(L.make_view(cam.w2c, cam.K, 1, 65535 * 16 + 1, output="u8"))


def test_render_degenerate_inputs(gpu_ctx):
    """Scenes with NaN and infinite means, zero, negative and huge covariances,
    opacities at and around the floor (0, 1/255, 1, NaN) and points on the near
    plane: the projection matches the oracle bit for bit (validity and values),
    and the frame's counts and image match the oracle's."""
    scene, cam, cov = _scene(20_000, 27)
    means = scene.means.copy()
    cov = cov.copy()
    op = scene.opacities.copy()
    rng = np.random.default_rng(27)
    idx = rng.permutation(means.shape[0])
    groups = np.array_split(idx[:2000], 10)
    means[groups[0], rng.integers(0, 3, groups[0].size)] = np.nan
    means[groups[1], rng.integers(0, 3, groups[1].size)] = np.inf
    means[groups[2], 2] = -np.inf
    cov[groups[3]] = 0.0
    c = cov[groups[4]].reshape(-1, 9)
    c[:, [0, 4, 8]] *= -1.0
    cov[groups[4]] = c.reshape(cov[groups[4]].shape)
    cov[groups[5]] *= np.float32(1e4)
    op[groups[6][0::4]] = 0.0
    op[groups[6][1::4]] = np.float32(1.0 / 255.0)
    op[groups[6][2::4]] = 1.0
    op[groups[6][3::4]] = np.nan
    # camera-space z exactly 0.2 (the near plane) for a group: the camera is the
    # identity rotation plus translation in this scene's view
    R = cam.w2c[:3, :3].astype(np.float64)
    t = cam.w2c[:3, 3].astype(np.float64)
    cam_pts = (means[groups[7]].astype(np.float64) @ R.T) + t
    cam_pts[:, 2] = 0.2
    means[groups[7]] = ((cam_pts - t) @ R).astype(np.float32)
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, output="f32")
    g = gpu_ctx.project(means, cov, op, scene.colors, view)
    o = O.project(means, cov, cam.w2c, cam.K, scene.colors, op, cam.height, cam.width)
    assert np.array_equal(g["valid"], o["valid"])
    for k in ("means2d", "covs2d", "depths", "radii", "colors", "opacities"):
        assert np.array_equal(_bits(g[k]), _bits(o[k])), k
    img_o, st_o, _ = O.render_full(means, cov, op, scene.colors, cam.w2c, cam.K, cam.height,
                                   cam.width, tile_size=16)
    gpu_ctx.set_scene(means, cov, op, scene.colors)
    img, st = gpu_ctx.render(view)
    print("degenerate: M", st["num_visible"], "P", st["num_entries"], flush=True)
    assert st["num_visible"] == st_o["num_visible"]
    assert st["num_entries"] == st_o["num_entries"]
    assert np.array_equal(np.isnan(img), np.isnan(img_o))
    assert np.nanmax(np.abs(img - img_o)) <= 1e-5


def test_sort_u64(gpu_ctx):
    rng = np.random.default_rng(7)
    for n in (0, 1, 4095, 4096, 4097, 100_003):
        tiles = rng.integers(0, 37, n).astype(np.uint64)
        depth = rng.uniform(0.2, 100, n).astype(np.float32)
        depth[: n // 3] = 1.5  # many ties
        keys = (tiles << np.uint64(32)) | depth.view(np.uint32).astype(np.uint64)
        vals = np.arange(n, dtype=np.uint32)
        ko, vo, passes = gpu_ctx.sort_pairs_u64(keys, vals, 0, 38)
        order = np.argsort(keys, kind="stable")
        assert np.array_equal(ko, keys[order]) and np.array_equal(vo, vals[order]), n


def test_sort_u64_partitions_and_skipped_passes(gpu_ctx):
    """64-bit sorts spanning several counting workgroups (64 partitions each),
    with constant digits (their passes skipped: the first pass then counts from
    the keys), all keys equal (no pass), and full 64-bit keys (8 passes)."""
    rng = np.random.default_rng(11)
    n = 1_000_003
    z = np.minimum(rng.zipf(1.1, n), 5000).astype(np.uint64) - np.uint64(1)
    d = np.exp(rng.uniform(np.log(0.2), np.log(100.0), n)).astype(np.float32)
    keys = (z << np.uint64(32)) | d.view(np.uint32).astype(np.uint64)
    vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    cases = [(keys, 45, None),
             ((keys >> np.uint64(16)) << np.uint64(16), 45, 4),   # bytes 0, 1 constant
             (np.full(200_000, 0x1234_5678_9ABC_DEF0, np.uint64), 64, 0),
             (rng.integers(0, 2**63, 500_000, dtype=np.uint64) * np.uint64(2) + np.uint64(1), 64, 8)]
    for k, end_bit, want_passes in cases:
        v = vals[: k.shape[0]]
        ko, vo, passes = gpu_ctx.sort_pairs_u64(k, v, 0, end_bit)
        order = np.argsort(k, kind="stable")
        assert np.array_equal(ko, k[order]) and np.array_equal(vo, v[order]), (k.shape, end_bit)
        if want_passes is not None:
            assert passes == want_passes


def test_sort_u64_config4_20m(gpu_ctx):
    """The standalone sort's key distribution (Zipf 1.1 tiles over 5000, log-uniform
    depths) at 20M keys: exact against numpy's stable sort."""
    keys, vals = scenes.config4_keys(n=20_000_000)
    ko, vo, passes = gpu_ctx.sort_pairs_u64(keys, vals, 0, 45)
    order = np.argsort(keys, kind="stable")
    assert passes == 6
    assert np.array_equal(ko, keys[order]) and np.array_equal(vo, vals[order])


def test_sort_tile_depth_partition_counts(gpu_ctx):
    """gs_sort_tile_depth_dev (8192-key partitions, a histogram of the first
    digit, each pass counting the next one's) at key counts on both sides of
    partition boundaries and with one to many partitions: exact against
    numpy's stable sort, with the per-tile ranges."""
    rng = np.random.default_rng(19)
    tiles = 300
    for n in (1, 8191, 8193, 3 * 8192 + 5, 8 * 8192, 9 * 8192 + 1, 100_003, 1_000_003):
        t = np.minimum(rng.zipf(1.3, n), tiles).astype(np.uint64) - np.uint64(1)
        d = np.exp(rng.uniform(np.log(0.2), np.log(100.0), n)).astype(np.float32)
        d[: n // 4] = 2.0  # ties
        keys = (t << np.uint64(32)) | d.view(np.uint32).astype(np.uint64)
        vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        dk, dv = gpu_ctx.dev_alloc(n * 8), gpu_ctx.dev_alloc(n * 4)
        dr = gpu_ctx.dev_alloc(tiles * 8)
        try:
            gpu_ctx.h2d(dk, keys)
            gpu_ctx.h2d(dv, vals)
            gpu_ctx.sort_tile_depth_dev(dk, dv, n, tiles, dr)
            ko, vo = np.empty_like(keys), np.empty_like(vals)
            rg = np.empty((tiles, 2), np.uint32)
            gpu_ctx.d2h(ko, dk)
            gpu_ctx.d2h(vo, dv)
            gpu_ctx.d2h(rg, dr)
        finally:
            for q in (dk, dv, dr):
                gpu_ctx.dev_free(q)
        order = np.argsort(keys, kind="stable")
        assert np.array_equal(ko, keys[order]) and np.array_equal(vo, vals[order]), n
        tk = (ko >> np.uint64(32)).astype(np.int64)
        lo = np.searchsorted(tk, np.arange(tiles), "left")
        hi = np.searchsorted(tk, np.arange(tiles), "right")
        exp = np.stack([np.where(lo == hi, 0, lo), np.where(lo == hi, 0, hi)], 1)
        assert np.array_equal(rg.astype(np.int64), exp), n


def test_render_opacity_prune_is_exact(gpu_ctx):
    """Dropping the Gaussians below min_opacity at load leaves the frame bit for
    bit unchanged (the projection drops them and compacts in source order)."""
    from gsplat_tt_amd import prep
    scene, cam, cov = _scene(30_000, 71)
    op = scene.opacities.copy()
    op[::3] = 0.002  # a third of the scene below 1/255
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16, output="f32")
    gpu_ctx.set_scene(scene.means, cov, op, scene.colors)
    img_a, st_a = gpu_ctx.render(view)
    pr = prep.opacity_prune({"means": scene.means, "cov": cov, "opacities": op,
                             "colors": scene.colors})
    assert pr["means"].shape[0] == 20_000
    gpu_ctx.set_scene(pr["means"], pr["cov"], pr["opacities"], pr["colors"])
    img_b, st_b = gpu_ctx.render(view)
    assert st_a["num_visible"] == st_b["num_visible"]
    assert st_a["num_entries"] == st_b["num_entries"]
    assert np.array_equal(_bits(img_a), _bits(img_b))


def test_render_morton_reordered_scene(gpu_ctx):
    """A Morton-reordered scene renders as the oracle renders the same reordered
    scene (counts bit-exact, image within the f32 bar)."""
    from gsplat_tt_amd import prep
    scene, cam, cov = _scene(40_000, 72)
    arrays, order = prep.morton_reorder({"means": scene.means, "cov": cov,
                                         "opacities": scene.opacities,
                                         "colors": scene.colors})
    assert not np.array_equal(order, np.arange(order.size))
    img_o, st_o, _ = O.render_full(arrays["means"], arrays["cov"], arrays["opacities"],
                                   arrays["colors"], cam.w2c, cam.K, cam.height, cam.width,
                                   tile_size=16)
    gpu_ctx.set_scene(arrays["means"], arrays["cov"], arrays["opacities"], arrays["colors"])
    img, st = gpu_ctx.render(L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16,
                                         output="f32"))
    assert st["num_visible"] == st_o["num_visible"]
    assert st["num_entries"] == st_o["num_entries"]
    assert np.abs(img - img_o).max() <= 1e-5


def test_render_batch_matches_single_frames(gpu_ctx):
    """Frames in flight (gs_render_batch) give each view the image and
    counts of its own gs_render, for device and host outputs."""
    scene, cams = scenes.config3(seed=73, n=60_000, views=8)
    cov = O.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
    H, W = cams[0].height, cams[0].width
    views = [L.make_view(c.w2c, c.K, H, W, tile_size=16, output="bf16") for c in cams]
    single = [gpu_ctx.render(v) for v in views]
    outs = [np.empty((H, W, 3), np.uint16) for _ in views]
    stats = gpu_ctx.render_batch(views, outs, out_on_device=False)
    for (img, st), out, sb in zip(single, outs, stats):
        assert np.array_equal(img, out)
        assert (st["num_visible"], st["num_entries"]) == (sb["num_visible"], sb["num_entries"])
    ptrs = [gpu_ctx.dev_alloc(H * W * 6) for _ in range(3)]
    try:
        stats = gpu_ctx.render_batch(views[:3], ptrs)
        for (img, st), p, sb in zip(single[:3], ptrs, stats):
            got = np.empty((H, W, 3), np.uint16)
            gpu_ctx.d2h(got, p)
            assert np.array_equal(img, got) and st["num_entries"] == sb["num_entries"]
    finally:
        for p in ptrs:
            gpu_ctx.dev_free(p)


def test_render_batch_capacity_retry():
    """A batch on a fresh context whose first frames overflow the pair capacity
    in every slot: every frame is re-run and equals the oracle's."""
    rng = np.random.default_rng(31)
    n = 4200
    means = np.stack([rng.uniform(-1.5, 1.5, n), rng.uniform(-1.1, 1.1, n),
                      rng.uniform(3.0, 6.0, n)], 1).astype(np.float32)
    scales = np.exp(rng.normal(np.log(0.4), 0.25, (n, 3))).astype(np.float32)
    q = rng.standard_normal((n, 4))
    quats = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    opac = rng.uniform(0.05, 0.35, n).astype(np.float32)
    rgb = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    cov = O.cov3d(scales, quats)
    K = scenes.intrinsics(500, 500, 320, 240)
    w2cs = []
    for k in range(4):  # one view per frame slot of gs_render_batch
        w2c = np.eye(4, dtype=np.float32)
        w2c[0, 3] = 0.05 * k
        w2cs.append(w2c)
    ctx = L.Context(0)
    try:
        ctx.set_scene(means, cov, opac, rgb)
        views = [L.make_view(w, K, 480, 640, tile_size=16, output="f32") for w in w2cs]
        outs = [np.empty((480, 640, 3), np.float32) for _ in views]
        stats = ctx.render_batch(views, outs, out_on_device=False)
        for w2c, img, st in zip(w2cs, outs, stats):
            ref, st_o, _ = O.render_full(means, cov, opac, rgb, w2c, K, 480, 640, tile_size=16)
            assert st["pairs_pre"] > (1 << 20)
            assert st["num_entries"] == st_o["num_entries"]
            assert np.abs(img - ref).max() <= 1e-5
    finally:
        ctx.close()


def test_render_next_pipelines_exactly(gpu_ctx):
    """gs_render_next with the next view announced: every frame equals its own
    gs_render, also when the announced view is not the one asked for next, and
    when the scene changes in between."""
    scene, cams = scenes.config3(seed=74, n=50_000, views=6)
    cov = O.cov3d(scene.scales, scene.quats)
    gpu_ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
    H, W = cams[0].height, cams[0].width
    views = [L.make_view(c.w2c, c.K, H, W, tile_size=16, output="bf16") for c in cams]
    single = [gpu_ctx.render(v) for v in views]
    for i, v in enumerate(views):
        nxt = views[i + 1] if i + 1 < len(views) else None
        img, st = gpu_ctx.render_next(v, nxt)
        assert np.array_equal(img, single[i][0]), i
        assert st["num_entries"] == single[i][1]["num_entries"], i
    # announced 1, asked for 3: the announced frame is dropped
    gpu_ctx.render_next(views[0], views[1])
    img, st = gpu_ctx.render_next(views[3], views[4])
    assert np.array_equal(img, single[3][0])
    # the scene changes while view 4 is announced
    op2 = scene.opacities * np.float32(0.5)
    gpu_ctx.set_scene(scene.means, cov, op2, scene.sh, sh_degree=3)
    img, st = gpu_ctx.render_next(views[4], None)
    ref, _ = gpu_ctx.render(views[4])
    assert np.array_equal(img, ref) and not np.array_equal(img, single[4][0])


def test_render_clean_next_extrinsics():
    """render_view(..., next_extrinsics=...) renders exactly what render_view
    renders without it, view after view."""
    import gsplat_tt_amd
    rc = gsplat_tt_amd.render_clean_module()
    scene, cams = scenes.config3(seed=75, n=40_000, views=4)
    cov = O.cov3d(scene.scales, scene.quats)
    args = dict(image_height=cams[0].height, image_width=cams[0].width, tile_size=16,
                min_opacity=1.0 / 255.0, contrib_floor=1.0 / 16384.0,
                mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
                use_isoellipse=False)
    plain = [rc.render_view(scene.means, cov, scene.opacities, scene.sh, c.w2c, c.K,
                            **args)[0] for c in cams]
    for i, c in enumerate(cams):
        nxt = cams[i + 1].w2c if i + 1 < len(cams) else None
        img, st = rc.render_view(scene.means, cov, scene.opacities, scene.sh, c.w2c, c.K,
                                 next_extrinsics=nxt, **args)
        assert np.array_equal(img, plain[i]), i
