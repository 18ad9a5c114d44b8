"""Benchmark: forward render of the 6M-Gaussian scene (SH degree 3, 1237x822,
16x16 tiles, 64-view orbit) on one MI355X, plus the 100K and 1M single-view
renders, the standalone 50M-key tile/depth radix sort with its per-tile ranges
and the 1M-Gaussian training step, with roofline figures and the CPU baselines.

Contract: `python bench.py --gpus N --steps K --warmup W` prints ONE JSON line.
A step is one frame: the whole five-stage pipeline of one orbit view, from the
HBM-resident scene to a bf16 image in HBM (inputs resident before timing).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP32_PEAK_TFLOPS = 157.3     # MI355X FP32 peak (packed FP32 VALU issue)
# per pixel x Gaussian evaluation: dx, dy (2 sub), quadratic form (3 mul + 2 FMA),
# clamp, exp, alpha (mul + min), alpha*T, 3 colour FMA, T update; FMA = 2 flops
BLEND_FLOPS_PER_EVAL = 20
# the training backward per (pixel, entry) pair it evaluates (k_train_bwd): the
# forward's recomputation for every pair up to the pixel's stop (dx, dy 2;
# quadratic form 3 mul + 2 FMA; clamp 1; exp 1; opacity product 1; alpha clamp
# 1) and, for the blended pairs, the gradient terms (1 - alpha, reciprocal, T
# update 3; dL/dalpha 3 sub + dot 5 + scale 1 + background FMA 2; alpha T 1;
# colour terms 3; opacity term 1; dp 1; mean terms 2 x (mul + FMA + mul) = 8;
# conic terms 9; colour-behind recursion 3 x (mul + FMA) = 9; the nine sums 9);
# FMA = 2 flops
TRAIN_BWD_FLOPS_CONSIDERED = 13
TRAIN_BWD_FLOPS_BLENDED = 55
# frame slots of gs_render_batch; one output buffer per slot
FRAMES_IN_FLIGHT = 4
# host threads of one GPU's share of the box (its worker pools are sized to it)
BOX_CPU_SHARE = 16


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--views", type=int, default=64)
    ap.add_argument("--n", type=int, default=6_000_000)
    ap.add_argument("--sort-keys", type=int, default=50_000_000)
    ap.add_argument("--no-sort", action="store_true")
    ap.add_argument("--sort-only", action="store_true",
                    help="only the 50M-key tile/depth sort leg (for profiling)")
    ap.add_argument("--train-only", action="store_true",
                    help="only the training leg (for profiling)")
    ap.add_argument("--no-train", action="store_true")
    ap.add_argument("--train-steps", type=int, default=20)
    ap.add_argument("--train-n", type=int, default=1_000_000)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-morton", action="store_true",
                    help="skip the Morton-ordered orbit with the chunk frustum skip")
    ap.add_argument("--cpu-frames", type=int, default=10)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU baseline threads (0: the process's logical cores, at most the "
                         "box's share of one GPU)")
    ap.add_argument("--no-views", action="store_true",
                    help="skip the 100K and 1M single-view legs")
    ap.add_argument("--view-steps", type=int, default=64)
    ap.add_argument("--workload", choices=("c1", "c2", "c3"), default="c3",
                    help="the workload of --sequential-frames")
    ap.add_argument("--sequential-frames", type=int, default=0, metavar="K",
                    help="only render K orbit views one at a time (device output, no frames "
                         "in flight): the per-kernel split of a frame under a kernel trace")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run device-to-device copies of BYTES (PMC byte-counter scale)")
    return ap.parse_args()


def bench_frames(args):
    """The orbit: `warmup` untimed frames, then `steps` frames timed as one camera
    path through gs_render_batch (four frames in flight on four streams), with the
    per-stage hipEvents off; then 16 frames one at a time with the events on,
    for the per-stage times and the blend diagnostics."""
    from gsplat_tt_amd import _lib as L
    from gsplat_tt_amd import scenes

    t = time.time()
    scene, cams = scenes.config3(n=args.n, views=args.views)
    cov = scenes.cov3d(scene.scales, scene.quats)
    log(f"scene generated in {time.time() - t:.1f}s (N={scene.n})")
    ctx = L.Context(0, timing=False)
    cus, _ = ctx.device_info()
    t = time.time()
    ctx.set_scene(scene.means, cov, scene.opacities, scene.sh, sh_degree=3)
    log(f"scene resident in HBM in {time.time() - t:.1f}s ({cus} CUs)")
    H, W = cams[0].height, cams[0].width
    outs = [ctx.dev_alloc(H * W * 3 * 2) for _ in range(FRAMES_IN_FLIGHT)]
    views = [L.make_view(c.w2c, c.K, H, W, tile_size=16, output="bf16") for c in cams]

    def path(first, count):
        return [views[(first + i) % len(views)] for i in range(count)]

    if args.warmup > 0:
        ctx.render_batch(path(0, args.warmup), [outs[i % FRAMES_IN_FLIGHT] for i in range(args.warmup)])
    log(f"warmup {args.warmup} frames done")
    seq = path(args.warmup, args.steps)
    t0 = time.perf_counter()
    ctx.render_batch(seq, [outs[i % FRAMES_IN_FLIGHT] for i in range(args.steps)])
    ctx._L.gs_sync(ctx.handle)
    dt = time.perf_counter() - t0
    log(f"timed {args.steps} frames in {dt:.3f}s")
    _check = L._check
    _check(ctx._L.gs_set_timing(ctx.handle, 2))  # stage events + blend counters
    stats = [ctx.render_dev(views[i % len(views)], outs[0]) for i in range(16)]
    for o in outs:
        ctx.dev_free(o)
    return ctx, scene, cov, cams, stats, dt


def stage_summary(n, sh_degree, tiles, stats):
    """Per-stage times (hipEvents on the render stream, frames rendered one at a
    time) and roofline figures from the per-unit algorithmic work:
    projection N*(12+24+4+12*(d+1)^2) B read + M*48 B written (d+1)^2 = 1 for RGB);
    depth sort 16 B per key per pass, 4 passes over the M depth keys; tile
    assignment M*40 B read + P*12 B written; tile sort 16 B per pair per pass over
    P (passes: the tile bits spread over 8-bit-or-less digits); blend 20 FP32 flops
    per pixel-Gaussian evaluation."""
    keys = ("ms_project", "ms_depth_sort", "ms_tile_assign", "ms_tile_sort", "ms_blend",
            "ms_total")
    avg = {k: float(np.mean([s[k] for s in stats])) for k in keys}
    M = float(np.mean([s["num_visible"] for s in stats]))
    P = float(np.mean([s["num_entries"] for s in stats]))
    Ppre = float(np.mean([s["pairs_pre"] for s in stats]))
    evals = float(np.mean([s["blend_evals"] for s in stats]))
    diag = {k: float(np.mean([s[k] for s in stats])) for k in ("blend_batches", "blend_iters",
                                                                 "blend_kept", "blend_max_iters")}
    K = 1 if sh_degree < 0 else (sh_degree + 1) ** 2
    tile_bits = max(1, math.ceil(math.log2(tiles)))
    tile_passes = (tile_bits + 7) // 8
    work = {
        "project": ("GB/s", n * (12 + 24 + 4 + 12 * K) + M * 48),
        "depth_sort": ("GB/s", M * 16 * 4),
        "tile_assign": ("GB/s", M * 40 + P * 12),
        "tile_sort": ("GB/s", P * 16 * tile_passes),
        "blend": ("TFLOP/s", evals * BLEND_FLOPS_PER_EVAL),
    }
    roof = {}
    for k, (unit, amount) in work.items():
        sec = avg["ms_" + k] * 1e-3
        if sec <= 0:
            continue
        if unit == "GB/s":
            ach = amount / sec / 1e9
            roof[k] = {"ms": round(avg["ms_" + k], 4), "bytes": round(amount),
                       "achieved_gbs": round(ach, 1), "frac_hbm": round(ach / HBM_PEAK_GBS, 4)}
        else:
            ach = amount / sec / 1e12
            roof[k] = {"ms": round(avg["ms_" + k], 4), "flops": round(amount),
                       "achieved_tflops": round(ach, 3),
                       "frac_fp32": round(ach / FP32_PEAK_TFLOPS, 4)}
    return {
        "N": n, "M_avg": M, "pairs_avg": P, "pairs_pre_avg": Ppre, "blend_evals_avg": evals,
        "blend_diag": diag, "ms": {k[3:]: round(v, 4) for k, v in avg.items()},
        "roofline": roof,
    }


def dominant_roofline(st, tag, deg, out):
    """The roofline object of the frame's dominant kernel: k_project (the project
    stage is that one kernel plus a small histogram reduction, HBM-bound) or
    k_blend (FP32 VALU-bound; no MFMA on this path), whichever takes longer.
    `traffic` is the kernel's PMC-measured HBM bytes per dispatch for this
    workload (profiles/frame_<tag>_pmc_traffic.md), for the kernel instance the
    workload runs (k_project<sh degree>, k_blend<tile, output format>)."""
    proj_k = f"k_project<{deg}>"
    blend_k = f"k_blend<16, {ORDER_OUT.index(out)}>"
    r = st["roofline"]
    proj_ms, blend_ms = r["project"]["ms"], r["blend"]["ms"]
    if blend_ms >= proj_ms:
        b = r["blend"]
        return {"kernel": "k_blend", "bound": "valu", "pipe": "fp32 VALU (no MFMA issued)",
                "achieved": b["achieved_tflops"], "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": b["frac_fp32"], "traffic": pmc_traffic(blend_k, tag),
                "flops_per_launch": b["flops"], "ms_per_launch": b["ms"],
                "work_model": "20 FP32 flops per pixel-Gaussian evaluation"}
    p = r["project"]
    return {"kernel": "k_project", "bound": "hbm", "achieved": p["achieved_gbs"],
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": p["frac_hbm"],
            "traffic": pmc_traffic(proj_k, tag), "bytes_per_launch": p["bytes"],
            "ms_per_launch": p["ms"],
            "work_model": "N*(12+24+4+12*(d+1)^2) B read + M*48 B written"}


ORDER_OUT = ("u8", "bf16", "f32")  # k_blend's output-format template argument


def pmc_traffic(kernel, tag):
    """HBM bytes per dispatch of `kernel` in workload `tag` from the committed
    rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE scaled by a copy-kernel
    calibration), or None when no summary holds it."""
    import re
    path = os.path.join(ROOT, "profiles", f"frame_{tag}_pmc_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_dispatch\[" + re.escape(kernel) + r"\]\s*=\s*([0-9]+)",
                  open(path).read())
    return int(m.group(1)) if m else None


def sort_traffic():
    """HBM bytes of one 50M-key tile/depth sort call from its PMC summary, or None."""
    import re
    path = os.path.join(ROOT, "profiles", "sort_50M_pmc_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_call\s*=\s*([0-9]+)", open(path).read())
    return int(m.group(1)) if m else None


def copy_calibration(nbytes):
    """Device-to-device copies of a known size: the reference reading for the PMC
    byte counters (FETCH_SIZE / WRITE_SIZE per dispatch vs nbytes)."""
    from gsplat_tt_amd import _lib as L
    ctx = L.Context(0)
    a, b = ctx.dev_alloc(nbytes), ctx.dev_alloc(nbytes)
    for _ in range(5):
        ctx.d2d(b, a, nbytes)
    ctx._L.gs_sync(ctx.handle)
    ctx.dev_free(a)
    ctx.dev_free(b)
    ctx.close()
    print(json.dumps({"copy_calibration_bytes": nbytes, "dispatches": 5}), flush=True)


def bench_morton(scene, cov, cams, steps, warmup):
    """The same orbit on the scene in Morton order with the chunk frustum skip
    on (render/run.py:1011-1057 + render/host/chunk_cull.h): a secondary figure,
    not the headline value (the headline scene is in its generated order)."""
    from gsplat_tt_amd import _lib as L
    from gsplat_tt_amd import prep

    t = time.time()
    a, _ = prep.morton_reorder({"means": scene.means, "cov": cov,
                                "opacities": scene.opacities, "sh": scene.sh})
    reorder_s = time.time() - t
    ctx = L.Context(0, timing=False)
    try:
        ctx.set_chunk_cull(True)
        ctx.set_scene(a["means"], a["cov"], a["opacities"], a["sh"], sh_degree=3)
        H, W = cams[0].height, cams[0].width
        outs = [ctx.dev_alloc(H * W * 3 * 2) for _ in range(FRAMES_IN_FLIGHT)]
        views = [L.make_view(c.w2c, c.K, H, W, tile_size=16, output="bf16") for c in cams]
        seq = [views[i % len(views)] for i in range(warmup + steps)]
        ctx.render_batch(seq[:warmup], [outs[i % FRAMES_IN_FLIGHT] for i in range(warmup)])
        t0 = time.perf_counter()
        sts = ctx.render_batch(seq[warmup:], [outs[i % FRAMES_IN_FLIGHT] for i in range(steps)])
        ctx._L.gs_sync(ctx.handle)
        dt = time.perf_counter() - t0
        for o in outs:
            ctx.dev_free(o)
    finally:
        ctx.close()
    nparts = -(-scene.n // L.PROJECT_PARTITION)
    return {"frames_per_s": round(steps / dt, 1), "partitions": nparts,
            "partitions_skipped_avg": round(float(np.mean([s["chunks_skipped"] for s in sts])), 1),
            "num_visible_avg": round(float(np.mean([s["num_visible"] for s in sts])), 1),
            "reorder_s": round(reorder_s, 2)}


def sequential_frames(args):
    """Frames of one workload rendered one at a time (gs_render, device output),
    nothing else: what a kernel trace splits into per-kernel frame times.
    --workload c3: the 6M-Gaussian orbit views; c1: the 100K-Gaussian view
    (f32 out); c2: the 1M-Gaussian SH3 view (bf16 out)."""
    from gsplat_tt_amd import _lib as L
    from gsplat_tt_amd import scenes

    if args.workload == "c1":
        scene, cams = scenes.config1()
        sh, deg, fmt = scene.colors, -1, "f32"
    elif args.workload == "c2":
        scene, cams = scenes.config2()
        sh, deg, fmt = scene.sh, 3, "bf16"
    else:
        scene, cams = scenes.config3(n=args.n, views=args.views)
        sh, deg, fmt = scene.sh, 3, "bf16"
    cov = scenes.cov3d(scene.scales, scene.quats)
    ctx = L.Context(0, timing=True)
    ctx.set_scene(scene.means, cov, scene.opacities, sh, sh_degree=deg)
    H, W = cams[0].height, cams[0].width
    out = ctx.dev_alloc(H * W * 12)
    sts = [ctx.render_dev(L.make_view(c.w2c, c.K, H, W, tile_size=16, output=fmt), out)
           for c in (cams[i % len(cams)] for i in range(args.sequential_frames))]
    ctx.dev_free(out)
    ctx.close()
    keys = ("ms_project", "ms_depth_sort", "ms_tile_assign", "ms_tile_sort", "ms_blend")
    print(json.dumps({"workload": args.workload, "sequential_frames": len(sts),
                      "ms": {k[3:]: round(float(np.mean([s[k] for s in sts[4:]])), 4) for k in keys}}),
          flush=True)


def bench_host_out(ctx, cams, frames):
    """The orbit with images delivered to host memory (PCIe-inclusive, the
    render_view path): u8 images into the pinned output ring with the next view
    announced (gs_render_out_ring), and, for comparison, copied into a fresh
    pageable numpy array per frame (gs_render_next). Not the headline value."""
    from gsplat_tt_amd import _lib as L

    L._check(ctx._L.gs_set_timing(ctx.handle, 0))
    H, W = cams[0].height, cams[0].width
    views = [L.make_view(c.w2c, c.K, H, W, tile_size=16, output="u8") for c in cams]
    res = {"format": "u8", "frames": frames}
    for name in ("ring", "pageable"):
        for rep in range(2):  # the first pass warms the ring's pinned buffers
            t0 = time.perf_counter()
            for i in range(frames):
                nxt = views[(i + 1) % len(views)] if i + 1 < frames else None
                if name == "ring":
                    img, _ = ctx.render_ring(views[i % len(views)], nxt)
                else:
                    img, _ = ctx.render_next(views[i % len(views)], nxt)
                del img
            dt = time.perf_counter() - t0
        res[f"{name}_frames_per_s"] = round(frames / dt, 1)
    L._check(ctx._L.gs_set_timing(ctx.handle, 1))  # the sort and training report stage times
    return res


def bench_render_view(scene, cov, cams, frames):
    """The drop-in call itself: render_clean.render_view over the orbit with the
    module's defaults (u8 zero-copy images from its pinned output ring) and the
    next view announced (next_extrinsics), the scene passed as host arrays on
    every call as render/run.py does (a scene-cache hit after the first call).
    PCIe-inclusive, through the module's own context; not the headline value.
    Also the module's host spans per view (stage_timings: head, frame, tail)."""
    import gsplat_tt_amd

    rc = gsplat_tt_amd.render_clean_module()
    H, W = cams[0].height, cams[0].width
    args = (scene.means, cov, scene.opacities, scene.sh)
    kw = dict(image_height=H, image_width=W, tile_size=16, min_opacity=1.0 / 255.0,
              contrib_floor=1.0 / 16384.0, mb_contrib_floor=1.0 / 16384.0,
              cull_disabled=False, transmittance_threshold=1.0 / 255.0, max_radius=0,
              k_cap=3.0, use_isoellipse=False)

    def run(first, count):
        for i in range(first, first + count):
            c, nx = cams[i % len(cams)], cams[(i + 1) % len(cams)]
            img, _ = rc.render_view(*args, c.w2c, c.K, **kw, next_extrinsics=nx.w2c)
            del img

    try:
        run(0, 8)  # scene upload, ring buffers, the first frames
        rc.reset_stage_timings()
        t0 = time.perf_counter()
        run(8, frames)
        dt = time.perf_counter() - t0
        t = rc.stage_timings()
    finally:
        rc.device_shutdown()
    n = max(int(t["views"]), 1)
    return {"format": "u8", "zero_copy": True, "next_extrinsics": True, "frames": frames,
            "frames_per_s": round(frames / dt, 1),
            "host_ms_per_view": {k: round(t[k] / n, 4) for k in ("head", "frame", "tail",
                                                                 "view_total")},
            "xview_hits": int(t["xview_hits"])}


def bench_view(ctx, name, tag, scene, cam, steps, warmup, cpu_frames, cpu_threads, out="bf16"):
    """One workload's single view, rendered `steps` times through gs_render_batch
    (four frames in flight), then 8 frames one at a time with per-stage events;
    the reference's CPU renderer on the same view for the CPU figure."""
    from gsplat_tt_amd import _lib as L
    from gsplat_tt_amd import scenes

    deg = scene.sh_degree if scene.sh is not None else -1
    colors = scene.sh if scene.sh is not None else scene.colors
    cov = scenes.cov3d(scene.scales, scene.quats)
    ctx.set_scene(scene.means, cov, scene.opacities, colors, sh_degree=deg)
    H, W = cam.height, cam.width
    view = L.make_view(cam.w2c, cam.K, H, W, tile_size=16, output=out)
    eb = {"bf16": 2, "f32": 4, "u8": 1}[out]
    outs = [ctx.dev_alloc(H * W * 3 * eb) for _ in range(FRAMES_IN_FLIGHT)]
    L._check(ctx._L.gs_set_timing(ctx.handle, 0))
    ctx.render_batch([view] * warmup, [outs[i % FRAMES_IN_FLIGHT] for i in range(warmup)])
    t0 = time.perf_counter()
    ctx.render_batch([view] * steps, [outs[i % FRAMES_IN_FLIGHT] for i in range(steps)])
    ctx._L.gs_sync(ctx.handle)
    dt = time.perf_counter() - t0
    L._check(ctx._L.gs_set_timing(ctx.handle, 2))  # stage events + blend counters
    stats = [ctx.render_dev(view, outs[0]) for _ in range(8)]
    for o in outs:
        ctx.dev_free(o)
    tiles = ((W + 15) // 16) * ((H + 15) // 16)
    st = stage_summary(scene.n, deg, tiles, stats)
    res = {"workload": f"{scene.n} Gaussians, {W}x{H}, "
                       f"{'SH degree %d' % deg if deg >= 0 else 'RGB'}, 16x16 tiles, {out} out, "
                       "one view", "frames": steps, "frames_per_s": round(steps / dt, 1),
           "ms_per_frame": round(dt / steps * 1e3, 4), "stages": st,
           "roofline": dominant_roofline(st, tag, deg, out)}
    if cpu_frames > 0:
        res["cpu_baseline"] = cpu_baseline(scene, cov, [cam], cpu_frames, cpu_threads,
                                           f"{cpu_frames} renders of the {name} view after 1 "
                                           "warm-up")
    log(f"{name}: {res['frames_per_s']} frames/s, stages {st['ms']}")
    return res


def sort_moved_bytes(n, tiles, num_gaussians):
    """HBM bytes that gs_sort_tile_depth_ids_dev moves by design over n keys with
    ids below num_gaussians: the first digit's histogram reads 8 B a key; a pass
    over keys and ids reads and writes 8 + 4 B a key, the one that joins them
    into 8-byte words (the first after which the key bits left and the id fit
    64 bits) writes 8; a pass over the words moves 16 B, the last (ids only
    written) 12 B."""
    tb = max(1, (tiles - 1).bit_length())
    vb = max(1, (num_gaussians - 1).bit_length()) if num_gaussians else 32
    end = 32 + tb
    npass = (end + 7) // 8
    dw = -(-end // npass)
    q = 1
    while end - q * dw + vb > 64:
        q += 1
    per = 8 + 24 * (q - 1) + 20 + 16 * (npass - q - 1) + 12
    return n * per


def bench_sort(ctx, n, tiles=5000, cpu_threads=0, cpu=True):
    """The 50M-key tile/depth sort with the outputs of the reference's
    sort_and_bin, sorted ids and per-tile ranges (gs_sort_tile_depth_ids_dev,
    ids = the keys' indices, below M = 50M): wall time from the host around the
    call (inputs restored outside it), the bytes model keys*(24*passes + 8) over
    that wall time, the bytes the passes move by design (after the first pass
    each key's unsorted bits and its id travel as one 8-byte word), the
    onesweep passes' own event times and the range extraction's; then the
    reference's CPU sort of the same keys (cpu_baseline)."""
    from gsplat_tt_amd import scenes

    t = time.time()
    keys, vals = scenes.config4_keys(n=n, tiles=tiles)
    log(f"sort keys generated in {time.time() - t:.1f}s")
    dk, dv, dr = ctx.dev_alloc(n * 8), ctx.dev_alloc(n * 4), ctx.dev_alloc(tiles * 8)
    L = ctx._L
    times, passes, pass_ms, ranges_ms = [], 0, [], []
    # wall times with the per-pass events off (events between passes add
    # gaps), then the same calls with them on for the per-pass split
    from gsplat_tt_amd import _lib as Lm
    for timed in (0, 1):
        Lm._check(L.gs_set_timing(ctx.handle, timed))
        for rep in range(5):
            ctx.h2d(dk, keys)   # restore the unsorted input, outside the timed region
            ctx.h2d(dv, vals)
            L.gs_sync(ctx.handle)
            t0 = time.perf_counter()
            passes = ctx.sort_tile_depth_ids_dev(dk, dv, n, tiles, dr, num_gaussians=n)
            dt = time.perf_counter() - t0
            if timed:
                if rep > 0:
                    pass_ms.append(ctx.last_sort_pass_ms())
                    ranges_ms.append(ctx.last_ranges_ms())
            else:
                times.append(dt)
    # the later legs (training) report stage times: leave the events on
    # the ids (input values 0..n-1) are the stable order of the keys: the keys
    # they pick are non-decreasing, equal keys keep increasing ids (so no id
    # repeats), every id is below n; the ranges are the per-tile counts' scan
    vo = np.empty(n, np.uint32)
    rg = np.empty((tiles, 2), np.uint32)
    ctx.d2h(vo, dv)
    ctx.d2h(rg, dr)
    ok = int(vo.max()) < n
    ko = keys[np.minimum(vo, n - 1)]
    eq = ko[1:] == ko[:-1]
    ok = ok and bool(np.all(ko[1:] >= ko[:-1])) and bool(np.all(vo[1:][eq] > vo[:-1][eq]))
    del ko, eq
    cnt = np.bincount((keys >> np.uint64(32)).astype(np.int64), minlength=tiles)[:tiles]
    end = np.cumsum(cnt)
    start = end - cnt
    ok = ok and bool(np.array_equal(rg[:, 0], np.where(cnt > 0, start, 0))) and bool(
        np.array_equal(rg[:, 1], np.where(cnt > 0, end, 0)))
    for p in (dk, dv, dr):
        ctx.dev_free(p)
    cpu_res = cpu_sort_baseline(keys, vo, cpu_threads) if cpu else None
    del vo
    best = min(times[1:])
    kernel_ms = float(np.mean([sum(p) for p in pass_ms]))
    per_pass_ms = np.mean(np.array([p for p in pass_ms if len(p) == passes]), axis=0)
    pass_bytes = sort_moved_bytes(n, tiles, n) - 8 * n
    bytes_total = n * (24 * passes + 8)
    moved = sort_moved_bytes(n, tiles, n)
    traffic = sort_traffic() if n == 50_000_000 else None
    ach = bytes_total / best / 1e9
    return {
        "keys": n, "tiles": tiles, "zipf_s": 1.1, "passes": passes, "ok": ok,
        "wall_ms": round(best * 1e3, 3), "passes_ms": round(kernel_ms, 3),
        "ranges_ms": round(float(np.mean(ranges_ms)), 4),
        "gkeys_per_s": round(n / best / 1e9, 3),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "bytes_model": f"keys*(24*passes+8) = {bytes_total}, over the wall time "
                                    "of the sort call (histogram, passes, ranges)",
                     "moved": {"bytes": moved,
                               "achieved": round(moved / best / 1e9, 1),
                               "frac": round(moved / best / 1e9 / HBM_PEAK_GBS, 4),
                               "note": "bytes the passes move by design: keys and ids "
                                       "for one pass, then words of the key bits left "
                                       "and the id (ids < 2^26), only ids written by "
                                       "the last"},
                     "passes": {"ms": [round(float(x), 4) for x in per_pass_ms],
                                "achieved": round(pass_bytes / (kernel_ms * 1e-3) / 1e9, 1),
                                "frac": round(pass_bytes / (kernel_ms * 1e-3) / 1e9
                                              / HBM_PEAK_GBS, 4),
                                "note": "the moved bytes of the passes over their summed "
                                        "event times"}},
        "cpu_baseline": cpu_res,
    }


def bench_train(ctx, n, steps):
    """Config 5: one training step = forward (3DGS rules) + L1 against a target +
    blend/projection backward + sparse Adam, fp32, 1M Gaussians, SH degree 1,
    1280x720. The target is the GPU forward of the perturbed copy. Rooflines:
    sparse Adam reads param, m, v, grad (16 B) and writes param, m, v (12 B) per
    scalar of the visible rows; the backward reads the 48-B forward record per
    pair and adds 9 gradient terms per (Gaussian, tile) by atomics."""
    from gsplat_tt_amd import _lib as L
    from gsplat_tt_amd import scenes

    L._check(ctx._L.gs_set_timing(ctx.handle, 1))  # per-phase events for the rooflines
    t = time.time()
    scene, tgt_scene, cams = scenes.config5(n=n)
    cam = cams[0]
    log(f"train scene generated in {time.time() - t:.1f}s")
    cfg = L.make_train_cfg()
    view = L.make_view(cam.w2c, cam.K, cam.height, cam.width, tile_size=16)
    tr = L.Trainer(ctx, scenes.train_params(tgt_scene), 1)
    target, _, _, _ = tr.forward(view, cfg)
    tr = L.Trainer(ctx, scenes.train_params(scene), 1)
    _, _, proj, _ = tr.forward(view, cfg, target, want_proj=True)
    visible = int(proj["visible"].sum())
    H, W = cam.height, cam.width
    dt = ctx.dev_alloc(H * W * 12)
    ctx.h2d(dt, np.ascontiguousarray(target, np.float32))
    for _ in range(2):
        tr.step(view, cfg, dt, target_on_device=True)
    stats = []
    t0 = time.perf_counter()
    for _ in range(steps):
        stats.append(tr.step(view, cfg, dt, target_on_device=True))
    el = time.perf_counter() - t0
    # the same steps with the full 3DGS loss 0.8 L1 + 0.2 (1 - SSIM)
    cfg_s = L.make_train_cfg(lambda_dssim=0.2)
    tr.step(view, cfg_s, dt, target_on_device=True)
    stats_s = []
    t1 = time.perf_counter()
    for _ in range(steps):
        stats_s.append(tr.step(view, cfg_s, dt, target_on_device=True))
    el_s = time.perf_counter() - t1
    # the L1 steps again with the moments stored as bf16 (the reference's
    # device step default): Adam moves 4 B less per moment
    tr.set_moments(True)
    tr.step(view, cfg, dt, target_on_device=True)
    stats_b = []
    t2 = time.perf_counter()
    for _ in range(steps):
        stats_b.append(tr.step(view, cfg, dt, target_on_device=True))
    el_b = time.perf_counter() - t2
    tr.set_moments(False)
    ctx.dev_free(dt)
    keys = ("ms_forward", "ms_backward", "ms_adam")
    avg = {k: float(np.mean([s[k] for s in stats])) for k in keys}
    avg_s = {k: float(np.mean([s[k] for s in stats_s])) for k in keys}
    avg_b = {k: float(np.mean([s[k] for s in stats_b])) for k in keys}
    planes = 11 + 3 * 4
    adam_bytes = visible * planes * 28
    adam_bytes_b = visible * planes * 20
    P = stats[-1]["num_entries"]
    bwd_bytes = P * 48 + stats[-1]["num_blendable"] * 9 * 4 * 2
    considered = float(np.mean([s["pixel_pairs"] for s in stats]))
    blended = float(np.mean([s["pixel_blended"] for s in stats]))
    bwd_flops = TRAIN_BWD_FLOPS_CONSIDERED * considered + TRAIN_BWD_FLOPS_BLENDED * blended
    bwd_tf = bwd_flops / (avg["ms_backward"] * 1e-3) / 1e12
    return {"workload": "training step, 1M Gaussians (64-component mixture), SH degree 1, "
                        "1280x720, L1 vs render of a perturbed copy, sparse Adam, fp32",
            "steps": steps, "ms_per_step": round(el / steps * 1e3, 4),
            "steps_per_s": round(steps / el, 2),
            "ms": {k[3:]: round(v, 4) for k, v in avg.items()},
            "M": stats[-1]["num_blendable"], "pairs": P, "visible_rows": visible,
            "loss_first": round(stats[0]["loss"], 6), "loss_last": round(stats[-1]["loss"], 6),
            "roofline": {
                "adam": {"bound": "hbm", "bytes": adam_bytes,
                         "achieved": round(adam_bytes / (avg["ms_adam"] * 1e-3) / 1e9, 1),
                         "frac": round(adam_bytes / (avg["ms_adam"] * 1e-3) / 1e9
                                       / HBM_PEAK_GBS, 4),
                         "model": "visible rows x 23 planes x (16 B read + 12 B write)"},
                "backward": {"bound": "valu", "pipe": "fp32 VALU (no MFMA issued)",
                             "achieved": round(bwd_tf, 3), "peak": FP32_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(bwd_tf / FP32_PEAK_TFLOPS, 4),
                             "flops": bwd_flops, "pixel_pairs": considered,
                             "pixel_blended": blended,
                             "model": f"{TRAIN_BWD_FLOPS_CONSIDERED} flops per (pixel, entry) "
                                      f"pair up to the pixel's stop + "
                                      f"{TRAIN_BWD_FLOPS_BLENDED} per blended pair",
                             "hbm": {"bytes": bwd_bytes,
                                     "achieved": round(bwd_bytes / (avg["ms_backward"] * 1e-3)
                                                       / 1e9, 1),
                                     "frac": round(bwd_bytes / (avg["ms_backward"] * 1e-3) / 1e9
                                                   / HBM_PEAK_GBS, 4),
                                     "model": "pairs x 48 B records + M x 9 gradient terms "
                                              "(read + write)"}}},
            "full_loss": {"loss": "0.8 L1 + 0.2 (1 - SSIM)",
                          "ms_per_step": round(el_s / steps * 1e3, 4),
                          "steps_per_s": round(steps / el_s, 2),
                          "ms": {k[3:]: round(v, 4) for k, v in avg_s.items()},
                          "ssim_last": round(stats_s[-1]["ssim"], 6),
                          "loss_last": round(stats_s[-1]["loss"], 6)},
            "bf16_moments": {"ms_per_step": round(el_b / steps * 1e3, 4),
                             "steps_per_s": round(steps / el_b, 2),
                             "ms": {k[3:]: round(v, 4) for k, v in avg_b.items()},
                             "adam_roofline": {
                                 "bound": "hbm", "bytes": adam_bytes_b,
                                 "achieved": round(adam_bytes_b / (avg_b["ms_adam"] * 1e-3)
                                                   / 1e9, 1),
                                 "frac": round(adam_bytes_b / (avg_b["ms_adam"] * 1e-3) / 1e9
                                               / HBM_PEAK_GBS, 4),
                                 "model": "visible rows x 23 planes x (12 B read + 8 B write)"},
                             "loss_last": round(stats_b[-1]["loss"], 6)}}


def cpu_info():
    """Logical cores this process may run on, the host's count, and the CPU model."""
    n_os = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = n_os
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": aff, "os_cpu_count": n_os, "model": model}


def sh_rgb_parallel(O, means, sh, deg, w2c, threads):
    """The oracle's SH colour in `threads` slices at once (the C call releases
    the GIL), so the CPU figure does not run its colour stage on one core."""
    from concurrent.futures import ThreadPoolExecutor
    n = means.shape[0]
    cuts = np.linspace(0, n, threads + 1).astype(np.int64)
    with ThreadPoolExecutor(threads) as ex:
        parts = list(ex.map(lambda k: O.sh_rgb(means[cuts[k]:cuts[k + 1]],
                                               sh[cuts[k]:cuts[k + 1]], deg, w2c),
                            range(threads)))
    return np.concatenate(parts, 0)


def cpu_baseline(scene, cov, cams, frames, threads, sample):
    """The reference's own CPU renderer (_gsplat_cpu.render_full, compiled from its
    sources into oracle/_ref) on a bounded sample of the same workload; SH colour
    (when the scene has SH) evaluated first on the same threads and included."""
    info = cpu_info()
    if threads <= 0:
        threads = max(1, min(info["nproc"], BOX_CPU_SHARE))
    os.environ["GSPLAT_TT_NUM_THREADS"] = str(threads)
    from oracle import oracle as O

    R = O.ref_module()
    kind = "reference" if R is not None else "port"
    times, stages = [], []
    for i in range(frames + 1):
        cam = cams[(i * 7) % len(cams)]
        t0 = time.perf_counter()
        if scene.sh is not None:
            rgb = sh_rgb_parallel(O, scene.means, scene.sh, scene.sh_degree, cam.w2c, threads)
        else:
            rgb = scene.colors
        t1 = time.perf_counter()
        if R is not None:
            _, st = R.render_full(scene.means, cov, scene.opacities, rgb, cam.w2c, cam.K,
                                  cam.height, cam.width, tile_size=16)
        else:
            _, st, _ = O.render_full(scene.means, cov, scene.opacities, rgb, cam.w2c, cam.K,
                                     cam.height, cam.width, tile_size=16)
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
            st = dict(st)
            st["sh_ms"] = (t1 - t0) * 1e3
            stages.append(st)
    med = float(np.median(times))
    # the reference's own per-stage wall times (render_full's stats dict,
    # pybind_module.cpp:1537-1566), medians over the sample
    split = {k: round(float(np.median([float(s.get(k, 0.0)) for s in stages])), 3)
             for k in ("sh_ms", "project_ms", "tile_assign_ms", "sort_ms", "cull_ms",
                       "blend_ms", "total_ms")}
    log(f"cpu baseline ({sample}): {med * 1e3:.0f} ms/frame on {threads} threads; {split}")
    return {"value": round(1.0 / med, 4), "unit": "frames/s",
            "cores": threads if kind == "reference" else 1, "kind": kind,
            "nproc": info["nproc"], "os_cpu_count": info["os_cpu_count"],
            "cpu_model": info["model"], "stages_ms": split,
            "sample": f"{sample}: median {med * 1e3:.1f} ms/frame (SH colour + render_full, "
                      f"16x16 tiles, {threads} threads; the box's share of one GPU is "
                      f"{BOX_CPU_SHARE} threads)"}


def cpu_sort_baseline(keys, vals_gpu, threads, reps=3):
    """The reference's own stable bin-and-radix sort (_gsplat_cpu.sort, i.e.
    sort_and_bin of src/gsplat_cpu/sort.cpp:89-263, compiled from its sources into
    oracle/_ref) on the same 50M keys: gaussian id = key index, tile id = the
    key's high word, depth = the fp32 of its low word; its sorted ids are the
    stable order of the keys. `reps` timed calls after one warm-up, median, on
    `threads` threads; the result is checked against the GPU's sorted values."""
    info = cpu_info()
    if threads <= 0:
        threads = max(1, min(info["nproc"], BOX_CPU_SHARE))
    os.environ["GSPLAT_TT_NUM_THREADS"] = str(threads)
    from oracle import oracle as O

    R = O.ref_module()
    if R is None:
        return None
    n = keys.shape[0]
    tiles = int(keys.max() >> np.uint64(32)) + 1
    gids = np.arange(n, dtype=np.int64)
    tids = (keys >> np.uint64(32)).astype(np.int64)
    depths = (keys & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    times = []
    sid = None
    for i in range(reps + 1):
        t0 = time.perf_counter()
        sid, _ = R.sort(gids, tids, depths, tiles, 1)
        if i > 0:
            times.append(time.perf_counter() - t0)
    same = bool(np.array_equal(np.asarray(sid), vals_gpu.astype(np.int64)))
    med = float(np.median(times))
    log(f"cpu sort baseline: {med * 1e3:.0f} ms for {n} keys on {threads} threads "
        f"(equal to the GPU order: {same})")
    return {"value": round(n / med / 1e9, 4), "unit": "Gkeys/s", "cores": threads,
            "kind": "reference", "nproc": info["nproc"], "os_cpu_count": info["os_cpu_count"],
            "cpu_model": info["model"], "equal_to_gpu": same,
            "sample": f"the {n}-key sort, {reps} calls after 1 warm-up: median "
                      f"{med * 1e3:.1f} ms (_gsplat_cpu.sort, {threads} threads)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); multi-GPU "
              "sharding is not part of this build", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.sequential_frames:
        sequential_frames(args)
        return
    if args.train_only:
        from gsplat_tt_amd import _lib as L
        ctx = L.Context(0, timing=False)
        print(json.dumps({"train": bench_train(ctx, args.train_n, args.train_steps)}), flush=True)
        ctx.close()
        return
    if args.sort_only:
        from gsplat_tt_amd import _lib as L
        ctx = L.Context(0, timing=False)
        print(json.dumps({"sort": bench_sort(ctx, args.sort_keys, cpu=False)}), flush=True)
        ctx.close()
        return
    ctx, scene, cov, cams, stats, dt = bench_frames(args)
    tiles = ((cams[0].width + 15) // 16) * ((cams[0].height + 15) // 16)
    st = stage_summary(scene.n, 3, tiles, stats)
    fps = args.steps / dt
    log(f"{fps:.1f} frames/s; stages {st['ms']}")
    res = {
        "metric": "frames/sec @6M Gaussians 1237x822; sort Gkeys/s; blend frac of FP32 peak",
        "value": round(fps, 3), "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "forward render, 6M Gaussians (slab+shell), SH degree 3, "
                               "1237x822, 16x16 tiles, 64-view orbit r=4m h=1m fx=fy=1100, "
                               "bf16 out",
                   "parallelism": "single GPU", "n_gaussians": scene.n, "views": len(cams),
                   "frames_in_flight": FRAMES_IN_FLIGHT,
                   "stage_times": "16 frames one at a time with per-stage hipEvents"},
        "stages": st,
        "roofline": dominant_roofline(st, "6M", 3, "bf16"),
        "blend": {"ms": st["roofline"]["blend"]["ms"],
                  "achieved_tflops": st["roofline"]["blend"]["achieved_tflops"],
                  "frac_fp32": st["roofline"]["blend"]["frac_fp32"]},
    }
    res["host_out"] = bench_host_out(ctx, cams, min(args.steps, 64))
    log(f"host_out: {res['host_out']}")
    res["render_view"] = bench_render_view(scene, cov, cams, min(args.steps, 64))
    log(f"render_view: {res['render_view']}")
    if not args.no_morton:
        res["morton_chunk_cull"] = bench_morton(scene, cov, cams, args.steps, args.warmup)
        log(f"morton_chunk_cull: {res['morton_chunk_cull']}")
    cpu_c3 = None
    if not args.no_cpu:
        cpu_c3 = cpu_baseline(scene, cov, cams, args.cpu_frames, args.cpu_threads,
                              f"{args.cpu_frames} orbit views of the 6M-Gaussian scene after 1 "
                              "warm-up")
    del scene, cov
    if not args.no_views:
        from gsplat_tt_amd import scenes
        s1, c1 = scenes.config1()
        res["c1_100k"] = bench_view(ctx, "100K", "100K", s1, c1[0], args.view_steps, 8,
                                    0 if args.no_cpu else 5, args.cpu_threads, out="f32")
        s2, c2 = scenes.config2()
        res["c2_1m"] = bench_view(ctx, "1M SH3", "1M", s2, c2[0], args.view_steps, 8,
                                  0 if args.no_cpu else 3, args.cpu_threads, out="bf16")
        del s1, s2
    if not args.no_sort:
        res["sort"] = bench_sort(ctx, args.sort_keys, cpu_threads=args.cpu_threads,
                                 cpu=not args.no_cpu)
        log(f"sort: {res['sort']}")
    if not args.no_train:
        res["train"] = bench_train(ctx, args.train_n, args.train_steps)
        log(f"train: {res['train']}")
    res["cpu_baseline"] = cpu_c3
    ctx.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
