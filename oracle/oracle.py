"""ctypes wrapper around the plain-C oracle (liboracle.so) and the reference's
own CPU module built from source into oracle/_ref/.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing measured
or shipped. The function names mirror the reference's stages
(src/gsplat_cpu/{project,tile_assign,sort,cull_and_blend}.cpp).
"""
from __future__ import annotations

import ctypes
import glob
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.orc_project.restype = ctypes.c_int64
        L.orc_tile_count.restype = ctypes.c_int64
        L.orc_tile_assign.restype = ctypes.c_int64
        L.orc_exp4.restype = ctypes.c_float
        L.orc_exp4.argtypes = [ctypes.c_float]
        _LIB = L
    return _LIB


def _p(a, t):
    if a is None:
        return ctypes.cast(None, t)
    return a.ctypes.data_as(t)


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def cov3d(scales, quats):
    """types.h:68-97 build_covariance_3d -> (N, 9) float32."""
    scales, quats = _f(scales), _f(quats)
    n = scales.shape[0]
    out = np.empty((n, 9), np.float32)
    lib().orc_cov3d(_p(scales, _f32p), _p(quats, _f32p), ctypes.c_int64(n), _p(out, _f32p))
    return out


def sh_rgb(means, sh, degree, w2c, clamp_hi=True):
    """gsplat/train_oracle.py:99-122,163-173 SH colour, fp32."""
    means = _f(means)
    sh = _f(sh).reshape(means.shape[0], -1)
    w2c = _f(w2c)
    out = np.empty((means.shape[0], 3), np.float32)
    lib().orc_sh_rgb(_p(means, _f32p), _p(sh, _f32p), ctypes.c_int64(means.shape[0]),
                     ctypes.c_int(degree), _p(w2c, _f32p), ctypes.c_int(int(clamp_hi)),
                     _p(out, _f32p))
    return out


def project(means, cov3d9, w2c, intr, colors, opac, H, W, min_opacity=1.0 / 255.0,
            max_radius=0, contrib_floor=1.0 / 16384.0, k_cap=3.0, use_isoellipse=False):
    """project.cpp:484-798 project_full_fused. Returns dict of compact arrays."""
    means, cov3d9, w2c, intr = _f(means), _f(cov3d9).reshape(-1, 9), _f(w2c), _f(intr)
    colors = None if colors is None else _f(colors)
    opac = None if opac is None else _f(opac)
    n = means.shape[0]
    valid = np.empty(n, np.uint8)
    m2 = np.empty((n, 2), np.float32)
    c2 = np.empty((n, 4), np.float32)
    dp = np.empty(n, np.float32)
    rd = np.empty((n, 2), np.float32)
    co = np.empty((n, 3), np.float32)
    op = np.empty(n, np.float32)
    M = lib().orc_project(
        _p(means, _f32p), _p(cov3d9, _f32p), _p(w2c, _f32p), _p(intr, _f32p),
        _p(colors, _f32p), _p(opac, _f32p), ctypes.c_float(min_opacity), ctypes.c_int64(n),
        ctypes.c_int(H), ctypes.c_int(W), ctypes.c_int(max_radius),
        ctypes.c_float(contrib_floor), ctypes.c_float(k_cap), ctypes.c_int(int(use_isoellipse)),
        _p(valid, _u8p), _p(m2, _f32p), _p(c2, _f32p), _p(dp, _f32p), _p(rd, _f32p),
        _p(co, _f32p), _p(op, _f32p))
    return dict(valid=valid.astype(bool), means2d=m2[:M].copy(), covs2d=c2[:M].copy(),
                depths=dp[:M].copy(), radii=rd[:M].copy(),
                colors=co[:M].copy() if colors is not None else None,
                opacities=op[:M].copy() if opac is not None else None)


def tile_count(means2d, radii, H, W, tile_size):
    """tile_assign.cpp:60-111: candidate pairs before the per-pair cull (the sum
    of the rectangle areas)."""
    means2d, radii = _f(means2d), _f(radii)
    return int(lib().orc_tile_count(_p(means2d, _f32p), _p(radii, _f32p),
                                    ctypes.c_int64(means2d.shape[0]), ctypes.c_int(H),
                                    ctypes.c_int(W), ctypes.c_int(tile_size)))


def pack_u8(img_f32):
    """The u8 image that the reference's render_view returns for an fp32 colour
    image: bf16 round-to-nearest-even, then uint8(clip(float(bf16), 0, 1) * 255)
    with truncation (render/kernels/dataflow/img_pack_u8.h:9-14; the product of
    a bf16 and 255 is exact in fp32, so float arithmetic gives the integer rule's
    result)."""
    u = np.ascontiguousarray(img_f32, np.float32).view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) & 0xFFFF
    f = (b << 16).astype(np.uint32).view(np.float32)
    return (np.clip(f, np.float32(0), np.float32(1)) * np.float32(255)).astype(np.uint8)


def tile_assign(means2d, radii, H, W, tile_size, covs2d=None, opac=None,
                contrib_floor=1.0 / 16384.0):
    """tile_assign.cpp:26-368 -> (gaussian_ids, tile_ids) int64."""
    means2d, radii = _f(means2d), _f(radii)
    covs2d = None if covs2d is None else _f(covs2d).reshape(-1, 4)
    opac = None if opac is None else _f(opac)
    M = means2d.shape[0]
    ppre = lib().orc_tile_count(_p(means2d, _f32p), _p(radii, _f32p), ctypes.c_int64(M),
                                ctypes.c_int(H), ctypes.c_int(W), ctypes.c_int(tile_size))
    g = np.empty(max(ppre, 1), np.int64)
    t = np.empty(max(ppre, 1), np.int64)
    P = lib().orc_tile_assign(_p(means2d, _f32p), _p(radii, _f32p), ctypes.c_int64(M),
                              ctypes.c_int(H), ctypes.c_int(W), ctypes.c_int(tile_size),
                              _p(covs2d, _f32p), _p(opac, _f32p), ctypes.c_float(contrib_floor),
                              _p(g, _i64p), _p(t, _i64p))
    return g[:P].copy(), t[:P].copy(), int(ppre)


def sort_and_bin(gids, tids, depths, tiles_x, tiles_y):
    """sort.cpp:89-263 -> (sorted_gaussian_ids int64 (P,), tile_ranges int64 (T,2))."""
    gids = np.ascontiguousarray(gids, np.int64)
    tids = np.ascontiguousarray(tids, np.int64)
    depths = _f(depths)
    P = gids.shape[0]
    s = np.empty(max(P, 1), np.int64)
    r = np.empty((tiles_x * tiles_y, 2), np.int64)
    lib().orc_sort_and_bin(_p(gids, _i64p), _p(tids, _i64p), _p(depths, _f32p),
                           ctypes.c_int64(P), ctypes.c_int(tiles_x), ctypes.c_int(tiles_y),
                           _p(s, _i64p), _p(r, _i64p))
    return s[:P].copy(), r


def cull_and_blend(means2d, covs2d, colors, opac, sorted_ids, tile_ranges, tiles_x, tiles_y,
                   tile_size, H, W, mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                   transmittance_threshold=1.0 / 255.0):
    """cull_and_blend.cpp:678-838 (AVX2 semantics) -> (image f32 (H,W,3), stats)."""
    means2d, covs2d, colors, opac = _f(means2d), _f(covs2d).reshape(-1, 4), _f(colors), _f(opac)
    sorted_ids = np.ascontiguousarray(sorted_ids, np.int64)
    tile_ranges = np.ascontiguousarray(tile_ranges, np.int64)
    img = np.empty((H, W, 3), np.float32)
    st = np.zeros(3, np.int64)
    lib().orc_cull_and_blend(
        _p(means2d, _f32p), _p(covs2d, _f32p), _p(colors, _f32p), _p(opac, _f32p),
        _p(sorted_ids, _i64p), _p(tile_ranges, _i64p), ctypes.c_int64(means2d.shape[0]),
        ctypes.c_int64(sorted_ids.shape[0]), ctypes.c_int(tiles_x), ctypes.c_int(tiles_y),
        ctypes.c_int(tile_size), ctypes.c_int(H), ctypes.c_int(W),
        ctypes.c_float(mb_contrib_floor), ctypes.c_int(int(cull_disabled)),
        ctypes.c_float(transmittance_threshold), _p(img, _f32p), _p(st, _i64p))
    return img, dict(pairs_in=int(st[0]), pairs_dropped=int(st[1]), pairs_kept_per_mb=int(st[2]))


def render_full(means, cov3d9, opacities, colors, extrinsics, intrinsics, image_height,
                image_width, tile_size=32, min_opacity=1.0 / 255.0, contrib_floor=1.0 / 16384.0,
                mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
                transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
                use_isoellipse=False):
    """backends/cpu_cpp/pybind_module.cpp:1149-1575 render_full_py, same arguments and
    defaults (:2071-2091). Returns (image f32 (H,W,3), stats, intermediates)."""
    H, W = image_height, image_width
    pr = project(means, cov3d9, extrinsics, intrinsics, colors, opacities, H, W,
                 min_opacity, max_radius, contrib_floor, k_cap, use_isoellipse)
    M = pr["depths"].shape[0]
    tx = (W + tile_size - 1) // tile_size
    ty = (H + tile_size - 1) // tile_size
    if M == 0:
        return (np.zeros((H, W, 3), np.float32),
                dict(num_visible=0, num_entries=0, pairs_in=0, pairs_dropped=0,
                     pairs_kept_per_mb=0), dict(project=pr))
    g, t, ppre = tile_assign(pr["means2d"], pr["radii"], H, W, tile_size,
                             None if cull_disabled else pr["covs2d"],
                             None if cull_disabled else pr["opacities"], contrib_floor)
    s, r = sort_and_bin(g, t, pr["depths"], tx, ty)
    img, st = cull_and_blend(pr["means2d"], pr["covs2d"], pr["colors"], pr["opacities"], s, r,
                             tx, ty, tile_size, H, W, mb_contrib_floor, cull_disabled,
                             transmittance_threshold)
    stats = dict(num_visible=M, num_entries=int(s.shape[0]), **st)
    return img, stats, dict(project=pr, gids=g, tids=t, pairs_pre=ppre, sorted_ids=s,
                            tile_ranges=r)


def stable_sort_u64(keys, vals):
    keys = np.ascontiguousarray(keys, np.uint64)
    vals = np.ascontiguousarray(vals, np.uint32)
    n = keys.shape[0]
    ko = np.empty(n, np.uint64)
    vo = np.empty(n, np.uint32)
    lib().orc_stable_sort_u64(_p(keys, _u64p), _p(vals, _u32p), ctypes.c_int64(n),
                              _p(ko, _u64p), _p(vo, _u32p))
    return ko, vo


def exp4(x: float) -> float:
    return float(lib().orc_exp4(ctypes.c_float(x)))


def ref_module():
    """The reference's own CPU module (_gsplat_cpu) built from its sources into
    oracle/_ref by oracle/Makefile, or None when it was not built."""
    d = os.path.join(HERE, "_ref")
    if not glob.glob(os.path.join(d, "_gsplat_cpu*.so")):
        return None
    if d not in sys.path:
        sys.path.insert(0, d)
    import _gsplat_cpu  # noqa: E402
    return _gsplat_cpu
