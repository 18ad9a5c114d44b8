"""Plugin backend: the GPU rasterizer behind the reference's `Backend` interface.

`HipBackend` implements the stage methods of gsplat/backend.py:40-158
(`project`, `tile_assign`, `sort`, `blend`, `close`) with the same argument
names, defaults, tensor shapes and dtypes as the CPU-PyTorch defaults it
replaces (gsplat/rasterization.py:30-195 project_gaussians, :198-356
get_tile_assignments, :359-435 sort_and_bin), plus the fused single-call path
`render_fused` / `has_render_fused` that gsplat/pipeline.py:149-182 prefers when
present, with the keyword arguments and stats keys of
backends/cpu_cpp/backend.py:319-380. Every stage runs on the GPU through the
C ABI (gsplat_tt_amd._lib); there is no CPU fallback: without the built library
or a GPU the constructor raises.

Registration mirrors backends/__init__.py:20-60: `register(REGISTRY)` adds the
class under "hip", so `get_backend("hip", **kwargs)` constructs it.
"""
from __future__ import annotations

import time

import numpy as np

from . import _lib as L
from .scenes import cov3d as _cov3d

NAME = "hip"


def _np(t, dtype=None):
    """torch tensor or array -> contiguous numpy (host)."""
    if hasattr(t, "detach"):
        t = t.detach().cpu().numpy()
    a = np.asarray(t)
    return np.ascontiguousarray(a, dtype) if dtype is not None else np.ascontiguousarray(a)


def _torch(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a))


def _tile_size_for(tile_ranges, image_height, image_width):
    """The tile size whose grid has as many tiles as `tile_ranges` rows."""
    n = int(tile_ranges.shape[0])
    for ts in (32, 16):
        if ((image_height + ts - 1) // ts) * ((image_width + ts - 1) // ts) == n:
            return ts
    raise ValueError(f"tile_ranges has {n} rows: no 16- or 32-pixel tile grid of "
                     f"{image_height}x{image_width} has that many tiles")


class HipBackend:
    """The reference's `Backend` (gsplat/backend.py:40) on one GPU.

    Constructor keywords are those of CpuCppBackend (backends/cpu_cpp/backend.py:
    24-40) plus `device` (GPU index), `tile_size` (16 or 32; the reference's
    fused path uses 32) and `cull_stats`: render_fused's microblock-cull counts
    (pairs_dropped, pairs_kept_per_mb) take one more pass over the frame's pairs
    (k_mb_stats), so they are collected only when asked for; without them those
    two keys are left out of the stats (the reference's pipeline then reads 0)."""

    name = NAME

    def __init__(self, microblock: bool = True, mb_contrib_floor: float = 1.0 / 16384.0,
                 fused: bool = True, render_fused: bool = True, verbose: bool = False,
                 cull_disabled: bool = False, transmittance_threshold: float = 1.0 / 255.0,
                 min_opacity: float = 1.0 / 255.0, max_radius: int = 0,
                 contrib_floor: float | None = None, k_cap: float = 3.0,
                 use_isoellipse: bool = False, device: int = 0, tile_size: int = 32,
                 cull_stats: bool = False):
        if tile_size not in (16, 32):
            raise ValueError("tile_size must be 16 or 32")
        self.verbose = verbose
        self.microblock = bool(microblock)
        self.mb_contrib_floor = float(mb_contrib_floor)
        self.fused = bool(fused)
        self._render_fused = bool(render_fused)
        self.cull_disabled = bool(cull_disabled)
        self.transmittance_threshold = float(transmittance_threshold)
        self.min_opacity = float(min_opacity)
        self.max_radius = int(max_radius)
        self.contrib_floor_override = contrib_floor
        self.k_cap = float(k_cap)
        self.use_isoellipse = bool(use_isoellipse)
        self.tile_size = int(tile_size)
        # per-stage device times (hipEvents) for render_fused's *_ms keys; raises
        # without the library or a GPU
        self.ctx = L.Context(device, timing=True)
        self.cull_stats = bool(cull_stats)
        if self.cull_stats:
            self.ctx.set_cull_stats(True)
        self._cov_key = None
        self._cov = None

    # ------------------------------------------------------------ helpers
    def _contrib_floor(self, override=None):
        if override is not None:
            return float(override)
        if self.contrib_floor_override is not None:
            return float(self.contrib_floor_override)
        return self.mb_contrib_floor

    def _view(self, extrinsics, intrinsics, image_height, image_width, tile_size=None,
              contrib_floor=None, k_cap=None, use_isoellipse=None, output="f32"):
        return L.make_view(
            _np(extrinsics, np.float32).reshape(4, 4), _np(intrinsics, np.float32).reshape(3, 3),
            int(image_height), int(image_width), tile_size=tile_size or self.tile_size,
            min_opacity=self.min_opacity, contrib_floor=self._contrib_floor(contrib_floor),
            mb_contrib_floor=self.mb_contrib_floor, cull_disabled=self.cull_disabled,
            transmittance_threshold=self.transmittance_threshold, max_radius=self.max_radius,
            k_cap=self.k_cap if k_cap is None else float(k_cap),
            use_isoellipse=self.use_isoellipse if use_isoellipse is None else bool(use_isoellipse),
            output=output)

    def _cached_cov3d(self, scales, rotations):
        """cov3d depends only on (scales, rotations): cached across views, keyed
        like backends/cpu_cpp/backend.py's cache (buffer address and shape)."""
        key = (scales.__array_interface__["data"][0], scales.shape,
               rotations.__array_interface__["data"][0], rotations.shape)
        if key != self._cov_key:
            self._cov = _cov3d(scales, rotations)
            self._cov_key = key
        return self._cov

    # ------------------------------------------------------------ stages
    def project(self, means, scales, rotations, extrinsics, intrinsics, image_height: int,
                image_width: int, opacities=None, sub_timings: dict | None = None):
        """gsplat/rasterization.py:30-195: (means_2d (M,2), covs_2d (M,2,2), depths (M),
        radii (M,2), valid_mask (N) bool) for the visible Gaussians."""
        t0 = time.perf_counter()
        m = _np(means, np.float32)
        cov = self._cached_cov3d(_np(scales, np.float32), _np(rotations, np.float32))
        op = None if opacities is None else _np(opacities, np.float32)
        colors = np.zeros((m.shape[0], 3), np.float32)  # not part of this stage's outputs
        view = self._view(extrinsics, intrinsics, image_height, image_width)
        r = self.ctx.project(m, cov, op, colors, view)
        M = r["means2d"].shape[0]
        if sub_timings is not None:
            sub_timings["project.gpu"] = (time.perf_counter() - t0) * 1e3
        return (_torch(r["means2d"]), _torch(r["covs2d"].reshape(M, 2, 2)),
                _torch(r["depths"]), _torch(r["radii"]), _torch(r["valid"]))

    def tile_assign(self, means_2d, radii, image_height: int, image_width: int,
                    tile_size: int = 32, covs_2d=None, opacities=None,
                    contrib_floor: float = 1.0 / 16384.0, sub_timings: dict | None = None):
        """gsplat/rasterization.py:198-356: (gaussian_ids, tile_ids, tiles_per_gaussian),
        int64; the per-pair cull runs when covs_2d and opacities are given."""
        t0 = time.perf_counter()
        m2 = _np(means_2d, np.float32)
        M = m2.shape[0]
        c2 = None if covs_2d is None else _np(covs_2d, np.float32).reshape(M, 4)
        op = None if opacities is None else _np(opacities, np.float32)
        g, t, _ = self.ctx.tile_assign(m2, _np(radii, np.float32), int(image_height),
                                       int(image_width), int(tile_size),
                                       c2 if op is not None else None,
                                       op if c2 is not None else None, float(contrib_floor))
        tpg = np.bincount(g, minlength=M).astype(np.int64)
        if sub_timings is not None:
            sub_timings["tile_assign.gpu"] = (time.perf_counter() - t0) * 1e3
        return _torch(g), _torch(t), _torch(tpg)

    def sort(self, gaussian_ids, tile_ids, depths, tiles_x: int, tiles_y: int,
             sub_timings: dict | None = None):
        """gsplat/rasterization.py:359-435: (sorted_gaussian_ids int64, tile_ranges
        (tiles_x*tiles_y, 2) int64, (0,0) for empty tiles); stable by
        (tile, depth bits), ties in input order."""
        t0 = time.perf_counter()
        s, r = self.ctx.sort_and_bin(_np(gaussian_ids, np.int64), _np(tile_ids, np.int64),
                                     _np(depths, np.float32), int(tiles_x), int(tiles_y))
        if sub_timings is not None:
            sub_timings["sort.gpu"] = (time.perf_counter() - t0) * 1e3
        return _torch(s), _torch(r)

    def blend(self, means_2d, covs_2d, colors, opacities, sorted_gaussian_ids, tile_ranges,
              image_height: int, image_width: int):
        """gsplat/backend.py:128-151: (image (H,W,3) float32 numpy, sub_timings_ms)
        with the per-microblock cull; synchronous (returns after the GPU is done)."""
        t0 = time.perf_counter()
        ranges = _np(tile_ranges, np.int64)
        ts = _tile_size_for(ranges, int(image_height), int(image_width))
        view = L.make_view(np.eye(4, dtype=np.float32), np.eye(3, dtype=np.float32),
                           int(image_height), int(image_width), tile_size=ts,
                           mb_contrib_floor=self.mb_contrib_floor,
                           cull_disabled=self.cull_disabled,
                           transmittance_threshold=self.transmittance_threshold,
                           output="f32")
        M = int(np.asarray(_np(means_2d)).shape[0])
        img = self.ctx.cull_and_blend(_np(means_2d, np.float32), _np(covs_2d, np.float32)
                                      .reshape(M, 4), _np(colors, np.float32),
                                      _np(opacities, np.float32), _np(sorted_gaussian_ids,
                                                                      np.int64), ranges, view)
        return img, {"kernel": (time.perf_counter() - t0) * 1e3}

    # ------------------------------------------------------------ fused path
    def has_render_fused(self) -> bool:
        return self._render_fused

    def render_fused(self, gaussians, extrinsics, intrinsics, image_height: int,
                     image_width: int, contrib_floor: float | None = None, k_cap: float = 3.0,
                     use_isoellipse: bool = False):
        """backends/cpu_cpp/backend.py:319-380: one call from the Gaussians to the
        (H,W,3) float32 image and a stats dict (project_ms, tile_assign_ms,
        sort_ms, cull_ms, blend_ms, total_ms, num_visible, num_entries, pairs_in, and
        with cull_stats pairs_dropped, pairs_kept_per_mb). `gaussians` has means, scales,
        rotations, opacities and colors (N,3) RGB. As in the reference, the
        contrib_floor / k_cap / use_isoellipse arguments of this call are not
        read: the constructor's settings apply (the per-pair floor is the
        microblock floor unless the constructor overrode it)."""
        del contrib_floor, k_cap, use_isoellipse  # the reference ignores them too
        means = _np(gaussians.means, np.float32)
        cov = self._cached_cov3d(_np(gaussians.scales, np.float32),
                                 _np(gaussians.rotations, np.float32))
        op = _np(gaussians.opacities, np.float32).reshape(-1)
        col = _np(gaussians.colors, np.float32).reshape(means.shape[0], 3)
        self.ctx.set_scene(means, cov, op, col)
        view = self._view(extrinsics, intrinsics, image_height, image_width)
        img, st = self.ctx.render(view)
        # pairs_in = the tile-sorted pairs the microblock cull reads
        # (cull_and_blend.cpp:700); dropped / kept_per_mb from its counts
        stats = {"project_ms": st["ms_project"] + st["ms_depth_sort"],
                 "tile_assign_ms": st["ms_tile_assign"], "sort_ms": st["ms_tile_sort"],
                 "cull_ms": 0.0, "blend_ms": st["ms_blend"], "total_ms": st["ms_total"],
                 "num_visible": int(st["num_visible"]), "num_entries": int(st["num_entries"]),
                 "pairs_in": int(st["num_entries"])}
        if self.cull_stats:
            stats["pairs_dropped"] = int(st["pairs_dropped_mb"])
            stats["pairs_kept_per_mb"] = int(st["pairs_kept_mb"])
        return img, stats

    def close(self) -> None:
        if self.ctx is not None:
            self.ctx.close()
            self.ctx = None


def register(registry: dict) -> dict:
    """Add the GPU backend to a backends/__init__.py-style REGISTRY (name -> class)."""
    registry[NAME] = HipBackend
    return registry


def get_backend(name: str, registry: dict | None = None, **kwargs):
    """backends/__init__.py:50-60 get_backend: construct the backend registered
    under `name` (KeyError listing the available names otherwise)."""
    reg = register({}) if registry is None else registry
    try:
        cls = reg[name]
    except KeyError:
        raise KeyError(f"unknown backend {name!r}; available: {', '.join(sorted(reg))}") from None
    return cls(**kwargs)
