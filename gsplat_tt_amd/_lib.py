"""ctypes binding of the C ABI in include/gsplat_hip.h (libgsplat_hip.so).

This is the Python-side mirror of the reference's per-stage operators
(_gsplat_cpu.project / tile_assign / sort / cull_and_blend / render_full,
backends/cpu_cpp/pybind_module.cpp) running on the GPU. There is no CPU
fallback: if the library is missing, importing raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgsplat_hip.so")

GS_OK, GS_E_INVALID, GS_E_DEVICE, GS_E_CAPACITY = 0, -1, -2, -3
OUT_FORMATS = {"u8": 0, "bf16": 1, "f32": 2}
# Gaussians per projection partition (the unit of the visibility compaction and
# of the chunk frustum skip; csrc/gs_internal.h kProjPartition)
PROJECT_PARTITION = 2048

EXPORTED = (
    "gs_create", "gs_destroy", "gs_last_error", "gs_set_timing", "gs_device_info",
    "gs_scene_set", "gs_render", "gs_project", "gs_tile_assign", "gs_sort_and_bin",
    "gs_cull_and_blend", "gs_sort_pairs_u64_dev", "gs_last_sort_pass_ms", "gs_dev_alloc",
    "gs_dev_free", "gs_memcpy_h2d", "gs_memcpy_d2h", "gs_memcpy_d2d", "gs_sync",
    "gs_train_init", "gs_train_read", "gs_train_write", "gs_train_set_step",
    "gs_train_set_visible", "gs_train_forward", "gs_train_backward", "gs_train_adam",
    "gs_train_set_moments",
    "gs_train_step",
    "gs_train_loss",
    "gs_render_batch",
    "gs_render_next",
    "gs_render_out_ring", "gs_out_release", "gs_out_ring_config", "gs_out_ring_info",
    "gs_set_chunk_cull",
    "gs_frame_readback", "gs_frame_readback_info", "gs_set_cull_stats", "gs_set_spin_limit",
    "gs_set_graphs", "gs_set_pair_limit", "gs_overflow_next_floor",
    "gs_graph_counts",
    "gs_sort_tile_depth_dev", "gs_sort_tile_depth_ids_dev", "gs_last_ranges_ms",
    "gs_sort_tile_depth_noalloc",
)
TRAIN_PARAMS = ("means", "log_scales", "quats", "opacity_logits", "sh")


class GsScene(ctypes.Structure):
    _fields_ = [("means", ctypes.c_void_p), ("cov3d", ctypes.c_void_p),
                ("cov3d_stride", ctypes.c_int), ("opacities", ctypes.c_void_p),
                ("colors", ctypes.c_void_p), ("sh_degree", ctypes.c_int),
                ("n", ctypes.c_int64), ("version", ctypes.c_uint64)]


class GsView(ctypes.Structure):
    _fields_ = [("extrinsics", ctypes.c_float * 16), ("intrinsics", ctypes.c_float * 9),
                ("image_height", ctypes.c_int), ("image_width", ctypes.c_int),
                ("tile_size", ctypes.c_int), ("min_opacity", ctypes.c_float),
                ("contrib_floor", ctypes.c_float), ("mb_contrib_floor", ctypes.c_float),
                ("cull_disabled", ctypes.c_int), ("transmittance_threshold", ctypes.c_float),
                ("max_radius", ctypes.c_int), ("k_cap", ctypes.c_float),
                ("use_isoellipse", ctypes.c_int), ("out_format", ctypes.c_int),
                ("sh_clamp_hi", ctypes.c_int)]


class GsStats(ctypes.Structure):
    _fields_ = [("num_visible", ctypes.c_int64), ("num_entries", ctypes.c_int64),
                ("pairs_pre", ctypes.c_int64), ("ms_project", ctypes.c_float),
                ("ms_depth_sort", ctypes.c_float), ("ms_tile_assign", ctypes.c_float),
                ("ms_tile_sort", ctypes.c_float), ("ms_blend", ctypes.c_float),
                ("ms_total", ctypes.c_float), ("blend_evals", ctypes.c_int64),
                ("blend_batches", ctypes.c_int64), ("blend_iters", ctypes.c_int64),
                ("blend_kept", ctypes.c_int64), ("blend_max_iters", ctypes.c_int64),
                ("chunks_skipped", ctypes.c_int64), ("pairs_dropped_mb", ctypes.c_int64),
                ("pairs_kept_mb", ctypes.c_int64), ("contrib_floor", ctypes.c_float),
                ("floor_retries", ctypes.c_int32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class GsOutImage(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("bytes", ctypes.c_int64), ("pitch", ctypes.c_int64),
                ("lease", ctypes.c_uint64)]


class GsTrainArrays(ctypes.Structure):
    _fields_ = [(k, ctypes.c_void_p) for k in ("means", "log_scales", "quats", "opacity_logits",
                                                "sh")]


class GsTrainCfg(ctypes.Structure):
    _fields_ = [("near_plane", ctypes.c_float), ("lowpass", ctypes.c_float),
                ("alpha_max", ctypes.c_float), ("alpha_min", ctypes.c_float),
                ("t_min", ctypes.c_float), ("background", ctypes.c_float * 3),
                ("loss_scale", ctypes.c_float), ("lambda_dssim", ctypes.c_float),
                ("lr_means", ctypes.c_double), ("lr_log_scales", ctypes.c_double),
                ("lr_quats", ctypes.c_double), ("lr_opacity", ctypes.c_double),
                ("lr_sh_dc", ctypes.c_double), ("lr_sh_rest", ctypes.c_double),
                ("beta1", ctypes.c_double), ("beta2", ctypes.c_double), ("eps", ctypes.c_double)]


class GsTrainStats(ctypes.Structure):
    _fields_ = [("num_blendable", ctypes.c_int64), ("num_entries", ctypes.c_int64),
                ("step", ctypes.c_int64), ("loss", ctypes.c_double),
                ("ms_forward", ctypes.c_float), ("ms_backward", ctypes.c_float),
                ("ms_adam", ctypes.c_float), ("ms_total", ctypes.c_float),
                ("l1", ctypes.c_double), ("ssim", ctypes.c_double),
                ("pairs_pre", ctypes.c_int64), ("pair_capacity", ctypes.c_int64),
                ("pixel_pairs", ctypes.c_int64), ("pixel_blended", ctypes.c_int64)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class GsTrainProj(ctypes.Structure):
    _fields_ = [(k, ctypes.c_void_p) for k in ("means2d", "conic", "opacity", "colors", "depth",
                                                "valid", "visible")]


def make_train_cfg(near=0.2, lowpass=0.3, alpha_max=0.99, alpha_min=1.0 / 255.0, t_min=1e-4,
                   background=(0.0, 0.0, 0.0), loss_scale=1.0, lr=None, betas=(0.9, 0.999),
                   eps=1e-15, lambda_dssim=0.0) -> GsTrainCfg:
    """Training configuration: gsplat/train_oracle.py RenderConfig (:63-71) and the
    3DGS learning rates of DEFAULT_LR (:421-423). lambda_dssim = 0: L1 loss;
    0.2: the full 3DGS loss 0.8 L1 + 0.2 (1 - SSIM) (train_oracle.py:276-279)."""
    lr = dict({"means": 1.6e-4, "log_scales": 5e-3, "quats": 1e-3, "opacity_logits": 0.05,
               "sh_dc": 2.5e-3, "sh_rest": 2.5e-3 / 20.0}, **(lr or {}))
    c = GsTrainCfg()
    c.near_plane, c.lowpass, c.alpha_max, c.alpha_min, c.t_min = near, lowpass, alpha_max, \
        alpha_min, t_min
    for i in range(3):
        c.background[i] = float(background[i])
    c.loss_scale = float(loss_scale)
    c.lambda_dssim = float(lambda_dssim)
    c.lr_means, c.lr_log_scales, c.lr_quats = lr["means"], lr["log_scales"], lr["quats"]
    c.lr_opacity, c.lr_sh_dc, c.lr_sh_rest = lr["opacity_logits"], lr["sh_dc"], lr["sh_rest"]
    c.beta1, c.beta2, c.eps = float(betas[0]), float(betas[1]), float(eps)
    return c


_LIB = None


def overflow_next_floor(floor: float, max_n: int, cap: int) -> float:
    """The floor ladder's next contribution floor (gs_overflow_next_floor)."""
    return float(load_library().gs_overflow_next_floor(float(floor), int(max_n), int(cap)))


def load_library():
    """Load libgsplat_hip.so (raises OSError when it was not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = ctypes.CDLL(LIB_PATH)
        L.gs_last_error.restype = ctypes.c_char_p
        L.gs_destroy.restype = None
        L.gs_out_release.argtypes = [ctypes.c_uint64]
        L.gs_set_spin_limit.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.gs_set_pair_limit.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.gs_overflow_next_floor.restype = ctypes.c_float
        L.gs_overflow_next_floor.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32]
        L.gs_last_ranges_ms.restype = ctypes.c_float
        L.gs_last_ranges_ms.argtypes = [ctypes.c_void_p]
        for name in EXPORTED:
            getattr(L, name)  # every declared symbol must resolve
        _LIB = L
    return _LIB


class GsError(RuntimeError):
    pass


def _check(rc):
    if rc != GS_OK:
        msg = load_library().gs_last_error().decode()
        if rc == GS_E_INVALID:
            raise ValueError(msg)
        raise GsError(f"[{rc}] {msg}")


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def make_view(extrinsics, intrinsics, H, W, tile_size=16, min_opacity=1.0 / 255.0,
              contrib_floor=1.0 / 16384.0, mb_contrib_floor=1.0 / 16384.0, cull_disabled=False,
              transmittance_threshold=1.0 / 255.0, max_radius=0, k_cap=3.0,
              use_isoellipse=False, output="f32", sh_clamp=True) -> GsView:
    v = GsView()
    e = _f32(extrinsics).reshape(16)
    k = _f32(intrinsics).reshape(9)
    for i in range(16):
        v.extrinsics[i] = float(e[i])
    for i in range(9):
        v.intrinsics[i] = float(k[i])
    v.image_height, v.image_width, v.tile_size = int(H), int(W), int(tile_size)
    v.min_opacity, v.contrib_floor = float(min_opacity), float(contrib_floor)
    v.mb_contrib_floor, v.cull_disabled = float(mb_contrib_floor), int(bool(cull_disabled))
    v.transmittance_threshold, v.max_radius = float(transmittance_threshold), int(max_radius)
    v.k_cap, v.use_isoellipse = float(k_cap), int(bool(use_isoellipse))
    v.out_format, v.sh_clamp_hi = OUT_FORMATS[output], int(bool(sh_clamp))
    return v


_OUT_DTYPE = {0: np.uint8, 1: np.uint16, 2: np.float32}


class _LeasedImage:
    """The base object of an array over a ring image: releases the lease when
    the last array over it is gone."""

    def __init__(self, lib, img, shape, dtype):
        self._lib = lib
        self._lease = int(img.lease)
        self.__array_interface__ = {"shape": shape, "typestr": np.dtype(dtype).str,
                                    "data": (int(img.data), False), "version": 3}

    def __del__(self):
        if self._lease:
            self._lib.gs_out_release(ctypes.c_uint64(self._lease))
            self._lease = 0


class Context:
    """One GPU context (device + stream + resident scene)."""

    def __init__(self, device: int = 0, timing: int = 0):
        """timing: 0 off, 1 (or True) per-stage hipEvent times in the stats, 2 also
        the blend's evaluation counters (gs_set_timing)."""
        self._L = load_library()
        self._c = ctypes.c_void_p()
        _check(self._L.gs_create(int(device), ctypes.byref(self._c)))
        if timing:
            _check(self._L.gs_set_timing(self._c, int(timing)))
        self._keep = None
        self._version = 0

    def close(self):
        if self._c:
            self._L.gs_destroy(self._c)
            self._c = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._c

    def device_info(self):
        cus, minor = ctypes.c_int(), ctypes.c_int()
        _check(self._L.gs_device_info(self._c, ctypes.byref(cus), ctypes.byref(minor)))
        return cus.value, minor.value

    # ---- scene + frame
    @staticmethod
    def _scene_struct(means, cov3d, opacities, colors, sh_degree=None, version=0):
        means = _f32(means)
        n = means.shape[0]
        cov3d = _f32(cov3d).reshape(n, -1)
        stride = cov3d.shape[1]
        colors = _f32(colors)
        if sh_degree is None:
            sh_degree = -1 if (colors.ndim == 2 and colors.shape[1] == 3) else \
                {1: 0, 4: 1, 9: 2, 16: 3}[colors.reshape(n, -1, 3).shape[1]]
        opac = None if opacities is None else _f32(opacities)
        s = GsScene(_ptr(means), _ptr(cov3d), stride, _ptr(opac), _ptr(colors), int(sh_degree),
                    n, int(version))
        return s, (means, cov3d, opac, colors)

    def set_scene(self, means, cov3d, opacities, colors, sh_degree=None):
        self._version += 1
        s, keep = self._scene_struct(means, cov3d, opacities, colors, sh_degree, self._version)
        _check(self._L.gs_scene_set(self._c, ctypes.byref(s)))
        self._keep = keep  # keep the host arrays alive for the pointer-keyed cache

    def render(self, view: GsView, out=None):
        H, W = view.image_height, view.image_width
        if out is None:
            out = np.empty((H, W, 3), _OUT_DTYPE[view.out_format])
        st = GsStats()
        _check(self._L.gs_render(self._c, ctypes.byref(view), _ptr(out), 0, ctypes.byref(st)))
        return out, st.as_dict()

    def train_loss(self, image, target, lambda_dssim=0.2, loss_scale=1.0):
        """(loss, l1, ssim, dL/dimage) of an (H,W,3) image against a target on the
        GPU: loss_scale ((1 - lambda) L1 + lambda (1 - SSIM))."""
        image, target = _f32(image), _f32(target)
        if image.shape != target.shape or image.ndim != 3 or image.shape[2] != 3:
            raise ValueError("image and target must both be (H, W, 3)")
        H, W = image.shape[:2]
        grad = np.empty_like(image)
        out = (ctypes.c_double * 3)()
        _check(self._L.gs_train_loss(self._c, _ptr(image), _ptr(target), int(H), int(W),
                                     ctypes.c_float(lambda_dssim), ctypes.c_float(loss_scale),
                                     _ptr(grad), out))
        return out[0], out[1], out[2], grad

    def render_next(self, view: GsView, next_view: GsView | None = None, out=None):
        """render() of `view` that also enqueues `next_view`'s frame on the second
        slot; a following render_next(next_view, ...) completes it."""
        H, W = view.image_height, view.image_width
        if out is None:
            out = np.empty((H, W, 3), _OUT_DTYPE[view.out_format])
        st = GsStats()
        _check(self._L.gs_render_next(self._c, ctypes.byref(view), _ptr(out), 0,
                                      ctypes.byref(next_view) if next_view is not None else None,
                                      ctypes.byref(st)))
        return out, st.as_dict()

    def render_ring(self, view: GsView, next_view: GsView | None = None):
        """render_next() whose image is a pinned buffer of the context's output
        ring, returned without a host copy: an (H,W,3) array that holds the
        buffer's lease until the array (and every view of it) is gone."""
        img, st = GsOutImage(), GsStats()
        _check(self._L.gs_render_out_ring(self._c, ctypes.byref(view),
                                          ctypes.byref(next_view) if next_view is not None
                                          else None, ctypes.byref(img), ctypes.byref(st)))
        shape = (view.image_height, view.image_width, 3)
        return np.asarray(_LeasedImage(self._L, img, shape, _OUT_DTYPE[view.out_format])), \
            st.as_dict()

    def set_chunk_cull(self, on: bool = True, k: float = 1.5):
        """Chunk frustum skip for the frames of this context (render/host/chunk_cull.h)."""
        _check(self._L.gs_set_chunk_cull(self._c, ctypes.c_int(1 if on else 0), ctypes.c_double(k)))

    def out_ring_config(self, cap: int):
        _check(self._L.gs_out_ring_config(self._c, ctypes.c_int(cap)))

    def out_ring_info(self):
        """(slots, slots whose image is held, slots made, slots replaced)."""
        size, held = ctypes.c_int(), ctypes.c_int()
        grows, replaced = ctypes.c_int64(), ctypes.c_int64()
        _check(self._L.gs_out_ring_info(self._c, ctypes.byref(size), ctypes.byref(held),
                                        ctypes.byref(grows), ctypes.byref(replaced)))
        return size.value, held.value, grows.value, replaced.value

    def render_batch(self, views, outs, out_on_device=True):
        """Views rendered with up to four frames in flight; outs: device pointers (or host
        arrays when out_on_device is False), one per view. Returns their stats."""
        n = len(views)
        varr = (GsView * n)(*views)
        if out_on_device:
            ptrs = (ctypes.c_void_p * n)(*[ctypes.c_void_p(int(p)) for p in outs])
        else:
            ptrs = (ctypes.c_void_p * n)(*[o.ctypes.data_as(ctypes.c_void_p) for o in outs])
        sts = (GsStats * n)()
        _check(self._L.gs_render_batch(self._c, varr, ctypes.c_int(n), ptrs,
                                       ctypes.c_int(1 if out_on_device else 0), sts))
        return [st.as_dict() for st in sts]

    def frame_readback(self, ids=True, ranges=True):
        """The frame held by the context's first slot (the last render(), or after
        render_batch the last view i with i % 4 == 0): dict(M, pairs_pre, P, T,
        batch_index, replayed, sorted_ids int64 (P,), tile_ranges int64 (T, 2)) -
        the tile-sorted compact ids and the tile ranges of the frame path itself
        (gs_frame_readback, sized by gs_frame_readback_info)."""
        info = np.zeros(6, np.int64)
        _check(self._L.gs_frame_readback_info(self._c, _ptr(info)))
        M, ppre, P, T, bi, rep = (int(x) for x in info)
        out = dict(M=M, pairs_pre=ppre, P=P, T=T, batch_index=bi, replayed=bool(rep))
        sid = np.empty(max(P, 1), np.int64) if ids else None
        rg = np.empty((T, 2), np.int64) if ranges else None
        _check(self._L.gs_frame_readback(self._c, None, _ptr(sid), ctypes.c_int64(P if ids else 0),
                                         _ptr(rg), ctypes.c_int64(T if ranges else 0)))
        if ids:
            out["sorted_ids"] = sid[:P]
        if ranges:
            out["tile_ranges"] = rg
        return out

    def set_cull_stats(self, on: bool = True):
        """Per-frame counts of the reference's microblock cull in the stats
        (pairs_dropped_mb, pairs_kept_mb)."""
        _check(self._L.gs_set_cull_stats(self._c, ctypes.c_int(1 if on else 0)))

    def set_graphs(self, on: bool = True):
        """render_batch frames replayed from captured HIP graphs (on by default)
        or every kernel enqueued directly; the results are the same."""
        _check(self._L.gs_set_graphs(self._c, ctypes.c_int(1 if on else 0)))

    def graph_counts(self):
        """(captures, replays) of frame graphs so far over the frame slots."""
        c = ctypes.c_int64(0)
        r = ctypes.c_int64(0)
        _check(self._L.gs_graph_counts(self._c, ctypes.byref(c), ctypes.byref(r)))
        return c.value, r.value

    def set_pair_limit(self, limit: int = 0):
        """Most candidate pairs a rendered frame may hold (0: 2^32-1). A frame with
        more is rendered again at a coarser contribution floor (gs_stats
        contrib_floor / floor_retries)."""
        _check(self._L.gs_set_pair_limit(self._c, ctypes.c_uint32(limit)))

    def set_spin_limit(self, limit: int = 0):
        """Spin limit of the kernels' bounded look-back waits (0: default); a tiny
        limit makes a wait give up, and the call then fails (tests of that path)."""
        _check(self._L.gs_set_spin_limit(self._c, ctypes.c_uint32(limit)))

    def sort_tile_depth_dev(self, keys_ptr: int, vals_ptr: int, n: int, num_tiles: int,
                            ranges_ptr: int):
        """Stable sort of (tile << 32 | depth bits, value) pairs on the device plus the
        per-tile [start, end) ranges (num_tiles x 2 u32 at ranges_ptr)."""
        passes = ctypes.c_int()
        _check(self._L.gs_sort_tile_depth_dev(self._c, ctypes.c_void_p(keys_ptr),
                                              ctypes.c_void_p(vals_ptr), ctypes.c_int64(n),
                                              ctypes.c_int64(num_tiles),
                                              ctypes.c_void_p(ranges_ptr), ctypes.byref(passes)))
        return passes.value

    def sort_tile_depth_ids_dev(self, keys_ptr: int, ids_ptr: int, n: int, num_tiles: int,
                                ranges_ptr: int, num_gaussians: int = 0):
        """The same sort with sort_and_bin's outputs only: the ids at ids_ptr
        (each below num_gaussians, sort_and_bin's M; 0: any 32-bit id) come back
        in sorted key order, the keys at keys_ptr are overwritten, and ranges_ptr
        receives the per-tile [start, end)."""
        passes = ctypes.c_int()
        _check(self._L.gs_sort_tile_depth_ids_dev(self._c, ctypes.c_void_p(keys_ptr),
                                                  ctypes.c_void_p(ids_ptr), ctypes.c_int64(n),
                                                  ctypes.c_int64(num_gaussians),
                                                  ctypes.c_int64(num_tiles),
                                                  ctypes.c_void_p(ranges_ptr),
                                                  ctypes.byref(passes)))
        return passes.value

    def last_ranges_ms(self) -> float:
        return float(self._L.gs_last_ranges_ms(self._c))

    def render_dev(self, view: GsView, dev_out_ptr: int):
        st = GsStats()
        _check(self._L.gs_render(self._c, ctypes.byref(view), ctypes.c_void_p(dev_out_ptr), 1,
                                 ctypes.byref(st)))
        return st.as_dict()

    # ---- stages (host arrays)
    def project(self, means, cov3d, opacities, colors, view: GsView, sh_degree=None):
        self._version += 1
        s, keep = self._scene_struct(means, cov3d, opacities, colors, sh_degree, self._version)
        n = s.n
        valid = np.empty(n, np.uint8)
        m2 = np.empty((n, 2), np.float32)
        c2 = np.empty((n, 4), np.float32)
        dp = np.empty(n, np.float32)
        rd = np.empty((n, 2), np.float32)
        co = np.empty((n, 3), np.float32)
        op = np.empty(n, np.float32)
        M = ctypes.c_int64()
        _check(self._L.gs_project(self._c, ctypes.byref(s), ctypes.byref(view), _ptr(valid),
                                  _ptr(m2), _ptr(c2), _ptr(dp), _ptr(rd), _ptr(co), _ptr(op),
                                  ctypes.byref(M)))
        self._keep = keep
        M = M.value
        return dict(valid=valid.astype(bool), means2d=m2[:M], covs2d=c2[:M], depths=dp[:M],
                    radii=rd[:M], colors=co[:M], opacities=op[:M])

    def tile_assign(self, means2d, radii, H, W, tile_size, covs2d=None, opac=None,
                    contrib_floor=1.0 / 16384.0):
        means2d, radii = _f32(means2d), _f32(radii)
        m = means2d.shape[0]
        covs2d = None if covs2d is None else _f32(covs2d).reshape(m, 4)
        opac = None if opac is None else _f32(opac)
        P, Ppre = ctypes.c_int64(), ctypes.c_int64()
        rc = self._L.gs_tile_assign(self._c, _ptr(means2d), _ptr(radii), ctypes.c_int64(m),
                                    int(H), int(W), int(tile_size), _ptr(covs2d), _ptr(opac),
                                    ctypes.c_float(contrib_floor), None, None, ctypes.c_int64(0),
                                    ctypes.byref(P), ctypes.byref(Ppre))
        if rc not in (GS_OK, GS_E_CAPACITY):
            _check(rc)
        g = np.empty(max(P.value, 1), np.int64)
        t = np.empty(max(P.value, 1), np.int64)
        if P.value > 0:
            _check(self._L.gs_tile_assign(self._c, _ptr(means2d), _ptr(radii), ctypes.c_int64(m),
                                          int(H), int(W), int(tile_size), _ptr(covs2d),
                                          _ptr(opac), ctypes.c_float(contrib_floor), _ptr(g),
                                          _ptr(t), ctypes.c_int64(P.value), ctypes.byref(P),
                                          ctypes.byref(Ppre)))
        return g[:P.value], t[:P.value], Ppre.value

    def sort_and_bin(self, gids, tids, depths, tiles_x, tiles_y):
        gids = np.ascontiguousarray(gids, np.int64)
        tids = np.ascontiguousarray(tids, np.int64)
        depths = _f32(depths)
        P = gids.shape[0]
        s = np.empty(max(P, 1), np.int64)
        r = np.empty((tiles_x * tiles_y, 2), np.int64)
        _check(self._L.gs_sort_and_bin(self._c, _ptr(gids), _ptr(tids), _ptr(depths),
                                       ctypes.c_int64(P), ctypes.c_int64(depths.shape[0]),
                                       int(tiles_x), int(tiles_y), _ptr(s), _ptr(r)))
        return s[:P], r

    def cull_and_blend(self, means2d, covs2d, colors, opac, sorted_ids, tile_ranges,
                       view: GsView):
        means2d, colors, opac = _f32(means2d), _f32(colors), _f32(opac)
        m = means2d.shape[0]
        covs2d = _f32(covs2d).reshape(m, 4)
        sorted_ids = np.ascontiguousarray(sorted_ids, np.int64)
        tile_ranges = np.ascontiguousarray(tile_ranges, np.int64)
        out = np.empty((view.image_height, view.image_width, 3), _OUT_DTYPE[view.out_format])
        _check(self._L.gs_cull_and_blend(self._c, _ptr(means2d), _ptr(covs2d), _ptr(colors),
                                         _ptr(opac), _ptr(sorted_ids), _ptr(tile_ranges),
                                         ctypes.c_int64(m), ctypes.c_int64(sorted_ids.shape[0]),
                                         ctypes.byref(view), _ptr(out)))
        return out

    # ---- device memory + standalone sort
    def dev_alloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        _check(self._L.gs_dev_alloc(self._c, ctypes.c_int64(nbytes), ctypes.byref(p)))
        return p.value

    def dev_free(self, ptr: int):
        _check(self._L.gs_dev_free(self._c, ctypes.c_void_p(ptr)))

    def h2d(self, dst: int, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        _check(self._L.gs_memcpy_h2d(self._c, ctypes.c_void_p(dst), _ptr(arr),
                                     ctypes.c_int64(arr.nbytes)))

    def d2h(self, arr: np.ndarray, src: int):
        _check(self._L.gs_memcpy_d2h(self._c, _ptr(arr), ctypes.c_void_p(src),
                                     ctypes.c_int64(arr.nbytes)))
        return arr

    def d2d(self, dst: int, src: int, nbytes: int):
        _check(self._L.gs_memcpy_d2d(self._c, ctypes.c_void_p(dst), ctypes.c_void_p(src),
                                     ctypes.c_int64(nbytes)))

    def sort_pairs_u64_dev(self, keys_ptr: int, vals_ptr: int, n: int, begin_bit=0, end_bit=64):
        passes = ctypes.c_int()
        _check(self._L.gs_sort_pairs_u64_dev(self._c, ctypes.c_void_p(keys_ptr),
                                             ctypes.c_void_p(vals_ptr), ctypes.c_int64(n),
                                             int(begin_bit), int(end_bit), ctypes.byref(passes)))
        return passes.value

    def last_sort_pass_ms(self):
        buf = (ctypes.c_float * 8)()
        k = self._L.gs_last_sort_pass_ms(self._c, buf, 8)
        return [buf[i] for i in range(k)]

    def sort_pairs_u64(self, keys, vals, begin_bit=0, end_bit=64):
        """Host convenience: stable sort of (u64 key, u32 value) on the GPU."""
        keys = np.ascontiguousarray(keys, np.uint64)
        vals = np.ascontiguousarray(vals, np.uint32)
        n = keys.shape[0]
        dk, dv = self.dev_alloc(max(n, 1) * 8), self.dev_alloc(max(n, 1) * 4)
        try:
            self.h2d(dk, keys)
            self.h2d(dv, vals)
            passes = self.sort_pairs_u64_dev(dk, dv, n, begin_bit, end_bit)
            ko, vo = np.empty_like(keys), np.empty_like(vals)
            self.d2h(ko, dk)
            self.d2h(vo, dv)
        finally:
            self.dev_free(dk)
            self.dev_free(dv)
        return ko, vo, passes


class Trainer:
    """Training on the GPU (forward with the 3DGS rules, L1, backward, sparse Adam)
    through the gs_train_* entry points of one Context. Parameters are dicts of
    numpy arrays in optimizer space: means (n,3), log_scales (n,3), quats (n,4),
    opacity_logits (n,), sh (n,(d+1)^2,3)."""

    def __init__(self, ctx: "Context", params: dict, sh_degree: int):
        self.ctx, self._L = ctx, ctx._L
        self.n = int(np.asarray(params["means"]).shape[0])
        self.deg = int(sh_degree)
        self.K = (self.deg + 1) ** 2
        arrs, keep = self._arrays(params)
        _check(self._L.gs_train_init(ctx.handle, ctypes.byref(arrs), ctypes.c_int64(self.n),
                                     self.deg))

    def _shapes(self):
        n, K = self.n, self.K
        return {"means": (n, 3), "log_scales": (n, 3), "quats": (n, 4), "opacity_logits": (n,),
                "sh": (n, K, 3)}

    def _arrays(self, params):
        keep = {}
        a = GsTrainArrays()
        for k, shp in self._shapes().items():
            arr = np.ascontiguousarray(np.asarray(params[k], np.float32).reshape(shp))
            keep[k] = arr
            setattr(a, k, arr.ctypes.data)
        return a, keep

    def read(self, which=0) -> dict:
        """which: 0 parameters, 1 first moments, 2 second moments, 3 gradients."""
        out = {k: np.empty(shp, np.float32) for k, shp in self._shapes().items()}
        a, _ = self._arrays(out)
        for k in out:   # _arrays copies only when needed; bind the real buffers
            setattr(a, k, out[k].ctypes.data)
        _check(self._L.gs_train_read(self.ctx.handle, int(which), ctypes.byref(a)))
        return out

    def write(self, which, arrays: dict):
        a, keep = self._arrays(arrays)
        _check(self._L.gs_train_write(self.ctx.handle, int(which), ctypes.byref(a)))

    def set_step(self, step: int):
        _check(self._L.gs_train_set_step(self.ctx.handle, ctypes.c_int64(step)))

    def set_visible(self, visible):
        v = np.ascontiguousarray(np.asarray(visible, bool).astype(np.uint8))
        _check(self._L.gs_train_set_visible(self.ctx.handle, _ptr(v)))

    def set_moments(self, bf16: bool):
        """Adam moments stored as bf16 (round to nearest even) or fp32 (default);
        the stored moments are carried over."""
        _check(self._L.gs_train_set_moments(self.ctx.handle, ctypes.c_int(1 if bf16 else 0)))

    def forward(self, view: GsView, cfg: GsTrainCfg, target=None, want_proj=False):
        H, W = view.image_height, view.image_width
        img = np.empty((H, W, 3), np.float32)
        T = np.empty((H, W), np.float32)
        tgt = None if target is None else _f32(target).reshape(H, W, 3)
        proj = None
        pj = None
        if want_proj:
            n = self.n
            proj = dict(means2d=np.empty((n, 2), np.float32), conic=np.empty((n, 3), np.float32),
                        opacity=np.empty(n, np.float32), colors=np.empty((n, 3), np.float32),
                        depth=np.empty(n, np.float32), valid=np.empty(n, np.uint8),
                        visible=np.empty(n, np.uint8))
            pj = GsTrainProj()
            for k, v in proj.items():
                setattr(pj, k, v.ctypes.data)
        st = GsTrainStats()
        _check(self._L.gs_train_forward(self.ctx.handle, ctypes.byref(view), ctypes.byref(cfg),
                                        _ptr(tgt), _ptr(img), _ptr(T),
                                        ctypes.byref(pj) if pj is not None else None,
                                        ctypes.byref(st)))
        if proj is not None:
            proj["valid"] = proj["valid"].astype(bool)
            proj["visible"] = proj["visible"].astype(bool)
        return img, T, proj, st.as_dict()

    def backward(self, cfg: GsTrainCfg, dimage=None, want_g2d=False):
        g2d = np.empty((self.n, 9), np.float32) if want_g2d else None
        d = None if dimage is None else _f32(dimage)
        st = GsTrainStats()
        _check(self._L.gs_train_backward(self.ctx.handle, ctypes.byref(cfg), _ptr(d), _ptr(g2d),
                                         ctypes.byref(st)))
        return g2d, st.as_dict()

    def adam(self, cfg: GsTrainCfg):
        st = GsTrainStats()
        _check(self._L.gs_train_adam(self.ctx.handle, ctypes.byref(cfg), ctypes.byref(st)))
        return st.as_dict()

    def step(self, view: GsView, cfg: GsTrainCfg, target, target_on_device=False):
        st = GsTrainStats()
        if target_on_device:
            ptr = ctypes.c_void_p(int(target))
            keep = None
        else:
            keep = _f32(target)
            ptr = _ptr(keep)
        _check(self._L.gs_train_step(self.ctx.handle, ctypes.byref(view), ctypes.byref(cfg), ptr,
                                     int(bool(target_on_device)), ctypes.byref(st)))
        return st.as_dict()
