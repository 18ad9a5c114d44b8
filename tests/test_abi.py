"""The C-ABI boundary without a GPU: the shared library loads, exports every
function include/gsplat_hip.h declares, the ctypes mirrors of the structs have
the C layout, the pybind module imports with the reference's surface, and with
no device every entry point fails loudly (no CPU fallback)."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from gsplat_tt_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gsplat_hip.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_][a-z0-9_]*\s*\**\s*(gs_[a-z0-9_]+)\s*\(",
                                 src, flags=re.M)))


def test_header_declares_the_known_entry_points():
    fns = declared_functions()
    assert set(fns) == set(L.EXPORTED), set(fns) ^ set(L.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = L.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", lib._name], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    for name in declared_functions():
        assert name in exported, name


def test_struct_layout_matches_header():
    prog = r"""
#include <stddef.h>
#include <stdio.h>
#include "gsplat_hip.h"
#define P(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  printf("gs_scene %zu\ngs_view %zu\ngs_stats %zu\n", sizeof(gs_scene), sizeof(gs_view),
         sizeof(gs_stats));
  printf("gs_train_cfg %zu\ngs_train_stats %zu\ngs_train_proj %zu\ngs_train_arrays %zu\n",
         sizeof(gs_train_cfg), sizeof(gs_train_stats), sizeof(gs_train_proj),
         sizeof(gs_train_arrays));
  P(gs_train_cfg, loss_scale) P(gs_train_cfg, lambda_dssim) P(gs_train_cfg, lr_means)
  P(gs_train_cfg, eps) P(gs_train_stats, loss) P(gs_train_stats, ms_total)
  P(gs_train_stats, l1) P(gs_train_stats, ssim) P(gs_train_stats, pair_capacity)
  P(gs_train_stats, pixel_blended)
  P(gs_train_proj, visible)
  P(gs_scene, n) P(gs_scene, version) P(gs_view, image_height) P(gs_view, tile_size)
  P(gs_view, k_cap) P(gs_view, out_format) P(gs_view, sh_clamp_hi)
  P(gs_stats, ms_project) P(gs_stats, blend_max_iters) P(gs_stats, contrib_floor)
  P(gs_stats, floor_retries)
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(c, "w").write(prog)
        subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), c, "-o", exe],
                       check=True)
        lines = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    got = dict(ln.rsplit(" ", 1) for ln in lines.strip().splitlines())
    assert int(got["gs_scene"]) == ctypes.sizeof(L.GsScene)
    assert int(got["gs_view"]) == ctypes.sizeof(L.GsView)
    assert int(got["gs_stats"]) == ctypes.sizeof(L.GsStats)
    classes = {"gs_scene": L.GsScene, "gs_view": L.GsView, "gs_stats": L.GsStats,
               "gs_train_cfg": L.GsTrainCfg, "gs_train_stats": L.GsTrainStats,
               "gs_train_proj": L.GsTrainProj, "gs_train_arrays": L.GsTrainArrays}
    for t, cls in classes.items():
        assert int(got[t]) == ctypes.sizeof(cls), t
    for key, val in got.items():
        if "." in key:
            t, f = key.split(".")
            cls = classes[t]
            assert getattr(cls, f).offset == int(val), key


def test_render_clean_module_surface():
    import gsplat_tt_amd
    rc = gsplat_tt_amd.render_clean_module()
    for name in ("render_view", "pfwc_num_cores", "bump_scene_version", "scene_version",
                 "device_shutdown", "stage_timings", "reset_stage_timings"):
        assert hasattr(rc, name), name
    v0 = rc.scene_version()
    rc.bump_scene_version()
    assert rc.scene_version() == v0 + 1


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_device_fails_loudly():
    with pytest.raises(RuntimeError):
        L.Context(0)
    import numpy as np
    import gsplat_tt_amd
    rc = gsplat_tt_amd.render_clean_module()
    with pytest.raises(RuntimeError):
        rc.render_view(np.zeros((1, 3), np.float32), np.eye(3, dtype=np.float32).reshape(1, 9),
                       np.ones(1, np.float32), np.ones((1, 3), np.float32),
                       np.eye(4, dtype=np.float32), np.eye(3, dtype=np.float32), 16, 16, 16,
                       1 / 255, 1 / 16384, 1 / 16384, False, 1 / 255, 0, 3.0, False)
