"""The plugin backend's interface (host side, no GPU): the stage methods and
their parameters are the reference's Backend ABC (gsplat/backend.py:53-151) and
the fused path's (backends/cpu_cpp/backend.py:319-338); registration follows
backends/__init__.py:20-60."""
import inspect

import pytest

from gsplat_tt_amd import backend as B

# parameter names in order, restated from the reference's signatures
REFERENCE_STAGES = {
    "project": ["means", "scales", "rotations", "extrinsics", "intrinsics", "image_height",
                "image_width", "opacities", "sub_timings"],           # backend.py:53-63
    "tile_assign": ["means_2d", "radii", "image_height", "image_width", "tile_size",
                    "covs_2d", "opacities", "contrib_floor", "sub_timings"],  # :78-88
    "sort": ["gaussian_ids", "tile_ids", "depths", "tiles_x", "tiles_y",
             "sub_timings"],                                          # :105-112
    "blend": ["means_2d", "covs_2d", "colors", "opacities", "sorted_gaussian_ids",
              "tile_ranges", "image_height", "image_width"],          # :128-138
    "render_fused": ["gaussians", "extrinsics", "intrinsics", "image_height", "image_width",
                     "contrib_floor", "k_cap", "use_isoellipse"],     # cpu_cpp:319-338
    "close": [],
}


@pytest.mark.parametrize("name,params", sorted(REFERENCE_STAGES.items()))
def test_stage_signatures_match_reference(name, params):
    sig = inspect.signature(getattr(B.HipBackend, name))
    got = [p for p in sig.parameters if p != "self"]
    assert got == params, (name, got)


def test_defaults_match_reference():
    ta = inspect.signature(B.HipBackend.tile_assign).parameters
    assert ta["tile_size"].default == 32 and ta["contrib_floor"].default == 1.0 / 16384.0
    rf = inspect.signature(B.HipBackend.render_fused).parameters
    assert rf["k_cap"].default == 3.0 and rf["use_isoellipse"].default is False
    init = inspect.signature(B.HipBackend.__init__).parameters
    for k, v in (("microblock", True), ("mb_contrib_floor", 1.0 / 16384.0),
                 ("cull_disabled", False), ("transmittance_threshold", 1.0 / 255.0),
                 ("min_opacity", 1.0 / 255.0), ("max_radius", 0), ("k_cap", 3.0),
                 ("use_isoellipse", False)):
        assert init[k].default == v, k


def test_registry():
    reg = {"cpu": object}
    assert B.register(reg)["hip"] is B.HipBackend and "cpu" in reg
    with pytest.raises(KeyError, match="available: cpu, hip"):
        B.get_backend("cuda", reg)


def test_tile_size_inference():
    import numpy as np
    assert B._tile_size_for(np.zeros((40 * 30, 2)), 480, 640) == 16
    assert B._tile_size_for(np.zeros((20 * 15, 2)), 480, 640) == 32
    with pytest.raises(ValueError):
        B._tile_size_for(np.zeros((7, 2)), 480, 640)


def test_no_gpu_fails_loudly():
    """No CPU fallback: without a GPU the constructor raises."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises((RuntimeError, OSError)):
        B.HipBackend()
