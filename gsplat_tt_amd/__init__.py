"""MI355X-native (gfx950) Gaussian-splat rasterizer.

Drop-in for the reference's render path: `gsplat_tt_amd.render_clean` is the
`render_clean` pybind module (render_view & co.), `gsplat_tt_amd._lib` binds
the C ABI of include/gsplat_hip.h, `gsplat_tt_amd.scenes` builds the seeded
benchmark workloads.
"""
from __future__ import annotations

import importlib
import os

HERE = os.path.dirname(os.path.abspath(__file__))

__all__ = ["build", "render_clean_module", "Context"]


def build(arch: str = "gfx950", jobs: int = 8) -> None:
    """Compile libgsplat_hip.so and the render_clean module in-tree."""
    from . import _build
    _build.build(arch=arch, jobs=jobs)


def render_clean_module():
    """Import the drop-in render_clean extension (raises if it was not built)."""
    return importlib.import_module("gsplat_tt_amd.render_clean")


def __getattr__(name):
    if name == "Context":
        from ._lib import Context
        return Context
    raise AttributeError(name)
