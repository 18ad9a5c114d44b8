"""The reference's known-answer cases (tests/kat_cases.py) through the HIP stage
entry points of the C ABI."""
import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from tests import kat_cases

pytestmark = pytest.mark.gpu


class GpuBackend:
    def __init__(self, ctx):
        self.ctx = ctx

    def project(self, means, cov3d9, w2c, K, colors, opac, H, W):
        view = L.make_view(w2c, K, H, W, tile_size=16)
        return self.ctx.project(means, cov3d9, opac, colors, view)

    def tile_assign(self, means2d, radii, H, W, ts, covs2d, opac, floor):
        return self.ctx.tile_assign(means2d, radii, H, W, ts, covs2d, opac, float(floor))

    def sort_and_bin(self, gids, tids, depths, tx, ty):
        return self.ctx.sort_and_bin(np.asarray(gids, np.int64), np.asarray(tids, np.int64),
                                     depths, tx, ty)

    def blend(self, means2d, covs2d, colors, opac, s, r, tx, ty, ts, H, W):
        view = L.make_view(np.eye(4, dtype=np.float32), np.eye(3, dtype=np.float32), H, W,
                           tile_size=ts, output="f32")
        return self.ctx.cull_and_blend(means2d, covs2d, colors, opac, s, r, view)


@pytest.mark.parametrize("case", kat_cases.ALL, ids=lambda f: f.__name__[4:])
def test_gpu_kat(gpu_ctx, case):
    print("kat", case.__name__, flush=True)
    case(GpuBackend(gpu_ctx))
