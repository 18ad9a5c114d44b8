"""gs_sort_tile_depth_noalloc, the entry point that allocates nothing, called
through the C ABI and checked against gs_sort_tile_depth_dev on the same keys:
sorted keys, values and per-tile ranges bit-exact, on two calls in a row (the
second smaller, over the same scratch array), and a size past the array's
maximum rejected with GS_E_CAPACITY."""
import ctypes

import numpy as np
import pytest

from gsplat_tt_amd import _lib as L
from gsplat_tt_amd import scenes

pytestmark = pytest.mark.gpu

MAX_KEYS = 1 << 20


def _sort(ctx, fn, keys, vals, tiles):
    n = keys.shape[0]
    dk, dv, dr = ctx.dev_alloc(max(n, 1) * 8), ctx.dev_alloc(max(n, 1) * 4), \
        ctx.dev_alloc(tiles * 8)
    try:
        ctx.h2d(dk, keys)
        ctx.h2d(dv, vals)
        passes = ctypes.c_int()
        rc = fn(ctx.handle, ctypes.c_void_p(dk), ctypes.c_void_p(dv), ctypes.c_int64(n),
                ctypes.c_int64(tiles), ctypes.c_void_p(dr), ctypes.byref(passes))
        L._check(rc)
        ko, vo = np.empty(n, np.uint64), np.empty(n, np.uint32)
        rg = np.empty((tiles, 2), np.uint32)
        ctx.d2h(ko, dk)
        ctx.d2h(vo, dv)
        ctx.d2h(rg, dr)
    finally:
        for p in (dk, dv, dr):
            ctx.dev_free(p)
    return ko, vo, rg, passes.value


@pytest.mark.parametrize("sizes", [(MAX_KEYS, 300_001), (700_000, 65_537)])
def test_noalloc_sort_matches_allocating_sort(sizes):
    ctx = L.Context(0)
    lib = L.load_library()
    try:
        for call, (n, tiles) in enumerate(zip(sizes, (5000, 1200))):
            print(f"noalloc call {call}: n={n} tiles={tiles}", flush=True)
            keys, vals = scenes.config4_keys(seed=40 + call, n=n, tiles=tiles)
            a = _sort(ctx, lib.gs_sort_tile_depth_noalloc, keys, vals, tiles)
            b = _sort(ctx, lib.gs_sort_tile_depth_dev, keys, vals, tiles)
            for x, y in zip(a[:3], b[:3]):
                assert np.array_equal(x, y)
            assert a[3] == (32 + int(np.ceil(np.log2(tiles))) + 7) // 8  # every pass runs
            order = np.argsort(keys, kind="stable").astype(np.uint32)
            assert np.array_equal(a[1], order)
    finally:
        ctx.close()


def test_noalloc_sort_rejects_beyond_maximum():
    ctx = L.Context(0)
    lib = L.load_library()
    try:
        # real buffers of the right size: the size check must refuse before any work
        n = MAX_KEYS + 1
        dk, dv, dr = ctx.dev_alloc(n * 8), ctx.dev_alloc(n * 4), ctx.dev_alloc(10 * 8)
        passes = ctypes.c_int()
        try:
            rc = lib.gs_sort_tile_depth_noalloc(ctx.handle, ctypes.c_void_p(dk),
                                                ctypes.c_void_p(dv), ctypes.c_int64(n),
                                                ctypes.c_int64(10), ctypes.c_void_p(dr),
                                                ctypes.byref(passes))
        finally:
            for p in (dk, dv, dr):
                ctx.dev_free(p)
        assert rc == L.GS_E_CAPACITY
        assert "beyond" in lib.gs_last_error().decode()
    finally:
        ctx.close()
