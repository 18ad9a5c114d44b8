"""The CPU oracle against the reference's own known-answer tests (restated in
tests/kat_cases.py) and against closed forms the mathematics fixes."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests import kat_cases


class OracleBackend:
    project = staticmethod(O.project)

    @staticmethod
    def tile_assign(means2d, radii, H, W, ts, covs2d, opac, floor):
        return O.tile_assign(means2d, radii, H, W, ts, covs2d, opac, float(floor))

    @staticmethod
    def sort_and_bin(gids, tids, depths, tx, ty):
        return O.sort_and_bin(np.asarray(gids, np.int64), np.asarray(tids, np.int64), depths,
                              tx, ty)

    @staticmethod
    def blend(means2d, covs2d, colors, opac, s, r, tx, ty, ts, H, W):
        img, _ = O.cull_and_blend(means2d, covs2d, colors, opac, s, r, tx, ty, ts, H, W)
        return img


@pytest.mark.parametrize("case", kat_cases.ALL, ids=lambda f: f.__name__[4:])
def test_oracle_kat(case):
    case(OracleBackend)


def test_exp4_closed_forms():
    """simd_exp_avx2.h:12-32: exact at 0, within the degree-4 Maclaurin bound
    |r|^5/120 * e^r (|r| <= ln2/2) relative error over [-30, 0]."""
    assert O.exp4(0.0) == 1.0
    for x in np.linspace(-30.0, 0.0, 2001, dtype=np.float32):
        e = math.exp(float(x))
        assert abs(O.exp4(float(x)) - e) <= e * 6e-5 + 1e-30, x


def test_cov3d_closed_form():
    """types.h:68-97: identity rotation gives diag(s^2); a 90-degree turn about z
    swaps the x and y variances."""
    s = np.array([[1.0, 2.0, 3.0], [1.0, 2.0, 3.0]], np.float32)
    h = np.float32(math.sqrt(0.5))
    q = np.array([[1, 0, 0, 0], [h, 0, 0, h]], np.float32)
    c = O.cov3d(s, q).reshape(2, 3, 3)
    assert np.array_equal(c[0], np.diag([1.0, 4.0, 9.0]).astype(np.float32))
    assert np.allclose(c[1], np.diag([4.0, 1.0, 9.0]), atol=1e-5)
    assert np.allclose(c[1], c[1].T)


def test_sh_degree0_closed_form():
    """Degree 0: rgb = C0 * dc + 0.5, independent of the view direction."""
    rng = np.random.default_rng(0)
    means = rng.normal(size=(64, 3)).astype(np.float32)
    sh = rng.normal(size=(64, 1, 3)).astype(np.float32)
    rgb = O.sh_rgb(means, sh, 0, np.eye(4, dtype=np.float32), clamp_hi=False)
    want = np.maximum(np.float32(0.28209479177387814) * sh[:, 0, :] + np.float32(0.5), 0)
    assert np.allclose(rgb, want, atol=1e-7)


def test_tile_assign_cull_vs_brute_force():
    """The per-pair cull keeps a pair iff the minimum Mahalanobis distance over the
    tile's closed rectangle is within the opacity threshold (tile_assign.cpp:151-290);
    brute force: dense sampling of the rectangle in float64."""
    rng = np.random.default_rng(3)
    H = W = 128
    ts = 16
    n = 40
    m2 = rng.uniform(10, 118, size=(n, 2)).astype(np.float32)
    a = rng.uniform(4, 60, size=n)
    c = rng.uniform(4, 60, size=n)
    b = rng.uniform(-0.8, 0.8, size=n) * np.sqrt(a * c)
    cov = np.stack([a, b, b, c], 1).astype(np.float32)
    op = rng.uniform(0.05, 1.0, size=n).astype(np.float32)
    radii = np.ceil(3 * np.sqrt(np.stack([a, c], 1))).astype(np.float32)
    floor = 1.0 / 255.0
    g_all, t_all, _ = O.tile_assign(m2, radii, H, W, ts, None, None, floor)
    g, t, _ = O.tile_assign(m2, radii, H, W, ts, cov, op, floor)
    kept = set(zip(g.tolist(), t.tolist()))
    tx = W // ts
    mismatches = 0
    for gi, ti in zip(g_all.tolist(), t_all.tolist()):
        A, Bc, C = (float(v) for v in (cov[gi, 0], cov[gi, 1], cov[gi, 3]))
        det = A * C - Bc * Bc
        ia, ib, ic = C / det, -Bc / det, A / det
        x0, y0 = (ti % tx) * ts, (ti // tx) * ts
        us = np.linspace(x0, x0 + ts, 129) - float(m2[gi, 0])
        vs = np.linspace(y0, y0 + ts, 129) - float(m2[gi, 1])
        U, V = np.meshgrid(us, vs)
        m2min = float(np.min(ia * U * U + 2 * ib * U * V + ic * V * V))
        thr = -2.0 * math.log(floor / float(op[gi])) if op[gi] > floor else -1.0
        want = m2min <= thr
        # sampling over-estimates the minimum slightly: only count clear disagreements
        if want != ((gi, ti) in kept) and abs(m2min - thr) > 1e-2 * max(thr, 1.0):
            mismatches += 1
    assert mismatches == 0


def test_pack_u8_matches_reference_header():
    """oracle.pack_u8 (bf16 round-to-nearest-even, then float clip * 255 with
    truncation) against the reference's integer rule compiled from its own header
    (render/kernels/dataflow/img_pack_u8.h:31-41, via oracle/img_pack_u8_dump.cpp)
    for every bf16 pattern except NaN, plus fixed points of the rule."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(O.__file__), "_ref", "img_pack_u8_dump")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/img_pack_u8_dump not built (reference sources absent)")
    ref = np.array(subprocess.run([exe], check=True, capture_output=True,
                                  text=True).stdout.split(), np.int64)
    assert ref.shape == (65536,)
    bits = np.arange(65536, dtype=np.uint32)
    f = (bits << 16).view(np.float32)
    ok = ~np.isnan(f)
    got = O.pack_u8(f).astype(np.int64)   # a bf16 value rounds to itself
    assert np.array_equal(got[ok], ref[ok])
    # fixed points: 1.0 -> 255, 0.5 -> 127 (truncation), negatives and tiny -> 0
    assert list(O.pack_u8(np.array([1.0, 0.5, -0.25, 1e-3, 2.0], np.float32))) == \
        [255, 127, 0, 0, 255]
    # rounding to bf16 happens first: 0.99999 rounds up to 1.0 -> 255
    assert O.pack_u8(np.array([0.99999], np.float32))[0] == 255
