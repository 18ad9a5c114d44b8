"""Oracle frames for the full-size parity tests: the reference pipeline's
intermediates (M, candidate pairs, tile-sorted ids, tile ranges) and image for
one view, from the reference's own CPU module where it was built (oracle/_ref,
multi-threaded: project_full_fused is restated by the C oracle, which is bit-exact
with it; tile_assign, sort and render_full are the reference's) and otherwise
from the single-threaded C oracle alone.

Test infrastructure only (imported by tests/)."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

FLOOR = 1.0 / 16384.0


def _bf16_to_f32(u16):
    return (np.asarray(u16).astype(np.uint32) << 16).view(np.float32)


def psnr(a, b):
    mse = float(np.mean((np.asarray(a, np.float64) - np.asarray(b, np.float64)) ** 2))
    return float("inf") if mse == 0 else 10 * np.log10(1.0 / mse)


def frame(means, cov9, opac, rgb, cam, ts, cull_disabled=False, use_isoellipse=False,
          want_image=True):
    """The reference's render_full (pybind_module.cpp:1149-1575) at its defaults,
    split so the intermediates can be compared: dict(project, M, pairs_pre, P,
    sorted_ids, tile_ranges, image f32 (H,W,3) or None, stats)."""
    H, W = cam.height, cam.width
    tx, ty = (W + ts - 1) // ts, (H + ts - 1) // ts
    pr = O.project(means, cov9, cam.w2c, cam.K, rgb, opac, H, W,
                   use_isoellipse=use_isoellipse)
    M = int(pr["depths"].shape[0])
    out = dict(project=pr, M=M, tiles=tx * ty)
    if M == 0:
        out.update(pairs_pre=0, P=0, sorted_ids=np.zeros(0, np.int64),
                   tile_ranges=np.zeros((tx * ty, 2), np.int64),
                   image=np.zeros((H, W, 3), np.float32), stats={})
        return out
    out["pairs_pre"] = O.tile_count(pr["means2d"], pr["radii"], H, W, ts)
    covs = None if cull_disabled else pr["covs2d"]
    ops = None if cull_disabled else pr["opacities"]
    R = O.ref_module()
    if R is not None:
        g, t, _ = R.tile_assign(pr["means2d"], pr["radii"], H, W, ts, covs, ops, FLOOR)
        s, r = R.sort(g, t, pr["depths"], tx, ty)
    else:
        g, t, _ = O.tile_assign(pr["means2d"], pr["radii"], H, W, ts, covs, ops, FLOOR)
        s, r = O.sort_and_bin(g, t, pr["depths"], tx, ty)
    out.update(P=int(s.shape[0]), sorted_ids=np.asarray(s, np.int64),
               tile_ranges=np.asarray(r, np.int64).reshape(tx * ty, 2))
    out["image"], out["stats"] = None, {}
    if want_image:
        if R is not None:
            img, st = R.render_full(means, cov9, opac, rgb, cam.w2c, cam.K, H, W, tile_size=ts,
                                    cull_disabled=cull_disabled,
                                    use_isoellipse=use_isoellipse)
        else:
            img, st = O.cull_and_blend(pr["means2d"], pr["covs2d"], pr["colors"],
                                       pr["opacities"], s, r, tx, ty, ts, H, W,
                                       cull_disabled=cull_disabled)
        out["image"], out["stats"] = np.asarray(img, np.float32), dict(st)
    return out


def check_frame(ctx, view, ref, img, st, bf16=True, label=""):
    """M, candidate pairs, P, tile-sorted ids and tile ranges of the GPU frame
    just rendered (gs_frame_readback) bit-exact against the oracle; the image
    within the stated tolerance (bf16: max-abs <= 2e-3 and PSNR >= 55 dB; f32:
    max-abs <= 1e-5)."""
    rb = ctx.frame_readback()
    print(f"{label}: M={rb['M']} pre={rb['pairs_pre']} P={rb['P']} "
          f"(oracle {ref['M']} {ref['pairs_pre']} {ref['P']})", flush=True)
    assert st["num_visible"] == ref["M"] and rb["M"] == ref["M"]
    assert rb["pairs_pre"] == ref["pairs_pre"]
    assert st["num_entries"] == ref["P"] and rb["P"] == ref["P"]
    assert np.array_equal(rb["tile_ranges"], ref["tile_ranges"])
    assert np.array_equal(rb["sorted_ids"], ref["sorted_ids"])
    if ref["image"] is not None:
        if bf16:
            g = _bf16_to_f32(img)
            d, p = float(np.abs(g - ref["image"]).max()), psnr(g, ref["image"])
            print(f"{label}: bf16 max_abs={d:.3g} psnr={p:.1f}", flush=True)
            assert d <= 2e-3 and p >= 55.0
        else:
            d = float(np.abs(img - ref["image"]).max())
            print(f"{label}: f32 max_abs={d:.3g}", flush=True)
            assert d <= 1e-5
    return rb
