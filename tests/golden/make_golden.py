"""Writes the golden vectors under tests/golden/ from the reference's own CPU
renderer (_gsplat_cpu.render_full and its stage functions, compiled from the
reference sources into oracle/_ref by oracle/Makefile). Run in a container that
has the reference checkout; the .npz files it writes are committed and are all
the tests read.

    make -C oracle ref && python tests/golden/make_golden.py

Also imports the reference's training-oracle dumps
(benchmarks/train_oracle/t0_sh{0,3}_64x64_n50.npz, fp64, written by
gsplat/train_oracle.py) with the per-pair `live` masks dropped.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

REF = "/root/reference"

# small C1/C2-shaped scenes (the full configs are exercised through invariants)
CASES = [
    dict(name="c1_n2000_128x96_ts16", kind="c1", n=2000, seed=101, H=96, W=128, ts=16),
    dict(name="c1_n2000_136x100_ts32", kind="c1", n=2000, seed=102, H=100, W=136, ts=32),
    dict(name="c2sh3_n1500_160x90_ts16", kind="c2", n=1500, seed=103, H=90, W=160, ts=16),
]


def _scene(case):
    from gsplat_tt_amd import scenes
    from oracle import oracle as O
    if case["kind"] == "c1":
        scene, cams = scenes.config1(seed=case["seed"], n=case["n"])
        cam = cams[0]
        f = 500.0 * case["W"] / 640.0
        K = scenes.intrinsics(f, f, case["W"] / 2, case["H"] / 2)
        return scene.means, scene.scales, scene.quats, scene.opacities, scene.colors, None, \
            cam.w2c, K
    scene, cams = scenes.config2(seed=case["seed"], n=case["n"])
    cam = cams[0]
    f = 0.5 * case["W"] / np.tan(np.deg2rad(25.0))
    K = scenes.intrinsics(f, f, case["W"] / 2, case["H"] / 2)
    rgb = O.sh_rgb(scene.means, scene.sh, 3, cam.w2c)
    return scene.means, scene.scales, scene.quats, scene.opacities, rgb, scene.sh, cam.w2c, K


def make_render_cases():
    from oracle import oracle as O
    R = O.ref_module()
    if R is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref)")
    for case in CASES:
        means, scales, quats, opac, rgb, sh, w2c, K = _scene(case)
        cov = np.asarray(R.compute_cov3d(scales, quats), np.float32).reshape(-1, 9)
        H, W, ts = case["H"], case["W"], case["ts"]
        img, st = R.render_full(means, cov, opac, rgb, w2c, K, H, W, tile_size=ts)
        m2, c2, d, r, v = R.project_full_with_cov3d(means, cov, w2c, K, H, W, opac)
        m2 = np.asarray(m2, np.float32).reshape(-1, 2)
        c2 = np.asarray(c2, np.float32).reshape(-1, 4)
        d = np.asarray(d, np.float32)
        r = np.asarray(r, np.float32).reshape(-1, 2)
        v = np.asarray(v).astype(bool)
        opv = opac[v]
        g, t, _ = R.tile_assign(m2, r, H, W, ts, c2, opv, 1.0 / 16384.0)
        tx, ty = (W + ts - 1) // ts, (H + ts - 1) // ts
        s, rr = R.sort(g, t, d, tx, ty)
        out = dict(
            means=means, cov3d=cov, opacities=opac, colors=np.asarray(rgb, np.float32),
            w2c=w2c, K=K, H=np.int32(H), W=np.int32(W), tile_size=np.int32(ts),
            image=np.asarray(img, np.float32), valid=v, means2d=m2, covs2d=c2, depths=d,
            radii=r, gaussian_ids=np.asarray(g, np.int64), tile_ids=np.asarray(t, np.int64),
            sorted_ids=np.asarray(s, np.int64),
            tile_ranges=np.asarray(rr, np.int64).reshape(-1, 2),
            stats=json.dumps({k: int(st[k]) for k in ("num_visible", "num_entries", "pairs_in",
                                                        "pairs_dropped", "pairs_kept_per_mb")}),
            params=json.dumps(dict(min_opacity=1 / 255, contrib_floor=1 / 16384,
                                   mb_contrib_floor=1 / 16384, cull_disabled=False,
                                   transmittance_threshold=1 / 255, max_radius=0, k_cap=3.0,
                                   use_isoellipse=False, generator=case)),
        )
        if sh is not None:
            out["sh"] = sh
        path = os.path.join(HERE, case["name"] + ".npz")
        np.savez_compressed(path, **out)
        print("wrote", path, json.loads(out["stats"]))


def import_train_fixtures():
    src = os.path.join(REF, "benchmarks", "train_oracle")
    for deg in (0, 3):
        name = f"t0_sh{deg}_64x64_n50.npz"
        d = np.load(os.path.join(src, name), allow_pickle=False)
        keep = {k: d[k] for k in d.files if k != "live"}
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **keep)
        print("wrote", path, len(keep), "arrays")


if __name__ == "__main__":
    make_render_cases()
    import_train_fixtures()
