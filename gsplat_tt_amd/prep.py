"""Order-preserving input preparation of a scene (host, once per scene).

* `opacity_prune` keeps the Gaussians whose opacity is not below min_opacity,
  in their order (render/opacity_prune.py:1-20): a Gaussian below the
  threshold is never visible (the projection's opacity test), so dropping it
  removes only bytes the projection would read per view. The projection
  compacts the visible Gaussians in source order, so the pruned scene's compact
  indices, depth-tie order, pairs and image are exactly the unpruned scene's.
* `morton_order` / `morton_reorder`: the stable argsort by a 30-bit Morton code
  (10 bits per axis over the 0.5-99.5 percentile box) of
  render/run.py:1011-1025, and the scene permuted by it, so that Gaussians near
  in space are near in memory (visible ones then share cache lines in the
  projection's reads). A reordered scene is a different input order: its
  render equals the reference's render of the same reordered scene (ties of
  equal depth follow the new order).
"""
from __future__ import annotations

import numpy as np


def opacity_keep_mask(opacities, min_opacity=1.0 / 255.0) -> np.ndarray:
    """True for the Gaussians the projection can keep: not (op < min_opacity)
    in fp32 (a NaN opacity passes the projection's test, so it is kept)."""
    op = np.asarray(opacities, np.float32).reshape(-1)
    return ~(op < np.float32(min_opacity))


def opacity_prune(arrays: dict, min_opacity=1.0 / 255.0, opacity_key="opacities") -> dict:
    """The per-Gaussian arrays (first axis = Gaussian) with the never-visible
    Gaussians removed, order kept."""
    keep = opacity_keep_mask(arrays[opacity_key], min_opacity)
    return {k: np.ascontiguousarray(np.asarray(v)[keep]) for k, v in arrays.items()}


def _spread10(x: np.ndarray) -> np.ndarray:
    """Bits 0..9 of x moved to bits 0, 3, 6, ..., 27."""
    x = x.astype(np.uint64)
    x = (x | (x << np.uint64(16))) & np.uint64(0x030000FF)
    x = (x | (x << np.uint64(8))) & np.uint64(0x0300F00F)
    x = (x | (x << np.uint64(4))) & np.uint64(0x030C30C3)
    x = (x | (x << np.uint64(2))) & np.uint64(0x09249249)
    return x


def morton_codes(means) -> np.ndarray:
    """30-bit Morton code per Gaussian: each axis quantised to 10 bits over its
    0.5-99.5 percentile range (clipped), x in bit 0, y in bit 1, z in bit 2."""
    m = np.nan_to_num(np.asarray(means, np.float64), nan=0.0, posinf=1e30, neginf=-1e30)
    lo = np.percentile(m, 0.5, axis=0)
    hi = np.percentile(m, 99.5, axis=0)
    u = np.clip((m - lo) / np.maximum(hi - lo, 1e-30), 0.0, 1.0)
    q = (u * 1023).astype(np.uint64)
    return _spread10(q[:, 0]) | (_spread10(q[:, 1]) << np.uint64(1)) | \
        (_spread10(q[:, 2]) << np.uint64(2))


def morton_order(means) -> np.ndarray:
    """Stable argsort of the Morton codes (int64 permutation)."""
    return np.argsort(morton_codes(means), kind="stable")


def morton_reorder(arrays: dict, means_key="means") -> tuple[dict, np.ndarray]:
    """(arrays permuted into Morton order, the permutation): new[i] = old[order[i]]."""
    order = morton_order(arrays[means_key])
    return {k: np.ascontiguousarray(np.asarray(v)[order]) for k, v in arrays.items()}, order
