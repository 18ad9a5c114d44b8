"""3D Gaussian scenes from .ply files, with the reference's activations.

gsplat/loading_gaussians.py:32-65 reads a trained scene with `plyfile` and
activates the optimizer-space parameters: scales = exp(scale_i), rotations =
rot_i / |rot| (w x y z), colours = clamp(0.5 + C0 * f_dc_i, 0, 1) with
C0 = 1 / (2 sqrt(pi)), opacities = sigmoid(opacity). `plyfile` is not a
dependency here: this module parses the PLY header itself and reads the vertex
element with one numpy structured read (binary little/big endian) or a text
parse (ascii).

Beyond the reference, the higher-order SH coefficients (f_rest_*, stored
channel-major: all of red, then green, then blue) are returned as `sh`
(N, (d+1)^2, 3), coefficient-major, which is the colour layout the GPU renderer
evaluates per view (render_view / Context.set_scene with sh_degree=d).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SH_C0 = 0.28209479177387814

_PLY_TYPES = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}


@dataclass
class Gaussians:
    """Activated Gaussians, the fields of gsplat/data_structures.py's Gaussians
    as float32 numpy arrays, plus the SH coefficients when the file has them."""
    means: np.ndarray       # (N, 3)
    scales: np.ndarray      # (N, 3), exp of the stored log-scales
    rotations: np.ndarray   # (N, 4) unit quaternions, w x y z
    colors: np.ndarray      # (N, 3) in [0, 1] from the SH DC term
    opacities: np.ndarray   # (N,) sigmoid of the stored logits
    sh: np.ndarray | None = None  # (N, (d+1)^2, 3) raw SH coefficients (DC first)

    @property
    def num_gaussians(self) -> int:
        return int(self.means.shape[0])

    @property
    def sh_degree(self) -> int:
        return -1 if self.sh is None else int(round(np.sqrt(self.sh.shape[1]))) - 1


def _parse_header(f):
    """(format, [(element name, count, [(property, numpy type)])], header bytes)."""
    first = f.readline()
    if first.strip() != b"ply":
        raise ValueError("not a PLY file (no 'ply' magic line)")
    fmt, elements = None, []
    while True:
        line = f.readline()
        if not line:
            raise ValueError("PLY header has no end_header line")
        tok = line.decode("ascii", "replace").split()
        if not tok or tok[0] in ("comment", "obj_info"):
            continue
        if tok[0] == "end_header":
            break
        if tok[0] == "format":
            fmt = tok[1]
            if fmt not in ("binary_little_endian", "binary_big_endian", "ascii"):
                raise ValueError(f"unsupported PLY format {fmt!r}")
        elif tok[0] == "element":
            elements.append((tok[1], int(tok[2]), []))
        elif tok[0] == "property":
            if not elements:
                raise ValueError("PLY property before any element")
            if tok[1] == "list":
                elements[-1][2].append((tok[-1], None))
            else:
                if tok[1] not in _PLY_TYPES:
                    raise ValueError(f"unsupported PLY property type {tok[1]!r}")
                elements[-1][2].append((tok[2], _PLY_TYPES[tok[1]]))
    if fmt is None:
        raise ValueError("PLY header has no format line")
    return fmt, elements


def read_ply(path: str) -> dict:
    """The properties of the file's first element (the vertices), as a dict of
    1-D numpy arrays in their stored types."""
    with open(path, "rb") as f:
        fmt, elements = _parse_header(f)
        if not elements:
            raise ValueError("PLY file has no elements")
        name, count, props = elements[0]
        if any(t is None for _, t in props):
            raise ValueError(f"list properties in element {name!r} are not supported")
        if fmt == "ascii":
            rows = np.loadtxt(f, dtype=np.float64, max_rows=count, ndmin=2)
            if rows.shape != (count, len(props)):
                raise ValueError(f"PLY element {name!r}: expected {count} rows of "
                                 f"{len(props)} values")
            return {p: rows[:, i].astype(t) for i, (p, t) in enumerate(props)}
        order = "<" if fmt == "binary_little_endian" else ">"
        dt = np.dtype([(p, order + t) for p, t in props])
        data = np.fromfile(f, dtype=dt, count=count)
        if data.shape[0] != count:
            raise ValueError(f"PLY element {name!r}: file holds {data.shape[0]} of {count} rows")
        return {p: data[p] for p, _ in props}


def _stack(v, names):
    missing = [n for n in names if n not in v]
    if missing:
        raise ValueError(f"PLY vertex element lacks {', '.join(missing)}")
    return np.stack([np.asarray(v[n], np.float32) for n in names], axis=-1)


def load_ply(path: str) -> Gaussians:
    """gsplat/loading_gaussians.py:32-65 load_ply: the activated Gaussians of a
    trained scene (float32, through the same fp32 torch CPU ops)."""
    v = read_ply(path)
    means = _stack(v, ["x", "y", "z"])
    log_scales = _stack(v, ["scale_0", "scale_1", "scale_2"])
    rot = _stack(v, ["rot_0", "rot_1", "rot_2", "rot_3"])
    dc = _stack(v, ["f_dc_0", "f_dc_1", "f_dc_2"])
    if "opacity" not in v:
        raise ValueError("PLY vertex element lacks opacity")
    # contiguous, as the reference's torch.tensor(np.array(...)) copy is: torch's
    # CPU kernels can round differently on strided inputs
    logit = np.ascontiguousarray(v["opacity"], np.float32)

    # the reference's own fp32 CPU ops (torch), so the activated values are its
    # values bit for bit (numpy's exp differs from torch's in the last bit for
    # about a third of the inputs)
    import torch
    T = torch.from_numpy
    scales = torch.exp(T(log_scales)).numpy()
    q = T(rot)
    rotations = (q / q.norm(dim=-1, keepdim=True)).numpy()
    colors = torch.clamp(0.5 + SH_C0 * T(dc), 0.0, 1.0).numpy()
    opacities = torch.sigmoid(T(logit)).numpy()

    rest = sorted((k for k in v if k.startswith("f_rest_")), key=lambda k: int(k[7:]))
    sh = None
    if rest:
        if len(rest) % 3 != 0 or rest != [f"f_rest_{i}" for i in range(len(rest))]:
            raise ValueError("f_rest_* properties must be f_rest_0 .. f_rest_{3m-1}")
        K = len(rest) // 3 + 1
        if K not in (4, 9, 16):
            raise ValueError(f"{len(rest)} f_rest_* properties: not an SH degree 1-3 set")
        r = _stack(v, rest).reshape(-1, 3, K - 1)       # channel-major on file
        sh = np.empty((means.shape[0], K, 3), np.float32)
        sh[:, 0, :] = dc
        sh[:, 1:, :] = r.transpose(0, 2, 1)
    return Gaussians(means=means, scales=scales.astype(np.float32),
                     rotations=rotations.astype(np.float32), colors=colors.astype(np.float32),
                     opacities=opacities, sh=sh)


def write_ply(path: str, arrays: dict, fmt: str = "binary_little_endian") -> None:
    """Writes one vertex element of float32 properties (name -> (N,) array), in
    the layout 3DGS scenes use; the inverse of read_ply for such files."""
    names = list(arrays)
    n = int(np.asarray(arrays[names[0]]).shape[0])
    head = ["ply", f"format {fmt} 1.0", f"element vertex {n}"]
    head += [f"property float {k}" for k in names]
    head.append("end_header")
    with open(path, "wb") as f:
        f.write(("\n".join(head) + "\n").encode("ascii"))
        cols = np.stack([np.asarray(arrays[k], np.float32) for k in names], axis=-1)
        if fmt == "ascii":
            np.savetxt(f, cols, fmt="%.9g")
        else:
            f.write(cols.astype("<f4" if fmt == "binary_little_endian" else ">f4").tobytes())
