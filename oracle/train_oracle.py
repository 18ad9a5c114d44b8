"""CPU oracle of the training step (forward with 3DGS blend rules, L1 gradient,
blend backward, projection backward, sparse Adam), in numpy.

TEST INFRASTRUCTURE ONLY: imported by tests/ (and nothing in the product), as the
checker of the HIP training path. A restatement of the reference's training
oracle gsplat/train_oracle.py (torch autograd, fp64) with the gradients written
out analytically:

  * forward: train_oracle.py:125-233 (projection, SH colour clamped at 0 only,
    3-sigma visibility for sparse Adam, per-pixel front-to-back blend: skip
    alpha < alpha_min, stop - without blending - when T * (1 - alpha) < t_min,
    alpha clamp alpha_max, out = C + T * background);
  * L1 gradient: train_loss.py:166-171 (mean |x - y| over 3HW, sign(0) = 0; the
    reference's device step also scales it by 1 - lambda_dssim = 0.8, here a
    `scale` argument);
  * full 3DGS loss (1 - lambda) L1 + lambda (1 - SSIM): train_oracle.py:253-279
    (11-tap Gaussian window, sigma 1.5, zero padding, C1 = 0.01^2,
    C2 = 0.03^2, mean over 3HW) with the analytic image gradient of
    train_loss.py:5-19 (fused-SSIM form: three filtered maps forward, three
    backward);
  * blend backward: the reverse recursion over each pixel's live pairs;
  * projection backward: conic -> cov2d -> (J, cov3d) -> means / log-scales /
    quaternions, opacity logit, SH coefficients and the SH view direction;
  * sparse Adam: train_oracle.py:434-470 (visible rows only, bias correction
    with step + 1 for every row).

Pinned against the reference's dumps (tests/golden/t0_sh{0,3}_64x64_n50.npz:
forward arrays, the full loss and its image gradient, 2D gradients, parameter
gradients, fp32 Adam outputs) and against central finite differences
(tests/test_train_oracle.py).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

SH_C0 = 0.28209479177387814
SH_C1 = 0.4886025119029199
SH_C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005,
         -1.0925484305920792, 0.5462742152960396)
SH_C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658,
         0.3731763325901154, -0.4570457994644658, 1.445305721320277,
         -0.5900435899266435)
PARAM_NAMES = ("means", "log_scales", "quats", "opacity_logits", "sh")
DEFAULT_LR = {"means": 1.6e-4, "log_scales": 5e-3, "quats": 1e-3, "opacity_logits": 0.05,
              "sh_dc": 2.5e-3, "sh_rest": 2.5e-3 / 20.0}


@dataclass
class Cfg:
    """train_oracle.py:63-71 RenderConfig."""
    sh_degree: int = 0
    near: float = 0.2
    lowpass: float = 0.3
    alpha_max: float = 0.99
    alpha_min: float = 1.0 / 255.0
    t_min: float = 1e-4
    background: tuple = (0.0, 0.0, 0.0)


# ------------------------------------------------------------------ SH
def sh_basis(d, degree):
    """(N, (degree+1)^2) real SH basis of unit directions d (N,3) and its gradient
    (N, K, 3) with respect to d, the basis taken as a polynomial in (x, y, z)."""
    x, y, z = d[:, 0], d[:, 1], d[:, 2]
    n = d.shape[0]
    K = (degree + 1) ** 2
    b = np.zeros((n, K), d.dtype)
    g = np.zeros((n, K, 3), d.dtype)
    b[:, 0] = SH_C0
    if degree >= 1:
        b[:, 1], g[:, 1, 1] = -SH_C1 * y, -SH_C1
        b[:, 2], g[:, 2, 2] = SH_C1 * z, SH_C1
        b[:, 3], g[:, 3, 0] = -SH_C1 * x, -SH_C1
    if degree >= 2:
        xx, yy, zz = x * x, y * y, z * z
        c = SH_C2
        b[:, 4] = c[0] * x * y
        g[:, 4] = np.stack([c[0] * y, c[0] * x, 0 * x], 1)
        b[:, 5] = c[1] * y * z
        g[:, 5] = np.stack([0 * x, c[1] * z, c[1] * y], 1)
        b[:, 6] = c[2] * (2 * zz - xx - yy)
        g[:, 6] = np.stack([-2 * c[2] * x, -2 * c[2] * y, 4 * c[2] * z], 1)
        b[:, 7] = c[3] * x * z
        g[:, 7] = np.stack([c[3] * z, 0 * x, c[3] * x], 1)
        b[:, 8] = c[4] * (xx - yy)
        g[:, 8] = np.stack([2 * c[4] * x, -2 * c[4] * y, 0 * x], 1)
    if degree >= 3:
        c = SH_C3
        b[:, 9] = c[0] * y * (3 * xx - yy)
        g[:, 9] = np.stack([6 * c[0] * x * y, c[0] * (3 * xx - 3 * yy), 0 * x], 1)
        b[:, 10] = c[1] * x * y * z
        g[:, 10] = np.stack([c[1] * y * z, c[1] * x * z, c[1] * x * y], 1)
        b[:, 11] = c[2] * y * (4 * zz - xx - yy)
        g[:, 11] = np.stack([-2 * c[2] * x * y, c[2] * (4 * zz - xx - 3 * yy),
                             8 * c[2] * y * z], 1)
        b[:, 12] = c[3] * z * (2 * zz - 3 * xx - 3 * yy)
        g[:, 12] = np.stack([-6 * c[3] * x * z, -6 * c[3] * y * z,
                             c[3] * (6 * zz - 3 * xx - 3 * yy)], 1)
        b[:, 13] = c[4] * x * (4 * zz - xx - yy)
        g[:, 13] = np.stack([c[4] * (4 * zz - 3 * xx - yy), -2 * c[4] * x * y,
                             8 * c[4] * x * z], 1)
        b[:, 14] = c[5] * z * (xx - yy)
        g[:, 14] = np.stack([2 * c[5] * x * z, -2 * c[5] * y * z, c[5] * (xx - yy)], 1)
        b[:, 15] = c[6] * x * (xx - 3 * yy)
        g[:, 15] = np.stack([c[6] * (3 * xx - 3 * yy), -6 * c[6] * x * y, 0 * x], 1)
    return b, g


# ------------------------------------------------------------------ forward
def quat_rot(q):
    """Rotation matrices (N,3,3) of unit quaternions (w, x, y, z) (types.h:68-85)."""
    w, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    return np.stack([
        np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        np.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        np.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], 1)


def project(params, w2c, K, H, W, cfg: Cfg, dtype=np.float64):
    """Per-Gaussian forward values (train_oracle.py:125-181)."""
    f = lambda a: np.asarray(a, dtype)  # noqa: E731
    m, ls, qr, ol, sh = (f(params[k]) for k in PARAM_NAMES)
    R, t = f(w2c)[:3, :3], f(w2c)[:3, 3]
    fx, fy, cx, cy = f(K)[0, 0], f(K)[1, 1], f(K)[0, 2], f(K)[1, 2]
    pc = m @ R.T + t
    x, y, z = pc[:, 0], pc[:, 1], pc[:, 2]
    valid = z > cfg.near
    zs = np.where(valid, z, 1.0)
    means2d = np.stack([fx * x / zs + cx, fy * y / zs + cy], -1)
    qn_norm = np.sqrt((qr * qr).sum(1))
    q = qr / qn_norm[:, None]
    Rq = quat_rot(q)
    s = np.exp(ls)
    Mx = Rq * s[:, None, :]
    cov3 = Mx @ np.transpose(Mx, (0, 2, 1))
    J = np.zeros((m.shape[0], 2, 3), dtype)
    J[:, 0, 0] = fx / zs
    J[:, 0, 2] = -fx * x / (zs * zs)
    J[:, 1, 1] = fy / zs
    J[:, 1, 2] = -fy * y / (zs * zs)
    T = J @ R
    cov2 = T @ cov3 @ np.transpose(T, (0, 2, 1))
    a = cov2[:, 0, 0] + cfg.lowpass
    b = cov2[:, 0, 1]
    c = cov2[:, 1, 1] + cfg.lowpass
    det = a * c - b * b
    conic = np.stack([c / det, -b / det, a / det], -1)
    cc = -R.T @ t
    dvec = m - cc
    dn = np.sqrt((dvec * dvec).sum(1))
    d = dvec / dn[:, None]
    basis, dbasis = sh_basis(d, cfg.sh_degree)
    raw = np.einsum("nk,nkc->nc", basis, sh[:, :basis.shape[1], :]) + 0.5
    colors = np.where(raw < 0.0, 0.0, raw)
    op = 1.0 / (1.0 + np.exp(-ol))
    rx = np.ceil(3.0 * np.sqrt(np.maximum(a, 0.0)))
    ry = np.ceil(3.0 * np.sqrt(np.maximum(c, 0.0)))
    visible = (valid & (means2d[:, 0] + rx > 0) & (means2d[:, 0] - rx < W)
               & (means2d[:, 1] + ry > 0) & (means2d[:, 1] - ry < H))
    return dict(pc=pc, valid=valid, means2d=means2d, q=q, qnorm=qn_norm, Rq=Rq, s=s, M=Mx,
                cov3=cov3, J=J, T=T, R=R, fx=fx, fy=fy, a=a, b=b, c=c, conic=conic, d=d,
                dnorm=dn, basis=basis, dbasis=dbasis, raw=raw, colors=colors, opacity=op,
                depth=z, visible=visible, sh=sh)


def blend_forward(pr, H, W, cfg: Cfg):
    """Per-pixel front-to-back blend with the 3DGS rules (train_oracle.py:183-233).
    Returns image, final T, depth order and the live mask (N, H*W)."""
    dt = pr["means2d"].dtype
    N = pr["means2d"].shape[0]
    order = np.argsort(pr["depth"], kind="stable")
    py, px = np.meshgrid(np.arange(H, dtype=dt) + 0.5, np.arange(W, dtype=dt) + 0.5,
                         indexing="ij")
    px, py = px.reshape(-1), py.reshape(-1)
    P = H * W
    T = np.ones(P, dt)
    C = np.zeros((P, 3), dt)
    alive = np.ones(P, bool)
    live_all = np.zeros((N, P), bool)
    for g in order:
        if not pr["valid"][g]:
            continue
        A, B, Cc = pr["conic"][g]
        dx = px - pr["means2d"][g, 0]
        dy = py - pr["means2d"][g, 1]
        power = -0.5 * (A * dx * dx + 2.0 * B * dx * dy + Cc * dy * dy)
        alpha = np.minimum(pr["opacity"][g] * np.exp(np.minimum(power, 0.0)), cfg.alpha_max)
        live = alive & (alpha >= cfg.alpha_min)
        stop = live & (T * (1.0 - alpha) < cfg.t_min)
        live &= ~stop
        alive &= ~stop
        live_all[g] = live
        a_eff = np.where(live, alpha, 0.0)
        C += (a_eff * T)[:, None] * pr["colors"][g]
        T = T * (1.0 - a_eff)
    image = (C + T[:, None] * np.asarray(cfg.background, dt)).reshape(H, W, 3)
    return image, T.reshape(H, W), order, live_all


def forward(params, w2c, K, H, W, cfg: Cfg, dtype=np.float64):
    pr = project(params, w2c, K, H, W, cfg, dtype)
    image, final_T, order, live = blend_forward(pr, H, W, cfg)
    return pr, image, final_T, order, live


# ------------------------------------------------------------------ loss
def l1_loss_grad(image, target, scale=1.0):
    """mean |x - y| over 3HW and its gradient sign(x - y) * scale / (3HW)
    (train_loss.py:166-171; torch sign(0) = 0)."""
    n = image.size
    d = image - target
    return scale * float(np.abs(d).sum() / n), scale * np.sign(d) / n


# ------------------------------------------------------------------ backward
SSIM_WIN, SSIM_SIGMA = 11, 1.5
SSIM_C1, SSIM_C2 = 0.01 ** 2, 0.03 ** 2


def gauss_window(size=SSIM_WIN, sigma=SSIM_SIGMA):
    """Normalised 1D Gaussian taps (train_oracle.py:240-243)."""
    x = np.arange(size, dtype=np.float64) - size // 2
    g = np.exp(-(x * x) / (2.0 * sigma * sigma))
    return g / g.sum()


def gauss_filter(z, size=SSIM_WIN, sigma=SSIM_SIGMA):
    """Separable Gaussian filter of (H, W, ...) arrays with zero padding: the
    banded-matrix form G_h @ z @ G_w^T of train_oracle.py:246-266."""
    g = gauss_window(size, sigma)
    r = size // 2
    z = np.asarray(z, np.float64)
    H, W = z.shape[:2]
    zp = np.zeros((H + 2 * r, W) + z.shape[2:])
    zp[r:r + H] = z
    t = sum(g[k] * zp[k:k + H] for k in range(size))
    tp = np.zeros((H, W + 2 * r) + z.shape[2:])
    tp[:, r:r + W] = t
    return sum(g[k] * tp[:, k:k + W] for k in range(size))


def ssim_loss_grad(image, target, lambda_dssim=0.2):
    """(loss, l1, ssim, dL/dimage) of loss = (1 - lambda) mean|x - y| +
    lambda (1 - SSIM(x, y)) (train_oracle.py:269-279), fp64; the gradient is the
    analytic fused-SSIM form (train_loss.py:5-19): with S = A B / (C D),
    dL/dx = (1 - lambda) sign(x - y)/n + G*(w dS/dmu_x) + 2 x G*(w dS/dE_xx)
    + y G*(w dS/dE_xy), w = -lambda / n, n = 3HW (G is symmetric)."""
    x = np.asarray(image, np.float64)
    y = np.asarray(target, np.float64)
    n = float(x.size)
    mu_x, mu_y = gauss_filter(x), gauss_filter(y)
    e_xx, e_yy, e_xy = gauss_filter(x * x), gauss_filter(y * y), gauss_filter(x * y)
    A = 2.0 * mu_x * mu_y + SSIM_C1
    B = 2.0 * (e_xy - mu_x * mu_y) + SSIM_C2
    C = mu_x * mu_x + mu_y * mu_y + SSIM_C1
    D = (e_xx - mu_x * mu_x) + (e_yy - mu_y * mu_y) + SSIM_C2
    S = (A * B) / (C * D)
    w = -lambda_dssim / n
    d_mu = w * S * (2.0 * mu_y / A - 2.0 * mu_y / B - 2.0 * mu_x / C + 2.0 * mu_x / D)
    d_xx = -w * S / D
    d_xy = 2.0 * w * S / B
    grad = gauss_filter(d_mu) + 2.0 * x * gauss_filter(d_xx) + y * gauss_filter(d_xy)
    grad = grad + (1.0 - lambda_dssim) * np.sign(x - y) / n
    l1 = float(np.abs(x - y).sum() / n)
    ssim = float(S.sum() / n)
    loss = (1.0 - lambda_dssim) * l1 + lambda_dssim * (1.0 - ssim)
    return loss, l1, ssim, grad


def blend_backward(pr, order, live, final_T, dL_dimage, H, W, cfg: Cfg):
    """dL/d(means2d, conic, opacity, colors) of the blend with the forward's
    decisions (live pairs, alpha clamp) held fixed, by the reverse recursion per
    pixel: T_i = T_{i+1} / (1 - alpha_i); behind_i = alpha_{i+1} c_{i+1} +
    (1 - alpha_{i+1}) behind_{i+1}; dL/dalpha_i = T_i (c_i - behind_i) . g
    - T_final bg . g / (1 - alpha_i); dL/dc_i = alpha_i T_i g."""
    dt = pr["means2d"].dtype
    N = pr["means2d"].shape[0]
    py, px = np.meshgrid(np.arange(H, dtype=dt) + 0.5, np.arange(W, dtype=dt) + 0.5,
                         indexing="ij")
    px, py = px.reshape(-1), py.reshape(-1)
    g = dL_dimage.reshape(-1, 3).astype(dt)
    bg_dot = g @ np.asarray(cfg.background, dt)
    T = final_T.reshape(-1).astype(dt).copy()
    behind = np.zeros((H * W, 3), dt)
    d_m2 = np.zeros((N, 2), dt)
    d_con = np.zeros((N, 3), dt)
    d_op = np.zeros(N, dt)
    d_col = np.zeros((N, 3), dt)
    Tfin = T.copy()
    for gi in order[::-1]:
        lv = live[gi]
        if not lv.any():
            continue
        A, B, Cc = pr["conic"][gi]
        dx = px - pr["means2d"][gi, 0]
        dy = py - pr["means2d"][gi, 1]
        power = -0.5 * (A * dx * dx + 2.0 * B * dx * dy + Cc * dy * dy)
        wgt = np.exp(np.minimum(power, 0.0))
        raw = pr["opacity"][gi] * wgt
        clamp = raw > cfg.alpha_max
        alpha = np.where(clamp, cfg.alpha_max, raw)
        Ti = np.where(lv, T / (1.0 - alpha), T)
        col = pr["colors"][gi]
        dalpha = Ti * ((col[None, :] - behind) * g).sum(1) - Tfin * bg_dot / (1.0 - alpha)
        d_col[gi] = np.where(lv[:, None], (alpha * Ti)[:, None] * g, 0.0).sum(0)
        act = lv & ~clamp
        d_op[gi] = np.where(act, dalpha * wgt, 0.0).sum()
        dpow = np.where(act & (power <= 0.0), dalpha * raw, 0.0)
        # power = -0.5 (A dx^2 + 2B dx dy + C dy^2), dx = px - mx
        d_m2[gi, 0] = (dpow * (A * dx + B * dy)).sum()
        d_m2[gi, 1] = (dpow * (B * dx + Cc * dy)).sum()
        d_con[gi, 0] = (dpow * -0.5 * dx * dx).sum()
        d_con[gi, 1] = (dpow * -dx * dy).sum()
        d_con[gi, 2] = (dpow * -0.5 * dy * dy).sum()
        behind = np.where(lv[:, None], alpha[:, None] * col[None, :]
                          + (1.0 - alpha)[:, None] * behind, behind)
        T = Ti
    return dict(dL_dmeans2d=d_m2, dL_dconic=d_con, dL_dopacity=d_op, dL_dcolors=d_col)


def _dR_dq(q):
    """(N, 4, 3, 3): derivative of quat_rot with respect to each of (w, x, y, z)."""
    w, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    o = 0 * w
    m = lambda r: np.stack([np.stack(row, -1) for row in r], 1)  # noqa: E731
    dw = m([[o, -z, y], [z, o, -x], [-y, x, o]])
    dx = m([[o, y, z], [y, -2 * x, -w], [z, w, -2 * x]])
    dy = m([[-2 * y, x, w], [x, o, z], [-w, z, -2 * y]])
    dz = m([[-2 * z, -w, x], [w, -2 * z, y], [x, y, o]])
    return 2.0 * np.stack([dw, dx, dy, dz], 1)


def projection_backward(pr, g2, cfg: Cfg):
    """Optimizer-space gradients from the 2D ones (g2: dL_dmeans2d (N,2),
    dL_dconic (N,3), dL_dopacity (N,), dL_dcolors (N,3)); rows outside the
    near plane get none."""
    gA, gB, gC = (g2["dL_dconic"][:, i] for i in range(3))
    A, B, Cc = (pr["conic"][:, i] for i in range(3))
    # Q = inv(S2); dL/dS2 = -Q Gq Q with Gq = [[gA, gB/2], [gB/2, gC]]
    Q = np.stack([np.stack([A, B], -1), np.stack([B, Cc], -1)], 1)
    Gq = np.stack([np.stack([gA, 0.5 * gB], -1), np.stack([0.5 * gB, gC], -1)], 1)
    G2 = -Q @ Gq @ Q                       # symmetric dL/dS2 with S2 = T cov3 T^T + lp
    Tm, cov3, R = pr["T"], pr["cov3"], pr["R"]
    G3 = np.transpose(Tm, (0, 2, 1)) @ G2 @ Tm        # dL/dcov3
    dT = 2.0 * G2 @ Tm @ cov3                          # dL/dT
    dJ = dT @ R.T                                      # T = J R
    x, y, z = (pr["pc"][:, i] for i in range(3))
    fx, fy = pr["fx"], pr["fy"]
    gu, gv = g2["dL_dmeans2d"][:, 0], g2["dL_dmeans2d"][:, 1]
    iz = 1.0 / np.where(pr["valid"], z, 1.0)
    gx = gu * fx * iz + dJ[:, 0, 2] * (-fx * iz * iz)
    gy = gv * fy * iz + dJ[:, 1, 2] * (-fy * iz * iz)
    gz = (gu * (-fx * x * iz * iz) + gv * (-fy * y * iz * iz)
          + dJ[:, 0, 0] * (-fx * iz * iz) + dJ[:, 1, 1] * (-fy * iz * iz)
          + dJ[:, 0, 2] * (2.0 * fx * x * iz ** 3) + dJ[:, 1, 2] * (2.0 * fy * y * iz ** 3))
    v = pr["valid"]
    gpc = np.where(v[:, None], np.stack([gx, gy, gz], 1), 0.0)
    gmeans = gpc @ R                                   # pc = R m + t
    # cov3 = M M^T, M = Rq diag(s)
    Mx, Rq, s = pr["M"], pr["Rq"], pr["s"]
    dM = 2.0 * G3 @ Mx
    gs = (dM * Rq).sum(1)
    gls = gs * s
    gR = dM * s[:, None, :]
    gq_unit = np.einsum("nkij,nij->nk", _dR_dq(pr["q"]), gR)
    q = pr["q"]
    gq = (gq_unit - q * (q * gq_unit).sum(1, keepdims=True)) / pr["qnorm"][:, None]
    gq = np.where(v[:, None], gq, 0.0)
    gls = np.where(v[:, None], gls, 0.0)
    op = pr["opacity"]
    gol = g2["dL_dopacity"] * op * (1.0 - op)
    # colour = max(SH(d) + 0.5, 0): passes where raw >= 0
    gcol = np.where(pr["raw"] >= 0.0, g2["dL_dcolors"], 0.0)
    K = pr["basis"].shape[1]
    gsh = np.zeros_like(pr["sh"])
    gsh[:, :K, :] = pr["basis"][:, :, None] * gcol[:, None, :]
    gd = np.einsum("nkc,nc,nkj->nj", pr["sh"][:, :K, :], gcol, pr["dbasis"])
    d = pr["d"]
    gw = (gd - d * (d * gd).sum(1, keepdims=True)) / pr["dnorm"][:, None]
    gmeans = gmeans + gw
    return {"means": gmeans, "log_scales": gls, "quats": gq, "opacity_logits": gol, "sh": gsh}


# ------------------------------------------------------------------ Adam
def bf16_round(x):
    """fp32 -> bf16 -> fp32, round to nearest even (torch's float -> bfloat16
    conversion; a NaN stays NaN)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    nan = np.isnan(np.asarray(x, np.float32))
    r = np.where(nan, (u.astype(np.uint32) | 0x00400000) & 0xFFFF0000, r).astype(np.uint32)
    return r.view(np.float32)


def sparse_adam(params, grads, m, v, step, visible, lr=None, betas=(0.9, 0.999), eps=1e-15,
                bf16_moments=False):
    """train_oracle.py:434-470: rows where `visible` is set are updated, with
    bias correction t = step + 1; fp32 arithmetic. bf16_moments: the moments
    given are bf16 values (exact in fp32) and the new ones are stored rounded to
    nearest even (moment_dtype bfloat16, :445-470); the parameter update uses
    the fp32 values before rounding."""
    lr = DEFAULT_LR if lr is None else lr
    f32 = np.float32
    b1, b2 = betas
    t = step + 1
    bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t
    vis = np.asarray(visible, bool)
    out = {}
    for name in PARAM_NAMES:
        p = np.array(params[name], f32)
        mm = np.array(m[name], f32)
        vv = np.array(v[name], f32)
        gg = np.asarray(grads[name], f32)[vis]
        m1 = f32(b1) * mm[vis] + f32(1.0 - b1) * gg
        v1 = f32(b2) * vv[vis] + f32(1.0 - b2) * gg * gg
        den = np.sqrt(v1) / f32(math.sqrt(bc2)) + f32(eps)
        if name == "sh":
            ss = np.full((1, p.shape[1], 1), f32(lr["sh_rest"]), f32)
            ss[:, 0] = f32(lr["sh_dc"])
            ss = ss / f32(bc1)
        else:
            ss = f32(lr[name] / bc1)
        p[vis] = p[vis] - ss * (m1 / den)
        mm[vis] = bf16_round(m1) if bf16_moments else m1
        vv[vis] = bf16_round(v1) if bf16_moments else v1
        out[name] = (p, mm, vv)
    return out
