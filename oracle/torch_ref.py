"""Differentiable PyTorch-CPU restatement of the rasterizer -- TEST INFRASTRUCTURE ONLY.

Written from the reference's forward definitions only (no backward formulas), so autograd through it is an
independent check of the C oracle's analytic backward (efgs_oracle.c). Also provides the unfused appearance
evaluation that serves as the CPU baseline: AppearanceModel.forward (Appearance/Base.py:83-108) with the
per-model residual_colors of Appearance/SH.py:34-56, SV.py:55-62, NASG.py:43-68, NASGabor.py:44-71 and the
Neural MLP (Neural.py:102-111, tcnn replaced by a matmul with fp16-rounded weights).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
"""
from __future__ import annotations

import math

import numpy as np
import torch

import oracle as O

LOG2E = 1.44269504089


# ---------------------------------------------------------------------------------------------------------
# activations (Appearance/utils.py:241-292)
# ---------------------------------------------------------------------------------------------------------

def base_activation(x, act):
    return torch.exp(3.0 * x) if act == 'exp' else x


def residual_activation(x, act):
    if act == 'tanh':
        return torch.tanh(x)
    if act == 'softplus':
        return torch.nn.functional.softplus(x, beta=10.0)
    return x


def color_activation(x, act):
    if act == 'none':
        return x + 0.5
    if act == 'relu':
        return torch.relu(x + 0.5)
    if act == 'softplus':
        return torch.nn.functional.softplus(x + 0.5, beta=10.0)
    if act == 'sigmoid':
        return torch.sigmoid(4.0 * x)
    if act == 'hardsigmoid':
        return torch.nn.functional.hardsigmoid(6.0 * x)
    if act == 'satexp':
        return -torch.expm1(-x)
    raise ValueError(act)


# ---------------------------------------------------------------------------------------------------------
# residual models
# ---------------------------------------------------------------------------------------------------------

def sh_residual(coef, d, degree, act):
    """Appearance/SH.py:34-56; coef (N, 15, 3), d (N, 3)."""
    x, y, z = d[:, 0:1], d[:, 1:2], d[:, 2:3]
    r = -0.48860251190291987 * y * coef[:, 0] + 0.48860251190291987 * z * coef[:, 1] - 0.48860251190291987 * x * coef[:, 2]
    if degree > 1:
        xx, yy, zz, xy, xz, yz = x * x, y * y, z * z, x * y, x * z, y * z
        r = r + 1.0925484305920792 * xy * coef[:, 3] - 1.0925484305920792 * yz * coef[:, 4] \
            + (0.94617469575755997 * zz - 0.31539156525251999) * coef[:, 5] - 1.0925484305920792 * xz * coef[:, 6] \
            + 0.54627421529603959 * (xx - yy) * coef[:, 7]
        if degree > 2:
            r = r + y * (0.59004358992664352 * yy - 1.7701307697799304 * xx) * coef[:, 8] \
                + 2.8906114426405538 * xy * z * coef[:, 9] + y * (0.45704579946446572 - 2.2852289973223288 * zz) * coef[:, 10] \
                + z * (1.865881662950577 * zz - 1.1195289977703462) * coef[:, 11] \
                + x * (0.45704579946446572 - 2.2852289973223288 * zz) * coef[:, 12] \
                + 1.4453057213202769 * z * (xx - yy) * coef[:, 13] + x * (1.7701307697799304 * yy - 0.59004358992664352 * xx) * coef[:, 14]
    return residual_activation(r, act)


def sv_residual(p, d, sites, act):
    """Appearance/SV.py:55-62; p (N, S, 7)."""
    s = torch.nn.functional.normalize(p[:, :sites, 0:3], dim=-1, eps=1e-12)
    taus = p[:, :sites, 3].exp()
    dist = torch.linalg.norm(s - d[:, None], dim=-1)
    w = torch.softmax(-taus * dist, dim=-1)
    c = residual_activation(p[:, :sites, 4:7], act)
    return (w[..., None] * c).sum(1)


def lobe_residual(p, d, lobes, act, gabor):
    """Appearance/NASG.py:43-68 (gabor False) and NASGabor.py:44-71 (gabor True); p (N, L, 8|9)."""
    ct, cp, cu = p[:, :lobes, 0:3].tanh().clamp(-0.999999, 0.999999).unbind(-1)
    st, sp, su = torch.sqrt(1 - ct * ct), torch.sqrt(1 - cp * cp), torch.sqrt(1 - cu * cu)
    fx = torch.stack([ct * cp * cu - st * su, st * cp * cu + ct * su, -sp * cu], -1)
    fz = torch.stack([ct * sp, st * sp, cp], -1)
    lam = p[:, :lobes, 3].exp().clamp_max(1e4)
    a = p[:, :lobes, 4].exp().clamp_max(1e4)
    vz = (d[:, None] * fz).sum(-1)
    vx = (d[:, None] * fx).sum(-1)
    vzc = vz.clamp(-0.99999988, 0.99999988)
    K = 0.5 * (vzc + 1.0)
    Ke = 5e-6 + a * vx * vx / (1.0 - vzc * vzc)
    E = K ** Ke
    N = lam * torch.sqrt(1.0 + a) / (2.0 * math.pi * (1.0 + 1e-8 - torch.exp(-2.0 * lam)))
    P = torch.exp(2.0 * lam * (E * K - 1.0))
    if gabor:
        k = (p[:, :lobes, 5].tanh() + 1.0) * 20.0
        G = 0.5 * (1.0 + torch.cos(k * vx))
        val = P * E * G * N
        w = residual_activation(p[:, :lobes, 6:9], act)
    else:
        val = P * E * N
        w = residual_activation(p[:, :lobes, 5:8], act)
    pdf = torch.where(vz >= 0.99999988, torch.ones_like(val), torch.where(vz > -0.99999988, val, torch.zeros_like(val)))
    return (pdf[..., None] * w).sum(1)


def sh_degree_values(d, degrees, active_degree):
    """Direction encoding of the neural model (Appearance/utils.py:138-223), differentiable."""
    out, rank = [], 0
    for deg in degrees:
        vals = [torch.full_like(d[:, 0], O.SH_C0)] if deg == 0 else O._sh_degree_values(d, deg)
        if deg > 0:
            keep = rank < active_degree
            rank += 1
            if not keep:
                vals = [torch.zeros_like(v) for v in vals]
        out += vals
    return torch.stack(out, 1)


def neural_residual(feat, base, d, mlp_cfg, mats, active_degree, act):
    """Appearance/Neural.py:102-111 with the MLP as fp16-rounded-operand matmuls (see oracle.mlp_forward)."""
    f = torch.cat([feat, base], 1) if mlp_cfg.base_input else feat
    if mlp_cfg.n_frequencies > 0:
        scaled = f[..., None] * (2.0 ** torch.arange(mlp_cfg.n_frequencies, dtype=f.dtype))
        f = torch.stack([scaled.sin(), scaled.cos()], -1).flatten(start_dim=-3)
    x = torch.cat([f, sh_degree_values(d, mlp_cfg.sh_degrees, active_degree)], 1)
    pad = mlp_cfg.n_input_padded - x.shape[1]
    if pad:
        x = torch.cat([x, torch.zeros(x.shape[0], pad, dtype=x.dtype)], 1)
    h = round_fp16(x)
    for i, w in enumerate(mats):
        h = h @ (w if torch.is_tensor(w) else torch.as_tensor(w, dtype=x.dtype)).T
        if i < len(mats) - 1:
            h = torch.relu(h)
        h = round_fp16(h)
    return residual_activation(h[:, :3], act)


def round_fp16(t):
    """fp16 rounding in the forward, identity in the backward (straight-through)."""
    return t + (t.detach().to(torch.float16).to(t.dtype) - t.detach())


def mlp_matrices_torch(flat, mlp_cfg):
    """Differentiable tcnn flat layout -> fp16-rounded row-major [out x in] matrices."""
    w = round_fp16(flat)
    mats, off = [], 0
    for r, c in mlp_cfg.layer_shapes():
        mats.append(w[off:off + r * c].reshape(r, c))
        off += r * c
    return mats


def appearance_colors(means, cam_pos, base, residual, app, degree, render_base=True, mats=None):
    """AppearanceModel.forward (Appearance/Base.py:83-108) for one view."""
    b = base_activation(base, app.base_act)
    if degree == 0:
        res = torch.zeros_like(b)
    else:
        d = torch.nn.functional.normalize(means - cam_pos[None], dim=-1)
        if app.model == 'sh':
            res = sh_residual(residual, d, degree, app.res_act)
        elif app.model == 'sv':
            res = sv_residual(residual, d, degree, app.res_act)
        elif app.model == 'nasg':
            res = lobe_residual(residual, d, degree, app.res_act, False)
        elif app.model == 'nasgabor':
            res = lobe_residual(residual, d, degree, app.res_act, True)
        elif app.model == 'neural':
            res = neural_residual(residual, base, d, app.mlp, mats, degree, app.res_act)
        else:
            raise ValueError(app.model)
    full = color_activation(b + res, app.color_act)
    if not render_base:
        return (full - color_activation(b, app.color_act)).abs()
    return full


# ---------------------------------------------------------------------------------------------------------
# geometry (preprocess_forward.cu:62-167) and blending with the oracle's discrete decisions held fixed
# ---------------------------------------------------------------------------------------------------------

def project(means, scales, rotations, opacities, cam: O.Camera):
    W = torch.as_tensor(np.asarray(cam.w2c, np.float64).reshape(-1, 4)[:3], dtype=means.dtype)
    m_h = torch.cat([means, torch.ones_like(means[:, :1])], 1)
    v = m_h @ W.T
    depth = v[:, 2]
    x, y = v[:, 0] / depth, v[:, 1] / depth
    wf, hf = float(cam.width), float(cam.height)
    cl, cr = (-0.15 * wf - cam.center_x) / cam.focal_x, (1.15 * wf - cam.center_x) / cam.focal_x
    ct, cb = (-0.15 * hf - cam.center_y) / cam.focal_y, (1.15 * hf - cam.center_y) / cam.focal_y
    xc, yc = x.clamp(cl, cr), y.clamp(ct, cb)
    q = rotations
    r, qx, qy, qz = q.unbind(1)
    ns = 1.0 / (q * q).sum(1)
    R = torch.stack([
        1 - 2 * (qy * qy + qz * qz) * ns, 2 * (qx * qy - r * qz) * ns, 2 * (qx * qz + r * qy) * ns,
        2 * (qx * qy + r * qz) * ns, 1 - 2 * (qx * qx + qz * qz) * ns, 2 * (qy * qz - r * qx) * ns,
        2 * (qx * qz - r * qy) * ns, 2 * (qy * qz + r * qx) * ns, 1 - 2 * (qx * qx + qy * qy) * ns], 1).reshape(-1, 3, 3)
    var = torch.exp(2.0 * scales)
    cov3 = R @ torch.diag_embed(var) @ R.transpose(1, 2)
    j11, j22 = cam.focal_x / depth, cam.focal_y / depth
    J = torch.zeros(means.shape[0], 2, 3, dtype=means.dtype)
    J[:, 0, 0] = j11
    J[:, 0, 2] = -j11 * xc
    J[:, 1, 1] = j22
    J[:, 1, 2] = -j22 * yc
    JW = J @ W[:, :3]
    cov2 = JW @ cov3 @ JW.transpose(1, 2)
    ks = 0.1 if cam.proper_aa else 0.3
    a_raw, b, c_raw = cov2[:, 0, 0], cov2[:, 0, 1], cov2[:, 1, 1]
    a, c = a_raw + ks, c_raw + ks
    det = a * c - b * b
    conic = torch.stack([c / det, -b / det, a / det], 1)
    opacity = torch.sigmoid(opacities[:, 0])
    if cam.proper_aa:
        # the antialiasing factor is detached from the 2D covariance (rasterization_config.h:12)
        opacity = opacity * torch.sqrt(torch.clamp((a_raw * c_raw - b * b) / det, min=0.0)).detach()
    mean2d = torch.stack([x * cam.focal_x + cam.center_x, y * cam.focal_y + cam.center_y], 1)
    return mean2d, conic, opacity


def contributor_lists(fw: O.ForwardState, cam: O.Camera) -> tuple[np.ndarray, np.ndarray]:
    """(P, K) primitive indices (-1 padded) of every pixel's contributing Gaussians in blend order, as decided by
    the oracle forward (alpha >= 1/255 before the pixel's last contributor)."""
    W, H = cam.width, cam.height
    gw, _ = cam.grid()
    lists = []
    for py in range(H):
        for px in range(W):
            t = (py // O.TILE_H) * gw + px // O.TILE_W
            r0 = fw.ranges[t, 0]
            last = fw.n_contrib[py * W + px]
            cur = []
            for k in range(last):
                p = fw.inst_prims[r0 + k]
                if O.blend_alpha(fw.mean2d[p], fw.conic_opacity[p], px, py) >= np.float32(1.0 / 255.0):
                    cur.append(p)
            lists.append(cur)
    K = max([len(c) for c in lists] + [1])
    idx = np.full((W * H, K), -1, np.int64)
    for i, c in enumerate(lists):
        idx[i, :len(c)] = c
    return idx, (idx >= 0)


def blend(mean2d, conic, opacity, colors, idx, mask, cam: O.Camera):
    W, H = cam.width, cam.height
    ys, xs = np.meshgrid(np.arange(H), np.arange(W), indexing='ij')
    pix = torch.as_tensor(np.stack([xs.reshape(-1) + 0.5, ys.reshape(-1) + 0.5], 1), dtype=mean2d.dtype)
    safe = torch.as_tensor(np.where(mask, idx, 0))
    m = torch.as_tensor(mask, dtype=mean2d.dtype)
    d = mean2d[safe] - pix[:, None]
    co = conic[safe]
    power = -0.5 * (co[..., 0] * d[..., 0] ** 2 + co[..., 2] * d[..., 1] ** 2) - co[..., 1] * d[..., 0] * d[..., 1]
    alpha = opacity[safe] * torch.exp(torch.clamp(power, max=0.0)) * m
    one_minus = 1.0 - alpha
    T_before = torch.cat([torch.ones_like(alpha[:, :1]), torch.cumprod(one_minus, 1)[:, :-1]], 1)
    w = T_before * alpha
    color = (w[..., None] * colors[safe]).sum(1)
    T_final = torch.prod(one_minus, 1)
    bg = torch.as_tensor(np.asarray(cam.bg, np.float64), dtype=mean2d.dtype)
    img = color + T_final[:, None] * bg[None]
    return img.T.reshape(3, H, W)


def render(scene: O.Scene, app: O.Appearance, cam: O.Camera, fw: O.ForwardState, dtype=torch.float64, requires_grad=True):
    """Differentiable image with the discrete structure of the oracle forward `fw`; returns (image, leaves)."""
    def leaf(a):
        t = torch.tensor(np.asarray(a, np.float64), dtype=dtype)
        t.requires_grad_(requires_grad)
        return t
    leaves = dict(means=leaf(scene.means), scales=leaf(scene.scales), rotations=leaf(scene.rotations), opacities=leaf(scene.opacities))
    if app.model == 'precomputed':
        leaves['precomputed_colors'] = leaf(scene.precomputed_colors)
    else:
        leaves['base_colors'] = leaf(scene.base_colors)
        leaves['residual_params'] = leaf(scene.residual_params)
    mats = None
    if app.model == 'neural':
        leaves['mlp_weights'] = leaf(scene.mlp_weights)
        mats = mlp_matrices_torch(leaves['mlp_weights'], app.mlp)
    mean2d, conic, opacity = project(leaves['means'], leaves['scales'], leaves['rotations'], leaves['opacities'], cam)
    degree = cam.degree if cam.render_residual else 0
    if app.model == 'precomputed':
        colors = leaves['precomputed_colors']
    else:
        means_for_dir = leaves['means'] if app.direction_gradient else leaves['means'].detach()
        colors = appearance_colors(means_for_dir, torch.as_tensor(np.asarray(cam.position, np.float64), dtype=dtype),
                                   leaves['base_colors'], leaves['residual_params'], app, degree, cam.render_base, mats)
    idx, mask = contributor_lists(fw, cam)
    img = blend(mean2d, conic, opacity, colors, idx, mask, cam)
    return img, leaves
