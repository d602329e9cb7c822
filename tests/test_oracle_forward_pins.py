"""Pins the oracle's projection forward and the lobe / site appearance forms with what the mathematics fixes
(CPU only). Nothing here restates the oracle's scalar expressions: every expected value comes from a
different construction.

* quaternion -> rotation: Rodrigues' axis-angle matrix of the same rotation, for scaled quaternions;
* view depth and mean2d: the pinhole model x' = W x + t, u = f x'_x / x'_z + c, in float64 with numpy products;
* the EWA covariance: (a) a Monte-Carlo estimate, points drawn from the 3D Gaussian and projected through the
  pinhole, whose sample covariance converges to the linearised projection (no Jacobian is written down);
  (b) the float64 matrix product J W R S^2 R^T W^T J^T with R from axis-angle (catches transposed operands);
  (c) the on-axis isotropic closed form (f/z)^2 s^2 + dilation; (d) the Jacobian's evaluation point clamped to
  1.15x the image (the reference's guard band) for a splat whose centre lies outside it;
* the antialiasing opacity factor sqrt(det(cov) / det(cov + 0.1 I)) in float64;
* culling: near/far depth, opacity below 1/255, a degenerate quaternion, the AA factor pushing opacity under
  the threshold;
* screen bounds: every pixel where the float64 alpha reaches 1/255 lies inside the bounds and inside a tile
  the exact tile count includes; the bounds are no wider than the ellipse's extent plus a pixel per side;
* NASG: the normalised lobe integrates to one over the sphere (Gauss-Legendre quadrature);
* NASGabor: equal to NASG where the direction has no component along the lobe's x axis, zero where
  k v_x = pi (the lobe frame built as Z-Y-Z Euler rotations, independently of the oracle's expanded form);
* SV: a direct float64 softmax over the sites (the oracle uses a one-pass rescaled softmax), two sites
  symmetric about the direction average their colours, a large sharpness selects the nearest site;
* SH model: projecting the residual back onto the (quadrature-orthonormal) basis recovers the coefficients;
* neural frequency encoding: sin^2 + cos^2 = 1 per pair, the double-angle ladder between frequencies, and
  atan2 of the first pair returning the feature (feature-major, then frequency, then sin / cos);
* blend forward: the product form of front-to-back compositing, sum_i c_i a_i prod_{j<i} (1 - a_j) + T bg
  with T = prod (1 - a_i), in float64 with exact exp, skip and stop decisions away from their thresholds.
"""
import math

import numpy as np
import pytest

import oracle as O
from helpers import single_tile_state

TILE_W, TILE_H = 16, 12


def _rodrigues(axis, angle):
    a = np.asarray(axis, np.float64)
    a = a / np.linalg.norm(a)
    K = np.array([[0, -a[2], a[1]], [a[2], 0, -a[0]], [-a[1], a[0], 0]])
    return np.eye(3) + math.sin(angle) * K + (1 - math.cos(angle)) * K @ K


def _random_rotations(rng, n):
    axes = rng.normal(size=(n, 3))
    angles = rng.uniform(-math.pi, math.pi, n)
    return axes, angles, np.stack([_rodrigues(axes[i], angles[i]) for i in range(n)])


def _quat(axis, angle, scale):
    a = np.asarray(axis, np.float64) / np.linalg.norm(axis)
    return scale * np.array([math.cos(angle / 2), *(math.sin(angle / 2) * a)])


def _camera(rng, width=96, height=72, f=80.0, rotate=True, dist=6.0):
    """World-to-view matrix of a camera at distance `dist` from the origin, looking at it (random orientation)."""
    if rotate:
        _, _, Rc = _random_rotations(rng, 1)
        Rc = Rc[0]
    else:
        Rc = np.eye(3)
    t = np.array([0.0, 0.0, dist])
    w2c = np.zeros((4, 4))
    w2c[:3, :3] = Rc
    w2c[:3, 3] = t
    w2c[3, 3] = 1
    pos = -Rc.T @ t
    return O.Camera(w2c=w2c.astype(np.float32), position=pos.astype(np.float32), width=width, height=height,
                    focal_x=f, focal_y=f * 1.1, center_x=width / 2 + 1.5, center_y=height / 2 - 2.0, degree=0)


def _scene(means, log_scales, quats, logits):
    n = len(means)
    return O.Scene(means=np.asarray(means, np.float32), scales=np.asarray(log_scales, np.float32),
                   rotations=np.asarray(quats, np.float32), opacities=np.asarray(logits, np.float32).reshape(n, 1),
                   precomputed_colors=np.full((n, 3), 0.5, np.float32))


def _preprocess(scene, cam):
    return O.preprocess(scene, O.Appearance(model='precomputed'), cam)


def _view(cam, x):
    W = np.asarray(cam.w2c, np.float64).reshape(-1, 4)[:3]
    return W[:, :3] @ np.asarray(x, np.float64) + W[:, 3]


def _sigmoid(x):
    return 1.0 / (1.0 + math.exp(-float(x)))


def _ewa64(cam, mean, R, log_scale, guard=1.15):
    """float64 EWA covariance J Wr Sigma Wr^T J^T (no dilation), J at the guard-clamped normalised point."""
    Wr = np.asarray(cam.w2c, np.float64).reshape(-1, 4)[:3, :3]
    t = _view(cam, mean)
    z = t[2]
    xn, yn = t[0] / z, t[1] / z
    lx0, lx1 = (-(guard - 1) * cam.width - cam.center_x) / cam.focal_x, (guard * cam.width - cam.center_x) / cam.focal_x
    ly0, ly1 = (-(guard - 1) * cam.height - cam.center_y) / cam.focal_y, (guard * cam.height - cam.center_y) / cam.focal_y
    xc, yc = min(max(xn, lx0), lx1), min(max(yn, ly0), ly1)
    J = np.array([[cam.focal_x / z, 0.0, -cam.focal_x * xc / z], [0.0, cam.focal_y / z, -cam.focal_y * yc / z]])
    S = R @ np.diag(np.exp(2.0 * np.asarray(log_scale, np.float64))) @ R.T
    return J @ Wr @ S @ Wr.T @ J.T


def _conic_to_cov(co):
    C = np.array([[co[0], co[1]], [co[1], co[2]]], np.float64)
    return np.linalg.inv(C)


# ---------------------------------------------------------------------------------------------------------
# quaternion, depth, mean2d
# ---------------------------------------------------------------------------------------------------------

def test_quat_to_rot_is_axis_angle_rotation():
    rng = np.random.default_rng(0)
    axes, angles, R = _random_rotations(rng, 200)
    scales = rng.uniform(0.05, 20.0, 200)
    for i in range(200):
        got, nsq = O.quat_to_rot(_quat(axes[i], angles[i], scales[i]))
        np.testing.assert_allclose(got, R[i], atol=2e-6)
        assert nsq == pytest.approx(scales[i] ** 2, rel=1e-6)
    got, _ = O.quat_to_rot([1.0, 0.0, 0.0, 0.0])
    np.testing.assert_array_equal(got, np.eye(3, dtype=np.float32))
    got, _ = O.quat_to_rot([0.0, 0.0, 0.0, 1.0])   # half turn about z
    np.testing.assert_allclose(got, np.diag([-1.0, -1.0, 1.0]), atol=1e-7)


def test_depth_and_mean2d_follow_the_pinhole():
    rng = np.random.default_rng(1)
    cam = _camera(rng)
    n = 400
    means = rng.uniform(-1.5, 1.5, (n, 3))
    axes, angles, _ = _random_rotations(rng, n)
    q = np.stack([_quat(axes[i], angles[i], 1.0) for i in range(n)])
    pre = _preprocess(_scene(means, np.full((n, 3), -2.5), q, np.full(n, 2.0)), cam)
    vis = pre['n_touched'] > 0
    assert vis.sum() > 300
    for i in np.nonzero(vis)[0]:
        t = _view(cam, means[i].astype(np.float32))
        depth = pre['depth_key'][i:i + 1].view(np.float32)[0]
        assert abs(depth - t[2]) <= 2 * np.spacing(np.float32(t[2]))
        u = cam.focal_x * t[0] / t[2] + cam.center_x
        v = cam.focal_y * t[1] / t[2] + cam.center_y
        np.testing.assert_allclose(pre['mean2d'][i], [u, v], rtol=0, atol=4e-5 * max(1.0, abs(u), abs(v)))


# ---------------------------------------------------------------------------------------------------------
# EWA covariance, dilation, guard band, antialiasing factor
# ---------------------------------------------------------------------------------------------------------

def test_ewa_covariance_matches_monte_carlo_projection():
    """Points drawn from N(mean, Sigma) and projected through the pinhole have a sample covariance that converges
    to the EWA covariance (the linearised projection; second-order terms are (sigma/z)^2 ~ 1e-5 relative).
    The oracle's conic inverted, minus the 0.3 dilation, must match within the sampling error."""
    rng = np.random.default_rng(2)
    cam = _camera(rng, width=160, height=120, f=300.0)
    n_samples = 400_000
    checked = 0
    for _ in range(6):
        t = np.array([rng.uniform(-0.4, 0.4), rng.uniform(-0.3, 0.3), 1.0]) * rng.uniform(4.5, 7.5)
        Wr = np.asarray(cam.w2c, np.float64)[:3, :3]
        mean = (Wr.T @ (t - np.asarray(cam.w2c, np.float64)[:3, 3])).astype(np.float32)
        axis, angle = rng.normal(size=3), rng.uniform(-math.pi, math.pi)
        log_s = rng.uniform(-4.5, -3.3, 3).astype(np.float32)
        q = _quat(axis, angle, rng.uniform(0.5, 2.0))
        pre = _preprocess(_scene(mean[None], log_s[None], q[None], [3.0]), cam)
        assert pre['n_touched'][0] > 0
        cov = _conic_to_cov(pre['conic_opacity'][0]) - 0.3 * np.eye(2)
        R = _rodrigues(axis, angle)
        X = mean.astype(np.float64) + (rng.normal(size=(n_samples, 3)) * np.exp(log_s.astype(np.float64))) @ R.T
        V = X @ np.asarray(cam.w2c, np.float64)[:3, :3].T + np.asarray(cam.w2c, np.float64)[:3, 3]
        uv = np.stack([cam.focal_x * V[:, 0] / V[:, 2], cam.focal_y * V[:, 1] / V[:, 2]], 1)
        emp = np.cov(uv.T)
        err = np.linalg.norm(emp - cov) / np.linalg.norm(emp)
        assert err < 0.015, (err, emp, cov)
        checked += 1
    assert checked == 6


def test_ewa_covariance_matches_matrix_form():
    """float64 J Wr R S^2 R^T Wr^T J^T + 0.3 I (R from axis-angle) against the oracle's conic, to fp32 accuracy."""
    rng = np.random.default_rng(3)
    cam = _camera(rng)
    n = 300
    means = rng.uniform(-1.5, 1.5, (n, 3)).astype(np.float32)
    axes, angles, R = _random_rotations(rng, n)
    q = np.stack([_quat(axes[i], angles[i], rng.uniform(0.3, 3.0)) for i in range(n)])
    log_s = rng.normal(-2.5, 0.6, (n, 3)).astype(np.float32)
    pre = _preprocess(_scene(means, log_s, q, np.full(n, 1.0)), cam)
    vis = np.nonzero(pre['n_touched'] > 0)[0]
    assert len(vis) > 200
    for i in vis:
        cov = _ewa64(cam, means[i], R[i], log_s[i]) + 0.3 * np.eye(2)
        want = np.linalg.inv(cov)
        got = pre['conic_opacity'][i, :3]
        scale = np.abs(want).max()
        np.testing.assert_allclose(got, [want[0, 0], want[0, 1], want[1, 1]], rtol=0, atol=2e-4 * scale)


def test_isotropic_gaussian_on_the_optical_axis():
    """A sphere of radius s at depth z on the optical axis projects to (f s / z)^2 + 0.3 per axis, no correlation."""
    cam = O.Camera(w2c=np.eye(4, dtype=np.float32), position=np.zeros(3, np.float32), width=64, height=48,
                   focal_x=100.0, focal_y=100.0, center_x=32.0, center_y=24.0, degree=0)
    for z, s in [(2.0, 0.05), (5.0, 0.02), (10.0, 0.3), (3.0, 0.001)]:
        pre = _preprocess(_scene([[0.0, 0.0, z]], [[math.log(s)] * 3], [[1.0, 0.0, 0.0, 0.0]], [4.0]), cam)
        var = (100.0 * s / z) ** 2 + 0.3
        co = pre['conic_opacity'][0]
        np.testing.assert_allclose(co[[0, 2]], [1.0 / var, 1.0 / var], rtol=2e-6)
        assert co[1] == 0.0
        np.testing.assert_array_equal(pre['mean2d'][0], [32.0, 24.0])


def test_jacobian_uses_the_guard_band_clamp():
    """A wide splat whose centre projects outside 1.15x the image still touches it; its Jacobian is evaluated at
    the point clamped to the guard band (reference preprocess_forward.cu: the 1.15 limits)."""
    rng = np.random.default_rng(4)
    cam = O.Camera(w2c=np.eye(4, dtype=np.float32), position=np.zeros(3, np.float32), width=64, height=48,
                   focal_x=60.0, focal_y=60.0, center_x=32.0, center_y=24.0, degree=0)
    seen = 0
    for k in range(40):
        z = rng.uniform(3.0, 6.0)
        xn = rng.choice([-1, 1]) * rng.uniform(0.9, 1.4) * 32.0 / 60.0 * 1.3 / 0.65
        yn = rng.uniform(-0.2, 0.2)
        mean = np.array([xn * z, yn * z, z], np.float32)
        axis, angle = rng.normal(size=3), rng.uniform(-math.pi, math.pi)
        log_s = np.full(3, math.log(0.6 * z), np.float32) + rng.normal(0, 0.2, 3).astype(np.float32)
        pre = _preprocess(_scene(mean[None], log_s[None], _quat(axis, angle, 1.0)[None], [4.0]), cam)
        if pre['n_touched'][0] == 0:
            continue
        R = _rodrigues(axis, angle)
        want = np.linalg.inv(_ewa64(cam, mean, R, log_s) + 0.3 * np.eye(2))
        unclamped = np.linalg.inv(_ewa64(cam, mean, R, log_s, guard=1e9) + 0.3 * np.eye(2))
        got = pre['conic_opacity'][0, :3]
        scale = np.abs(want).max()
        np.testing.assert_allclose(got, [want[0, 0], want[0, 1], want[1, 1]], rtol=0, atol=2e-4 * scale)
        if abs(mean[0] / z * 60.0 + 32.0) > 1.15 * 64 + 5:
            assert np.abs(unclamped - want).max() > 1e-2 * scale  # the clamp changes the answer here
            seen += 1
    assert seen >= 5


def test_antialiasing_opacity_factor():
    """proper_aa: opacity x sqrt(det(cov) / det(cov + 0.1 I)) with cov the undilated EWA covariance."""
    rng = np.random.default_rng(5)
    cam = _camera(rng)
    cam.proper_aa = True
    n = 200
    means = rng.uniform(-1.2, 1.2, (n, 3)).astype(np.float32)
    axes, angles, R = _random_rotations(rng, n)
    q = np.stack([_quat(axes[i], angles[i], 1.0) for i in range(n)])
    log_s = rng.normal(-3.0, 0.5, (n, 3)).astype(np.float32)
    logits = rng.normal(1.0, 1.0, n).astype(np.float32)
    pre = _preprocess(_scene(means, log_s, q, logits), cam)
    vis = np.nonzero(pre['n_touched'] > 0)[0]
    assert len(vis) > 100
    small = 0
    for i in vis:
        cov = _ewa64(cam, means[i], R[i], log_s[i])
        f = math.sqrt(np.linalg.det(cov) / np.linalg.det(cov + 0.1 * np.eye(2)))
        small += f < 0.8
        assert pre['conic_opacity'][i, 3] == pytest.approx(_sigmoid(logits[i]) * f, rel=2e-4)
        want = np.linalg.inv(cov + 0.1 * np.eye(2))
        np.testing.assert_allclose(pre['conic_opacity'][i, :3], [want[0, 0], want[0, 1], want[1, 1]], rtol=0,
                                   atol=2e-4 * np.abs(want).max())
    assert small > 20   # the factor is exercised well away from 1


def test_culling_rules():
    cam = O.Camera(w2c=np.eye(4, dtype=np.float32), position=np.zeros(3, np.float32), width=64, height=48,
                   focal_x=60.0, focal_y=60.0, center_x=32.0, center_y=24.0, degree=0, near_plane=0.2, far_plane=100.0)
    # the opacity pair projects onto the centre of pixel (32, 24), so a threshold just above zero still passes
    c = 0.5 / 60.0 * 3.0
    means = [[0, 0, 0.19], [0, 0, 0.21], [0, 0, 99.0], [0, 0, 101.0], [c, c, 3.0], [c, c, 3.0], [0, 0, 3.0], [0, 0, 3.0]]
    log_s = [[math.log(0.01)] * 3] * 4 + [[math.log(0.05)] * 3] * 4
    log_s[2] = [math.log(5.0)] * 3
    quats = [[1, 0, 0, 0]] * 8
    quats[6] = [5e-5, 0, 0, 0]          # |q|^2 = 2.5e-9 < 1e-8: degenerate
    o_min = math.log((1 / 255) / (1 - 1 / 255))
    logits = [3.0, 3.0, 3.0, 3.0, o_min - 1e-3, o_min + 1e-2, 3.0, 3.0]
    pre = _preprocess(_scene(np.array(means), np.array(log_s), np.array(quats), np.array(logits)), cam)
    assert list(pre['n_touched'] > 0) == [False, True, True, False, False, True, False, True]
    # proper AA: a splat much smaller than a pixel loses opacity below 1/255 and is culled
    cam.proper_aa = True
    pre = _preprocess(_scene(np.array([[0, 0, 3.0], [0, 0, 3.0]]), np.array([[math.log(1e-4)] * 3, [math.log(0.05)] * 3]),
                             np.array([[1, 0, 0, 0]] * 2), np.array([-3.0, -3.0])), cam)
    assert list(pre['n_touched'] > 0) == [False, True]


# ---------------------------------------------------------------------------------------------------------
# bounds and exact tile counts against per-pixel float64 alpha
# ---------------------------------------------------------------------------------------------------------

def test_bounds_and_tiles_cover_every_contributing_pixel():
    rng = np.random.default_rng(6)
    cam = _camera(rng, width=80, height=60, f=70.0)
    n = 300
    means = rng.uniform(-1.5, 1.5, (n, 3)).astype(np.float32)
    axes, angles, _ = _random_rotations(rng, n)
    q = np.stack([_quat(axes[i], angles[i], 1.0) for i in range(n)])
    log_s = rng.normal(-2.3, 0.5, (n, 3)).astype(np.float32)
    logits = rng.normal(0.0, 1.5, n).astype(np.float32)
    pre = _preprocess(_scene(means, log_s, q, logits), cam)
    gw, gh = cam.grid()
    ys, xs = np.mgrid[0:gh * TILE_H, 0:gw * TILE_W]
    checked = 0
    for i in np.nonzero(pre['n_touched'] > 0)[0]:
        m = pre['mean2d'][i].astype(np.float64)
        co = pre['conic_opacity'][i].astype(np.float64)
        dx, dy = m[0] - (xs + 0.5), m[1] - (ys + 0.5)
        power = 0.5 * (co[0] * dx * dx + co[2] * dy * dy) + co[1] * dx * dy
        alpha = co[3] * np.exp(-power)
        hit = alpha >= (1.0 / 255.0) * (1 + 1e-4)
        b = pre['bounds'][i].astype(np.int64)
        inside = (xs >= b[0]) & (xs < b[1]) & (ys >= b[2]) & (ys < b[3])
        assert not np.any(hit & ~inside), i
        # the bounds are no wider than the alpha = 1/255 ellipse's extent plus a pixel on each side
        cov = _conic_to_cov(co[:3])
        cut = 2.0 * math.log(255.0 * co[3])
        ex, ey = math.sqrt(cov[0, 0] * cut), math.sqrt(cov[1, 1] * cut)
        pw, ph = gw * TILE_W, gh * TILE_H
        assert b[1] - b[0] <= min(2 * ex + 2, pw) and b[3] - b[2] <= min(2 * ey + 2, ph)
        # every tile holding a contributing pixel is counted; no more tiles than the bounds' rectangle
        tiles = {(int(y) // TILE_H, int(x) // TILE_W) for y, x in zip(ys[hit], xs[hit])}
        rect = ((b[1] + TILE_W - 1) // TILE_W - b[0] // TILE_W) * ((b[3] + TILE_H - 1) // TILE_H - b[2] // TILE_H)
        assert len(tiles) <= pre['n_touched'][i] <= rect
        checked += hit.any()
    assert checked > 150


# ---------------------------------------------------------------------------------------------------------
# NASG / NASGabor / SV forms
# ---------------------------------------------------------------------------------------------------------

def _sphere_quadrature(n_theta, n_phi):
    t, w = np.polynomial.legendre.leggauss(n_theta)
    phi = np.arange(n_phi) * 2 * np.pi / n_phi
    T, P = np.meshgrid(t, phi, indexing='ij')
    W = np.repeat(w[:, None], n_phi, 1) * (2 * np.pi / n_phi)
    s = np.sqrt(1 - T * T)
    return np.stack([s * np.cos(P), s * np.sin(P), T], -1).reshape(-1, 3), W.reshape(-1)


@pytest.mark.parametrize('lam_raw,an_raw', [(0.5, -3.0), (1.5, -1.0), (2.0, 0.5), (2.3, 1.5)])
def test_nasg_lobe_is_normalised(lam_raw, an_raw):
    """The NASG lobe with its normalisation lambda sqrt(1 + a) / (2 pi (1 - e^{-2 lambda})) integrates to one
    over the sphere (up to the 5e-6 exponent epsilon), for isotropic and anisotropic lobes alike."""
    d, w = _sphere_quadrature(128, 256)
    app = O.Appearance(model='nasg', max_degree=1, res_act='none')
    p = np.array([0.3, -0.2, 0.5, lam_raw, an_raw, 1.0, 0.0, 0.0], np.float32)
    vals = np.array([O.residual(app, p, x.astype(np.float32), 1)[0] for x in d], np.float64)
    assert abs((vals * w).sum() - 1.0) < 5e-5


def _zyz_frame(p):
    """Lobe frame of raw angles (cos theta, cos phi, cos psi) = tanh(raw): the rotation Rz(theta) Ry(phi) Rz(psi)
    applied to the coordinate axes (x axis, y axis, z axis = lobe direction)."""
    c = np.clip(np.tanh(np.asarray(p[:3], np.float64)), -0.999999, 0.999999)
    th, ph, ps = np.arccos(c)

    def rz(a):
        return np.array([[math.cos(a), -math.sin(a), 0], [math.sin(a), math.cos(a), 0], [0, 0, 1]])

    def ry(a):
        return np.array([[math.cos(a), 0, math.sin(a)], [0, 1, 0], [-math.sin(a), 0, math.cos(a)]])
    M = rz(th) @ ry(ph) @ rz(ps)
    return M[:, 0], M[:, 1], M[:, 2]


def test_nasgabor_reduces_to_nasg_and_vanishes_at_half_period():
    rng = np.random.default_rng(7)
    nasg = O.Appearance(model='nasg', max_degree=1, res_act='none')
    gabor = O.Appearance(model='nasgabor', max_degree=1, res_act='none')
    for _ in range(30):
        p = np.concatenate([rng.normal(0, 0.8, 3), [rng.normal(1.0, 0.4), rng.normal(0.5, 0.5)]]).astype(np.float32)
        freq_raw = np.float32(rng.normal(0.0, 1.0))
        col = rng.uniform(0.2, 1.0, 3).astype(np.float32)
        pg = np.concatenate([p, [freq_raw], col]).astype(np.float32)
        pn = np.concatenate([p, col]).astype(np.float32)
        x, y, z = _zyz_frame(p)
        # direction in the lobe's y-z plane: v_x = 0, the Gabor factor is 1
        a = rng.uniform(0.05, 1.2)
        v = (math.cos(a) * z + math.sin(a) * y).astype(np.float32)
        want = O.residual(nasg, pn, v, 1)
        np.testing.assert_allclose(O.residual(gabor, pg, v, 1), want, rtol=2e-5, atol=1e-7 * np.abs(want).max())
        # k v_x = pi: the Gabor factor 0.5 (1 + cos(k v_x)) vanishes
        k = (math.tanh(float(freq_raw)) + 1.0) * 20.0
        vx = math.pi / k
        if vx >= 0.9:
            continue
        # the rest of the unit vector in the y-z plane, mostly along the lobe axis so the lobe is not negligible
        rest = math.sqrt(1 - vx * vx)
        v = vx * x + rest * (0.9 * z + math.sqrt(0.19) * y * rng.choice([-1.0, 1.0]))
        v32 = v.astype(np.float32)
        ref = O.residual(nasg, pn, v32, 1)
        got = O.residual(gabor, pg, v32, 1)
        # first-order error of k v_x in float32 leaves G ~ (k dv)^2 / 4
        assert np.abs(got).max() <= 1e-8 * max(1.0, np.abs(ref).max()) + 1e-9, (got, ref)


def _sv_direct(params, d, act='none'):
    p = np.asarray(params, np.float64).reshape(-1, 7)
    s = p[:, :3] / np.linalg.norm(p[:, :3], axis=1, keepdims=True)
    logits = -np.exp(p[:, 3]) * np.linalg.norm(s - np.asarray(d, np.float64), axis=1)
    w = np.exp(logits - logits.max())
    w /= w.sum()
    c = np.tanh(p[:, 4:]) if act == 'tanh' else p[:, 4:]
    return w @ c


def test_sv_is_a_softmax_over_sites():
    rng = np.random.default_rng(8)
    for sites in (2, 3, 8):
        app = O.Appearance(model='sv', max_degree=sites, res_act='tanh')
        for _ in range(40):
            p = np.concatenate([rng.normal(size=(sites, 3)), rng.normal(1.0, 1.0, (sites, 1)), rng.normal(0, 0.5, (sites, 3))], 1)
            p = p.astype(np.float32)
            d = rng.normal(size=3)
            d /= np.linalg.norm(d)
            np.testing.assert_allclose(O.residual(app, p, d.astype(np.float32), sites), _sv_direct(p, d.astype(np.float32), 'tanh'),
                                       rtol=2e-5, atol=2e-6)


def test_sv_symmetric_sites_average_and_sharp_sites_select():
    app = O.Appearance(model='sv', max_degree=2, res_act='none')
    d = np.array([0.0, 0.0, 1.0], np.float32)
    a = 0.4
    c1, c2 = np.array([0.9, -0.2, 0.3], np.float32), np.array([-0.1, 0.5, 0.7], np.float32)
    p = np.array([[math.sin(a), 0.0, math.cos(a), 2.0, *c1], [-math.sin(a) * 3, 0.0, math.cos(a) * 3, 2.0, *c2]], np.float32)
    np.testing.assert_allclose(O.residual(app, p, d, 2), 0.5 * (c1 + c2), rtol=1e-5, atol=1e-6)
    # large sharpness: the nearest site's colour
    p = np.array([[0.1, 0.0, 1.0, 6.0, *c1], [0.6, 0.0, 1.0, 6.0, *c2]], np.float32)
    np.testing.assert_allclose(O.residual(app, p, d, 2), c1, rtol=1e-5, atol=1e-6)
    # the active degree gates the sites: one active site is that site's colour whatever the direction
    np.testing.assert_allclose(O.residual(app, p, np.array([0.0, 1.0, 0.0], np.float32), 1), c1, rtol=1e-6)


def test_sh_residual_projects_back_onto_its_coefficients():
    d, w = _sphere_quadrature(48, 96)
    app = O.Appearance(model='sh', max_degree=3, res_act='none')
    rng = np.random.default_rng(9)
    coef = rng.normal(0.0, 1.0, (15, 3)).astype(np.float32)
    res = np.array([O.residual(app, coef, x.astype(np.float32), 3) for x in d], np.float64)
    B = np.stack([O.sh_rest_basis(x.astype(np.float32), 3) for x in d]).astype(np.float64)
    np.testing.assert_allclose((B * w[:, None]).T @ res, coef, atol=2e-5)
    # degree 1 only keeps the first three coefficients
    res1 = np.array([O.residual(app, coef, x.astype(np.float32), 1) for x in d], np.float64)
    proj = (B * w[:, None]).T @ res1
    np.testing.assert_allclose(proj[:3], coef[:3], atol=2e-5)
    np.testing.assert_allclose(proj[3:], 0.0, atol=2e-5)


def test_frequency_encoding_identities():
    rng = np.random.default_rng(10)
    feat = rng.uniform(-1.5, 1.5, (200, 5)).astype(np.float32)
    for nf in (1, 2, 4):
        enc = O.frequency_encode(feat, nf).astype(np.float64).reshape(200, 5, nf, 2)
        sin, cos = enc[..., 0], enc[..., 1]
        np.testing.assert_allclose(sin * sin + cos * cos, 1.0, atol=1e-6)
        np.testing.assert_allclose(np.arctan2(sin[..., 0], cos[..., 0]), feat, atol=1e-6)
        for f in range(nf - 1):   # the argument doubles from one frequency to the next
            np.testing.assert_allclose(sin[..., f + 1], 2 * sin[..., f] * cos[..., f], atol=2e-6)
            np.testing.assert_allclose(cos[..., f + 1], cos[..., f] ** 2 - sin[..., f] ** 2, atol=2e-6)
    np.testing.assert_array_equal(O.frequency_encode(feat, 0), feat)


def test_blend_forward_is_the_product_composite():
    rng = np.random.default_rng(11)
    bg = np.array([0.2, 0.5, 0.1], np.float32)
    checked = 0
    for k, spread, o_min in ((1, 6.0, 0.5), (2, 6.0, 0.5), (3, 6.0, 0.5), (5, 6.0, 0.5), (8, 6.0, 0.5), (12, 40.0, 0.9)):
        mean2d = rng.uniform([1.0, 1.0], [15.0, 11.0], (k, 2)).astype(np.float32)
        co = np.zeros((k, 4), np.float32)
        for i in range(k):
            a = rng.normal(size=(2, 2))
            inv = np.linalg.inv(a @ a.T * spread + np.eye(2) * 2.0)
            co[i] = [inv[0, 0], inv[0, 1], inv[1, 1], rng.uniform(o_min, 0.995)]
        color = rng.uniform(0.0, 1.0, (k, 3)).astype(np.float32)
        _, fw = single_tile_state(mean2d, co, color, bg)
        ys, xs = np.mgrid[0:12, 0:16]
        px, py = xs.reshape(-1) + 0.5, ys.reshape(-1) + 0.5
        m, c = mean2d.astype(np.float64), co.astype(np.float64)
        dx, dy = m[:, 0:1] - px[None], m[:, 1:2] - py[None]
        alpha = c[:, 3:4] * np.exp(-(0.5 * (c[:, 0:1] * dx * dx + c[:, 2:3] * dy * dy) + c[:, 1:2] * dx * dy))  # (k, P)
        used = alpha >= 1.0 / 255.0
        a = np.where(used, alpha, 0.0)
        T_before = np.cumprod(np.vstack([np.ones((1, a.shape[1])), 1.0 - a[:-1]]), axis=0)
        T_after = T_before * (1.0 - a)
        # stop: the first contributor after which T < 1e-4 ends the walk
        stop = np.where((T_after < 1e-4) & used, np.arange(k)[:, None], k).min(0)
        keep = np.arange(k)[:, None] <= stop[None]
        w = np.where(keep, T_before * a, 0.0)
        T = np.where(stop < k, T_after[np.minimum(stop, k - 1), np.arange(a.shape[1])], T_after[-1])
        img = w.T @ color.astype(np.float64) + T[:, None] * bg[None].astype(np.float64)
        last = np.where(keep & used, np.arange(1, k + 1)[:, None], 0).max(0)
        # leave out pixels where a decision sits near its threshold (float32 exp2 against exact exp)
        near = (np.abs(alpha * 255.0 - 1.0) < 1e-4).any(0) | (np.abs(T_after / 1e-4 - 1.0) < 1e-3).any(0)
        ok = ~near
        np.testing.assert_allclose(fw.image.reshape(3, -1).T[ok], img[ok], atol=2e-6)
        np.testing.assert_allclose(fw.final_T[ok], T[ok], atol=2e-6)
        np.testing.assert_array_equal(fw.n_contrib[ok], last[ok])
        checked += ok.sum()
        if k == 12:
            assert (stop < k).sum() > 20   # the early stop is exercised
    assert checked > 900
