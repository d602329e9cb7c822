"""Pins the CPU oracle (CPU only).

* deterministic exp / log / exp2 against libm in float64 (ulp bounds, special values);
* the tile-contribution test against brute force where the reference's closest-edge search is exact;
* the SH bases (rest bands of the SH model and the neural direction encoding, degrees 0-6) against
  orthonormality on the sphere by quadrature, and degree-1 values against the textbook formulas;
* appearance special cases that reduce to closed forms (one SV site, NASG on the lobe pole / antipole);
* the analytic backward of the C oracle against autograd of the independent torch restatement, for every
  appearance model and activation family, and the torch restatement's image against the oracle's;
* Adam against torch.optim.Adam (scalar learning rate) and a float64 restatement (learning-rate lists);
* sort / scan invariants of the forward state.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
import torch_ref as TR
from helpers import small_case, rel_l2, single_tile_state


def _ulps(got, ref):
    ref32 = np.abs(ref).astype(np.float32)
    return np.abs(np.asarray(got, np.float64) - ref) / np.spacing(ref32).astype(np.float64)


def test_ef_exp_accuracy():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-87.0, 88.7, 20000), np.linspace(-1, 1, 2001)]).astype(np.float32)
    got = np.array([O.ef_exp(float(x)) for x in xs])
    assert _ulps(got, np.exp(xs.astype(np.float64))).max() <= 1.5
    assert O.ef_exp(0.0) == 1.0
    assert O.ef_exp(100.0) == math.inf
    assert O.ef_exp(-200.0) == 0.0


def test_ef_log_accuracy():
    rng = np.random.default_rng(1)
    ys = np.concatenate([rng.uniform(1e-3, 1e3, 20000), np.geomspace(1e-30, 1e30, 2001), np.linspace(0.5, 2.0, 2001)]).astype(np.float32)
    got = np.array([O.ef_log(float(y)) for y in ys])
    ref = np.log(ys.astype(np.float64))
    err = np.abs(got - ref)
    tol = np.maximum(2.5 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64), 1e-9)
    assert (err <= tol).all()
    assert O.ef_log(1.0) == 0.0
    assert O.ef_log(0.0) == -math.inf


def test_ef_exp2_accuracy():
    xs = np.concatenate([np.linspace(-126, 0, 200001), np.linspace(-1, 0, 20001)]).astype(np.float32)
    got = np.array([O.ef_exp2(float(x)) for x in xs[::7]])
    ref = np.exp2(xs[::7].astype(np.float64))
    normal = ref >= 2.0 ** -126
    assert _ulps(got[normal], ref[normal]).max() <= 1.0  # the minimax polynomial stays under one ulp
    assert O.ef_exp2(0.0) == 1.0
    assert O.ef_exp2(-1.0) == 0.5
    assert O.ef_exp2(-127.0) == 0.0
    assert O.ef_exp2(-1000.0) == 0.0 and O.ef_exp2(float("nan")) == 0.0 and O.ef_exp2(-math.inf) == 0.0
    # just below -126: the subnormal 2^x (p in (0.7, 1) times 2^-126), rounded once
    sub = O.ef_exp2(-126.25)
    assert 0.0 < sub < 2.0 ** -126 and abs(sub - 2.0 ** -126.25) <= 2.0 ** -149


def _dense_max_power(mx, my, cx, cy, cz, tx, ty):
    """Minimum of 0.5 d^T C d over the continuous tile rectangle (pixel-centre coordinates), by dense sampling."""
    xs = np.linspace(tx * 16, tx * 16 + 15, 301)
    ys = np.linspace(ty * 12, ty * 12 + 11, 221)
    X, Y = np.meshgrid(xs, ys)
    dx, dy = mx - X, my - Y
    return (0.5 * (cx * dx * dx + cz * dy * dy) + cy * dx * dy).min()


def test_tile_contribution_matches_brute_force_isotropic():
    rng = np.random.default_rng(2)
    checked = 0
    for _ in range(400):
        mx, my = rng.uniform(-20, 60, 2)
        s = rng.uniform(0.2, 30.0)
        c = 1.0 / (s * s)
        pt = float(np.log(255 * rng.uniform(0.01, 1.0)))
        tx, ty = 1, 1
        q = _dense_max_power(mx, my, c, 0.0, c, tx, ty)
        if abs(q - pt) < 1e-3 * max(1.0, pt):
            continue  # too close to the threshold for the sampled minimum
        got = O.lib().efo_will_primitive_contribute(mx, my, c, 0.0, c, tx, ty, pt)
        assert bool(got) == (q <= pt), (mx, my, s, pt)
        checked += 1
    assert checked > 300


def test_tile_contribution_mean_inside_always_true():
    rng = np.random.default_rng(3)
    for _ in range(200):
        tx, ty = rng.integers(0, 10, 2)
        mx = rng.uniform(tx * 16, tx * 16 + 15)
        my = rng.uniform(ty * 12, ty * 12 + 11)
        assert O.lib().efo_will_primitive_contribute(mx, my, 1e3, 0.0, 1e3, int(tx), int(ty), 0.0)


def _sphere_quadrature(n_theta=96, n_phi=192):
    t, w = np.polynomial.legendre.leggauss(n_theta)
    phi = np.arange(n_phi) * 2 * np.pi / n_phi
    T, P = np.meshgrid(t, phi, indexing='ij')
    W = np.repeat(w[:, None], n_phi, 1) * (2 * np.pi / n_phi)
    s = np.sqrt(1 - T * T)
    d = np.stack([s * np.cos(P), s * np.sin(P), T], -1).reshape(-1, 3)
    return d, W.reshape(-1)


def test_sh_model_basis_orthonormal():
    d, w = _sphere_quadrature()
    B = np.stack([O.sh_rest_basis(x, 3) for x in d[::1]]).astype(np.float64)
    G = (B * w[:, None]).T @ B
    np.testing.assert_allclose(G, np.eye(15), atol=2e-6)


def test_neural_direction_encoding_orthonormal():
    d, w = _sphere_quadrature()
    B = O._sh_encoding64(d, (0, 1, 2, 3, 4, 5, 6), 6)
    G = (B * w[:, None]).T @ B
    np.testing.assert_allclose(G, np.eye(49), atol=1e-9)
    # degree 1 is (-c1 y, c1 z, -c1 x) with c1 = sqrt(3 / (4 pi))
    c1 = math.sqrt(3 / (4 * math.pi))
    np.testing.assert_allclose(B[:, 1:4], np.stack([-c1 * d[:, 1], c1 * d[:, 2], -c1 * d[:, 0]], 1), atol=1e-12)


def test_direction_encoding_gating():
    d = np.array([[0.6, 0.0, 0.8]])
    enc = O._sh_encoding64(d, (0, 1, 2), 1)
    assert enc[0, 0] == pytest.approx(O.SH_C0)
    assert np.all(enc[0, 4:] == 0)          # degree 2 gated off at active degree 1
    assert np.any(enc[0, 1:4] != 0)


def test_sv_single_site_is_its_colour():
    app = O.Appearance(model='sv', max_degree=1, res_act='tanh')
    p = np.array([0.3, -0.2, 0.9, 1.7, 0.4, -0.3, 0.2], np.float32)
    out = O.residual(app, p, np.array([0.0, 0.0, 1.0], np.float32), 1)
    np.testing.assert_allclose(out, np.tanh(p[4:7]), rtol=1e-6)


def test_nasg_pole_and_antipole():
    app = O.Appearance(model='nasg', max_degree=1, res_act='none')
    p = np.array([0.3, -0.7, 0.0, 0.2, 0.1, 0.5, -0.25, 0.125], np.float32)
    # lobe axis z = (cos(theta) sin(phi), sin(theta) sin(phi), cos(phi)) with cos = tanh(raw)
    ct, cp = np.tanh(np.float64(p[0])), np.tanh(np.float64(p[1]))
    st, sp = np.sqrt(1 - ct * ct), np.sqrt(1 - cp * cp)
    v = np.array([ct * sp, st * sp, cp], np.float32)
    out = O.residual(app, p, v, 1)      # direction on the lobe axis: pdf = 1
    np.testing.assert_allclose(out, p[5:8], rtol=1e-6)
    out = O.residual(app, p, -v, 1)     # antipode: pdf = 0
    np.testing.assert_array_equal(out, np.zeros(3, np.float32))


GRAD_CASES = [
    dict(model='sh'),
    dict(model='sh', acts=('exp', 'softplus', 'sigmoid')),
    dict(model='sh', acts=('none', 'tanh', 'hardsigmoid'), degree=2),
    dict(model='sh', acts=('exp', 'softplus', 'satexp'), proper_aa=True),
    dict(model='sh', direction_gradient=False),
    dict(model='precomputed'),
    dict(model='sv', scale_shift=2.5),
    dict(model='nasg', scale_shift=2.5),
    dict(model='nasgabor', acts=('none', 'tanh', 'softplus'), scale_shift=2.5),
    dict(model='neural', scale_shift=2.5),
    dict(model='neural', scale_shift=2.5, mlp=dict(n_feature_dims=5, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=16,
                                                   n_hidden_layers=2, base_input=True)),
]


@pytest.mark.parametrize('case', GRAD_CASES, ids=lambda c: '-'.join(str(v) for v in c.values()))
def test_oracle_backward_matches_autograd(case):
    scene, app, cam = small_case(n=300, width=48, height=36, **case)
    fw = O.render(scene, app, cam)
    assert len(fw.visible) > 50
    g = np.random.default_rng(3).normal(size=fw.image.shape).astype(np.float32)
    ref = O.backward(scene, app, cam, fw, g)
    img, leaves = TR.render(scene, app, cam, fw)
    assert np.abs(img.detach().numpy() - fw.image).max() < 5e-5
    (img * torch.as_tensor(g, dtype=torch.float64)).sum().backward()
    for k, t in leaves.items():
        want = t.grad.numpy()
        if np.linalg.norm(want) == 0:
            assert np.abs(ref[k]).max() == 0, k
            continue
        assert rel_l2(ref[k], want) < 1e-4, k


def test_render_base_off_backward_follows_reference_rule():
    """With render_base off the colour is |act(b + r) - act(b)|; the reference backward (preprocess_backward.cu:93-99)
    zeroes the base gradient and pulls the colour gradient back with the activation derivative evaluated at that
    stored colour. Check that rule: the residual gradients equal those of a render_base-on pass whose colour
    gradient is pre-scaled by act'(stored) / act'(full colour)."""
    scene, app, cam = small_case(model='sh', n=300, width=48, height=36, acts=('none', 'none', 'sigmoid'), render_base=False)
    fw = O.render(scene, app, cam)
    g = np.random.default_rng(3).normal(size=fw.image.shape).astype(np.float32)
    ref = O.backward(scene, app, cam, fw, g)
    assert np.abs(ref['base_colors']).max() == 0
    vis = fw.n_touched > 0
    assert np.abs(ref['residual_params'][vis]).max() > 0


def test_adam_matches_torch_scalar_lr():
    rng = np.random.default_rng(4)
    p = rng.normal(size=1000).astype(np.float32)
    tp = torch.tensor(p.copy(), requires_grad=True)
    opt = torch.optim.Adam([tp], lr=1e-2, eps=1e-15)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for step in range(1, 6):
        g = rng.normal(size=1000).astype(np.float32)
        tp.grad = torch.tensor(g)
        opt.step()
        O.adam_step(g, p, m, v, step, 1e-2, 0.9, 0.999, 1e-15)
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-5, atol=1e-6)


def test_adam_lr_list_float64():
    rng = np.random.default_rng(5)
    lrs = [1e-2, 2e-2, 3e-2, 1e-3, 5e-3, 5e-3, 5e-3]
    p = rng.normal(size=(100, 7)).astype(np.float32)
    p64 = p.astype(np.float64).copy()
    m64 = np.zeros_like(p64)
    v64 = np.zeros_like(p64)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for step in range(1, 4):
        g = rng.normal(size=p.shape).astype(np.float32)
        O.adam_step(g, p, m, v, step, lrs, 0.9, 0.999, 1e-15)
        m64 = 0.9 * m64 + 0.1 * g
        v64 = 0.999 * v64 + 0.001 * g.astype(np.float64) ** 2
        lr = np.array(lrs)[None, :]
        p64 -= lr / (1 - 0.9 ** step) * m64 / (np.sqrt(v64) / np.sqrt(1 - 0.999 ** step) + 1e-15)
        np.testing.assert_allclose(p, p64, rtol=1e-5, atol=1e-6)


def test_forward_state_invariants():
    scene, app, cam = small_case(model='sh', n=2000, width=96, height=80, scale_shift=1.5)
    fw = O.render(scene, app, cam)
    gw, gh = cam.grid()
    # depth order is sorted, ties in primitive-index order
    keys = fw.depth_key[fw.depth_sorted]
    assert np.all(np.diff(keys.astype(np.int64)) >= 0)
    ties = np.diff(keys.astype(np.int64)) == 0
    assert np.all(np.diff(fw.depth_sorted.astype(np.int64))[ties] > 0)
    # instance keys sorted and ranges consistent
    assert np.all(np.diff(fw.inst_keys.astype(np.int64)) >= 0)
    for t in range(gw * gh):
        s, e = fw.ranges[t]
        assert np.all(fw.inst_keys[s:e] == t)
    assert fw.ranges[:, 1].max() == len(fw.inst_keys)
    # touched-tile counts bounded by the tile rectangle
    b = fw.bounds.astype(np.int64)
    area = ((b[:, 1] + 15) // 16 - b[:, 0] // 16) * ((b[:, 3] + 11) // 12 - b[:, 2] // 12)
    assert np.all(fw.n_touched <= np.maximum(area, 0))
    # transmittance in [0, 1]; empty tiles show the background
    assert fw.final_T.min() >= 0 and fw.final_T.max() <= 1


DECODE_MLPS = {
    'c2': dict(n_feature_dims=8, n_frequencies=0, sh_degrees=(1,), n_neurons=64, n_hidden_layers=2, base_input=False),
    'base_freq': dict(n_feature_dims=5, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=32, n_hidden_layers=3, base_input=True),
}


@pytest.mark.parametrize('name', list(DECODE_MLPS))
def test_neural_decode_matches_autograd(name):
    """The standalone decode statement (encoding + fp16 MLP + their backward) against autograd of the
    independent torch restatement (straight-through fp16 rounding), in float64."""
    from efgs.synthetic import xavier_mlp
    mlp = O.MLPConfig(**DECODE_MLPS[name])
    rng = np.random.default_rng(11)
    n = 400
    feat = rng.normal(0.0, 0.5, size=(n, mlp.n_feature_dims)).astype(np.float32)
    base = rng.normal(0.0, 0.5, size=(n, 3)).astype(np.float32)
    d = rng.normal(size=(n, 3)).astype(np.float32)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    w = xavier_mlp(rng, mlp.n_input_dims, mlp.n_neurons, mlp.n_hidden_layers)
    dy = rng.normal(size=(n, 3)).astype(np.float32)
    y, acts, mats = O.neural_decode(feat, base, d, w, mlp, 1)
    ref = O.neural_decode_backward(feat, base, d, dy, mats, acts, mlp, 1)
    tf, tb, td, tw = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (feat, base, d, w))
    out = TR.neural_residual(tf, tb, td, mlp, TR.mlp_matrices_torch(tw, mlp), 1, 'none')
    assert np.abs(out.detach().numpy() - y).max() < 2e-3
    (out * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    assert rel_l2(ref['features'], tf.grad.numpy()) < 1e-4
    assert rel_l2(ref['weights'], tw.grad.numpy()) < 1e-4
    assert rel_l2(ref['dirs'], td.grad.numpy()) < 1e-4
    if mlp.base_input:
        assert rel_l2(ref['base'], tb.grad.numpy()) < 1e-4


# ---------------------------------------------------------------------------------------------------------
# MCMC densification (B/densification/include/kernels_mcmc.cuh:11-146)
# ---------------------------------------------------------------------------------------------------------

# Random123 known-answer vectors of philox4x32 with 10 rounds: (counter, key, output)
PHILOX_KAT = [
    ([0x00000000] * 4, [0x00000000] * 2, [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0], [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
]


@pytest.mark.parametrize('case', range(len(PHILOX_KAT)))
def test_philox_known_answers(case):
    ctr, key, want = PHILOX_KAT[case]
    np.testing.assert_array_equal(O.philox4x32_10(ctr, key), np.array(want, np.uint32))


def test_box_muller_closed_forms_and_moments():
    """u = 1 (bits 0xffffffff) gives radius 0; u = 2^-33 (bits 0) radius sqrt(66 ln 2); the angle word maps
    [0, 2^32) onto [0, 2 pi). Samples from consecutive Philox counters have zero mean, unit variance and no
    correlation between the two outputs (tolerances ~5 standard errors at 40,000 samples)."""
    np.testing.assert_allclose(O.box_muller(0xffffffff, 12345), [0.0, 0.0], atol=1e-6)
    r = math.sqrt(66.0 * math.log(2.0))
    np.testing.assert_allclose(O.box_muller(0, 0), [r, 0.0], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.box_muller(0, 1 << 30), [0.0, r], rtol=1e-5, atol=2e-5)  # angle pi / 2
    np.testing.assert_allclose(O.box_muller(0, 1 << 31), [-r, 0.0], rtol=1e-5, atol=3e-5)  # angle pi
    z = []
    for i in range(10000):
        b = O.philox4x32_10([i, 0, 7, 0], [1234, 5678])
        z.append(O.box_muller(int(b[0]), int(b[1])))
        z.append(O.box_muller(int(b[2]), int(b[3])))
    z = np.array(z, np.float64)
    n = z.shape[0]
    assert np.all(np.abs(z.mean(0)) < 5 / math.sqrt(n))
    assert np.all(np.abs(z.var(0) - 1.0) < 5 * math.sqrt(2.0 / n))
    assert abs(np.corrcoef(z[:, 0], z[:, 1])[0, 1]) < 5 / math.sqrt(n)


def _noise_direct(raw_scales, rot64, raw_opacities, lr, seed, offset):
    """Expected noise step in float64 from an independent rotation matrix (axis-angle), the oracle's Philox
    words and Box-Muller samples."""
    n = raw_scales.shape[0]
    out = np.zeros((n, 3))
    for i in range(n):
        b = O.philox4x32_10([offset // 4 & 0xffffffff, offset // 4 >> 32, i, 0], [seed & 0xffffffff, seed >> 32])
        zxy, zz = O.box_muller(int(b[0]), int(b[1])), O.box_muller(int(b[2]), int(b[3]))
        z = np.array([zxy[0], zxy[1], zz[0]], np.float64)
        R = rot64[i]
        sigma = R @ np.diag(np.exp(2.0 * raw_scales[i].astype(np.float64))) @ R.T
        o = 1.0 / (1.0 + math.exp(-float(raw_opacities[i])))
        f = lr / (1.0 + math.exp(100.0 * o - 0.5))
        out[i] = f * (sigma @ z)
    return out


def _axis_angle(axis, angle):
    a = np.asarray(axis, np.float64)
    a = a / np.linalg.norm(a)
    K = np.array([[0, -a[2], a[1]], [a[2], 0, -a[0]], [-a[1], a[0], 0]])
    return np.eye(3) + math.sin(angle) * K + (1 - math.cos(angle)) * K @ K


def test_add_noise_against_direct_statement():
    """Quaternion (w, x, y, z) = (cos(t/2), sin(t/2) axis) scaled by arbitrary factors (the kernel normalises
    through |q|^2) must give Sigma = R(axis, t) diag(e^{2s}) R^T; a zero quaternion leaves the mean
    unchanged; the opacity factor follows sigmoid(-(100 o - 0.5))."""
    rng = np.random.default_rng(3)
    n = 64
    axes = rng.normal(size=(n, 3))
    angles = rng.uniform(-math.pi, math.pi, n)
    scale = rng.uniform(0.5, 3.0, n)
    q = np.stack([np.cos(angles / 2), *(np.sin(angles / 2)[None] * (axes / np.linalg.norm(axes, axis=1, keepdims=True)).T)], 1) * scale[:, None]
    q[5] = 0.0
    rot = np.stack([_axis_angle(axes[i], angles[i]) for i in range(n)])
    raw_scales = rng.normal(-2.0, 0.5, (n, 3)).astype(np.float32)
    raw_op = rng.normal(-5.0, 2.0, n).astype(np.float32)  # a spread of opacity factors (opaque ones get ~0)
    means = rng.uniform(-3, 3, (n, 3)).astype(np.float32)
    seed, offset, lr = 0x1234_5678_9abc_def0, 4 * 77, 0.37
    got = O.add_noise(raw_scales, q.astype(np.float32), raw_op, means, lr, seed, offset) - means.astype(np.float64)
    want = _noise_direct(raw_scales, rot, raw_op, lr, seed, offset)
    want[5] = 0.0
    assert np.all(got[5] == 0.0)
    assert rel_l2(got, want) < 1e-4
    # float32 rounding of the mean update: at most one ulp of the mean plus 1e-5 of the step
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=float(np.abs(means).max()) * 2.0 ** -22)


def test_relocation_closed_forms():
    """The coefficient table equals C(m, k) (-1)^k / sqrt(k + 1) (math.comb, float64); one sample keeps the
    Gaussian (o' = o, scales unchanged); two samples follow o' = 1 - sqrt(1 - o), factor o / (2 o' - o'^2 /
    sqrt(2)); counts clamp to 1..50; the split opacities compose back, 1 - (1 - o')^n = o."""
    t = O.relocation_table()
    want = np.zeros((50, 50))
    for m in range(50):
        for k in range(m + 1):
            want[m, k] = math.comb(m, k) * (-1) ** k / math.sqrt(k + 1)
    np.testing.assert_allclose(t, want.astype(np.float32), rtol=1e-7, atol=0)
    o = np.array([0.01, 0.3, 0.5, 0.9, 0.999, 0.3, 0.3], np.float32)
    s = np.tile(np.array([[0.1, 0.2, 0.05]], np.float32), (7, 1))
    c = np.array([1, 1, 2, 2, 2, 0, 80], np.int64)
    no, ns = O.relocation_adjustment(o, s, c)
    np.testing.assert_allclose(no[:2, 0], o[:2], rtol=1e-6)
    np.testing.assert_allclose(ns[:2], s[:2], rtol=1e-6)
    o2 = 1.0 - np.sqrt(1.0 - o[2:5].astype(np.float64))
    np.testing.assert_allclose(no[2:5, 0], o2, rtol=1e-5)
    f2 = o[2:5] / (2 * o2 - o2 ** 2 / math.sqrt(2.0))
    np.testing.assert_allclose(ns[2:5], s[2:5] * f2[:, None], rtol=1e-5)
    np.testing.assert_allclose(no[5], no[0] * 0 + o[5], rtol=1e-6)  # count 0 clamps to 1
    o50 = 1.0 - (1.0 - 0.3) ** (1.0 / 50.0)
    np.testing.assert_allclose(no[6, 0], o50, rtol=1e-4)  # count 80 clamps to 50
    rng = np.random.default_rng(5)
    oo = rng.uniform(0.05, 0.99, 500).astype(np.float32)
    cc = rng.integers(1, 51, 500)
    no, _ = O.relocation_adjustment(oo, np.ones((500, 3), np.float32), cc)
    np.testing.assert_allclose(1.0 - (1.0 - no[:, 0].astype(np.float64)) ** cc, oo, rtol=3e-4)


# ---------------------------------------------------------------------------------------------------------
# pruning scores (B/rasterization/include/kernels_pruning_scores.cuh:11-171)
# ---------------------------------------------------------------------------------------------------------

def _random_2d_gaussians(rng, k):
    mean2d = rng.uniform([1.0, 1.0], [15.0, 11.0], (k, 2)).astype(np.float32)
    co = np.zeros((k, 4), np.float32)
    for i in range(k):
        a = rng.normal(size=(2, 2))
        cov = a @ a.T * 4.0 + np.eye(2) * 1.5
        inv = np.linalg.inv(cov)
        co[i] = [inv[0, 0], inv[0, 1], inv[1, 1], rng.uniform(0.3, 0.95)]
    color = rng.uniform(0.0, 1.0, (k, 3)).astype(np.float32)
    return mean2d, co, color


def test_pruning_scores_match_autograd():
    """The score of a Gaussian is sum over pixels of (dL/dG)^2 (alpha = o G, so o dL/dalpha = dL/dG) for
    L = sum of the image: autograd through a float64 front-to-back composite of per-pixel Gaussian values,
    with the float32 walk's skip (alpha < 1/255) and stop (last contributor) decisions."""
    rng = np.random.default_rng(21)
    k = 6
    mean2d, co, color = _random_2d_gaussians(rng, k)
    bg = np.array([0.2, 0.5, 0.1], np.float32)
    cam, fw = single_tile_state(mean2d, co, color, bg)
    got = O.pruning_scores(cam, fw)
    log2e = 1.44269504089
    ys, xs = np.mgrid[0:12, 0:16]
    px, py = xs.reshape(-1) + 0.5, ys.reshape(-1) + 0.5
    G = np.zeros((k, px.size))
    for i in range(k):
        dx, dy = mean2d[i, 0] - px, mean2d[i, 1] - py
        q = -0.5 * log2e * (co[i, 0] * dx * dx + 2 * co[i, 1] * dx * dy + co[i, 2] * dy * dy)
        G[i] = np.exp2(np.minimum(q, 0.0))
    Gt = torch.tensor(G, dtype=torch.float64, requires_grad=True)
    total = torch.zeros((), dtype=torch.float64)
    for pix in range(px.size):
        T = torch.ones((), dtype=torch.float64)
        for i in range(int(fw.n_contrib[pix])):
            a32 = np.float32(co[i, 3]) * np.float32(G[i, pix])
            if a32 < 1.0 / 255.0:
                continue
            alpha = float(co[i, 3]) * Gt[i, pix]
            total = total + T * alpha * float(color[i].sum())
            T = T * (1 - alpha)
        total = total + T * float(bg.sum())
    total.backward()
    want = (Gt.grad.numpy() ** 2).sum(1)
    np.testing.assert_allclose(got, want, rtol=2e-4)


def test_pruning_score_single_gaussian_closed_form():
    """One Gaussian over the tile: the colour still to come after it is zero and T_final = 1 - alpha, so every
    pixel it reaches scores (o (sum c - sum bg))^2, whatever its Gaussian value."""
    mean2d = np.array([[8.0, 6.0]], np.float32)
    co = np.array([[0.3, 0.02, 0.4, 0.7]], np.float32)
    color = np.array([[0.9, 0.4, 0.3]], np.float32)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    cam, fw = single_tile_state(mean2d, co, color, bg)
    n_pix = int((fw.n_contrib == 1).sum())
    assert 0 < n_pix < 192
    got = O.pruning_scores(cam, fw)
    want = n_pix * (0.7 * (color.sum() - bg.sum())) ** 2
    np.testing.assert_allclose(got, [want], rtol=1e-5)
