"""The .ngsplat oracle (oracle/ngsplat_oracle.py) and the exporter's host-side planning (efgs.ngsplat) on the CPU.

Pins of the oracle's restatement of viewer/export_ngsplat.py:
  - hand-computed codes: log-scale codes at the range ends and mid-range, quaternion codes of the identity and
    of half turns, culling exactly at sigmoid(x) >= 1/255;
  - the viewer's decoders (viewer/shaders/splat_decode.glsl) invert the splat words within the quantisation
    steps: rgb8 base and a8 opacity within half a step, fp16 positions exactly, log scales within half a log step,
    rotations within the 8-bit axis / angle resolution;
  - SH fields read back with the shader's own shift expressions (viewer/shaders/eval_sh.glsl) dequantise to the
    coefficients within half a quantisation step;
  - the viewer's MLP loop over the weight texels (viewer/shaders/eval_neural.glsl) equals the matrix product of the
    fp16 weights, and the baked layout (stored h0_static + direction columns) equals the full evaluation up to the
    fp16 rounding of h0_static;
  - the NASG / NASGabor lobe frames are orthonormal, SV sites unit length (a dropped term or a wrong sign breaks
    these), the normalisation constant matches its closed form;
  - header fields written by the oracle come back through the viewer's parser (viewer/utils.js:230-330).
"""
import math

import numpy as np
import pytest

from efgs import ngsplat as NG
from efgs.synthetic import NGSPLAT_NEURAL_CASES as NEURAL_CASES, mlp_flat
from efgs.synthetic import ngsplat_model as make_case
import ngsplat_oracle as ON

def _export(m, plan):
    return ON.export(m['means'], m['raw_scales'], m['raw_rotations'], m['raw_opacities'], m['base_colors'], m['residual_params'], plan)


def test_scale_codes_known_values():
    s = np.array([[math.exp(-12.0), math.exp(9.0), 0.0], [math.exp(-1.5), math.exp(20.0), math.exp(-30.0)]], np.float32)
    code, _ = ON.encode_scales(s)
    # ln s = -12 -> 0 steps -> code 1; ln s = 9 -> 254 steps -> 255; exactly 0 -> 0; ln s = -1.5 -> 10.5 * 254 / 21 = 127 -> 128;
    # above the range clamps to 255; below it to 1
    assert code.tolist() == [[1, 255, 0], [128, 255, 1]]


def test_quaternion_codes_known_values():
    q = np.array([[0.0, 0.0, 0.0, 1.0],    # identity: degenerate axis -> (1, 0, 0), angle 0
                  [0.0, 0.0, 1.0, 0.0],    # half turn about z: axis (0, 0, 1) -> u = v = 127.5 -> 128 (half to even), angle 255
                  [1.0, 0.0, 0.0, 0.0],    # half turn about x: u = 255, v = 127.5 -> 128
                  [0.0, 0.0, -1.0, 0.0]],  # half turn about -z: w = 0 keeps the sign, z < 0 folds: u = v = (1 - 0) * 1 -> 255
                 np.float32)
    code, _ = ON.encode_quat(q)
    u, v, a = code & 0xFF, (code >> 8) & 0xFF, code >> 16
    assert u.tolist() == [255, 128, 255, 255]
    assert v.tolist() == [128, 128, 128, 255]
    assert a.tolist() == [0, 255, 255, 255]


def test_culling_threshold():
    x = np.array([-10.0, math.log((1 / 255) / (1 - 1 / 255)) + 1e-4, math.log((1 / 255) / (1 - 1 / 255)) - 1e-4, 0.0], np.float32)
    o, _, _ = ON.activated(np.zeros((4, 3), np.float32), np.tile([1, 0, 0, 0], (4, 1)).astype(np.float32), x)
    assert (o >= ON.MIN_ALPHA).tolist() == [False, True, False, True]


@pytest.mark.parametrize('name', ['sh3', 'baked'])
def test_splat_words_decode_within_quantisation(name):
    m, plan, _ = make_case(name, n=4000, seed=3)
    out = _export(m, plan)
    kept = out['kept']
    o, s, q = ON.activated(m['raw_scales'], m['raw_rotations'], m['raw_opacities'])
    np.testing.assert_array_equal(kept, np.nonzero(o >= ON.MIN_ALPHA)[0])
    n = out['n_kept']
    assert 0 < n < len(o) and out['rows'] % 2048 == 0 and np.all(out['splat_words'][n:] == 0)
    rgba, pos, scales, quat = ON.decode_splats(out['splat_words'][:n])
    base = plan['color_shift'] + m['base_colors'][kept].astype(np.float64)
    decoded_base = out['base_offset'] + (rgba[:, :3] * 255.0) * out['base_scale']
    assert np.abs(decoded_base - base).max() <= 0.5 * out['base_scale'] * (1 + 1e-4)
    assert np.abs(rgba[:, 3] - o[kept]).max() <= 0.5 / 255 + 1e-6
    np.testing.assert_array_equal(pos, m['means'][kept].astype(np.float16).astype(np.float32))
    ln = np.log(s[kept].astype(np.float64))
    inside = (ln > -12.0) & (ln < 9.0)
    assert np.abs(np.log(scales[inside]) - ln[inside]).max() <= 0.5 * 21.0 / 254.0 + 1e-4
    qk = q[kept].astype(np.float64)
    qk /= np.linalg.norm(qk, axis=1, keepdims=True)
    dot = np.abs((quat * qk).sum(axis=1))
    # 8-bit angle (pi / 255) and 8 + 8-bit octahedral axis: rotations agree within a few degrees
    assert 2.0 * np.degrees(np.arccos(np.minimum(dot, 1.0))).max() < 6.0


def test_sh_fields_through_the_shader_shifts():
    m, plan, _ = make_case('sh3', n=2000, seed=5)
    out = _export(m, plan)
    n, kept = out['n_kept'], out['kept']
    assert len(out['textures']) == 3 and [t.shape[1] for t in out['textures']] == [2, 4, 4]
    coefs = m['residual_params'][kept]
    offset = 0
    for (degree, bits, _), tex, scale in zip(ON.SH_LEVELS, out['textures'], out['sh_level_scales']):
        width = 2 * degree + 1
        qmax = (1 << (bits - 1)) - 1
        want = coefs[:, offset:offset + width, :].reshape(n, -1)
        fields = np.stack([ON.decode_sh_field(tex[:n], bits, f) for f in range(3 * width)], axis=1)
        assert np.abs(fields).max() <= qmax
        assert np.abs(fields * (scale / qmax) - want).max() <= 0.5 * scale / qmax * (1 + 1e-4)
        offset += width
    # fields 3 and 4 of degree 1, literally as eval_sh.glsl:30-31 decodes them
    w = out['textures'][0][:n].astype(np.uint32)
    f3 = (w[:, 0] << np.uint32(4)).astype(np.int32) >> 25
    f4 = ((w[:, 0] >> np.uint32(3)) | (w[:, 1] << np.uint32(29))).astype(np.int32) >> 25
    np.testing.assert_array_equal(f3, ON.decode_sh_field(w, 7, 3))
    np.testing.assert_array_equal(f4, ON.decode_sh_field(w, 7, 4))


def _direction_values(dirs, degrees):
    """Real SH basis values of degrees >= 1 for unit directions (closed forms of degrees 1 and 2, and the degree-3
    polynomials), in the tcnn order the rasterizer's MLP input uses."""
    x, y, z = dirs[:, 0], dirs[:, 1], dirs[:, 2]
    vals = {1: [-0.48860251190291987 * y, 0.48860251190291987 * z, -0.48860251190291987 * x],
            2: [1.0925484305920792 * x * y, -1.0925484305920792 * y * z, 0.94617469575755997 * z * z - 0.31539156525251999,
                -1.0925484305920792 * x * z, 0.54627421529603959 * (x * x - y * y)],
            3: [0.59004358992664352 * y * (-3.0 * x * x + y * y), 2.8906114426405538 * x * y * z, 0.45704579946446572 * y * (1.0 - 5.0 * z * z),
                0.3731763325901154 * z * (5.0 * z * z - 3.0), 0.45704579946446572 * x * (1.0 - 5.0 * z * z),
                1.4453057213202769 * z * (x * x - y * y), 0.59004358992664352 * x * (-x * x + 3.0 * y * y)]}
    return np.stack(sum((vals[d] for d in degrees), []), axis=1)


@pytest.mark.parametrize('name', list(NEURAL_CASES))
def test_weight_texels_through_the_viewer_mlp(name):
    m, plan, _ = make_case(name, n=600, seed=7)
    out = _export(m, plan)
    n, kept = out['n_kept'], out['kept']
    rng = np.random.default_rng(1)
    dirs = rng.normal(size=(n, 3))
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    degrees = plan['direction_degrees']
    dvals = _direction_values(dirs, degrees)
    feats = m['residual_params'][kept].astype(np.float64)
    if plan['base_input']:
        feats = np.concatenate([feats, m['base_colors'][kept]], axis=1)
    enc = ON.frequency_encode(feats.astype(np.float32), plan['n_frequencies']).astype(np.float64)
    full_in = np.concatenate([enc] + ([np.full((n, 1), ON.SH_C0)] if plan['sh0'] else []) + [dvals], axis=1)
    h = full_in
    for i, w in enumerate(plan['matrices']):
        h = h @ w.astype(np.float16).astype(np.float64).T
        if i < len(plan['matrices']) - 1:
            h = np.maximum(h, 0.0)
    nn, nh = plan['header_neurons'], plan['header_hidden']
    if plan['use_baked']:
        h0 = out['values'].astype(np.float16).astype(np.float64)
        l0 = -(-dvals.shape[1] // 4) * 4
        inputs = np.zeros((n, l0))
        inputs[:, :dvals.shape[1]] = dvals
        got = ON.shader_mlp(plan['weight_texels'], inputs, nn, nh, h0=h0)
        # h0_static is stored in fp16: the difference stays within its rounding, propagated through the layers
        assert np.abs(got - h).max() <= 2e-2 * max(1.0, np.abs(h).max())
        # and the unrounded bake equals the full layer 0 on the static inputs
        w0 = plan['matrices'][0].astype(np.float16).astype(np.float64)
        static = enc @ w0[:, :enc.shape[1]].T + (ON.SH_C0 * w0[:, enc.shape[1]] if plan['sh0'] else 0.0)
        np.testing.assert_allclose(out['values'], static, rtol=1e-5, atol=1e-5)
    else:
        l0 = full_in.shape[1]
        assert l0 % 4 == 0
        stored = out['values'].astype(np.float16).astype(np.float64)
        inputs = np.concatenate([stored] + ([np.full((n, 1), ON.SH_C0)] if plan['sh0'] else []) + [dvals], axis=1)
        got = ON.shader_mlp(plan['weight_texels'], inputs, nn, nh)
        h_stored = inputs
        for i, w in enumerate(plan['matrices']):
            h_stored = h_stored @ w.astype(np.float16).astype(np.float64).T
            if i < len(plan['matrices']) - 1:
                h_stored = np.maximum(h_stored, 0.0)
        np.testing.assert_allclose(got, h_stored, rtol=1e-9, atol=1e-9)


def test_weight_texel_order_is_not_transposed():
    """A 4 x 8 layer: texel j * out + o holds W[o, 4j:4j+4]."""
    w = np.arange(32, dtype=np.float32).reshape(4, 8)
    t = NG.pack_weight_texels([w]).view(np.float16).astype(np.float32)
    assert t.shape == (8, 4)
    np.testing.assert_array_equal(t[0], w[0, 0:4])
    np.testing.assert_array_equal(t[3], w[3, 0:4])
    np.testing.assert_array_equal(t[4], w[0, 4:8])
    np.testing.assert_array_equal(t[7], w[3, 4:8])


@pytest.mark.parametrize('name', ['nasg5', 'nasgabor2', 'sv7'])
def test_lobe_and_site_invariants(name):
    m, plan, _ = make_case(name, n=1500, seed=11)
    out = _export(m, plan)
    v = out['values'].astype(np.float64)
    kept = out['kept']
    if name == 'sv7':
        sites = v.reshape(len(kept), -1, 7)
        np.testing.assert_allclose(np.linalg.norm(sites[..., :3], axis=-1), 1.0, atol=1e-6)
        raw = m['residual_params'][kept].astype(np.float64)
        np.testing.assert_allclose(sites[..., 3], np.minimum(np.exp(raw[..., 3]), 60000.0), rtol=1e-6)
        np.testing.assert_allclose(sites[..., 4:], np.tanh(raw[..., 4:]), atol=1e-6)
        return
    per = 13 if name == 'nasgabor2' else 12
    lobes = v.reshape(len(kept), -1, per)
    fx, fz = lobes[..., 0:3], lobes[..., 3:6]
    np.testing.assert_allclose(np.linalg.norm(fx, axis=-1), 1.0, atol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(fz, axis=-1), 1.0, atol=1e-5)
    assert np.abs((fx * fz).sum(-1)).max() < 1e-5
    raw = m['residual_params'][kept].astype(np.float64)
    lam = np.minimum(np.exp(raw[..., 3]), 1e4)
    a = np.minimum(np.exp(raw[..., 4]), 1e4)
    np.testing.assert_allclose(lobes[..., 6], 2 * lam, rtol=1e-6)
    np.testing.assert_allclose(lobes[..., 7], a, rtol=1e-6)
    norm = lam * np.sqrt(1 + a) / (2 * np.pi * (1 - np.exp(-2 * lam)))
    np.testing.assert_allclose(lobes[..., per - 4], norm, rtol=1e-5)
    if per == 13:
        np.testing.assert_allclose(lobes[..., 8], (np.tanh(raw[..., 5]) + 1) * 20.0, rtol=1e-5)
    np.testing.assert_allclose(lobes[..., -3:], np.tanh(raw[..., -3:]), atol=1e-6)


@pytest.mark.parametrize('name', ['baked', 'full', 'sh3', 'sh1', 'sv7', 'nasg1', 'nasgabor2'])
def test_header_through_the_viewer_parser(tmp_path, name):
    m, plan, _ = make_case(name, n=2500, seed=13)
    out = _export(m, plan)
    cams = np.random.default_rng(2).normal(size=(3, 18)).astype(np.float32)
    path = str(tmp_path / 'o.ngsplat')
    ON.write_file(path, plan, out, [0.5, -1.0, 2.0], [0.0, -1.0, 0.0], 7.5, cams, proper_antialiasing=True)
    h, texels, splat, textures = ON.read_file(path)
    assert h['num_splats'] == out['n_kept'] and h['tex_height'] == out['rows'] // 2048
    assert h['appearance'] == plan['model'] and h['proper_aa'] and not h['base_exp']
    assert h['color_activation'] == 0 and h['residual_activation'] == 1
    assert h['base_scale'] == np.float32(out['base_scale']) and h['base_offset'] == np.float32(out['base_offset'])
    assert h['center'] == [0.5, -1.0, 2.0] and h['distance'] == 7.5
    np.testing.assert_array_equal(h['test_cameras'], cams)
    np.testing.assert_array_equal(splat, out['splat_words'])
    assert len(textures) == len(out['textures'])
    for a, b in zip(textures, out['textures']):
        np.testing.assert_array_equal(a, b)
    if plan['model'] == 'neural':
        assert h['baked'] == plan['use_baked'] and h['sh0_input'] == plan['sh0'] and h['n_neurons'] == plan['header_neurons']
        np.testing.assert_array_equal(texels, plan['weight_texels'])
    if plan['model'] == 'sh':
        assert h['sh_scales'] == [float(np.float32(s)) for s in out['sh_level_scales']]
        assert h['sh_degree_mask'] == (0b1110 if name == 'sh3' else 0b10)


def test_planning_rejects_what_the_viewer_cannot_read():
    rng = np.random.default_rng(0)
    base = dict(appearance_type='neural', sh_degrees=[0, 1], n_frequencies=0, n_neurons=32, n_hidden_layers=1)
    with pytest.raises(ValueError, match='unrepresentable'):
        NG.plan_export(base, (10, 20), mlp_flat(rng, 24, 32, 1))          # 20 stored features > 16 and 32 neurons > 16
    with pytest.raises(ValueError, match='multiple of 4'):
        NG.plan_export(base, (10, 8), mlp_flat(rng, 12, 32, 1))            # full layout: 8 + 1 + 3 = 12 ok ...
        NG.plan_export(dict(base, sh_degrees=[1]), (10, 8), mlp_flat(rng, 11, 32, 1))  # ... 8 + 3 = 11 is not
    with pytest.raises(ValueError, match='view-direction degree'):
        NG.plan_export(dict(base, sh_degrees=[0]), (10, 8), mlp_flat(rng, 9, 32, 1))
    with pytest.raises(ValueError, match='N_NEURONS'):
        NG.plan_export(dict(base, n_neurons=6), (10, 8), None)
    with pytest.raises(ValueError, match='color activation'):
        NG.plan_export(dict(appearance_type='sh', color_activation='gelu'), (10, 15, 3))
    with pytest.raises(ValueError, match='cap of 64'):
        NG.plan_export(dict(appearance_type='nasg'), (10, 6, 8))
    with pytest.raises(ValueError, match='degrees 1-3'):
        NG.plan_export(dict(appearance_type='sh'), (10, 24, 3))
    with pytest.raises(ValueError, match='softplus'):
        NG.plan_export(dict(base, n_neurons=16, residual_activation='softplus'), (10, 8), mlp_flat(rng, 12, 16, 1), active_degree=0)


def test_planning_schedule_and_flags():
    rng = np.random.default_rng(1)
    cfg = dict(appearance_type='neural', sh_degrees=[0, 1, 2, 3], n_frequencies=1, n_neurons=16, n_hidden_layers=2)
    mlp = mlp_flat(rng, 16 + 16, 16, 2)
    p = NG.plan_export(cfg, (10, 8), mlp, active_degree=1)
    # degrees 2 and 3 (layer-0 columns 16 + 1 + 3 .. 32) are zeroed, degree 1 kept
    assert np.all(p['matrices'][0][:, 20:32] == 0) and np.any(p['matrices'][0][:, 17:20] != 0)
    assert p['degree_mask'] == 0b1110 and p['flags'] == 4 and p['use_baked']
    p0 = NG.plan_export(cfg, (10, 8), mlp, active_degree=0)
    assert np.all(p0['matrices'][-1] == 0)
    sh = NG.plan_export(dict(appearance_type='sh', base_activation='exp'), (10, 15, 3), active_degree=2)
    assert sh['n_items'] == 8 and sh['degree_mask'] == 0b110 and sh['flags'] == (1 << 3) | 32 and sh['color_shift'] == 0.0
    g = NG.plan_export(dict(appearance_type='nasgabor', color_activation='sigmoid'), (10, 3, 9), active_degree=2)
    assert g['n_items'] == 2 and g['n_values'] == 26 and g['flags'] == (0 << 3) | (1 << 6) and g['color_shift'] == 0.0
    assert NG.plan_export(dict(appearance_type='sv'), (10, 7, 7))['flags'] == 2 << 3
