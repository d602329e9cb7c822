"""PLY export (efgs.export, reference Model.py:503-531 and Appearance/{Base,SH}.py ply_attributes) on the CPU:
the byte layout of the 3DGS convention, the property order, the standard SH column order, the baked base-only
columns of the other configurations, and a write/read round trip."""
import struct

import numpy as np
import pytest

from efgs import export as E


def _model(rng, n=37):
    return dict(means=rng.normal(size=(n, 3)).astype(np.float32), raw_scales=rng.normal(-3, 1, (n, 3)).astype(np.float32),
                raw_rotations=rng.normal(size=(n, 4)).astype(np.float32) * 3.0, raw_opacities=rng.normal(size=(n, 1)).astype(np.float32),
                base_colors=rng.normal(0, 0.3, (n, 3)).astype(np.float32), residual_params=rng.normal(0, 0.05, (n, 15, 3)).astype(np.float32))


def test_sh3_layout_bytes_and_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    m = _model(rng)
    path = str(tmp_path / 'm.ply')
    assert E.export_ply(path, **m) == 37
    raw = open(path, 'rb').read()
    names = (['x', 'y', 'z', 'f_dc_0', 'f_dc_1', 'f_dc_2'] + [f'f_rest_{i}' for i in range(45)] + ['opacity'] +
             [f'scale_{i}' for i in range(3)] + [f'rot_{i}' for i in range(4)])
    header = ('ply\nformat binary_little_endian 1.0\nelement vertex 37\n' + ''.join(f'property float {n}\n' for n in names) +
              'end_header\n').encode()
    assert raw.startswith(header) and len(raw) == len(header) + 37 * 59 * 4
    # row 5 from the raw bytes: mean, f_dc = base / SH_C0, f_rest channel-major, raw opacity and scales, unit quaternion
    row = struct.unpack('<59f', raw[len(header) + 5 * 236:len(header) + 6 * 236])
    np.testing.assert_array_equal(row[0:3], m['means'][5])
    np.testing.assert_allclose(row[3:6], m['base_colors'][5] / E.SH_C0, rtol=1e-6)
    np.testing.assert_array_equal(row[6:21], m['residual_params'][5, :, 0])   # red bands 1..15
    np.testing.assert_array_equal(row[21:36], m['residual_params'][5, :, 1])  # green
    np.testing.assert_array_equal(row[36:51], m['residual_params'][5, :, 2])  # blue
    assert row[51] == m['raw_opacities'][5, 0]
    np.testing.assert_array_equal(row[52:55], m['raw_scales'][5])
    q = m['raw_rotations'][5].astype(np.float64)
    np.testing.assert_allclose(row[55:59], q / np.linalg.norm(q), rtol=1e-6)
    back = E.read_ply(path)
    assert back.dtype.names == tuple(names)
    np.testing.assert_array_equal(back['f_rest_44'], m['residual_params'][:, 14, 2])


@pytest.mark.parametrize('cfg', [dict(model='sh', color_act='sigmoid'), dict(model='neural', base_act='none', residual_act='tanh',
                                                                                  color_act='relu'),
                                 dict(model='nasg', base_act='exp', residual_act='tanh', color_act='none'),
                                 dict(model='sv', color_act='softplus')])
def test_base_only_columns(tmp_path, cfg):
    """Non-standard configurations store the activated base colour as degree-0 SH: 0.5 + SH_C0 f_dc is the
    colour the rasterizer would produce without the residual."""
    rng = np.random.default_rng(1)
    m = _model(rng, n=9)
    v = E.ply_vertices(**m, **cfg)
    assert [n for n in v.dtype.names if n.startswith('f_')] == ['f_dc_0', 'f_dc_1', 'f_dc_2']
    base = m['base_colors'].astype(np.float64)
    if cfg.get('base_act') == 'exp':
        base = np.exp(3 * base)
    act = cfg['color_act']
    want = {'sigmoid': 1 / (1 + np.exp(-4 * base)), 'relu': np.maximum(base + 0.5, 0), 'none': base + 0.5,
            'softplus': np.log1p(np.exp(10 * (base + 0.5))) / 10}[act]
    got = 0.5 + E.SH_C0 * np.stack([v['f_dc_0'], v['f_dc_1'], v['f_dc_2']], 1).astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    path = str(tmp_path / 'b.ply')
    E.write_ply(path, v)
    np.testing.assert_array_equal(E.read_ply(path), v)


def test_empty_model(tmp_path):
    path = str(tmp_path / 'e.ply')
    z = np.zeros((0, 3), np.float32)
    assert E.export_ply(path, z, z, np.zeros((0, 4), np.float32), np.zeros((0, 1), np.float32), z, np.zeros((0, 15, 3), np.float32)) == 0
    assert E.read_ply(path).shape == (0,)
