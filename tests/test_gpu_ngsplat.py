"""GPU parity of the .ngsplat packing (efgs.ngsplat.pack_textures / export_ngsplat, through the C ABI
efgs_ngsplat_pack) against the CPU oracle (oracle/ngsplat_oracle.py, pinned in test_ngsplat_oracle).

Bars:
  culling         the kept set and its order equal the oracle's
  integer codes   rgb8 base, a8 opacity, log-scale, octahedral u / v / angle and SH codes equal the oracle's,
                  except a code one step away whose pre-round value lies within 1e-3 of a rounding boundary
                  (where a last-bit difference of exp / log / acos / sin decides); such cases stay below 0.1%
  fp16 positions  bit-exact
  fp16 payloads   within one fp16 ulp plus 2^-22 of the oracle's (SV / NASG / NASGabor / stored features: a
                  lobe frame component formed by cancellation carries the float32 rounding of its terms); the baked
                  layer 0 within one ulp plus 1e-6 of sum |e_j w_j| (the dot product's summation order)
  statistics      base offset / scale and the SH level scales equal the oracle's (float32)
  file            export_ngsplat's bytes equal the oracle writer's on the same packed arrays
"""
import numpy as np
import pytest

import ngsplat_oracle as ON
from efgs.synthetic import NGSPLAT_NEURAL_CASES as NEURAL_CASES, NGSPLAT_OTHER_CASES as OTHER_CASES
from efgs.synthetic import ngsplat_model as make_case

pytestmark = pytest.mark.gpu


def _device(m):
    import torch
    dev = torch.device('cuda:0')
    return {k: torch.tensor(v, device=dev) for k, v in m.items()}


def _pack(m, plan):
    from efgs import ngsplat as NG
    t = _device(m)
    out = NG.pack_textures(t['means'], t['raw_scales'], t['raw_rotations'], t['raw_opacities'], t['base_colors'], t['residual_params'], plan)
    host = dict(out)
    host['splat_words'] = out['splat_words'].cpu().numpy().view(np.uint32)
    host['textures'] = [x.cpu().numpy().view(np.uint32) for x in out['textures']]
    host['source_index'] = out['source_index'].cpu().numpy()
    return host


def _near_half(pre):
    f = np.asarray(pre, np.float64)
    return np.abs(f - np.floor(f) - 0.5) < 1e-3


def _codes(name, got, want, pre, stats):
    got, want = np.asarray(got, np.int64), np.asarray(want, np.int64)
    bad = got != want
    stats['fields'] += got.size
    if bad.any():
        assert np.all(np.abs(got[bad] - want[bad]) == 1), f'{name}: codes differ by more than one step'
        assert np.all(_near_half(np.broadcast_to(pre, got.shape)[bad])), f'{name}: a code differs away from a rounding boundary'
        stats['boundary'] += int(bad.sum())


def _fp16_ulps(got_bits, want_bits):
    g = np.asarray(got_bits, np.uint16).view(np.int16).astype(np.int64)
    w = np.asarray(want_bits, np.uint16).view(np.int16).astype(np.int64)
    # map sign-magnitude bit patterns to a monotone integer line
    g = np.where(g < 0, -(g & 0x7FFF), g)
    w = np.where(w < 0, -(w & 0x7FFF), w)
    return np.abs(g - w)


def _halves(textures, n, count):
    bits = np.concatenate([np.stack([t[:n] & 0xFFFF, t[:n] >> 16], axis=2).reshape(n, -1) for t in textures], axis=1)
    return bits[:, :count].astype(np.uint16)


def check_against_oracle(m, plan, case):
    want = ON.export(m['means'], m['raw_scales'], m['raw_rotations'], m['raw_opacities'], m['base_colors'], m['residual_params'], plan)
    got = _pack(m, plan)
    n = want['n_kept']
    print(f'case {case}: {len(m["means"])} splats, kept {n}, device kept {got["n_kept"]}', flush=True)
    assert got['n_kept'] == n
    np.testing.assert_array_equal(got['source_index'][:n], want['kept'])
    assert np.all(got['source_index'][n:] == -1)
    assert np.float32(got['base_offset']) == np.float32(want['base_offset'])
    assert np.float32(got['base_scale']) == np.float32(want['base_scale'])
    gw, ww = got['splat_words'], want['splat_words']
    assert gw.shape == ww.shape and np.all(gw[n:] == 0)
    gw, ww = gw[:n], ww[:n]
    stats = dict(fields=0, boundary=0)
    for c in range(3):
        _codes('base', (gw[:, 0] >> (8 * c)) & 0xFF, (ww[:, 0] >> (8 * c)) & 0xFF, want['base_pre'][:, c], stats)
    _codes('opacity', gw[:, 0] >> 24, ww[:, 0] >> 24, want['opacity_pre'], stats)
    np.testing.assert_array_equal(gw[:, 1], ww[:, 1])
    np.testing.assert_array_equal(gw[:, 2] & 0xFFFF, ww[:, 2] & 0xFFFF)
    for c in range(3):
        _codes('scale', (gw[:, 3] >> (8 * c)) & 0xFF, (ww[:, 3] >> (8 * c)) & 0xFF, want['scale_pre'][:, c], stats)
    _codes('quat u', (gw[:, 2] >> 16) & 0xFF, (ww[:, 2] >> 16) & 0xFF, want['quat_pre'][:, 0], stats)
    _codes('quat v', gw[:, 2] >> 24, ww[:, 2] >> 24, want['quat_pre'][:, 1], stats)
    _codes('quat angle', gw[:, 3] >> 24, ww[:, 3] >> 24, want['quat_pre'][:, 2], stats)
    assert len(got['textures']) == len(want['textures'])
    if plan['payload'] == 2:
        assert [np.float32(s) for s in got['sh_level_scales']] == [np.float32(s) for s in want['sh_level_scales']]
        for (degree, bits, _), gt, wt, pre in zip(ON.SH_LEVELS, got['textures'], want['textures'], want['sh_pre']):
            assert np.all(gt[n:] == 0)
            for f in range(3 * (2 * degree + 1)):
                _codes(f'sh{degree}', ON.decode_sh_field(gt[:n], bits, f), ON.decode_sh_field(wt[:n], bits, f), pre[:, f], stats)
    else:
        count = want['values'].shape[1]
        g16 = _halves(got['textures'], n, count)
        w16 = want['values'].astype(np.float16).view(np.uint16)
        for t in got['textures']:
            assert np.all(t[n:] == 0)
        if plan['payload'] == 1:
            g = g16.view(np.float16).astype(np.float64)
            w = want['values'].astype(np.float64)
            ulp = np.abs(np.spacing(want['values'].astype(np.float16))).astype(np.float64)
            tol = ulp + 1e-6 * want['bake_magnitude']
            assert np.all(np.abs(g - w) <= tol), f'baked layer 0: max excess {np.max(np.abs(g - w) - tol):.3e}'
        else:
            d = _fp16_ulps(g16, w16)
            g = g16.view(np.float16).astype(np.float64)
            w = w16.view(np.float16).astype(np.float64)
            tol = np.abs(np.spacing(w16.view(np.float16))).astype(np.float64) + 2.0 ** -22
            worst = np.unravel_index(np.argmax(np.abs(g - w) - tol), g.shape)
            print(f'case {case}: fp16 values differing: {int((d > 0).sum())} of {d.size}, max {int(d.max())} ulp; worst column '
                  f'{worst[1]}: {g[worst]:.6e} vs {w[worst]:.6e}', flush=True)
            assert np.all(np.abs(g - w) <= tol)
            assert (d > 0).mean() < 1e-2
    print(f'case {case}: boundary codes {stats["boundary"]} of {stats["fields"]}', flush=True)
    assert stats['boundary'] <= 1e-3 * stats['fields']
    return want, got


@pytest.mark.parametrize('name', list(NEURAL_CASES) + list(OTHER_CASES))
def test_pack_matches_oracle(name):
    m, plan, _ = make_case(name, n=20000, seed=21)
    check_against_oracle(m, plan, name)


@pytest.mark.parametrize('acts', [('softplus', 'softplus', 'none'), ('none', 'sigmoid', 'exp')])
def test_pack_activations(acts):
    residual_act, color_act, base_act = acts
    for name in ('sv7', 'nasgabor2', 'baked'):
        m, plan, _ = make_case(name, n=5000, seed=4, residual_act=residual_act, color_act=color_act, base_act=base_act)
        check_against_oracle(m, plan, f'{name}/{"/".join(acts)}')


@pytest.mark.parametrize('name', ['sh3', 'baked'])
def test_pack_full_size(name):
    """1M splats, a c3-sized model."""
    m, plan, _ = make_case(name, n=1_000_000, seed=9)
    check_against_oracle(m, plan, f'{name}_1M')


def test_export_file_matches_oracle_writer(tmp_path):
    import torch
    from efgs import ngsplat as NG
    for name in ('baked', 'sh3', 'nasg5'):
        m, plan, mlp = make_case(name, n=7000, seed=17)
        t = _device(m)
        cams = np.random.default_rng(3).normal(size=(2, 18)).astype(np.float32)
        path = str(tmp_path / f'{name}.ngsplat')
        summary = NG.export_ngsplat(path, t['means'], t['raw_scales'], t['raw_rotations'], t['raw_opacities'], t['base_colors'],
                                    t['residual_params'], plan['config'], mlp_params=mlp, test_cameras=cams, proper_antialiasing=True)
        got = _pack(m, plan)
        kept_means = m['means'][got['source_index'][:got['n_kept']]]
        c, u, d = NG.camera_hint(kept_means, cams)
        ref = str(tmp_path / f'{name}_oracle.ngsplat')
        ON.write_file(ref, plan, got, c, u, d, cams, proper_antialiasing=True)
        assert open(path, 'rb').read() == open(ref, 'rb').read()
        h, texels, splat, textures = ON.read_file(path)
        assert h['num_splats'] == summary['n_splats'] == got['n_kept']
        assert summary['bytes'] == len(open(path, 'rb').read())
        torch.cuda.synchronize()


def test_empty_and_all_culled(tmp_path):
    from efgs import ngsplat as NG
    m, plan, mlp = make_case('sh3', n=100, seed=1)
    m['raw_opacities'][:] = -20.0
    got = _pack(m, plan)
    assert got['n_kept'] == 0 and got['splat_words'].shape == (0, 4)
    e = {k: v[:0] for k, v in m.items()}
    got = _pack(e, plan)
    assert got['n_kept'] == 0
    t = _device(m)
    path = str(tmp_path / 'empty.ngsplat')
    NG.export_ngsplat(path, t['means'], t['raw_scales'], t['raw_rotations'], t['raw_opacities'], t['base_colors'], t['residual_params'],
                      plan['config'])
    h, _, splat, textures = ON.read_file(path)
    assert h['num_splats'] == 0 and splat.shape == (0, 4) and all(x.shape[0] == 0 for x in textures)
