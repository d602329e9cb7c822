"""GPU parity of the MCMC densification operators (efgs.add_noise / efgs.relocation_adjustment, through the C ABI)
against the CPU oracle (oracle.add_noise / oracle.relocation_adjustment, pinned by the Philox known-answer
vectors and the closed forms in test_oracle).

Bars:
  add_noise   the device's Philox words equal the oracle's (integer work), so the noise steps agree to the
              float rounding of exp / log / sin / cos: new means within rtol 1e-5 plus one ulp of the largest
              mean; rows with |q|^2 < 1e-8 unchanged bit for bit; each call advances the device generator's
              offset by 4 and a repeated (seed, offset) reproduces the step exactly.
  relocation  o' = 1 - (1 - o)^(1/n) is one rounding of powf away from the oracle's: |delta o'| <= 8 ulp of 1.0;
              the scale factor then differs by the same absolute amount relative to o' (rtol 1e-5 + 8 ulp / o').
Cases: a small scene with degenerate quaternions, the full c3 scene (1M Gaussians), counts outside 1..50, empty.
"""
import numpy as np
import pytest

import oracle as O
from efgs.synthetic import make_scene

pytestmark = pytest.mark.gpu

ULP1 = 2.0 ** -23


def _noise_inputs(n, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.normal(size=(n, 4)).astype(np.float32)
    q[::97] = 0.0  # degenerate quaternions leave the mean unchanged
    scales = rng.normal(-3.0, 1.0, (n, 3)).astype(np.float32)
    opacities = rng.normal(-4.0, 2.0, (n, 1)).astype(np.float32)
    means = rng.uniform(-5.0, 5.0, (n, 3)).astype(np.float32)
    return scales, q, opacities, means


def _check_noise(scales, q, opacities, means, lr):
    import torch
    import efgs
    dev = torch.device('cuda:0')
    ts, tq, to = (torch.tensor(a, device=dev) for a in (scales, q, opacities))
    tm = torch.tensor(means, device=dev)
    gen = torch.cuda.default_generators[0]
    seed, offset = gen.initial_seed(), gen.get_offset()
    efgs.add_noise(ts, tq, to, tm, lr)
    assert gen.get_offset() == offset + 4
    got = tm.cpu().numpy()
    want = O.add_noise(scales, q, opacities.reshape(-1), means, lr, seed, offset)
    atol = float(np.abs(means).max()) * 2.0 ** -23
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=atol)
    degenerate = (q.astype(np.float64) ** 2).sum(1) < 1e-8
    np.testing.assert_array_equal(got[degenerate], means[degenerate])
    moved = np.abs(want - means).max()
    print(f'add_noise n={len(means)} seed={seed} offset={offset}: max |step| {moved:.3e}, '
          f'max |gpu - oracle| {np.abs(got - want).max():.3e}', flush=True)
    assert moved > 0.0
    return ts, tq, to, seed, offset


def test_add_noise_small_scene_and_generator_offsets():
    import torch
    import efgs
    torch.cuda.manual_seed(2024)
    scales, q, opacities, means = _noise_inputs(4096)
    ts, tq, to, seed, offset = _check_noise(scales, q, opacities, means, 0.05)
    # the next call draws from the next Philox counter: different noise, again equal to the oracle's
    _check_noise(scales, q, opacities, means, 0.05)
    # a repeated (seed, offset) reproduces the step bit for bit
    gen = torch.cuda.default_generators[0]
    tm1 = torch.tensor(means, device='cuda:0')
    gen.set_offset(offset)
    efgs.add_noise(ts, tq, to, tm1, 0.05)
    tm2 = torch.tensor(means, device='cuda:0')
    gen.set_offset(offset)
    efgs.add_noise(ts, tq, to, tm2, 0.05)
    assert torch.equal(tm1, tm2)


def test_add_noise_full_c3_scene():
    import torch
    torch.cuda.manual_seed(7)
    sc = make_scene('c3')
    n = sc['means'].shape[0]
    print(f'c3 add_noise: n={n}', flush=True)
    _check_noise(sc['scales'], sc['rotations'], sc['opacities'].reshape(n, 1), sc['means'], 5e5 * 1.6e-4 * 0.01)


def test_add_noise_empty_and_rejections():
    import torch
    import efgs
    e3 = torch.empty((0, 3), device='cuda:0')
    efgs.add_noise(e3, torch.empty((0, 4), device='cuda:0'), torch.empty((0, 1), device='cuda:0'), e3.clone(), 0.1)
    with pytest.raises(ValueError):
        efgs.add_noise(torch.zeros((4, 3), device='cuda:0'), torch.zeros((4, 4), device='cuda:0'), torch.zeros((4, 1), device='cuda:0'),
                       torch.zeros((4, 3), device='cuda:0', dtype=torch.float64), 0.1)
    with pytest.raises(ValueError):
        efgs.add_noise(torch.zeros((4, 3), device='cuda:0'), torch.zeros((4, 4), device='cuda:0'), torch.zeros((4, 1), device='cuda:0'),
                       torch.zeros((3, 4), device='cuda:0').t(), 0.1)


@pytest.mark.parametrize('n', [1, 1000, 100_000])
def test_relocation_matches_oracle(n):
    import torch
    import efgs
    rng = np.random.default_rng(n)
    o = rng.uniform(0.005, 0.999, (n, 1)).astype(np.float32)
    s = np.exp(rng.normal(-4.0, 1.0, (n, 3))).astype(np.float32)
    c = rng.integers(-1, 61, n).astype(np.int64)  # counts outside 1..50 clamp
    dev = torch.device('cuda:0')
    new_o, new_s = efgs.relocation_adjustment(torch.tensor(o, device=dev), torch.tensor(s, device=dev), torch.tensor(c, device=dev))
    assert new_o.shape == (n, 1) and new_s.shape == (n, 3)
    want_o, want_s = O.relocation_adjustment(o, s, c)
    got_o, got_s = new_o.cpu().numpy(), new_s.cpu().numpy()
    print(f'relocation n={n}: max |delta o\'| {np.abs(got_o - want_o).max():.3e}', flush=True)
    assert np.abs(got_o - want_o).max() <= 8 * ULP1
    rtol = 1e-5 + 8 * ULP1 / want_o
    assert np.all(np.abs(got_s - want_s) <= rtol * np.abs(want_s))


def test_relocation_shapes_and_empty():
    import torch
    import efgs
    dev = torch.device('cuda:0')
    o = torch.tensor([0.3, 0.6], device=dev)  # (N,) opacities are accepted, as the reference reads size(0)
    s = torch.tensor([[0.1, 0.2, 0.3], [0.3, 0.2, 0.1]], device=dev)
    new_o, new_s = efgs.relocation_adjustment(o, s, torch.tensor([1, 3], device=dev))
    np.testing.assert_allclose(new_o.cpu().numpy()[:, 0], O.relocation_adjustment(o.cpu().numpy(), s.cpu().numpy(), [1, 3])[0][:, 0],
                               atol=8 * ULP1)
    e_o, e_s = efgs.relocation_adjustment(torch.empty((0, 1), device=dev), torch.empty((0, 3), device=dev),
                                          torch.empty((0,), dtype=torch.int64, device=dev))
    assert e_o.shape == (0, 1) and e_s.shape == (0, 3)
    with pytest.raises(ValueError):
        efgs.relocation_adjustment(o, s, torch.tensor([1, 3], device=dev, dtype=torch.int32))
