"""GPU parity of the Speedy-Splat pruning scores (efgs.update_pruning_scores, through the C ABI) against the CPU
oracle (oracle.pruning_scores, pinned against autograd and a closed form in test_oracle).

The device sums each primitive's per-pixel terms in a fixed order different from the oracle's pixel order,
and evaluates alpha with the hardware exp2 and the reciprocal with v_rcp_f32, so scores agree to float
rounding: rel-L2 <= 1e-4 over all primitives and every score within rtol 1e-3 (atol 1e-6 of the largest).
The scores accumulate into the given tensor; repeated calls are bit-identical (no atomics).
"""
import numpy as np
import pytest

import oracle as O
from helpers import small_case, rel_l2, configure, torch_inputs, settings

pytestmark = pytest.mark.gpu


def _scores(scene, app, cam, init=None):
    import torch
    import efgs
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    scores = torch.tensor(init, device=dev) if init is not None else torch.zeros(scene.n, dtype=torch.float32, device=dev)
    efgs.update_pruning_scores(scores, inp['means'], inp['scales'], inp['rotations'], inp['opacities'], settings(cam, dev),
                               base_colors=inp['base_colors'], residual_params=inp['residual_params'],
                               mlp_weights=inp['mlp_weights'])
    torch.cuda.synchronize()
    return scores.cpu().numpy()


def _check(got, want, name):
    e = rel_l2(got, want)
    print(f'case {name}: pruning scores rel-L2 {e:.3e}, max {want.max():.3e}, nonzero {(want > 0).sum()}', flush=True)
    assert e <= 1e-4
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-6 * float(np.abs(want).max()))


CASES = {
    'sh3': dict(model='sh', n=500),
    'sh3_dense': dict(model='sh', n=3000, scale_shift=2.0),
    'neural': dict(model='neural', n=800),
    'nasg': dict(model='nasg', n=600),
}


@pytest.mark.parametrize('name', list(CASES))
def test_pruning_scores_match_oracle(name):
    scene, app, cam = small_case(**CASES[name])
    fw = O.render(scene, app, cam)
    want = O.pruning_scores(cam, fw)
    got = _scores(scene, app, cam)
    _check(got, want, name)
    assert np.all(got[fw.n_touched == 0] == 0.0)


def test_pruning_scores_accumulate_and_repeat_exactly():
    scene, app, cam = small_case(model='sh', n=500)
    fw = O.render(scene, app, cam)
    init = np.random.default_rng(1).uniform(0.0, 5.0, scene.n).astype(np.float32)
    want = O.pruning_scores(cam, fw, init)
    a = _scores(scene, app, cam, init)
    b = _scores(scene, app, cam, init)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_allclose(a, want, rtol=1e-4, atol=1e-5)


def test_pruning_scores_full_c3_scene():
    """c3 (1M Gaussians, 1920 x 1080, neural) at full size."""
    from test_gpu_full_size import _scene
    scene, app, cam = _scene('c3_neural')
    print('case c3: oracle forward', flush=True)
    fw = O.render(scene, app, cam)
    want = O.pruning_scores(cam, fw)
    print('case c3: device scores', flush=True)
    got = _scores(scene, app, cam)
    _check(got, want, 'c3')


def test_pruning_scores_rejects_bad_score_tensor():
    import torch
    import efgs
    scene, app, cam = small_case(model='sh', n=50)
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    for bad in (torch.zeros(scene.n + 1, device=dev), torch.zeros(scene.n, device=dev, dtype=torch.float64)):
        with pytest.raises(ValueError):
            efgs.update_pruning_scores(bad, inp['means'], inp['scales'], inp['rotations'], inp['opacities'], settings(cam, dev),
                                       base_colors=inp['base_colors'], residual_params=inp['residual_params'])
