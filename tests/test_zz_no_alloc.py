"""The allocation-free decode backward (efgs_neural_decode_backward_no_alloc, through the C ABI) against the
allocating entry point (efgs_neural_decode_backward) on the same inputs: two calls in a row on the c2 network, the
second with a smaller input (the static scratch keeps the first call's partial rows; every row the second call's
reduction reads is rewritten by it), and a three-layer base-input network whose 11,264 parameters leave room for 372
partial rows of the 16 MiB scratch instead of 512 blocks (a different summation order).

Bars: feature, base, direction and weight gradients rel-L2 <= 1e-3 (the decode's gradient bar); with the same block
count (c2: 6,144 parameters) the results are bit-identical.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from efgs.synthetic import xavier_mlp
from helpers import rel_l2

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-3

MLPS = {
    'c2': dict(n_feature_dims=8, n_frequencies=0, sh_degrees=(1,), n_neurons=64, n_hidden_layers=2, base_input=False),
    'deep_base_input': dict(n_feature_dims=5, n_frequencies=1, sh_degrees=(0, 1, 2), n_neurons=64, n_hidden_layers=3, base_input=True),
}


def _configure(mlp: O.MLPConfig):
    import efgs
    efgs.initialize_appearance('neural', 0, 'none', 'none', 'relu', True)
    efgs.initialize_residual_mlp(mlp.n_input_dims, 3, {'otype': 'Identity'},
                                 {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None',
                                  'n_neurons': mlp.n_neurons, 'n_hidden_layers': mlp.n_hidden_layers},
                                 mlp.base_input, mlp.n_frequencies, list(mlp.sh_degrees))


def _backward_both(mlp: O.MLPConfig, n: int, seed: int):
    """Gradients of both entry points for one seeded input of n primitives (c2's draw order)."""
    import torch
    from efgs import _lib
    from efgs import rasterization as R
    rng = np.random.default_rng(seed)
    dev = torch.device('cuda:0')
    feat = torch.tensor(rng.normal(0.0, 0.1, size=(n, mlp.n_feature_dims)).astype(np.float32), device=dev)
    d = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    d /= np.maximum(np.linalg.norm(d, axis=1, keepdims=True), 1e-12)
    dirs = torch.tensor(d, device=dev)
    w = torch.tensor(xavier_mlp(rng, mlp.n_input_dims, mlp.n_neurons, mlp.n_hidden_layers), device=dev).half().contiguous()
    dy = torch.tensor(rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32), device=dev)
    base = torch.tensor(rng.normal(0.0, 0.5, size=(n, 3)).astype(np.float32), device=dev)
    handle = R._rasterizer.handle
    stream = torch.cuda.current_stream(dev).cuda_stream
    assert w.numel() == R._rasterizer.mlp_param_count()
    out = {}
    for name in ('alloc', 'no_alloc'):
        g = dict(features=torch.full_like(feat, float('nan')), base=torch.full_like(base, float('nan')),
                 dirs=torch.full_like(dirs, float('nan')), weights=torch.full((w.numel(),), float('nan'), device=dev))
        args = [handle, n, feat.data_ptr(), base.data_ptr(), dirs.data_ptr(), w.data_ptr(), 1, dy.data_ptr(), g['features'].data_ptr(),
                g['base'].data_ptr(), g['dirs'].data_ptr(), g['weights'].data_ptr()]
        print(f'calling efgs_neural_decode_backward{"_no_alloc" if name == "no_alloc" else ""}: n={n} '
              f'params={w.numel()}', flush=True)
        if name == 'alloc':
            alloc = _lib.WorkspaceAllocator(dev, 'decode')
            status = _lib.lib.efgs_neural_decode_backward(*args, alloc.fn, alloc.ctx, ctypes.c_void_p(stream))
            torch.cuda.synchronize()
            alloc.done()
        else:
            status = _lib.lib.efgs_neural_decode_backward_no_alloc(*args, ctypes.c_void_p(stream))
            torch.cuda.synchronize()
        assert status == 0, _lib.lib.efgs_last_error()
        out[name] = {k: v.cpu().numpy() for k, v in g.items()}
    keys = ['features', 'dirs', 'weights'] + (['base'] if mlp.base_input else [])
    return out['alloc'], out['no_alloc'], keys


@pytest.mark.parametrize('name', list(MLPS))
def test_decode_backward_no_alloc_matches_the_allocating_entry_point(name):
    mlp = O.MLPConfig(**MLPS[name])
    _configure(mlp)
    params = sum(r * c for r, c in mlp.layer_shapes())
    for n, seed in ((200_000, 0), (7_001, 1)):   # the second call is smaller
        ref, got, keys = _backward_both(mlp, n, seed)
        for k in keys:
            assert np.isfinite(got[k]).all(), k
            e = rel_l2(got[k], ref[k])
            print(f'case {name}: n={n} grad {k} rel-L2 {e:.3e}', flush=True)
            assert e <= GRAD_TOL, (k, e)
            if params <= 8192:   # same block count: the same kernels and summation order
                np.testing.assert_array_equal(got[k], ref[k])


def test_decode_backward_no_alloc_rejects_bad_input():
    import torch
    from efgs import _lib
    from efgs import rasterization as R
    mlp = O.MLPConfig(**MLPS['c2'])
    _configure(mlp)
    dev = torch.device('cuda:0')
    g = torch.zeros(R._rasterizer.mlp_param_count(), device=dev)
    status = _lib.lib.efgs_neural_decode_backward_no_alloc(R._rasterizer.handle, 10, None, None, None, None, 1, None, None, None,
                                                           None, g.data_ptr(), None)
    assert status != 0 and b'null' in _lib.lib.efgs_last_error()
    # n = 0: the weight gradient is cleared, nothing else is touched
    g.fill_(5.0)
    status = _lib.lib.efgs_neural_decode_backward_no_alloc(R._rasterizer.handle, 0, None, None, None, None, 1, None, None, None, None,
                                                           g.data_ptr(), None)
    torch.cuda.synchronize()
    assert status == 0 and float(g.abs().max()) == 0.0
