"""GPU parity of the standalone neural decode (efgs_neural_decode_forward / _backward through the C ABI)
against the CPU oracle's statement of the same MLP (oracle.neural_decode, pinned against autograd in
test_oracle): configuration c2 at its full size (1M primitives, 8 latents ~ N(0, 0.1), unit directions,
11 -> 64 -> 64 -> 3 fp16 Xavier MLP, upstream gradients N(0, 1)), the reference's default network
(frequency-encoded features, SH degrees 0-3, 16 neurons) and a base-input network, plus ragged and empty
inputs and a gated direction encoding.

Bars: outputs max-abs <= 2e-3 (fp16 MLP path); feature, base, direction and weight gradients rel-L2 <= 1e-3.
"""
import numpy as np
import pytest

import oracle as O
from efgs.synthetic import xavier_mlp
from helpers import rel_l2

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-3
GRAD_TOL = 1e-3

MLPS = {
    'c2': dict(n_feature_dims=8, n_frequencies=0, sh_degrees=(1,), n_neurons=64, n_hidden_layers=2, base_input=False),
    'reference_default': dict(n_feature_dims=8, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=16, n_hidden_layers=2,
                              base_input=False),
    'base_input': dict(n_feature_dims=5, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=32, n_hidden_layers=3, base_input=True),
}


def _configure(mlp: O.MLPConfig):
    import efgs
    efgs.initialize_appearance('neural', 0, 'none', 'none', 'relu', True)
    efgs.initialize_residual_mlp(mlp.n_input_dims, 3, {'otype': 'Identity'},
                                 {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None',
                                  'n_neurons': mlp.n_neurons, 'n_hidden_layers': mlp.n_hidden_layers},
                                 mlp.base_input, mlp.n_frequencies, list(mlp.sh_degrees))


def _inputs(mlp: O.MLPConfig, n: int, seed: int = 0):
    """c2's draw order: latents N(0, 0.1), directions normalize(N(0, 1)^3), Xavier weights, upstream N(0, 1)."""
    rng = np.random.default_rng(seed)
    feat = rng.normal(0.0, 0.1, size=(n, mlp.n_feature_dims)).astype(np.float32)
    d = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    d /= np.maximum(np.linalg.norm(d, axis=1, keepdims=True), 1e-12)
    w = xavier_mlp(rng, mlp.n_input_dims, mlp.n_neurons, mlp.n_hidden_layers)
    dy = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    base = rng.normal(0.0, 0.5, size=(n, 3)).astype(np.float32)
    return feat, d.astype(np.float32), w, dy, base


def _run(name, n, degree=1):
    import torch
    from efgs.rasterization import neural_decode
    mlp = O.MLPConfig(**MLPS[name])
    _configure(mlp)
    feat, d, w, dy, base = _inputs(mlp, n)
    dev = torch.device('cuda:0')
    tf = torch.tensor(feat, device=dev, requires_grad=True)
    td = torch.tensor(d, device=dev, requires_grad=True)
    tw = torch.tensor(w, device=dev, requires_grad=True)
    tb = torch.tensor(base, device=dev, requires_grad=True) if mlp.base_input else None
    out = neural_decode(tf, td, tw, degree, tb)
    out.backward(torch.tensor(dy, device=dev))
    torch.cuda.synchronize()
    return mlp, (feat, d, w, dy, base), out.detach().cpu().numpy(), tf, td, tw, tb


def _check(name, n, degree=1):
    print(f'case {name}: n={n} degree={degree}', flush=True)
    mlp, (feat, d, w, dy, base), out, tf, td, tw, tb = _run(name, n, degree)
    y, acts, mats = O.neural_decode(feat, base, d, w, mlp, degree)
    ref = O.neural_decode_backward(feat, base, d, dy, mats, acts, mlp, degree)
    err = float(np.abs(out - y).max()) if n else 0.0
    print(f'case {name}: output max-abs {err:.3e}', flush=True)
    assert err <= OUT_TOL
    grads = dict(features=tf.grad, weights=tw.grad, dirs=td.grad)
    if mlp.base_input:
        grads['base'] = tb.grad
    for k, g in grads.items():
        got = g.cpu().numpy()
        want = ref[k]
        if np.linalg.norm(want) == 0:
            assert np.abs(got).max() == 0, k
            continue
        e = rel_l2(got, want)
        print(f'case {name}: grad {k} rel-L2 {e:.3e}', flush=True)
        assert e <= GRAD_TOL, f'{k}: rel-L2 {e}'


def test_c2_full_size():
    _check('c2', 1_000_000)


@pytest.mark.parametrize('name', ['reference_default', 'base_input'])
def test_other_networks(name):
    _check(name, 20_000)


def test_ragged_count():
    _check('c2', 64 * 1000 + 37)


def test_direction_encoding_gated():
    """degree 0 zeroes the SH degree >= 1 inputs (the rasterizer's render_residual = False / degree 0 case)."""
    _check('reference_default', 5_000, degree=0)


def test_empty_input_zeroes_weight_gradients():
    import torch
    from efgs.rasterization import neural_decode
    mlp = O.MLPConfig(**MLPS['c2'])
    _configure(mlp)
    dev = torch.device('cuda:0')
    w = torch.tensor(_inputs(mlp, 1)[2], device=dev, requires_grad=True)
    f = torch.zeros((0, mlp.n_feature_dims), device=dev, requires_grad=True)
    d = torch.zeros((0, 3), device=dev, requires_grad=True)
    out = neural_decode(f, d, w, 1)
    assert out.shape == (0, 3)
    out.sum().backward()
    torch.cuda.synchronize()
    assert float(w.grad.abs().max()) == 0.0
