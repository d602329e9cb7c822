"""The tiny-cuda-nn surface (efgs.tcnn) without a GPU: the object the neural appearance plugin builds
(Appearance/Neural.py:40-66) constructs from the plugin's own configuration, holds its flat parameter vector in the
layout the rasterizer and the oracle read (tcnn FullyFusedMLP: output layer padded to 16 rows and stored last, so
Neural.py:53's slice is exactly that layer), carries the attributes Neural.py:55-66 hand to
initialize_residual_mlp, and rejects what the kernels cannot run."""
import math

import pytest

import oracle as O

NEURAL_NETWORK = {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None', 'n_neurons': 16, 'n_hidden_layers': 2}


def _net(n_in=32, **kw):
    from efgs import tcnn
    cfg = dict(NEURAL_NETWORK, **kw)
    return tcnn.NetworkWithInputEncoding(n_in, 3, {'otype': 'Identity'}, cfg, device='cpu')


def test_reference_default_network_has_1024_params():
    net = _net()
    assert net.params.numel() == net.n_params == 16 * 32 + 16 * 16 + 16 * 16 == 1024
    assert net.params.dtype.is_floating_point and net.params.dtype.itemsize == 4 and net.params.requires_grad


@pytest.mark.parametrize('n_in,n_neurons,n_hidden', [(32, 16, 2), (11, 64, 2), (25, 32, 3), (48, 32, 4)])
def test_param_count_matches_the_oracle_layout(n_in, n_neurons, n_hidden):
    net = _net(n_in, n_neurons=n_neurons, n_hidden_layers=n_hidden)
    from efgs import tcnn
    shapes = tcnn.layer_shapes(n_in, n_neurons, n_hidden)
    # the oracle's layer shapes for a network whose encoded input is n_in wide
    mlp = O.MLPConfig(n_feature_dims=n_in, n_frequencies=0, sh_degrees=(), n_neurons=n_neurons, n_hidden_layers=n_hidden)
    assert shapes == mlp.layer_shapes()
    assert net.params.numel() == mlp.n_params == sum(r * c for r, c in shapes)


def test_neural_py_zero_slice_is_exactly_the_output_layer():
    net = _net()
    n_out_padded = (net.n_output_dims + 15) // 16 * 16
    before = net.params.detach().clone()
    net.params.data[-net.network_config['n_neurons'] * n_out_padded:].zero_()   # Neural.py:53
    from efgs import tcnn
    shapes = tcnn.layer_shapes(32, 16, 2)
    out_start = sum(r * c for r, c in shapes[:-1])
    assert (net.params[out_start:] == 0).all()
    assert (net.params[:out_start] == before[:out_start]).all()
    assert (before[:out_start] != 0).all()


def test_attributes_feed_initialize_residual_mlp():
    """Neural.py:58-66 passes the network's attributes to initialize_residual_mlp: the configured rasterizer then
    expects exactly this many weights."""
    from efgs import rasterization as R
    net = _net(32)
    r = R.Rasterizer()
    r.set_appearance(5, 0, 0, 1, 1, True)
    # what initialize_residual_mlp does with the attributes (frequency encoding 1, SH degrees 0..3: 16 + 16 inputs)
    r.set_residual_mlp(net.n_input_dims, net.n_output_dims, int(net.network_config['n_neurons']),
                       int(net.network_config['n_hidden_layers']), 1, False, 1, 0b1111)
    assert r.mlp_param_count() == net.params.numel()
    assert net.encoding_config == {'otype': 'Identity'}


def test_initialisation_is_xavier_uniform_per_matrix_and_seeded():
    from efgs import tcnn
    a = tcnn.NetworkWithInputEncoding(11, 3, {'otype': 'Identity'}, dict(NEURAL_NETWORK, n_neurons=64), seed=7, device='cpu')
    b = tcnn.NetworkWithInputEncoding(11, 3, {'otype': 'Identity'}, dict(NEURAL_NETWORK, n_neurons=64), seed=7, device='cpu')
    c = tcnn.NetworkWithInputEncoding(11, 3, {'otype': 'Identity'}, dict(NEURAL_NETWORK, n_neurons=64), seed=8, device='cpu')
    assert (a.params == b.params).all() and not (a.params == c.params).all()
    off = 0
    for rows, cols in tcnn.layer_shapes(11, 64, 2):
        w = a.params.detach()[off:off + rows * cols]
        bound = math.sqrt(6.0 / (rows + cols))
        assert float(w.abs().max()) <= bound
        # uniform on [-bound, bound]: variance bound^2 / 3
        assert abs(float(w.var()) - bound * bound / 3.0) < 0.15 * bound * bound / 3.0
        off += rows * cols


@pytest.mark.parametrize('enc,net_cfg,n_out,match', [
    ({'otype': 'HashGrid'}, NEURAL_NETWORK, 3, 'encoding'),
    ({'otype': 'Identity', 'n_dims_to_encode': 4}, NEURAL_NETWORK, 3, 'Identity encoding options'),
    ({'otype': 'Identity'}, dict(NEURAL_NETWORK, otype='CutlassMLP'), 3, 'network'),
    ({'otype': 'Identity'}, dict(NEURAL_NETWORK, activation='Sine'), 3, 'hidden activation'),
    ({'otype': 'Identity'}, dict(NEURAL_NETWORK, output_activation='Sigmoid'), 3, 'output activation'),
    ({'otype': 'Identity'}, dict(NEURAL_NETWORK, n_neurons=48), 3, 'n_neurons'),
    ({'otype': 'Identity'}, dict(NEURAL_NETWORK, n_hidden_layers=0), 3, 'n_hidden_layers'),
    ({'otype': 'Identity'}, NEURAL_NETWORK, 4, 'outputs'),
])
def test_unsupported_configurations_raise(enc, net_cfg, n_out, match):
    from efgs import tcnn
    with pytest.raises(ValueError, match=match):
        tcnn.NetworkWithInputEncoding(32, n_out, enc, net_cfg, device='cpu')


def test_calls_need_a_gpu_device():
    import torch
    net = _net()
    with pytest.raises(ValueError, match='GPU'):
        net(torch.zeros(4, 32))
    with pytest.raises(ValueError, match=r'\(batch, 32\)'):
        net(torch.zeros(4, 31))


def test_state_dict_and_pickling_keep_the_weights():
    import pickle
    import torch
    net = _net()
    sd = net.state_dict()
    assert list(sd) == ['params'] and sd['params'].numel() == 1024
    clone = pickle.loads(pickle.dumps(net))
    assert torch.equal(clone.params, net.params) and clone.n_params == 1024
