"""GPU parity of the tiny-cuda-nn surface (efgs.tcnn.NetworkWithInputEncoding) that the neural appearance plugin
builds (Appearance/Neural.py:40-66) and calls for its unfused evaluation (Neural.py:102-111), through the library's
decode entry points on a rasterizer handle of the network's own.

Checked against the oracle's MLP statement (oracle.mlp_forward / mlp_backward: fp16-rounded weights and activations,
fp32 accumulation, pinned against torch matmul and autograd in test_oracle): outputs max-abs <= 2e-3 (the fp16 MLP
path), input and weight gradients rel-L2 <= 1e-3, for the reference default network (32 inputs, 16 neurons, 2 hidden
layers) and an odd input width; the Neural.py:53 zeroing gives exact zero outputs; and the network's `params`, passed
to diff_rasterize after the plugin's own initialize_residual_mlp call, reproduce the neural_reference_default parity
case (image <= 2e-3, MLP weight gradient rel-L2 <= 1e-3), while its unfused call on the plugin's encoded inputs gives
the fused kernels' MLP outputs."""
import numpy as np
import pytest

import oracle as O
from efgs.synthetic import xavier_mlp
from helpers import small_case, rel_l2, torch_inputs, settings

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-3
GRAD_TOL = 1e-3
NETWORK = {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None', 'n_neurons': 16, 'n_hidden_layers': 2}


def _oracle_config(n_in, n_neurons, n_hidden):
    return O.MLPConfig(n_feature_dims=n_in, n_frequencies=0, sh_degrees=(), n_neurons=n_neurons, n_hidden_layers=n_hidden)


def _check_call(n_in, n_neurons, n_hidden, n, x_requires_grad=True):
    import torch
    from efgs import tcnn
    dev = torch.device('cuda:0')
    print(f'tcnn call: n_in={n_in} neurons={n_neurons} hidden={n_hidden} n={n}', flush=True)
    net = tcnn.NetworkWithInputEncoding(n_in, 3, {'otype': 'Identity'}, dict(NETWORK, n_neurons=n_neurons, n_hidden_layers=n_hidden))
    rng = np.random.default_rng(3)
    w = xavier_mlp(rng, n_in, n_neurons, n_hidden)
    x = rng.uniform(-1.0, 1.0, size=(n, n_in)).astype(np.float32)
    dy = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    with torch.no_grad():
        net.params.copy_(torch.tensor(w, device=dev))
    tx = torch.tensor(x, device=dev, requires_grad=x_requires_grad)
    out = net(tx)
    assert out.dtype == torch.float16 and out.shape == (n, 3)
    out.float().backward(torch.tensor(dy, device=dev))   # as Neural.py:110: mlp(x).float()
    torch.cuda.synchronize()
    mlp = _oracle_config(n_in, n_neurons, n_hidden)
    xp = np.concatenate([x, np.zeros((n, mlp.n_input_padded - n_in), np.float32)], 1)
    mats = O.mlp_matrices(w, mlp)
    y, acts = O.mlp_forward(xp, mats)
    err = float(np.abs(out.detach().float().cpu().numpy() - y).max())
    print(f'tcnn call: output max-abs {err:.3e}', flush=True)
    assert err <= OUT_TOL
    # the upstream gradient reaches the half-precision output as fp16 (autograd's cast of .float())
    dy16 = dy.astype(np.float16).astype(np.float32)
    dx, dW = O.mlp_backward(dy16, mats, acts)
    e_w = rel_l2(net.params.grad.cpu().numpy(), np.concatenate([g.reshape(-1) for g in dW]))
    print(f'tcnn call: weight grad rel-L2 {e_w:.3e}', flush=True)
    assert e_w <= GRAD_TOL
    if x_requires_grad:
        assert tx.grad.dtype == torch.float32
        e_x = rel_l2(tx.grad.cpu().numpy(), dx[:, :n_in])
        print(f'tcnn call: input grad rel-L2 {e_x:.3e}', flush=True)
        assert e_x <= GRAD_TOL
    return net


def test_reference_default_network():
    net = _check_call(32, 16, 2, 20_000)
    assert net.params.numel() == 1024


def test_odd_input_width_c2_network():
    _check_call(11, 64, 2, 64 * 300 + 5)


def test_weights_only_gradient():
    _check_call(32, 32, 3, 4_000, x_requires_grad=False)


def test_zeroed_output_rows_give_zero_outputs():
    import torch
    from efgs import tcnn
    dev = torch.device('cuda:0')
    net = tcnn.NetworkWithInputEncoding(32, 3, {'otype': 'Identity'}, NETWORK)
    net.params.data[-NETWORK['n_neurons'] * 16:].zero_()   # Neural.py:53
    x = torch.randn(1000, 32, device=dev)
    out = net(x)
    torch.cuda.synchronize()
    assert out.shape == (1000, 3) and float(out.detach().abs().max()) == 0.0


def test_empty_batch():
    import torch
    from efgs import tcnn
    dev = torch.device('cuda:0')
    net = tcnn.NetworkWithInputEncoding(32, 3, {'otype': 'Identity'}, NETWORK)
    x = torch.zeros((0, 32), device=dev, requires_grad=True)
    out = net(x)
    assert out.shape == (0, 3)
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert float(net.params.grad.abs().max()) == 0.0 and x.grad.shape == (0, 32)


def test_params_drive_the_rasterizer_and_the_unfused_call_matches_the_fused_kernels():
    """The plugin's sequence: build the network (Neural.py:40-53), initialize_residual_mlp with its attributes
    (:58-66), pass `params` as mlp_weights (:100) -- on the neural_reference_default parity scene (8 latents, one
    frequency, SH degrees 0..3: 32 inputs, 16 neurons, 2 hidden layers). Then the unfused path (:102-111): the
    network on the plugin's encoded inputs gives the fused preprocess's MLP outputs."""
    import torch
    import efgs
    from efgs import tcnn
    mlp_cfg = dict(n_feature_dims=8, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=16, n_hidden_layers=2, base_input=False)
    scene, app, cam = small_case(model='neural', scale_shift=2.5, acts=('none', 'tanh', 'relu'), mlp=mlp_cfg)
    dev = torch.device('cuda:0')
    m = app.mlp
    net = tcnn.NetworkWithInputEncoding(m.n_input_dims, 3, {'otype': 'Identity'},
                                        dict(NETWORK, n_neurons=m.n_neurons, n_hidden_layers=m.n_hidden_layers))
    assert net.n_input_dims == 32
    efgs.initialize_appearance(app.model, app.max_degree, app.base_act, app.res_act, app.color_act, app.direction_gradient)
    efgs.initialize_residual_mlp(net.n_input_dims, net.n_output_dims, net.encoding_config, net.network_config, m.base_input,
                                 m.n_frequencies, list(m.sh_degrees))
    with torch.no_grad():
        net.params.copy_(torch.tensor(scene.mlp_weights, device=dev))
    inp = torch_inputs(scene, dev, requires_grad=True)
    img = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], torch.empty(0, device=dev),
                              settings(cam, dev), base_colors=inp['base_colors'], residual_params=inp['residual_params'],
                              mlp_weights=net.params)
    fw = O.render(scene, app, cam)
    g = np.random.default_rng(7).normal(size=fw.image.shape).astype(np.float32)
    img.backward(torch.tensor(g, device=dev))
    torch.cuda.synchronize()
    err = float(np.abs(img.detach().cpu().numpy() - fw.image).max())
    print(f'tcnn params in diff_rasterize: image max-abs {err:.3e}', flush=True)
    assert err <= OUT_TOL
    ref = O.backward(scene, app, cam, fw, g, densify_rows=0, densification_info=np.zeros((1, scene.n), np.float32))
    for k, got in (('mlp_weights', net.params.grad), ('residual_params', inp['residual_params'].grad), ('means', inp['means'].grad)):
        e = rel_l2(got.cpu().numpy(), ref[k])
        print(f'tcnn params in diff_rasterize: grad {k} rel-L2 {e:.3e}', flush=True)
        assert e <= GRAD_TOL, k
    # unfused: the plugin's encoded inputs (frequency-encoded latents, SH degree values of the view direction)
    x = O.mlp_inputs(scene, m, cam, cam.degree)[:, :m.n_input_dims]
    out = net(torch.tensor(x, device=dev)).detach().float().cpu().numpy()
    y, _, _ = O.neural_outputs(scene, app, cam)
    err = float(np.abs(out - y).max())
    print(f'tcnn unfused call vs fused MLP outputs: max-abs {err:.3e}', flush=True)
    assert err <= OUT_TOL
