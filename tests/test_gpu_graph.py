"""The neural decode's forward + backward (neural_decode and autograd's backward through the C ABI) captured as one
HIP graph with torch.cuda.graph, as a caller with a launch-bound loop would run it: every replay must give the
eager path's outputs and gradients bit for bit (the same kernels on the same inputs). Between replays the test
writes new values into the graph's static inputs and runs the eager path on copies of them, so each replay is
checked against its own eager result, with the program's eager work and synchronisations between the replays.
No hipMemsetAsync is recorded: the decode's launches are kernels, its scratch comes from torch's graph pool."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

C2_MLP = dict(n_feature_dims=8, n_frequencies=0, sh_degrees=(1,), n_neurons=64, n_hidden_layers=2, base_input=False)


def _inputs(rng, n, n_in):
    from efgs.synthetic import xavier_mlp
    feat = rng.normal(0.0, 0.1, size=(n, 8)).astype(np.float32)
    d = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    d /= np.maximum(np.linalg.norm(d, axis=1, keepdims=True), 1e-12)
    w = xavier_mlp(rng, n_in, 64, 2)
    dy = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    return feat, d.astype(np.float32), w, dy


def _eager(tf, td, tw, tdy):
    from efgs.rasterization import neural_decode
    f, d, w = (t.detach().clone().requires_grad_(True) for t in (tf, td, tw))
    out = neural_decode(f, d, w, 1)
    out.backward(tdy.clone())
    return out.detach(), f.grad, d.grad, w.grad


def test_decode_graph_replays_match_eager():
    import torch
    import efgs
    from efgs.rasterization import neural_decode
    n, n_in = 100_003, 8 + 3
    print(f'case decode graph: n={n}', flush=True)
    efgs.initialize_appearance('neural', 0, 'none', 'none', 'relu', True)
    efgs.initialize_residual_mlp(n_in, 3, {'otype': 'Identity'},
                                 {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None',
                                  'n_neurons': 64, 'n_hidden_layers': 2}, False, 0, [1])
    dev = torch.device('cuda:0')
    rng = np.random.default_rng(7)
    feat, d, w, dy = _inputs(rng, n, n_in)
    tf = torch.tensor(feat, device=dev, requires_grad=True)
    td = torch.tensor(d, device=dev, requires_grad=True)
    tw = torch.tensor(w, device=dev, requires_grad=True)
    tdy = torch.tensor(dy, device=dev)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            neural_decode(tf, td, tw, 1).backward(tdy)
            tf.grad = td.grad = tw.grad = None
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g = neural_decode(tf, td, tw, 1)
        out_g.backward(tdy)
    torch.cuda.synchronize()
    grads_g = (tf.grad, td.grad, tw.grad)

    for r in range(4):
        if r > 0:
            feat, d, w, dy = _inputs(rng, n, n_in)
            with torch.no_grad():
                tf.copy_(torch.tensor(feat, device=dev))
                td.copy_(torch.tensor(d, device=dev))
                tw.copy_(torch.tensor(w, device=dev))
                tdy.copy_(torch.tensor(dy, device=dev))
        ref = _eager(tf, td, tw, tdy)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = (out_g,) + grads_g
        for name, a, b in zip(('output', 'features grad', 'dirs grad', 'weights grad'), got, ref):
            same = torch.equal(a, b)
            print(f'replay {r}: {name} bit-exact {same}', flush=True)
            assert same, f'replay {r}: {name} differs from the eager path (max-abs {float((a - b).abs().max()):.3e})'
