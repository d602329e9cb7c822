"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on identical seeded scenes.

Bars: integer / key / index / range arrays bit-exact; per-primitive projection records (mean2d, conic,
opacity, bounds) bit-exact (shared decision-path arithmetic); image max-abs <= 1e-4 (fp32 path; the blend's
alpha uses the hardware exp2) and <= 2e-3 (fp16 neural MLP path); last-contributor indices equal up to
near-threshold decisions (at most 2 + 1e-5 of the pixels, every appearance model); gradients rel-L2 <= 1e-3, including the MLP weight
gradients. The c0 colour configuration: fused preprocess colours against the unfused torch appearance within 1e-5.
"""
import numpy as np
import pytest

import oracle as O
from helpers import small_case, rel_l2, configure, torch_inputs, settings, read_device, check_emission, check_first_tiles, \
    check_image, device_contributors

pytestmark = pytest.mark.gpu

IMAGE_TOL = 1e-4
IMAGE_TOL_FP16 = 2e-3   # neural: fp16 MLP path
GRAD_TOL = 1e-3

CASES = {
    'sh3_relu': dict(model='sh'),
    'sh3_exp_softplus_sigmoid': dict(model='sh', acts=('exp', 'softplus', 'sigmoid')),
    'sh1_tanh_hardsigmoid': dict(model='sh', acts=('none', 'tanh', 'hardsigmoid'), degree=1),
    'sh2_satexp': dict(model='sh', acts=('exp', 'softplus', 'satexp'), degree=2),
    'sh_degree0': dict(model='sh', degree=0),
    'sh_residual_off': dict(model='sh', render_residual=False),
    'sh_render_base_off_aa': dict(model='sh', render_base=False, proper_aa=True),
    'sh_no_direction_gradient': dict(model='sh', direction_gradient=False),
    'precomputed': dict(model='precomputed'),
    'sv': dict(model='sv'),
    'nasg': dict(model='nasg'),
    'nasgabor': dict(model='nasgabor', acts=('none', 'tanh', 'softplus')),
    # the remaining model x colour-activation pairs of the c4 sweep (the others run here or at full size)
    'sv_softplus': dict(model='sv', acts=('none', 'none', 'softplus')),
    'nasg_sigmoid': dict(model='nasg', acts=('none', 'tanh', 'sigmoid')),
    'nasgabor_sigmoid': dict(model='nasgabor', acts=('none', 'tanh', 'sigmoid')),
    'ragged_image': dict(model='sh', width=50, height=37),
    'dense_2k': dict(model='sh', n=2000, width=96, height=80, scale_shift=1.5),
    # tiles of 171-632 and of 716-2549 instances: every path of the per-tile sort (registers, LDS slab,
    # chunks merged by rank) and many staging batches in the blends
    'dense_tiles_3k': dict(model='sh', n=3000, scale_shift=2.0),
    'dense_tiles_12k': dict(model='sh', n=12000, scale_shift=2.0),
    'neural_c3_mlp': dict(model='neural', scale_shift=2.5),
    'neural_reference_default': dict(model='neural', scale_shift=2.5, acts=('none', 'tanh', 'relu'),
                                     mlp=dict(n_feature_dims=8, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=16,
                                              n_hidden_layers=2, base_input=False)),
    'neural_base_input_softplus': dict(model='neural', scale_shift=2.5, acts=('exp', 'softplus', 'satexp'),
                                       mlp=dict(n_feature_dims=5, n_frequencies=1, sh_degrees=(0, 1, 2, 3), n_neurons=32,
                                                n_hidden_layers=3, base_input=True)),
    'neural_degree0': dict(model='neural', scale_shift=2.5, degree=0),
}


def _image_tol(case):
    return IMAGE_TOL_FP16 if case.get('model') == 'neural' else IMAGE_TOL


def _run(case):
    import torch
    import efgs
    from efgs.rasterization import forward_with_frame, frame_views
    scene, app, cam = small_case(**case)
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    st = settings(cam, dev)
    image, frame, bufs = forward_with_frame(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], st,
                                            precomputed_colors=inp['precomputed_colors'], base_colors=inp['base_colors'],
                                            residual_params=inp['residual_params'], mlp_weights=inp['mlp_weights'])
    torch.cuda.synchronize()
    return scene, app, cam, image, frame, bufs, frame_views(frame), efgs


@pytest.mark.parametrize('name', list(CASES))
def test_forward_parity(name):
    scene, app, cam, image, frame, bufs, v, _ = _run(CASES[name])
    fw = O.render(scene, app, cam)
    n = scene.n
    V, I = int(frame.n_visible), int(frame.n_instances)
    print(f'case {name}: N={n} V={V} I={I}', flush=True)
    assert V == len(fw.visible) and I == len(fw.inst_keys)
    n_touched = read_device(bufs, v.n_touched, n, np.uint32)
    np.testing.assert_array_equal(n_touched, fw.n_touched)
    vis = fw.n_touched > 0
    np.testing.assert_array_equal(read_device(bufs, v.depth_keys, n, np.uint32)[vis], fw.depth_key[vis])
    rec = read_device(bufs, v.records, 12 * n, np.float32).reshape(n, 12)[vis]
    np.testing.assert_array_equal(rec[:, 0:2], fw.mean2d[vis])
    np.testing.assert_array_equal(rec[:, 2:5], fw.conic_opacity[vis][:, 0:3])
    np.testing.assert_array_equal(rec[:, 5], fw.conic_opacity[vis][:, 3])
    bx, by = rec[:, 9].view(np.uint32), rec[:, 10].view(np.uint32)
    b = fw.bounds[vis].astype(np.uint32)
    np.testing.assert_array_equal(np.stack([bx & 0xffff, bx >> 16, by & 0xffff, by >> 16], 1), b)
    np.testing.assert_allclose(rec[:, 6:9], fw.color[vis], rtol=0, atol=_image_tol(CASES[name]) / 10 if CASES[name].get('model') != 'neural' else IMAGE_TOL_FP16)
    counters = read_device(bufs, v.counters, 8, np.uint32)
    if V > 0:
        assert counters[3] == fw.depth_key[vis].min() and counters[4] == fw.depth_key[vis].max()
    check_emission(bufs, v, frame, fw, n)
    check_first_tiles(rec, fw, vis, *cam.grid())
    kt = np.uint16 if frame.key_bytes == 2 else np.uint32
    np.testing.assert_array_equal(read_device(bufs, v.tile_sorted_keys, I, kt).astype(np.uint32), fw.inst_keys)
    sorted_inst = read_device(bufs, v.tile_sorted_instances, I, np.uint32)
    inst_prim = read_device(bufs, v.instance_primitive, I, np.uint32)
    np.testing.assert_array_equal(inst_prim[sorted_inst], fw.inst_prims)
    gw, gh = cam.grid()
    np.testing.assert_array_equal(read_device(bufs, v.tile_ranges, 2 * gw * gh, np.uint32).reshape(-1, 2), fw.ranges)
    counters = read_device(bufs, v.counters, 4, np.uint32)
    assert counters[2] == 0, 'instance emission disagreed with the preprocess counts'
    # alpha uses the hardware exp2 (the oracle a correctly rounded one): a skip or stop decision can flip where
    # alpha sits within an ulp of 1/255 or T of 1e-4. The decisions depend on the fp32 geometry alone, which is
    # bit-exact for every appearance model (the neural colours do not enter them).
    check_image(image.cpu().numpy(), fw, device_contributors(bufs, v, cam), _image_tol(CASES[name]), name)


def _check_backward(name, densify_rows):
    import torch
    import efgs
    case = CASES[name]
    scene, app, cam = small_case(**case)
    dev = torch.device('cuda:0')
    configure(app)
    fw = O.render(scene, app, cam)
    g = np.random.default_rng(7).normal(size=fw.image.shape).astype(np.float32)
    ref = O.backward(scene, app, cam, fw, g, densify_rows=densify_rows,
                     densification_info=np.zeros((max(densify_rows, 1), scene.n), np.float32))
    inp = torch_inputs(scene, dev, requires_grad=True)
    if densify_rows:
        dinfo = torch.zeros((densify_rows, scene.n), dtype=torch.float32, device=dev)
    else:
        dinfo = torch.empty(0, device=dev)
    img = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], dinfo, settings(cam, dev),
                              precomputed_colors=inp['precomputed_colors'], base_colors=inp['base_colors'],
                              residual_params=inp['residual_params'], mlp_weights=inp['mlp_weights'])
    img.backward(torch.tensor(g, device=dev))
    torch.cuda.synchronize()
    keys = ['means', 'scales', 'rotations', 'opacities']
    keys += ['precomputed_colors'] if app.model == 'precomputed' else ['base_colors', 'residual_params']
    if app.model == 'neural':
        keys.append('mlp_weights')
    for k in keys:
        got = inp[k].grad.cpu().numpy()
        want = ref[k]
        if np.linalg.norm(want) == 0:
            assert np.abs(got).max() == 0, k
            continue
        e = rel_l2(got, want)
        print(f'case {name} (densification rows {densify_rows}) grad {k}: rel-L2 {e:.3e}', flush=True)
        assert e <= GRAD_TOL, f'{k}: rel-L2 {e}'
    if densify_rows:
        np.testing.assert_allclose(dinfo.cpu().numpy()[0], ref['densification_info'][0], rtol=0, atol=0)
        for row in range(1, densify_rows):
            e = rel_l2(dinfo.cpu().numpy()[row], ref['densification_info'][row])
            assert e <= GRAD_TOL, f'densification row {row}: {e}'


@pytest.mark.parametrize('name', list(CASES))
def test_backward_parity(name):
    """Gradients and all three densification rows (|dL/dmean2d| reduced as well)."""
    _check_backward(name, 3)


@pytest.mark.parametrize('name', ['sh3_relu', 'dense_2k', 'neural_c3_mlp', 'nasgabor'])
@pytest.mark.parametrize('rows', [0, 2])
def test_backward_parity_fewer_densification_rows(name, rows):
    """Without the third densification row the blend backward reduces 9 values instead of 11."""
    _check_backward(name, rows)


def test_backward_is_deterministic():
    import torch
    import efgs
    scene, app, cam = small_case(model='sh', n=2000, width=96, height=80, scale_shift=1.5)
    dev = torch.device('cuda:0')
    configure(app)
    outs = []
    for _ in range(2):
        inp = torch_inputs(scene, dev, requires_grad=True)
        img = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], torch.empty(0, device=dev),
                                  settings(cam, dev), base_colors=inp['base_colors'], residual_params=inp['residual_params'])
        img.sum().backward()
        outs.append([img.detach().cpu().numpy()] + [inp[k].grad.cpu().numpy() for k in ('means', 'scales', 'rotations', 'opacities',
                                                                                         'base_colors', 'residual_params')])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)


def test_c0_fused_colours_match_the_unfused_appearance():
    """BASELINE configuration c0: 10k Gaussians with SH degree 3, colour sigmoid(4 (base + residual(dir))), camera at
    the origin. The fused preprocess colours (every Gaussian visible: small, opaque, inside a wide view) equal the
    reference's unfused evaluation (AppearanceModel.forward restated in torch on the CPU) and the oracle's."""
    import math
    import torch
    from efgs.rasterization import forward_with_frame, frame_views
    from efgs.synthetic import c0_inputs
    import torch_ref as TR
    c0 = c0_inputs()
    n = c0['means'].shape[0]
    a = c0['appearance']
    app = O.Appearance(model='sh', base_act=a['base_act'], res_act=a['res_act'], color_act=a['color_act'], max_degree=3)
    width = height = 512
    f = (width / 2) / 0.7            # |x / z| <= 2 / 3 lands inside the image
    cam = O.Camera(w2c=np.eye(4, dtype=np.float32), position=c0['cam_position'], width=width, height=height, focal_x=f,
                   focal_y=f, center_x=width / 2, center_y=height / 2, degree=3)
    scene = O.Scene(means=c0['means'], scales=np.full((n, 3), math.log(0.01), np.float32),
                    rotations=np.tile(np.array([1, 0, 0, 0], np.float32), (n, 1)), opacities=np.full((n, 1), 2.0, np.float32),
                    base_colors=c0['base_colors'], residual_params=c0['residual_params'])
    unfused = TR.appearance_colors(torch.tensor(c0['means']), torch.tensor(c0['cam_position']), torch.tensor(c0['base_colors']),
                                   torch.tensor(c0['residual_params']), app, 3).numpy()
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    image, frame, bufs = forward_with_frame(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], settings(cam, dev),
                                            base_colors=inp['base_colors'], residual_params=inp['residual_params'])
    torch.cuda.synchronize()
    v = frame_views(frame)
    assert int(frame.n_visible) == n
    rec = read_device(bufs, v.records, 12 * n, np.float32).reshape(n, 12)
    err = float(np.abs(rec[:, 6:9] - unfused).max())
    print(f'c0: fused vs unfused colour max-abs {err:.3e}', flush=True)
    assert err <= 1e-5
    fw = O.render(scene, app, cam)
    np.testing.assert_allclose(rec[:, 6:9], fw.color, rtol=0, atol=1e-5)
