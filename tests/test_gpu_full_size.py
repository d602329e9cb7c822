"""GPU parity at the benchmark configurations' full sizes: the HIP path (through the C ABI) against the CPU
oracle on the seeded synthetic scenes of c1 (100k Gaussians, 800 x 800, SH degree 3), c3 (1M Gaussians,
1920 x 1080, neural appearance) and the c4 appearance sweep (c3 geometry, SV / NASG / NASGabor with 8 sites
or lobes, two colour activations each from {sigmoid, softplus, relu}; the third pair of each model runs at
test size in test_gpu_parity).

Bars (as in test_gpu_parity): counts, per-primitive tile counts and depth keys, projection records, the
index-ordered emission, tile keys, the tile-sorted primitive order and tile ranges bit-exact; image max-abs <= 1e-4
(fp32 appearance) or 2e-3 (fp16 MLP); last-contributor indices equal up to near-threshold decisions
(at most 2 + 1e-5 of the pixels, the neural path included: alpha comes from the bit-exact fp32 geometry); every gradient and
densification row rel-L2 <= 1e-3. Size-independent invariants (sorted tile keys, ranges partitioning the
instance list, per-tile counts summing to the instance count) are checked on the device arrays as well.
"""
import numpy as np
import pytest

import oracle as O
from efgs.synthetic import make_scene
from helpers import rel_l2, configure, torch_inputs, settings, read_device, check_emission, check_first_tiles, check_image, device_contributors

pytestmark = pytest.mark.gpu

IMAGE_TOL = 1e-4
IMAGE_TOL_FP16 = 2e-3
GRAD_TOL = 1e-3

# (configuration, colour activation override or None)
CONFIGS = {
    'c1_sh3': ('c1', None),
    'c3_neural': ('c3', None),
    'c4_sv_sigmoid': ('c4_sv', 'sigmoid'),
    'c4_nasg_softplus': ('c4_nasg', 'softplus'),
    'c4_nasgabor_relu': ('c4_nasgabor', 'relu'),
    'c4_sv_softplus': ('c4_sv', 'softplus'),
    'c4_nasg_sigmoid': ('c4_nasg', 'sigmoid'),
    'c4_nasgabor_sigmoid': ('c4_nasgabor', 'sigmoid'),
}


def _scene(name):
    cfg, color_act = CONFIGS[name]
    sc = make_scene(cfg)
    cam0 = sc['camera']
    app = dict(sc['appearance'])
    if color_act is not None:
        app['color_act'] = color_act
    cam = O.Camera(w2c=cam0['w2c'], position=cam0['position'], width=cam0['width'], height=cam0['height'],
                   focal_x=cam0['focal_x'], focal_y=cam0['focal_y'], center_x=cam0['center_x'], center_y=cam0['center_y'],
                   bg=np.array([0.1, 0.2, 0.3], np.float32), degree=app['max_degree'] if app['model'] != 'neural' else 1,
                   near_plane=cam0['near_plane'], far_plane=cam0['far_plane'])
    mlp = O.MLPConfig(**app['mlp']) if app.get('mlp') else None
    scene = O.Scene(means=sc['means'], scales=sc['scales'], rotations=sc['rotations'], opacities=sc['opacities'],
                    base_colors=sc['base_colors'], residual_params=sc['residual_params'], mlp_weights=sc['mlp_weights'])
    oapp = O.Appearance(model=app['model'], base_act=app['base_act'], res_act=app['res_act'], color_act=app['color_act'],
                        direction_gradient=app['direction_gradient'], max_degree=app['max_degree'], mlp=mlp)
    return scene, oapp, cam


@pytest.mark.parametrize('name', list(CONFIGS))
def test_full_size_parity(name):
    import torch
    import efgs
    from efgs.rasterization import forward_with_frame, frame_views

    scene, app, cam = _scene(name)
    neural = app.model == 'neural'
    n = scene.n
    print(f'case {name}: N={n} {cam.width}x{cam.height} {app.model}/{app.color_act}: oracle forward', flush=True)
    fw = O.render(scene, app, cam)
    g = np.random.default_rng(7).normal(size=fw.image.shape).astype(np.float32)
    print(f'case {name}: oracle backward', flush=True)
    ref = O.backward(scene, app, cam, fw, g, densify_rows=3, densification_info=np.zeros((3, n), np.float32))

    print(f'case {name}: device forward', flush=True)
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    st = settings(cam, dev)
    image, frame, bufs = forward_with_frame(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], st,
                                            base_colors=inp['base_colors'], residual_params=inp['residual_params'],
                                            mlp_weights=inp['mlp_weights'])
    torch.cuda.synchronize()
    v = frame_views(frame)
    V, I = int(frame.n_visible), int(frame.n_instances)
    print(f'case {name}: V={V} I={I} (oracle V={len(fw.visible)} I={len(fw.inst_keys)})', flush=True)
    assert V == len(fw.visible) and I == len(fw.inst_keys)

    # per primitive
    n_touched = read_device(bufs, v.n_touched, n, np.uint32)
    np.testing.assert_array_equal(n_touched, fw.n_touched)
    vis = fw.n_touched > 0
    np.testing.assert_array_equal(read_device(bufs, v.depth_keys, n, np.uint32)[vis], fw.depth_key[vis])
    rec = read_device(bufs, v.records, 12 * n, np.float32).reshape(n, 12)[vis]
    np.testing.assert_array_equal(rec[:, 0:2], fw.mean2d[vis])
    np.testing.assert_array_equal(rec[:, 2:5], fw.conic_opacity[vis][:, 0:3])
    np.testing.assert_array_equal(rec[:, 5], fw.conic_opacity[vis][:, 3])
    bx, by = rec[:, 9].view(np.uint32), rec[:, 10].view(np.uint32)
    np.testing.assert_array_equal(np.stack([bx & 0xffff, bx >> 16, by & 0xffff, by >> 16], 1), fw.bounds[vis].astype(np.uint32))
    # appearance colours: transcendental-heavy, compared to a tolerance (the image bar applies downstream)
    np.testing.assert_allclose(rec[:, 6:9], fw.color[vis], rtol=0, atol=IMAGE_TOL_FP16 if neural else IMAGE_TOL / 10)

    # index-ordered emission, tile order and ranges
    check_emission(bufs, v, frame, fw, n)
    check_first_tiles(rec, fw, vis, *cam.grid())
    kdt = np.uint16 if frame.key_bytes == 2 else np.uint32
    keys = read_device(bufs, v.tile_sorted_keys, I, kdt).astype(np.uint32)
    assert np.all(np.diff(keys.astype(np.int64)) >= 0), 'tile keys not sorted'
    np.testing.assert_array_equal(keys, fw.inst_keys)
    sorted_inst = read_device(bufs, v.tile_sorted_instances, I, np.uint32)
    inst_prim = read_device(bufs, v.instance_primitive, I, np.uint32)
    np.testing.assert_array_equal(inst_prim[sorted_inst], fw.inst_prims)
    gw, gh = cam.grid()
    ranges = read_device(bufs, v.tile_ranges, 2 * gw * gh, np.uint32).reshape(-1, 2)
    np.testing.assert_array_equal(ranges, fw.ranges)
    nonempty = ranges[:, 1] > ranges[:, 0]
    assert int((ranges[:, 1] - ranges[:, 0]).sum()) == I and int(n_touched.sum()) == I
    starts = ranges[nonempty, 0]
    assert starts[0] == 0 and np.all(starts[1:] == ranges[nonempty, 1][:-1]), 'ranges do not partition the instances'
    assert read_device(bufs, v.counters, 4, np.uint32)[2] == 0, 'instance emission disagreed with the preprocess counts'

    # image and last contributors
    check_image(image.cpu().numpy(), fw, device_contributors(bufs, v, cam), IMAGE_TOL_FP16 if neural else IMAGE_TOL, name)
    del image, frame, bufs

    # gradients through the autograd path
    print(f'case {name}: device backward', flush=True)
    inp = torch_inputs(scene, dev, requires_grad=True)
    dinfo = torch.zeros((3, n), dtype=torch.float32, device=dev)
    img = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], dinfo, st,
                              base_colors=inp['base_colors'], residual_params=inp['residual_params'],
                              mlp_weights=inp['mlp_weights'])
    img.backward(torch.tensor(g, device=dev))
    torch.cuda.synchronize()
    keys_grad = ['means', 'scales', 'rotations', 'opacities', 'base_colors', 'residual_params'] + (['mlp_weights'] if neural else [])
    for k in keys_grad:
        e = rel_l2(inp[k].grad.cpu().numpy(), ref[k])
        print(f'case {name}: grad {k} rel-L2 {e:.3e}', flush=True)
        assert e <= GRAD_TOL, f'{k}: rel-L2 {e}'
    d = dinfo.cpu().numpy()
    np.testing.assert_array_equal(d[0], ref['densification_info'][0])
    for row in (1, 2):
        e = rel_l2(d[row], ref['densification_info'][row])
        assert e <= GRAD_TOL, f'densification row {row}: rel-L2 {e}'
