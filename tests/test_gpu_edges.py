"""GPU edge cases of the boundary: empty and fully culled scenes, degenerate quaternions, 32-bit tile keys,
primitives straddling the near plane, error behaviour, and Adam through the C ABI."""
import numpy as np
import pytest

import oracle as O
from helpers import small_case, configure, torch_inputs, settings, read_device, rel_l2, check_image, device_contributors

pytestmark = pytest.mark.gpu


def _render(scene, app, cam):
    import torch
    from efgs.rasterization import forward_with_frame
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    image, frame, bufs = forward_with_frame(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], settings(cam, dev),
                                            precomputed_colors=inp['precomputed_colors'], base_colors=inp['base_colors'],
                                            residual_params=inp['residual_params'], mlp_weights=inp['mlp_weights'])
    torch.cuda.synchronize()
    return image.cpu().numpy(), frame, bufs


def test_empty_scene_renders_background():
    scene, app, cam = small_case(model='sh', n=10)
    empty = O.Scene(means=scene.means[:0], scales=scene.scales[:0], rotations=scene.rotations[:0], opacities=scene.opacities[:0],
                    base_colors=scene.base_colors[:0], residual_params=scene.residual_params[:0])
    image, frame, _ = _render(empty, app, cam)
    assert frame.n_visible == 0 and frame.n_instances == 0
    np.testing.assert_array_equal(image, np.broadcast_to(cam.bg[:, None, None], image.shape))


def test_all_culled_behind_camera_and_degenerate():
    scene, app, cam = small_case(model='sh', n=300)
    means = scene.means.copy()
    means[:150, 2] = -50.0                       # behind the camera (depth < near)
    rot = scene.rotations.copy()
    rot[150:] = 0.0                              # zero quaternions are culled
    s2 = O.Scene(means=means, scales=scene.scales, rotations=rot, opacities=scene.opacities, base_colors=scene.base_colors,
                 residual_params=scene.residual_params)
    image, frame, _ = _render(s2, app, cam)
    fw = O.render(s2, app, cam)
    assert frame.n_visible == 0 == len(fw.visible)
    np.testing.assert_allclose(image, fw.image, atol=0)


def test_thirty_two_bit_tile_keys():
    # 4200 x 3000 px -> 263 x 250 = 65750 tiles, beyond 16-bit keys
    scene, app, cam = small_case(model='sh', n=3000, width=4200, height=3000, scale_shift=4.0, distance=5.0)
    image, frame, bufs = _render(scene, app, cam)
    assert frame.key_bytes == 4
    fw = O.render(scene, app, cam)
    assert frame.n_instances == len(fw.inst_keys)
    from efgs.rasterization import frame_views
    v = frame_views(frame)
    np.testing.assert_array_equal(read_device(bufs, v.tile_sorted_keys, int(frame.n_instances), np.uint32), fw.inst_keys)
    gw, gh = cam.grid()
    np.testing.assert_array_equal(read_device(bufs, v.tile_ranges, 2 * gw * gh, np.uint32).reshape(-1, 2), fw.ranges)
    # (a dense scene: almost every pixel ends within a few fragments of T = 1e-4)
    check_image(image, fw, device_contributors(bufs, v, cam), 1e-4, '4200x3000')


def test_long_tile_runs():
    # Tile runs longer than the forward blend sorts itself (256): the tile sort's LDS-slab (<= 512) and chunked paths,
    # beside runs the forward sorts; the order, ranges, the blend's primitives and the image match the oracle.
    scene, app, cam = small_case(model='precomputed', n=3000, width=96, height=72, scale_shift=3.0)
    fw = O.render(scene, app, cam)
    runs = np.diff(np.asarray(fw.ranges).reshape(-1, 2), axis=1)[:, 0]
    assert (runs > 512).any() and ((runs > 256) & (runs <= 512)).any() and ((runs > 0) & (runs <= 256)).any()
    image, frame, bufs = _render(scene, app, cam)
    from efgs.rasterization import frame_views
    v = frame_views(frame)
    I = int(frame.n_instances)
    assert I == len(fw.inst_keys)
    gw, gh = cam.grid()
    np.testing.assert_array_equal(read_device(bufs, v.tile_ranges, 2 * gw * gh, np.uint32).reshape(-1, 2), fw.ranges)
    kt = np.uint16 if frame.key_bytes == 2 else np.uint32
    np.testing.assert_array_equal(read_device(bufs, v.tile_sorted_keys, I, kt).astype(np.uint32), fw.inst_keys)
    sorted_inst = read_device(bufs, v.tile_sorted_instances, I, np.uint32)
    inst_prim = read_device(bufs, v.instance_primitive, I, np.uint32)
    np.testing.assert_array_equal(inst_prim[sorted_inst], fw.inst_prims)
    check_image(image, fw, device_contributors(bufs, v, cam), 1e-4, 'long runs')


def test_sort_beyond_24_bit_emission_indices():
    # 60k large Gaussians at 4200x3000 (65,750 tiles, 32-bit tile keys, global-atomic binning): 19.3M instances, more
    # than the 2^24 - 1 emission indices that the forward's packed sort keys hold, so runs of <= 256 are sorted with
    # (depth, emission index) keys and their primitives gathered, beside the LDS-slab sorts of longer runs.
    # Too large for the oracle's blend: checked by the properties that define the result. Emission: primitives in
    # index order, each one's tiles ascending, as many as its count. Sorted arrays: the same (tile, primitive) pairs,
    # grouped by the tile ranges, and within each tile strictly increasing in (depth key, primitive index).
    scene, app, cam = small_case(model='precomputed', n=60000, width=4200, height=3000, scale_shift=1.5)
    print('case sort beyond 24-bit emission indices: n=60000 4200x3000', flush=True)
    _, frame, bufs = _render(scene, app, cam)
    from efgs.rasterization import frame_views
    v = frame_views(frame)
    I, n = int(frame.n_instances), 60000
    gw, gh = cam.grid()
    T = gw * gh
    assert frame.key_bytes == 4 and I >= (1 << 24)
    inst_key = read_device(bufs, v.instance_keys, I, np.uint32).astype(np.int64)
    inst_prim = read_device(bufs, v.instance_primitive, I, np.uint32).astype(np.int64)
    n_touched = read_device(bufs, v.n_touched, n, np.uint32).astype(np.int64)
    depth = read_device(bufs, v.depth_keys, n, np.uint32).astype(np.int64)
    ranges = read_device(bufs, v.tile_ranges, 2 * T, np.uint32).reshape(-1, 2).astype(np.int64)
    sorted_key = read_device(bufs, v.tile_sorted_keys, I, np.uint32).astype(np.int64)
    sorted_inst = read_device(bufs, v.tile_sorted_instances, I, np.uint32).astype(np.int64)
    # emission
    assert np.all(np.diff(inst_prim) >= 0)
    same = np.diff(inst_prim) == 0
    assert np.all(np.diff(inst_key)[same] > 0)
    np.testing.assert_array_equal(np.bincount(inst_prim, minlength=n), n_touched)
    # ranges partition the instances in tile order; every tile's run sorted by (depth key, primitive)
    runs = ranges[:, 1] - ranges[:, 0]
    assert ranges[0, 0] == 0 and ranges[-1, 1] == I and np.all(ranges[1:, 0] == ranges[:-1, 1])
    assert ((runs > 0) & (runs <= 256)).sum() > 1000 and (runs > 256).sum() > 1000
    np.testing.assert_array_equal(sorted_key, np.repeat(np.arange(T), runs))
    sorted_prim = inst_prim[sorted_inst]
    np.testing.assert_array_equal(np.sort(sorted_key * n + sorted_prim), np.sort(inst_key * n + inst_prim))
    d = depth[sorted_prim]
    within = sorted_key[1:] == sorted_key[:-1]
    increasing = (d[1:] > d[:-1]) | ((d[1:] == d[:-1]) & (sorted_prim[1:] > sorted_prim[:-1]))
    assert np.all(increasing[within])


def test_near_plane_straddle():
    scene, app, cam = small_case(model='sh', n=400, distance=2.0)  # camera inside the cube: many behind / near
    image, frame, _ = _render(scene, app, cam)
    fw = O.render(scene, app, cam)
    assert frame.n_visible == len(fw.visible)
    assert np.abs(image - fw.image).max() <= 1e-4


def test_forward_before_set_appearance_raises():
    import torch
    import efgs
    from efgs import rasterization as R
    fresh = R.Rasterizer()
    saved = R._rasterizer
    R._rasterizer = fresh
    try:
        scene, app, cam = small_case(model='sh', n=10)
        dev = torch.device('cuda:0')
        inp = torch_inputs(scene, dev)
        with pytest.raises(RuntimeError, match='not initialized'):
            efgs.rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], settings(cam, dev), True, False,
                           base_colors=inp['base_colors'], residual_params=inp['residual_params'])
    finally:
        R._rasterizer = saved


def test_fused_adam_matches_oracle_bitwise():
    import torch
    import efgs
    dev = torch.device('cuda:0')
    rng = np.random.default_rng(0)
    # an LR list cycling over a trailing dimension of 7, and an odd-sized group with a 3-entry list
    shapes = [(1000, 3), (1000, 8, 7), (6144,), (1001,)]
    lrs = [1e-3, [1e-2, 1e-2, 1e-2, 5e-3, 2e-3, 2e-3, 2e-3], 4e-4, [3e-3, 1e-3, 2e-3]]
    betas = [(0.9, 0.999), (0.9, 0.999), (0.9, 0.99), (0.8, 0.99)]
    params = [torch.tensor(rng.normal(size=s).astype(np.float32), device=dev, requires_grad=True) for s in shapes]
    groups = [{'params': [p], 'lr': lr, 'betas': b} for p, lr, b in zip(params, lrs, betas)]
    opt = efgs.FusedAdam(groups, lr=0.0, eps=1e-15)
    ref_p = [p.detach().cpu().numpy().copy() for p in params]
    ref_m = [np.zeros_like(r) for r in ref_p]
    ref_v = [np.zeros_like(r) for r in ref_p]
    for step in range(1, 4):
        for i, p in enumerate(params):
            g = rng.normal(size=p.shape).astype(np.float32)
            p.grad = torch.tensor(g, device=dev)
            O.adam_step(g, ref_p[i], ref_m[i], ref_v[i], step, lrs[i], betas[i][0], betas[i][1], 1e-15)
        opt.step()
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            np.testing.assert_array_equal(p.detach().cpu().numpy(), ref_p[i])
            st = opt.state[p]
            np.testing.assert_array_equal(st['exp_avg'].cpu().numpy(), ref_m[i])
            np.testing.assert_array_equal(st['exp_avg_sq'].cpu().numpy(), ref_v[i])


def test_rasterize_inference_layouts():
    """efgs_render writes CHW or HWC, clamped or not, in the blend kernel: every combination equals the oracle's
    image (clamped to [0, 1] where asked) and, unclamped CHW, the training forward's image bit for bit."""
    import torch
    import efgs
    scene, app, cam = small_case(model='sh', n=500)
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    st = settings(cam, dev)
    fw = O.render(scene, app, cam)
    imgs = {}
    for to_chw in (True, False):
        for clamp in (True, False):
            img = efgs.rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], st, to_chw, clamp,
                                 base_colors=inp['base_colors'], residual_params=inp['residual_params'])
            assert img.shape == ((3, cam.height, cam.width) if to_chw else (cam.height, cam.width, 3))
            got = img.cpu().numpy() if to_chw else img.cpu().numpy().transpose(2, 0, 1)
            want = np.clip(fw.image, 0, 1) if clamp else fw.image
            assert np.abs(got - want).max() <= 1e-4
            imgs[(to_chw, clamp)] = got
    assert np.array_equal(imgs[(True, False)], imgs[(False, False)]) and np.array_equal(imgs[(True, True)], imgs[(False, True)])
    train = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], torch.empty(0, device=dev), st,
                                base_colors=inp['base_colors'], residual_params=inp['residual_params'])
    assert np.array_equal(train.detach().cpu().numpy(), imgs[(True, False)])


def test_rasterize_neural_inference_matches_training_forward():
    import torch
    import efgs
    scene, app, cam = small_case(model='neural', n=800)
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev)
    st = settings(cam, dev)
    hwc = efgs.rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], st, False, True,
                         base_colors=inp['base_colors'], residual_params=inp['residual_params'], mlp_weights=inp['mlp_weights'])
    train = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], torch.empty(0, device=dev), st,
                                base_colors=inp['base_colors'], residual_params=inp['residual_params'], mlp_weights=inp['mlp_weights'])
    assert np.array_equal(hwc.cpu().numpy(), np.clip(train.detach().cpu().numpy(), 0, 1).transpose(1, 2, 0))

def test_backward_twice_through_a_retained_graph():
    """The backward's outputs are prepared during the forward; a second backward of the same graph
    (retain_graph) gets fresh outputs, so the gradients the first one produced stay intact."""
    import torch
    import efgs
    scene, app, cam = small_case(model='neural', n=400)
    dev = torch.device('cuda:0')
    configure(app)
    inp = torch_inputs(scene, dev, requires_grad=True)
    img = efgs.diff_rasterize(inp['means'], inp['scales'], inp['rotations'], inp['opacities'], torch.empty(0, device=dev),
                              settings(cam, dev), base_colors=inp['base_colors'], residual_params=inp['residual_params'],
                              mlp_weights=inp['mlp_weights'])
    g = torch.randn_like(img)
    img.backward(g, retain_graph=True)
    first = {k: v.grad.clone() for k, v in inp.items() if v is not None and v.grad is not None}
    held = {k: v.grad for k, v in inp.items() if v is not None and v.grad is not None}
    for v in inp.values():
        if v is not None:
            v.grad = None
    img.backward(g)
    torch.cuda.synchronize()
    assert set(first) == {'means', 'scales', 'rotations', 'opacities', 'base_colors', 'residual_params', 'mlp_weights'}
    for k in first:
        assert torch.equal(inp[k].grad, first[k]), k
        assert torch.equal(held[k], first[k]), k  # the first call's tensors were not written again
        assert inp[k].grad.data_ptr() != held[k].data_ptr(), k


@pytest.mark.parametrize('n_total', [1_500_000, 1_900_000])
def test_block_count_scan_at_large_primitive_counts(n_total):
    # The per-block count scan over 5860 / 7422 preprocess blocks (several blocks per scan thread): the same
    # 400 visible primitives, spread through a scene padded with primitives behind the camera, must render
    # exactly as the 400 alone (same visible set, order and keys).
    scene, app, cam = small_case(model='sh', n=400)
    m = len(scene.means)
    slots = np.linspace(17, n_total - 5, m).astype(np.int64)
    src = np.arange(n_total) % m

    def pad(a):
        out = a[src].copy()
        out[slots] = a
        return out
    means = pad(scene.means)
    hidden = np.ones(n_total, bool)
    hidden[slots] = False
    means[hidden, 2] = -50.0
    big = O.Scene(means=means, scales=pad(scene.scales), rotations=pad(scene.rotations), opacities=pad(scene.opacities),
                  base_colors=pad(scene.base_colors), residual_params=pad(scene.residual_params))
    small_img, small_frame, _ = _render(scene, app, cam)
    big_img, big_frame, _ = _render(big, app, cam)
    assert small_frame.n_visible > 0
    assert (big_frame.n_visible, big_frame.n_instances) == (small_frame.n_visible, small_frame.n_instances)
    np.testing.assert_array_equal(big_img, small_img)


# (width, height, primitives, sparse and dense scale shifts): fused-emission grids, a small one and one of 13,400
# tiles (its histogram near the LDS limit of 16,384 tiles), and a 32-bit-key grid (global-atomic counting)
SPECULATION_GRIDS = {
    'fused_64x48': (64, 48, 600, 1.0, 3.5),
    'fused_1600x1600': (1600, 1600, 600, 0.5, 2.0),
    'global_4200x3000': (4200, 3000, 800, 0.5, 1.5),
}


@pytest.mark.parametrize('grid', list(SPECULATION_GRIDS))
def test_instance_buffers_sized_from_the_previous_frame(grid):
    # After a frame of a scene size the forward launches the binning and the blend into instance buffers sized
    # from that frame's count (+12.5 % + 1024) before it reads the counters. A second scene of the same primitive
    # count and image size with far larger Gaussians overflows them: the device skips the binning and the blend and
    # the host re-runs them with exact buffers. A third, sparse one fits the (now large) speculative buffers; the
    # fourth, dense again, fits them too. Every frame's keys, order, ranges and image match the oracle and the
    # overflow flag ends cleared, on each binning path.
    from efgs.rasterization import frame_views
    width, height, n, s_sparse, s_dense = SPECULATION_GRIDS[grid]
    sparse, app, cam = small_case(model='sh', n=n, width=width, height=height, scale_shift=s_sparse)
    dense = O.Scene(means=sparse.means, scales=sparse.scales + (s_dense - s_sparse), rotations=sparse.rotations,
                    opacities=sparse.opacities, base_colors=sparse.base_colors, residual_params=sparse.residual_params)
    gw, gh = cam.grid()
    counts = []
    for k, scene in enumerate((sparse, dense, sparse, dense)):
        print(f'speculation {grid}: frame {k}', flush=True)
        image, frame, bufs = _render(scene, app, cam)
        fw = O.render(scene, app, cam)
        assert frame.n_instances == len(fw.inst_keys)
        assert frame.instance_capacity >= frame.n_instances
        v = frame_views(frame)
        kt = np.uint16 if frame.key_bytes == 2 else np.uint32
        assert frame.key_bytes == (2 if gw * gh <= 65535 else 4)
        np.testing.assert_array_equal(read_device(bufs, v.tile_sorted_keys, int(frame.n_instances), kt).astype(np.uint32), fw.inst_keys)
        sorted_inst = read_device(bufs, v.tile_sorted_instances, int(frame.n_instances), np.uint32)
        inst_prim = read_device(bufs, v.instance_primitive, int(frame.n_instances), np.uint32)
        np.testing.assert_array_equal(inst_prim[sorted_inst], fw.inst_prims)
        np.testing.assert_array_equal(read_device(bufs, v.tile_ranges, 2 * gw * gh, np.uint32).reshape(-1, 2), fw.ranges)
        check_image(image, fw, device_contributors(bufs, v, cam), 1e-4)
        assert read_device(bufs, v.counters, 8, np.uint32)[5] == 0  # overflow flag cleared by the re-run
        counts.append(int(frame.n_instances))
    assert counts[1] > counts[0] + counts[0] // 8 + 1024  # the dense frame did overflow the sparse frame's buffers
