"""Shared builders for the parity tests: small seeded scenes in oracle form, their torch counterparts and
settings, device-buffer readers for frame inspection."""
from __future__ import annotations

import numpy as np

import oracle as O
from efgs.synthetic import make_scene, xavier_mlp

MODEL_CONFIG = {'sh': 'c1', 'sv': 'c4_sv', 'nasg': 'c4_nasg', 'nasgabor': 'c4_nasgabor', 'neural': 'c3', 'precomputed': 'c1'}


def small_case(model='sh', n=500, width=64, height=48, seed=0, scale_shift=2.0, acts=None, degree=None, bg=(0.1, 0.2, 0.3),
               proper_aa=False, render_base=True, render_residual=True, direction_gradient=True, distance=None, mlp=None):
    """Oracle (scene, appearance, camera) of a seeded scene with Gaussians enlarged by exp(scale_shift) so
    they cover several pixels at test resolutions."""
    cfg = MODEL_CONFIG[model]
    sc = make_scene(cfg, n=n, seed=seed, width=width, height=height)
    cam0 = sc['camera']
    app_cfg = sc['appearance']
    default_degree = {'sh': 3, 'sv': 8, 'nasg': 8, 'nasgabor': 8, 'neural': 1, 'precomputed': 0}[model]
    w2c = cam0['w2c'].copy()
    pos = cam0['position'].copy()
    if distance is not None:
        w2c[2, 3] = distance
        pos[2] = -distance
    cam = O.Camera(w2c=w2c, position=pos, width=width, height=height, focal_x=cam0['focal_x'], focal_y=cam0['focal_y'],
                   center_x=width / 2.0, center_y=height / 2.0, bg=np.array(bg, np.float32),
                   degree=default_degree if degree is None else degree, proper_aa=proper_aa, render_base=render_base,
                   render_residual=render_residual)
    base_act, res_act, color_act = acts if acts is not None else (app_cfg['base_act'], app_cfg['res_act'], app_cfg['color_act'])
    if model == 'precomputed':
        rng = np.random.default_rng(seed + 100)
        scene = O.Scene(means=sc['means'], scales=sc['scales'] + scale_shift, rotations=sc['rotations'], opacities=sc['opacities'],
                        precomputed_colors=rng.uniform(0, 1, size=(n, 3)).astype(np.float32))
        app = O.Appearance(model='precomputed')
        return scene, app, cam
    mlp_cfg = None
    residual, weights = sc['residual_params'], sc['mlp_weights']
    if model == 'neural':
        mlp_cfg = O.MLPConfig(**(mlp if mlp is not None else app_cfg['mlp']))
        if mlp is not None:
            rng = np.random.default_rng(seed + 200)
            residual = rng.normal(0.0, 0.1, size=(n, mlp_cfg.n_feature_dims)).astype(np.float32)
            weights = xavier_mlp(rng, mlp_cfg.n_input_dims, mlp_cfg.n_neurons, mlp_cfg.n_hidden_layers)
    scene = O.Scene(means=sc['means'], scales=sc['scales'] + scale_shift, rotations=sc['rotations'], opacities=sc['opacities'],
                    base_colors=sc['base_colors'], residual_params=residual, mlp_weights=weights)
    app = O.Appearance(model=model, base_act=base_act, res_act=res_act, color_act=color_act, direction_gradient=direction_gradient,
                       max_degree=app_cfg['max_degree'], mlp=mlp_cfg)
    return scene, app, cam


def single_tile_state(mean2d, conic_opacity, color, bg):
    """Forward state of one 16 x 12 tile whose instances are the given 2D Gaussians in order."""
    import ctypes
    from types import SimpleNamespace
    k = mean2d.shape[0]
    W, H = 16, 12
    ranges = np.array([0, k], np.uint32)
    inst = np.arange(k, dtype=np.uint32)
    bounds = np.tile(np.array([0, W, 0, H], np.uint16), (k, 1))
    image = np.zeros((3, H, W), np.float32)
    final_T = np.zeros(H * W, np.float32)
    n_contrib = np.zeros(H * W, np.uint32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    O.lib().efo_blend_forward(ctypes.c_int(W), ctypes.c_int(H), ctypes.c_int(1), ctypes.c_int(1), p(ranges), p(inst), p(bounds), p(mean2d),
                              p(conic_opacity), p(color), p(bg), p(image), p(final_T), p(n_contrib))
    cam = SimpleNamespace(width=W, height=H, bg=bg, grid=lambda: (1, 1))
    fw = SimpleNamespace(n_touched=np.ones(k, np.uint32), ranges=ranges, inst_prims=inst, mean2d=mean2d, conic_opacity=conic_opacity,
                         color=color, image=image, final_T=final_T, n_contrib=n_contrib)
    return cam, fw


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def contributor_tolerance(n_pixels: int) -> int:
    """Pixels whose last-contributor index may differ from the oracle's: the blend evaluates alpha with the
    hardware exp2 (within 1 ulp of the oracle's), which can flip an alpha >= 1/255 or T < 1e-4 decision only
    where the value sits within an ulp of the threshold."""
    return 2 + n_pixels // 100000


# Image difference allowed at a pixel where a near-threshold decision flipped (the device's alpha uses the hardware
# exp2, the oracle's a correctly rounded one): at the stop, the one fragment taken or skipped has weight T alpha <= 0.99 T
# with T (1 - alpha) at the 1e-4 threshold (<= 1e-2); at a skip (alpha within an ulp of 1/255, the last contributor
# unchanged), the fragment's weight is <= 4e-3 T and the later fragments are rescaled by the same factor; times colours
# and background of magnitude <= 2.
FLIPPED_PIXEL_TOL = 2e-2


def device_contributors(bufs, v, cam) -> np.ndarray:
    """The device's last-contributor indices in image order (H * W): the blend stores them per tile (16 x 12
    row-major)."""
    gw, gh = cam.grid()
    nc = read_device(bufs, v.n_contributors, gw * gh * 192, np.uint32).reshape(gh, gw, 12, 16).transpose(0, 2, 1, 3)
    return nc.reshape(gh * 12, gw * 16)[:cam.height, :cam.width].reshape(-1)


def check_image(image, fw, nc, tol: float, name: str = '') -> int:
    """Image parity: max-abs <= tol at every pixel but at most contributor_tolerance ones, where a near-threshold
    skip or stop decision flipped (those differ by at most FLIPPED_PIXEL_TOL); the last-contributor indices nc (image
    order) equal the oracle's at all but at most contributor_tolerance pixels. Returns the number of pixels over tol."""
    image = np.asarray(image)
    diff = np.abs(image - fw.image).reshape(3, -1).max(axis=0)
    mism = int(np.count_nonzero(nc != fw.n_contrib))
    over = diff > tol
    n_over = int(np.count_nonzero(over))
    err = float(diff[~over].max()) if diff.size > n_over else 0.0
    print(f'case {name}: image max-abs {err:.3e} at all but {n_over} of {diff.size} pixels'
          + (f' (max-abs {float(diff[over].max()):.3e} there)' if n_over else '') + f', {mism} last-contributor mismatches',
          flush=True)
    assert mism <= contributor_tolerance(nc.size), f'{mism} last-contributor mismatches'
    assert n_over <= contributor_tolerance(diff.size), f'{n_over} pixels with image max-abs above {tol}'
    if n_over:
        assert float(diff[over].max()) <= FLIPPED_PIXEL_TOL
    return n_over


# ---------------------------------------------------------------------------------------------------------
# torch side (GPU tests only)
# ---------------------------------------------------------------------------------------------------------

def configure(app: O.Appearance) -> None:
    import efgs
    if app.model == 'precomputed':
        return
    efgs.initialize_appearance(app.model, app.max_degree, app.base_act, app.res_act, app.color_act, app.direction_gradient)
    if app.model == 'neural':
        m = app.mlp
        efgs.initialize_residual_mlp(m.n_input_dims, 3, {'otype': 'Identity'},
                                     {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None',
                                      'n_neurons': m.n_neurons, 'n_hidden_layers': m.n_hidden_layers},
                                     m.base_input, m.n_frequencies, list(m.sh_degrees))


def torch_inputs(scene: O.Scene, device, requires_grad=False) -> dict:
    import torch

    def t(a):
        if a is None:
            return None
        x = torch.tensor(np.ascontiguousarray(a, np.float32), device=device)
        x.requires_grad_(requires_grad)
        return x
    return dict(means=t(scene.means), scales=t(scene.scales), rotations=t(scene.rotations), opacities=t(scene.opacities),
                precomputed_colors=t(scene.precomputed_colors), base_colors=t(scene.base_colors),
                residual_params=t(scene.residual_params), mlp_weights=t(scene.mlp_weights))


def settings(cam: O.Camera, device):
    import torch
    import efgs
    return efgs.RasterizerSettings(
        w2c=torch.tensor(np.asarray(cam.w2c, np.float32), device=device),
        cam_position=torch.tensor(np.asarray(cam.position, np.float32), device=device),
        bg_color=torch.tensor(np.asarray(cam.bg, np.float32), device=device),
        appearance_degree=cam.degree, width=cam.width, height=cam.height, focal_x=cam.focal_x, focal_y=cam.focal_y,
        center_x=cam.center_x, center_y=cam.center_y, near_plane=cam.near_plane, far_plane=cam.far_plane,
        proper_antialiasing=cam.proper_aa, render_base=cam.render_base, render_residual=cam.render_residual)


def read_device(buffers, ptr: int, count: int, dtype) -> np.ndarray:
    """Copies `count` elements of `dtype` at device address `ptr` (inside one of the frame's buffers) to numpy."""
    nbytes = count * np.dtype(dtype).itemsize
    if nbytes == 0:
        return np.zeros(0, dtype)
    for b in buffers:
        base = b.data_ptr()
        if base <= ptr and ptr + nbytes <= base + b.numel():
            return b[ptr - base: ptr - base + nbytes].cpu().numpy().view(dtype).copy()
    raise AssertionError('pointer outside the frame buffers')


def check_emission(bufs, v, frame, fw, n: int) -> None:
    """Index-ordered emission against the oracle: the visible primitives in index order, each one's first
    emission slot (exclusive scan of the tile counts in index order) and, at the emission slots, every
    primitive's tiles in ascending order (its tile rectangle in row-major order)."""
    V, I = int(frame.n_visible), int(frame.n_instances)
    np.testing.assert_array_equal(read_device(bufs, v.visible_prims, V, np.uint32), fw.visible)
    counts = fw.n_touched.astype(np.int64)
    offsets = np.cumsum(counts) - counts
    vis = fw.n_touched > 0
    np.testing.assert_array_equal(read_device(bufs, v.prim_offset, n, np.uint32)[vis], offsets[vis])
    order = np.lexsort((fw.inst_keys, fw.inst_prims))  # by primitive, then tile
    kt = np.uint16 if frame.key_bytes == 2 else np.uint32
    np.testing.assert_array_equal(read_device(bufs, v.instance_keys, I, kt).astype(np.uint32), fw.inst_keys[order])
    np.testing.assert_array_equal(read_device(bufs, v.instance_primitive, I, np.uint32), fw.inst_prims[order])


# tiles of a primitive's rectangle whose test results the preprocess records in the record's spare word
SEQUENTIAL_TILES = 8


def check_first_tiles(rec: np.ndarray, fw, vis: np.ndarray, grid_w: int, grid_h: int) -> None:
    """The record's spare word (column 11): bit j (j < SEQUENTIAL_TILES) set exactly when tile j of the primitive's
    tile rectangle (row-major) is one of the tiles the oracle emits for it (the preprocess's tile-test results that
    instance emission reads instead of testing again). rec: the device records of the visible primitives."""
    prims = np.nonzero(vis)[0]
    b = fw.bounds[vis].astype(np.int64)
    x0, x1 = b[:, 0] // 16, (b[:, 1] + 15) // 16
    y0, y1 = b[:, 2] // 12, (b[:, 3] + 11) // 12
    bw = x1 - x0
    cnt = bw * (y1 - y0)
    n_tiles_max = int(grid_w) * int(grid_h)
    emitted = np.sort(fw.inst_prims.astype(np.int64) * n_tiles_max + fw.inst_keys.astype(np.int64))
    expected = np.zeros(len(prims), np.uint32)
    for j in range(SEQUENTIAL_TILES):
        tile = (y0 + j // np.maximum(bw, 1)) * grid_w + x0 + j % np.maximum(bw, 1)
        code = prims * n_tiles_max + tile
        pos = np.minimum(np.searchsorted(emitted, code), len(emitted) - 1)
        hit = (j < cnt) & (emitted[pos] == code) if len(emitted) else np.zeros(len(prims), bool)
        expected |= hit.astype(np.uint32) << np.uint32(j)
    np.testing.assert_array_equal(rec[:, 11].view(np.uint32), expected)
