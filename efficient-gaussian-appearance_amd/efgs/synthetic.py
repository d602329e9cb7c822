"""Seeded synthetic scenes for the benchmark configurations (numpy PCG64, fixed draw order).

c0_inputs gives the colour-only configuration c0. Rasterisation configurations (camera looking along +z from
(0, 0, -distance), horizontal field of view 60 degrees,
principal point at the image centre, near 0.2, far 1e4, black background):
  c1          100k Gaussians, means U[-2, 2]^3, 800 x 800, SH degree 3 (none / none / relu)
  c3          1M Gaussians, means U[-10, 10]^3, 1920 x 1080, neural (8 latents, SH degree 1 direction,
              2 x 64 ReLU, tanh residual, relu colour)
  c4_sv / c4_nasg / c4_nasgabor   c3 geometry with 8 sites / lobes
Per Gaussian, in draw order: means, log-scales N(-4.5, 0.5), quaternions normalize(N(0, 1)^4), opacity logits
N(0, 1), base colours N(0, 0.5), then the appearance parameters (SH rest N(0, 0.05); latents N(0, 0.1);
lobe models as documented in make_scene). The MLP is Xavier-uniform per layer (unpadded fan-in), rounded
to fp16 and packed in the tcnn flat layout with zero padding.
"""
from __future__ import annotations

import math

import numpy as np

CONFIGS = {
    'c1': dict(n=100_000, extent=2.0, distance=5.0, width=800, height=800, model='sh'),
    'c3': dict(n=1_000_000, extent=10.0, distance=22.0, width=1920, height=1080, model='neural'),
    'c4_sv': dict(n=1_000_000, extent=10.0, distance=22.0, width=1920, height=1080, model='sv'),
    'c4_nasg': dict(n=1_000_000, extent=10.0, distance=22.0, width=1920, height=1080, model='nasg'),
    'c4_nasgabor': dict(n=1_000_000, extent=10.0, distance=22.0, width=1920, height=1080, model='nasgabor'),
}

NEURAL_MLP = dict(n_feature_dims=8, n_frequencies=0, sh_degrees=(1,), n_neurons=64, n_hidden_layers=2, base_input=False)


def camera(width: int, height: int, distance: float, fov_deg: float = 60.0) -> dict:
    f = (width / 2.0) / math.tan(math.radians(fov_deg) / 2.0)
    w2c = np.eye(4, dtype=np.float32)
    w2c[2, 3] = distance
    return dict(w2c=w2c, position=np.array([0.0, 0.0, -distance], np.float32), width=width, height=height,
                focal_x=f, focal_y=f, center_x=width / 2.0, center_y=height / 2.0, near_plane=0.2, far_plane=1e4)


def mlp_layer_shapes(n_in: int, n_neurons: int, n_hidden_layers: int) -> list[tuple[int, int]]:
    n_in_pad = (n_in + 15) // 16 * 16
    return [(n_neurons, n_in_pad)] + [(n_neurons, n_neurons)] * (n_hidden_layers - 1) + [(16, n_neurons)]


def xavier_mlp(rng: np.random.Generator, n_in: int, n_neurons: int, n_hidden_layers: int, n_out: int = 3) -> np.ndarray:
    """Flat tcnn-layout parameters (fp16-representable fp32) with Xavier-uniform layers and zero padding."""
    parts = []
    layer_in = n_in
    shapes = mlp_layer_shapes(n_in, n_neurons, n_hidden_layers)
    for i, (rows, cols) in enumerate(shapes):
        fan_out = n_out if i == len(shapes) - 1 else rows
        limit = math.sqrt(6.0 / (layer_in + fan_out))
        w = np.zeros((rows, cols), np.float32)
        w[:fan_out, :layer_in] = rng.uniform(-limit, limit, size=(fan_out, layer_in)).astype(np.float32)
        parts.append(w.reshape(-1))
        layer_in = n_neurons
    return np.concatenate(parts).astype(np.float16).astype(np.float32)


def make_scene(config: str, n: int | None = None, seed: int = 0, width: int | None = None, height: int | None = None) -> dict:
    cfg = dict(CONFIGS[config])
    if n is not None:
        cfg['n'] = n
    if width is not None:
        cfg['width'] = width
    if height is not None:
        cfg['height'] = height
    rng = np.random.default_rng(seed)
    N, e = cfg['n'], cfg['extent']
    means = rng.uniform(-e, e, size=(N, 3)).astype(np.float32)
    scales = rng.normal(-4.5, 0.5, size=(N, 3)).astype(np.float32)
    q = rng.normal(0.0, 1.0, size=(N, 4)).astype(np.float32)
    rotations = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)
    opacities = rng.normal(0.0, 1.0, size=(N, 1)).astype(np.float32)
    base = rng.normal(0.0, 0.5, size=(N, 3)).astype(np.float32)
    model = cfg['model']
    out = dict(means=means, scales=scales, rotations=rotations, opacities=opacities, base_colors=base, mlp_weights=None,
               camera=camera(cfg['width'], cfg['height'], cfg['distance']), model=model)
    if model == 'sh':
        out['residual_params'] = rng.normal(0.0, 0.05, size=(N, 15, 3)).astype(np.float32)
        out['appearance'] = dict(model='sh', max_degree=3, base_act='none', res_act='none', color_act='relu', direction_gradient=True)
    elif model == 'neural':
        mlp = NEURAL_MLP
        out['residual_params'] = rng.normal(0.0, 0.1, size=(N, mlp['n_feature_dims'])).astype(np.float32)
        n_in = mlp['n_feature_dims'] + sum(2 * d + 1 for d in mlp['sh_degrees'])
        out['mlp_weights'] = xavier_mlp(rng, n_in, mlp['n_neurons'], mlp['n_hidden_layers'])
        out['appearance'] = dict(model='neural', max_degree=len([d for d in mlp['sh_degrees'] if d > 0]), base_act='none',
                                 res_act='tanh', color_act='relu', direction_gradient=True, mlp=dict(mlp))
    elif model == 'sv':
        sites = rng.normal(0.0, 1.0, size=(N, 8, 3)).astype(np.float32)
        sites /= np.linalg.norm(sites, axis=-1, keepdims=True)
        tau = rng.normal(1.0, 0.5, size=(N, 8, 1)).astype(np.float32)
        col = rng.normal(0.0, 0.1, size=(N, 8, 3)).astype(np.float32)
        out['residual_params'] = np.concatenate([sites, tau, col], axis=-1).astype(np.float32)
        out['appearance'] = dict(model='sv', max_degree=8, base_act='none', res_act='none', color_act='relu', direction_gradient=True)
    elif model in ('nasg', 'nasgabor'):
        frame = rng.normal(0.0, 1.0, size=(N, 8, 3)).astype(np.float32)
        shape = rng.normal(1.0, 0.5, size=(N, 8, 2)).astype(np.float32)
        extra = [rng.normal(0.0, 1.0, size=(N, 8, 1)).astype(np.float32)] if model == 'nasgabor' else []
        amp = rng.normal(0.0, 0.1, size=(N, 8, 3)).astype(np.float32)
        out['residual_params'] = np.concatenate([frame, shape] + extra + [amp], axis=-1).astype(np.float32)
        out['appearance'] = dict(model=model, max_degree=8, base_act='none', res_act='tanh', color_act='relu', direction_gradient=True)
    else:
        raise ValueError(model)
    return out


def c0_inputs(n: int = 10_000, seed: int = 0) -> dict:
    """Configuration c0 (the unfused appearance on the host): a camera at the origin looking along +z, means
    U[-2, 2]^3 + (0, 0, 5), base colours (the SH DC term) N(0, 0.5) (n, 3), SH rest bands N(0, 0.05) (n, 15, 3);
    draw order as listed. Colour = sigmoid(4 (base + residual(dir))), base and residual activations none."""
    rng = np.random.default_rng(seed)
    means = (rng.uniform(-2.0, 2.0, (n, 3)) + np.array([0.0, 0.0, 5.0])).astype(np.float32)
    base = rng.normal(0.0, 0.5, (n, 3)).astype(np.float32)
    rest = rng.normal(0.0, 0.05, (n, 15, 3)).astype(np.float32)
    return dict(means=means, base_colors=base, residual_params=rest, cam_position=np.zeros(3, np.float32),
                appearance=dict(model='sh', max_degree=3, base_act='none', res_act='none', color_act='sigmoid'))


def target_image(width: int, height: int, seed: int = 1) -> np.ndarray:
    return np.random.default_rng(seed).uniform(0.0, 1.0, size=(3, height, width)).astype(np.float32)


# ---- .ngsplat export models ----

NGSPLAT_NEURAL_CASES = {
    # encoded 16 = 8 features x (sin, cos); degrees 0..3: 48 inputs; 16 neurons -> baked (the viewer's default model)
    'baked': dict(n_features=8, n_frequencies=1, sh_degrees=[0, 1, 2, 3], n_neurons=16, n_hidden_layers=2, base_input=False),
    # 32 neurons exceed the baked cache -> stored features + full layer 0 (16 + 1 + 15 = 32 inputs)
    'full': dict(n_features=8, n_frequencies=1, sh_degrees=[0, 1, 2, 3], n_neurons=32, n_hidden_layers=2, base_input=False),
    # raw base colours appended to 5 features, identity encoding, no constant input, input padded 20 -> 32
    'base_input': dict(n_features=5, n_frequencies=0, sh_degrees=[1, 2], n_neurons=16, n_hidden_layers=3, base_input=True),
}
NGSPLAT_OTHER_CASES = {'sh3': ('sh', (15, 3)), 'sh1': ('sh', (3, 3)), 'sv7': ('sv', (7, 7)), 'nasg1': ('nasg', (1, 8)), 'nasg5': ('nasg', (5, 8)),
               'nasgabor2': ('nasgabor', (2, 9))}


def mlp_flat(rng, n_in, n_neurons, n_hidden_layers, scale=0.4):
    """Random fp16 residual-MLP parameters in the flat layout (layer-0 input padded to a multiple of 16)."""
    n_in_pad = -(-n_in // 16) * 16
    size = n_in_pad * n_neurons + (n_hidden_layers - 1) * n_neurons * n_neurons + 16 * n_neurons
    return rng.normal(0.0, scale, size).astype(np.float16)


def ngsplat_model(name: str, n: int = 3000, seed: int = 0, residual_act: str = 'tanh', color_act: str = 'relu', base_act: str = 'none'):
    """A random model (raw parameters as numpy arrays) and its .ngsplat export plan for one of the named
    configurations of NGSPLAT_NEURAL_CASES / NGSPLAT_OTHER_CASES; about 12% of the splats fall below the opacity
    threshold."""
    from . import ngsplat as NG
    rng = np.random.default_rng(seed)
    m = dict(means=rng.normal(0.0, 3.0, (n, 3)).astype(np.float32), raw_scales=rng.normal(-4.0, 1.5, (n, 3)).astype(np.float32),
             raw_rotations=rng.normal(size=(n, 4)).astype(np.float32), raw_opacities=rng.normal(-2.0, 3.0, (n, 1)).astype(np.float32),
             base_colors=rng.normal(0.0, 0.4, (n, 3)).astype(np.float32))
    cfg = dict(base_activation=base_act, residual_activation=residual_act, color_activation=color_act)
    mlp = None
    if name in NGSPLAT_NEURAL_CASES:
        c = NGSPLAT_NEURAL_CASES[name]
        cfg.update(appearance_type='neural', n_frequencies=c['n_frequencies'], sh_degrees=c['sh_degrees'], n_neurons=c['n_neurons'],
                   n_hidden_layers=c['n_hidden_layers'], base_input=c['base_input'])
        m['residual_params'] = rng.normal(0.0, 0.5, (n, c['n_features'])).astype(np.float32)
        enc = (c['n_features'] + (3 if c['base_input'] else 0)) * (2 * c['n_frequencies'] if c['n_frequencies'] else 1)
        n_in = enc + sum(2 * d + 1 for d in c['sh_degrees'])
        mlp = mlp_flat(rng, n_in, c['n_neurons'], c['n_hidden_layers'])
    else:
        model, shape = NGSPLAT_OTHER_CASES[name]
        cfg['appearance_type'] = model
        m['residual_params'] = rng.normal(0.0, 0.6, (n,) + shape).astype(np.float32)
    plan = NG.plan_export(cfg, m['residual_params'].shape, mlp)
    return m, plan, mlp
