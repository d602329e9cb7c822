"""PLY export of a Gaussian model in the layout 3DGS viewers read, as the reference's model writes it
(Model.as_ply_dict, reference Model.py:503-531; appearance columns Appearance/Base.py:230-236 and
Appearance/SH.py:59-70): one `vertex` element of float32 properties

    x y z | appearance columns | opacity | scale_0 scale_1 scale_2 | rot_0 rot_1 rot_2 rot_3

with the raw (pre-activation) opacity and log-scales and the normalised quaternion (w, x, y, z). The appearance
columns are the standard SH layout f_dc_0..2 = base / SH_C0, f_rest_i = the residual coefficients
channel-major (all red bands, then green, then blue) for an SH model with identity base and residual
activations and the relu colour activation; every other configuration stores only the base colour baked to
degree-0 SH, f_dc = (colour_activation(base_activation(base)) - 0.5) / SH_C0 (viewers reconstruct the diffuse
colour as 0.5 + SH_C0 f_dc), without the view-dependent residual.

File format: `ply` / `format binary_little_endian 1.0` / `element vertex N` / one `property float <name>` line
per column / `end_header`, then N rows of little-endian float32.
"""
from __future__ import annotations

import numpy as np

SH_C0 = 0.28209479177387814


def _base_activation(x: np.ndarray, act: str) -> np.ndarray:
    if act == 'none':
        return x
    if act == 'exp':
        return np.exp(3.0 * x)
    raise ValueError(f'unsupported base activation: {act}')


def _color_activation(x: np.ndarray, act: str) -> np.ndarray:
    """The rasterizer's colour activations (the shifted forms: relu(x + 0.5), softplus_10(x + 0.5), ...)."""
    x = x.astype(np.float64)
    if act == 'none':
        return x + 0.5
    if act == 'relu':
        return np.maximum(x + 0.5, 0.0)
    if act == 'softplus':
        y = 10.0 * (x + 0.5)
        return (np.maximum(y, 0.0) + np.log1p(np.exp(-np.abs(y)))) / 10.0
    if act == 'sigmoid':
        return 1.0 / (1.0 + np.exp(-4.0 * x))
    if act == 'hardsigmoid':
        return np.clip(x + 0.5, 0.0, 1.0)
    if act == 'satexp':
        return -np.expm1(-x)
    raise ValueError(f'unsupported colour activation: {act}')


def ply_attributes(base_colors: np.ndarray, residual_params: np.ndarray | None, model: str, base_act: str, residual_act: str,
                   color_act: str) -> tuple[np.ndarray, list[str]]:
    """Appearance columns (N, C) and their names."""
    base = np.asarray(base_colors, np.float32).reshape(-1, 3)
    if model == 'sh' and base_act == 'none' and residual_act == 'none' and color_act == 'relu':
        rest = np.asarray(residual_params, np.float32)
        n_rest = rest.size // (3 * base.shape[0]) if base.shape[0] else (rest.shape[1] if rest.ndim == 3 else 0)
        rest = rest.reshape(base.shape[0], n_rest, 3).transpose(0, 2, 1).reshape(base.shape[0], 3 * n_rest)
        names = ['f_dc_0', 'f_dc_1', 'f_dc_2'] + [f'f_rest_{i}' for i in range(rest.shape[1])]
        return np.concatenate([(base / np.float32(SH_C0)).astype(np.float32), rest], axis=1), names
    baked = (_color_activation(_base_activation(base.astype(np.float64), base_act), color_act) - 0.5) / SH_C0
    return baked.astype(np.float32), ['f_dc_0', 'f_dc_1', 'f_dc_2']


def ply_vertices(means: np.ndarray, raw_scales: np.ndarray, raw_rotations: np.ndarray, raw_opacities: np.ndarray, base_colors: np.ndarray,
                 residual_params: np.ndarray | None = None, model: str = 'sh', base_act: str = 'none', residual_act: str = 'none',
                 color_act: str = 'relu') -> np.ndarray:
    """The structured `vertex` array (one float32 field per property, in file order)."""
    means = np.asarray(means, np.float32).reshape(-1, 3)
    n = means.shape[0]
    q = np.asarray(raw_rotations, np.float64).reshape(n, 4)
    q = (q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-12)).astype(np.float32)  # torch normalize (eps 1e-12)
    app, app_names = ply_attributes(base_colors, residual_params, model, base_act, residual_act, color_act)
    cols = np.concatenate([means, app, np.asarray(raw_opacities, np.float32).reshape(n, 1), np.asarray(raw_scales, np.float32).reshape(n, 3), q],
                          axis=1)
    names = ['x', 'y', 'z'] + app_names + ['opacity', 'scale_0', 'scale_1', 'scale_2', 'rot_0', 'rot_1', 'rot_2', 'rot_3']
    vertices = np.empty(n, dtype=[(name, '<f4') for name in names])
    for i, name in enumerate(names):
        vertices[name] = cols[:, i]
    return vertices


def write_ply(path: str, vertices: np.ndarray) -> None:
    """Binary little-endian PLY with one `vertex` element of float32 properties."""
    names = vertices.dtype.names
    if any(vertices.dtype[name] != np.dtype('<f4') for name in names):
        raise ValueError('write_ply stores float32 properties only')
    header = 'ply\nformat binary_little_endian 1.0\n' + f'element vertex {vertices.shape[0]}\n'
    header += ''.join(f'property float {name}\n' for name in names) + 'end_header\n'
    with open(path, 'wb') as f:
        f.write(header.encode('ascii'))
        f.write(np.ascontiguousarray(vertices).tobytes())


def read_ply(path: str) -> np.ndarray:
    """Reads a file written by write_ply (binary little-endian, one float32 `vertex` element)."""
    with open(path, 'rb') as f:
        data = f.read()
    end = data.index(b'end_header\n') + len(b'end_header\n')
    lines = data[:end].decode('ascii').splitlines()
    if lines[0] != 'ply' or lines[1] != 'format binary_little_endian 1.0':
        raise ValueError('not a binary little-endian PLY file')
    n = None
    names = []
    for line in lines[2:]:
        parts = line.split()
        if parts[0] == 'element':
            if parts[1] != 'vertex' or n is not None:
                raise ValueError('expected a single vertex element')
            n = int(parts[2])
        elif parts[0] == 'property':
            if parts[1] != 'float':
                raise ValueError(f'unsupported property type {parts[1]}')
            names.append(parts[2])
    dtype = np.dtype([(name, '<f4') for name in names])
    return np.frombuffer(data, dtype=dtype, count=n, offset=end).copy()


def export_ply(path: str, means, raw_scales, raw_rotations, raw_opacities, base_colors, residual_params=None, model: str = 'sh',
               base_act: str = 'none', residual_act: str = 'none', color_act: str = 'relu') -> int:
    """Writes the model (torch tensors or arrays) to `path`; returns the number of Gaussians written."""
    def host(t):
        if t is None:
            return None
        return t.detach().cpu().numpy() if hasattr(t, 'detach') else np.asarray(t)
    vertices = ply_vertices(host(means), host(raw_scales), host(raw_rotations), host(raw_opacities), host(base_colors), host(residual_params),
                            model, base_act, residual_act, color_act)
    write_ply(path, vertices)
    return int(vertices.shape[0])
