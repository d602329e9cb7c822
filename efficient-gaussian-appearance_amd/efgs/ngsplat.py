"""Export of a Gaussian model to the WebGL viewer's `.ngsplat` file, as the reference's numpy script
viewer/export_ngsplat.py writes it (main :1309-1644), with the per-splat work on the GPU: culling
(sigmoid(opacity) < 1/255), the rgb8 base / a8 opacity / fp16 position / 24-bit rotation / 8-bit log-scale splat
words and the appearance payload textures are computed by libefgs_hip.so (efgs_ngsplat_pack) from the model's
tensors where they already live. This module plans the layout from the appearance configuration, slices and
orders the residual MLP weights, and writes the header and the textures.

File (little-endian): b'NGSPLAT\\n'; 11 u32 (numSplats, texWidth 2048, texHeight, featureDim, nFrequencies,
shBandMask, colorActivation, residualActivation, nNeurons, nHiddenLayers, flags); f32 baseScale, baseOffset;
SH files only 3 f32 level scales; f32x3 camCenter, f32x3 camUp, f32 camDistance; u32 nTestCameras and
18 f32 per camera; u32 nWeightTexels and 4 fp16 per texel; the splat texture (4 u32 per row) and the payload
textures, each texWidth x texHeight rows (viewer/export_ngsplat.py:88-170, parsed by viewer/utils.js:230-330).

Differences from the script: a model is passed as tensors (the checkpoint loading, dataset-based test cameras
and PPISP baking of the script stay with the caller: test cameras may be passed in, PPISP is not written); an
MLP whose input width is not a multiple of 16 is accepted (the flat parameters pad layer 0's input to a
multiple of 16 and the rasterizer feeds zeros there, so the padded columns are dropped); a model without a
splat above the opacity threshold gives a file without splats rather than an error.
"""
from __future__ import annotations

import ctypes
import math
import struct
from typing import Any

import numpy as np
import torch

from ._lib import NgsplatInput, NgsplatOutput, WorkspaceAllocator, check, lib

SH_C0 = 0.28209479177387814
TEX_WIDTH = 2048
MAGIC = b'NGSPLAT\n'
COLOR_ACTIVATION_CODES = {'relu': 0, 'softplus': 1, 'sigmoid': 2, 'satexp': 3, 'hardsigmoid': 4, 'none': 5}
SHIFTED_COLOR_ACTIVATIONS = {'none', 'relu', 'softplus', 'hardsigmoid'}
RESIDUAL_CODES = {'none': 0, 'tanh': 1, 'softplus': 2}
FILE_MODEL_IDS = {'sh': 1, 'sv': 2, 'nasg': 3, 'nasgabor': 4, 'neural': 0}
PARAM_VALUE_CAP = 64
# payload kinds of efgs_ngsplat_pack (include/efgs.h)
NEURAL_FEATURES, NEURAL_BAKED, SH, SV, NASG, NASGABOR = range(6)
# defaults of the appearance configuration (the tracked configs' values, viewer/export_ngsplat.py:281-296)
CONFIG_DEFAULTS = {
    'appearance_type': 'neural', 'base_activation': 'none', 'residual_activation': 'tanh', 'color_activation': 'relu',
    'base_input': False, 'n_frequencies': 1, 'sh_degrees': [0, 1, 2, 3], 'n_neurons': 16, 'n_hidden_layers': 2,
    'hidden_activation': 'relu',
}


def slice_mlp_params(params: np.ndarray, n_in: int, n_neurons: int, n_hidden_layers: int, n_out: int = 3,
                     out_padded: int = 16) -> list[np.ndarray]:
    """Flat tcnn-layout parameters -> row-major [out x in] float32 matrices, output layer trimmed to n_out rows
    (viewer/export_ngsplat.py:1013-1029). Layer 0 may be stored with its input padded to a multiple of 16."""
    params = np.asarray(params).astype(np.float32).reshape(-1)
    hidden = (n_hidden_layers - 1) * n_neurons * n_neurons + out_padded * n_neurons
    for n_in_stored in (n_in, -(-n_in // 16) * 16):
        if params.size == n_in_stored * n_neurons + hidden:
            break
    else:
        raise ValueError(f'mlp params length {params.size} does not match a {n_in}-wide input (padded to 16 or not), '
                         f'{n_neurons} neurons and {n_hidden_layers} hidden layers')
    dims = [(n_neurons, n_in_stored)] + [(n_neurons, n_neurons)] * (n_hidden_layers - 1) + [(out_padded, n_neurons)]
    matrices, offset = [], 0
    for rows, cols in dims:
        matrices.append(params[offset:offset + rows * cols].reshape(rows, cols).copy())
        offset += rows * cols
    matrices[0] = np.ascontiguousarray(matrices[0][:, :n_in])
    matrices[-1] = matrices[-1][:n_out]
    return matrices


def pack_weight_texels(matrices: list[np.ndarray]) -> np.ndarray:
    """fp16 weight stream [T, 4] (uint16 bits): per layer, texel j * out + o = W[o, 4j:4j+4]
    (viewer/export_ngsplat.py:388-400; read by viewer/shaders/eval_neural.glsl)."""
    blocks = []
    for w in matrices:
        out_dim, in_dim = w.shape
        if in_dim % 4:
            raise ValueError(f'layer input dim must be a multiple of 4, got {w.shape}')
        blocks.append(np.asarray(w, np.float32).reshape(out_dim, in_dim // 4, 4).transpose(1, 0, 2).reshape(-1, 4))
    if not blocks:
        return np.zeros((0, 4), np.uint16)
    return np.concatenate(blocks).astype(np.float16).view(np.uint16)


def gate_inactive_degrees(matrices: list[np.ndarray], encoded_dim: int, sh_degrees: list[int], active_degree: int) -> list[int]:
    """Zeroes the layer-0 columns of the view-direction degrees the appearance schedule has not enabled yet
    (viewer/export_ngsplat.py:1254-1268); returns the gated degrees."""
    gated, offset, rank = [], encoded_dim, 0
    for degree in sh_degrees:
        width = 2 * degree + 1
        if degree > 0:
            if rank >= active_degree:
                matrices[0][:, offset:offset + width] = 0.0
                gated.append(degree)
            rank += 1
        offset += width
    return gated


def plan_export(config: dict[str, Any], residual_shape: tuple[int, ...], mlp_params: np.ndarray | None = None,
                active_degree: int | None = None) -> dict[str, Any]:
    """The payload kind, its parameters, the header fields and the weight stream for a model's appearance
    configuration (the validation and planning of viewer/export_ngsplat.py:1337-1530)."""
    cfg = dict(CONFIG_DEFAULTS)
    cfg.update(config)
    model = str(cfg['appearance_type']).lower()
    if model not in FILE_MODEL_IDS:
        raise ValueError(f'unknown appearance type {model!r} (supported: {", ".join(FILE_MODEL_IDS)})')
    if cfg['color_activation'] not in COLOR_ACTIVATION_CODES:
        raise ValueError(f'unknown color activation {cfg["color_activation"]!r}')
    if cfg['base_activation'] not in ('none', 'exp'):
        raise ValueError(f'unknown base activation {cfg["base_activation"]!r} (supported: none, exp)')
    if cfg['residual_activation'] not in RESIDUAL_CODES:
        raise ValueError(f'unknown residual activation {cfg["residual_activation"]!r}')
    residual_code = RESIDUAL_CODES[cfg['residual_activation']]
    p: dict[str, Any] = dict(model=model, config=cfg, n_items=0, base_input=0, n_frequencies=0, n_neurons=0, residual_act=0,
                             bake_matrix=None, bake_bias=None, weight_texels=np.zeros((0, 4), np.uint16), degree_mask=0,
                             model_dims=0, header_frequencies=0, header_neurons=0, header_hidden=0, flags=0)
    p['color_shift'] = 0.5 if cfg['color_activation'] in SHIFTED_COLOR_ACTIVATIONS and cfg['base_activation'] == 'none' else 0.0
    n_cols = residual_shape[1] if len(residual_shape) > 1 else 0
    if model == 'neural':
        if cfg['n_hidden_layers'] < 1:
            raise ValueError(f'N_HIDDEN_LAYERS must be >= 1, got {cfg["n_hidden_layers"]}')
        if str(cfg['hidden_activation']).lower() != 'relu':
            raise ValueError(f'unsupported hidden activation {cfg["hidden_activation"]!r} (the viewer implements relu)')
        n_neurons = int(cfg['n_neurons'])
        if n_neurons % 4 or n_neurons < 4:
            raise ValueError(f'N_NEURONS must be a multiple of 4 >= 4, got {n_neurons}')
        degrees = [int(d) for d in cfg['sh_degrees']]
        if degrees != sorted(set(degrees)) or any(d < 0 or d > 6 for d in degrees):
            raise ValueError(f'SH_DEGREES must be strictly ascending in [0, 6], got {degrees}')
        direction_degrees = [d for d in degrees if d > 0]
        if not direction_degrees:
            raise ValueError(f'SH_DEGREES must contain at least one view-direction degree (>= 1), got {degrees}')
        if mlp_params is None:
            raise ValueError('the neural appearance model needs the residual mlp parameters')
        k = int(cfg['n_frequencies'])
        base_input = bool(cfg['base_input'])
        encoded_dim = (n_cols + (3 if base_input else 0)) * (2 * k if k else 1)
        sh0 = 0 in degrees
        n_direction_values = sum(2 * d + 1 for d in direction_degrees)
        n_in = encoded_dim + sum(2 * d + 1 for d in degrees)
        # the fused kernels evaluate the mlp with fp16 weights, so the export rounds the same way
        matrices = slice_mlp_params(np.asarray(mlp_params).astype(np.float16), n_in, n_neurons, int(cfg['n_hidden_layers']))
        if active_degree is None:
            active_degree = len(direction_degrees)
        if active_degree == 0:
            if cfg['residual_activation'] == 'softplus':
                raise ValueError('no active view-direction degree and RESIDUAL_ACTIVATION softplus: the rasterizer skips the mlp, '
                                 'which zeroed weights cannot reproduce (softplus(0) != 0)')
            matrices[-1][:] = 0.0
        elif active_degree < len(direction_degrees):
            gate_inactive_degrees(matrices, encoded_dim, degrees, active_degree)
        use_baked = n_neurons <= 16 and -(-n_neurons // 8) <= -(-encoded_dim // 8)
        p.update(n_items=n_cols, base_input=int(base_input), n_frequencies=k, matrices=matrices, use_baked=use_baked, sh0=sh0,
                 encoded_dim=encoded_dim, direction_degrees=direction_degrees)
        if use_baked:
            w0 = matrices[0]
            p['payload'] = NEURAL_BAKED
            p['n_neurons'] = n_neurons
            p['bake_matrix'] = np.ascontiguousarray(w0[:, :encoded_dim], np.float32)
            p['bake_bias'] = (np.float32(SH_C0) * w0[:, encoded_dim]).astype(np.float32) if sh0 else None
            n_static = encoded_dim + (1 if sh0 else 0)
            w0_dyn = np.zeros((n_neurons, (n_direction_values + 3) // 4 * 4), np.float32)
            w0_dyn[:, :n_direction_values] = w0[:, n_static:]
            p['weight_texels'] = pack_weight_texels([w0_dyn] + matrices[1:])
            p['n_values'] = n_neurons
        else:
            if encoded_dim > 16:
                raise ValueError(f'{encoded_dim} encoded feature dims exceed the viewer\'s cap of 16 and {n_neurons} neurons exceed '
                                 f'the baked h0_static cache: this configuration is unrepresentable')
            p['payload'] = NEURAL_FEATURES
            p['weight_texels'] = pack_weight_texels(matrices)
            p['n_values'] = encoded_dim
        p['degree_mask'] = sum(1 << d for d in direction_degrees)
        p.update(model_dims=encoded_dim, header_frequencies=k, header_neurons=n_neurons, header_hidden=int(cfg['n_hidden_layers']))
        p['flags'] |= (0 if sh0 else 2) | (4 if use_baked else 0)
    elif model == 'sh':
        max_degree = int(round(math.sqrt(n_cols + 1))) - 1
        if (max_degree + 1) ** 2 - 1 != n_cols:
            raise ValueError(f'{n_cols} sh coefficients do not form complete degrees 1..D')
        if max_degree > 3:
            raise ValueError(f'the viewer\'s quantized sh layout covers degrees 1-3, got degree {max_degree}')
        export_degree = max_degree if active_degree is None else min(active_degree, max_degree)
        p.update(payload=SH, n_items=(export_degree + 1) ** 2 - 1, n_values=0,
                 degree_mask=sum(1 << d for d in range(1, export_degree + 1)))
    else:
        payload, per_item = {'sv': (SV, 7), 'nasg': (NASG, 12), 'nasgabor': (NASGABOR, 13)}[model]
        n_items = n_cols if model == 'sv' or active_degree is None else min(active_degree, n_cols)
        if per_item * n_items > PARAM_VALUE_CAP:
            raise ValueError(f'{per_item * n_items} residual values per splat exceed the viewer\'s cap of {PARAM_VALUE_CAP}')
        p.update(payload=payload, n_items=n_items, n_values=per_item * n_items, residual_act=residual_code, model_dims=n_items)
    model_id = FILE_MODEL_IDS[model]
    p['flags'] |= ((model_id & 3) << 3) | ((model_id >> 2) << 6) | (32 if cfg['base_activation'] == 'exp' else 0)
    p['color_code'] = COLOR_ACTIVATION_CODES[cfg['color_activation']]
    p['residual_code'] = residual_code
    return p


def _device_f32(name: str, t, device: torch.device, shape_tail: tuple[int, ...] | None = None) -> torch.Tensor:
    t = torch.as_tensor(t)
    if t.dtype != torch.float32:
        raise ValueError(f'efgs: {name} must be float32, got {t.dtype}')
    if t.device.type != 'cuda':
        raise ValueError(f'efgs: {name} must be on a GPU device, got {t.device}')
    if t.device != device:
        raise ValueError(f'efgs: {name} is on {t.device}, expected {device}')
    if shape_tail is not None and tuple(t.shape[1:]) != shape_tail:
        raise ValueError(f'efgs: {name} must have shape (N, {", ".join(map(str, shape_tail))}), got {tuple(t.shape)}')
    return t.contiguous()


def pack_textures(means: torch.Tensor, raw_scales: torch.Tensor, raw_rotations: torch.Tensor, raw_opacities: torch.Tensor,
                  base_colors: torch.Tensor, residual_params: torch.Tensor, plan: dict[str, Any], timing: bool = False) -> dict[str, Any]:
    """Culls, quantises and packs the splat and payload textures on the device (efgs_ngsplat_pack). Returns the
    kept count, the statistics and device tensors: splat_words (P, 4) and the payload textures (P, words) as
    uint32 bit patterns in int32 tensors, source_index (P,), with P = 2048 * ceil(kept / 2048); with `timing`, the
    milliseconds of the statistics + combine kernels and of the pack kernel (HIP events) as kernel_ms."""
    device = means.device
    n = means.shape[0]
    means = _device_f32('means', means, device, (3,))
    raw_scales = _device_f32('scales', raw_scales, device, (3,))
    raw_rotations = _device_f32('rotations', raw_rotations, device, (4,))
    raw_opacities = _device_f32('opacities', raw_opacities, device).reshape(-1)
    base_colors = _device_f32('base_colors', base_colors, device).reshape(n, 3) if base_colors.numel() == 3 * n else None
    residual = _device_f32('residual_params', residual_params, device)
    residual = residual.reshape(n, int(np.prod(residual.shape[1:])))
    if raw_scales.shape[0] != n or raw_rotations.shape[0] != n or raw_opacities.numel() != n or base_colors is None:
        raise ValueError('efgs: inconsistent splat counts or base colours not (N, 3)')
    inp = NgsplatInput()
    inp.n = n
    inp.means, inp.raw_scales, inp.raw_rotations = means.data_ptr(), raw_scales.data_ptr(), raw_rotations.data_ptr()
    inp.raw_opacities, inp.base_colors = raw_opacities.data_ptr(), base_colors.data_ptr()
    inp.residual_params = residual.data_ptr() if residual.numel() else None
    inp.residual_row_stride = residual.shape[1]
    inp.payload = plan['payload']
    inp.n_items = plan['n_items']
    inp.base_input = plan['base_input']
    inp.n_frequencies = plan['n_frequencies']
    inp.n_neurons = plan['n_neurons']
    inp.residual_act = plan['residual_act']
    inp.color_shift = plan['color_shift']
    if plan['bake_matrix'] is not None:
        # the layer-0 bake on the device, uploaded once per plan and device
        cache = plan.setdefault('_device_bake', {})
        if device not in cache:
            cache[device] = (torch.from_numpy(plan['bake_matrix']).to(device),
                             torch.from_numpy(plan['bake_bias']).to(device) if plan['bake_bias'] is not None else None)
        m, b = cache[device]
        inp.bake_matrix = m.data_ptr()
        inp.bake_bias = b.data_ptr() if b is not None else None
    n_textures = ctypes.c_int()
    texel_words = (ctypes.c_int * 8)()
    check(lib.efgs_ngsplat_layout(ctypes.byref(inp), ctypes.byref(n_textures), texel_words))
    words = [texel_words[k] for k in range(n_textures.value)]
    capacity = max(1, -(-n // TEX_WIDTH)) * TEX_WIDTH
    splat_words = torch.empty((capacity, 4), dtype=torch.int32, device=device)
    params = torch.empty(capacity * sum(words), dtype=torch.int32, device=device) if words else None
    source_index = torch.empty(capacity, dtype=torch.int32, device=device)
    out = NgsplatOutput()
    out.capacity = capacity
    out.splat_words = splat_words.data_ptr()
    out.params = params.data_ptr() if params is not None else None
    out.source_index = source_index.data_ptr()
    kernel_ms = (ctypes.c_float * 2)()
    out.kernel_ms = kernel_ms if timing else None
    with torch.cuda.device(device):
        alloc = WorkspaceAllocator(device, 'ngsplat')
        check(lib.efgs_ngsplat_pack(ctypes.byref(inp), ctypes.byref(out), alloc.fn, alloc.ctx, torch.cuda.current_stream(device).cuda_stream))
        alloc.done()
    n_kept = int(out.n_kept)
    rows = -(-n_kept // TEX_WIDTH) * TEX_WIDTH
    textures, offset = [], 0
    for w in words:
        textures.append(params[offset:offset + capacity * w].view(capacity, w)[:rows])
        offset += capacity * w
    return dict(n_kept=n_kept, base_offset=float(out.base_offset), base_scale=float(out.base_scale),
                sh_level_scales=[float(out.sh_level_scale[i]) for i in range(3)] if plan['payload'] == SH else None,
                splat_words=splat_words[:rows], textures=textures, source_index=source_index[:rows],
                kernel_ms=(float(kernel_ms[0]), float(kernel_ms[1])) if timing else None)


def camera_hint(kept_means: np.ndarray, test_cameras: np.ndarray | None = None, center=None, up=None, distance=None):
    """Orbit target, up vector and distance (viewer/export_ngsplat.py:1190-1212, :1533-1553): the per-axis median
    of the kept means, the mean camera up (else -y) and the median camera distance (else 1.5 x the median radius)."""
    kept_means = np.asarray(kept_means, np.float32)
    n = kept_means.shape[0]
    c = np.array(center, np.float32) if center is not None else (np.median(kept_means, axis=0).astype(np.float32) if n
                                                                    else np.zeros(3, np.float32))
    median_radius = float(np.median(np.linalg.norm(kept_means - c, axis=1))) if n else 1.0
    hint_up, hint_distance = None, None
    if test_cameras is not None and len(test_cameras):
        cams = np.asarray(test_cameras, np.float32)
        ups = -cams[:, [1, 5, 9]].astype(np.float64)
        ups /= np.maximum(np.linalg.norm(ups, axis=1, keepdims=True), 1e-12)
        mean_up = ups.sum(axis=0)
        norm = float(np.linalg.norm(mean_up))
        hint_distance = float(np.median(np.linalg.norm(cams[:, [3, 7, 11]].astype(np.float64) - c, axis=1)))
        if norm >= 1e-6:
            hint_up = (mean_up / norm).astype(np.float32)
    if up is not None:
        hint_up = np.array(up, np.float32)
    elif hint_up is None:
        hint_up = np.array([0.0, -1.0, 0.0], np.float32)
    hint_up = hint_up / np.linalg.norm(hint_up)
    if distance is not None:
        hint_distance = float(distance)
    elif hint_distance is None:
        hint_distance = 1.5 * median_radius
    return c, hint_up.astype(np.float32), hint_distance


def write_ngsplat(path: str, plan: dict[str, Any], packed: dict[str, Any], center: np.ndarray, up: np.ndarray, distance: float,
                  test_cameras: np.ndarray | None = None, proper_antialiasing: bool = False) -> int:
    """Writes the header, the weight stream and the textures (viewer/export_ngsplat.py:1581-1623); returns the
    file size in bytes."""
    n_kept = packed['n_kept']
    tex_height = -(-n_kept // TEX_WIDTH)
    flags = plan['flags'] | (1 if proper_antialiasing else 0)
    cams = np.zeros((0, 18), np.float32) if test_cameras is None else np.asarray(test_cameras, '<f4').reshape(-1, 18)
    texels = np.ascontiguousarray(plan['weight_texels'], '<u2')
    parts = [MAGIC, struct.pack('<11I', n_kept, TEX_WIDTH, tex_height, plan['model_dims'], plan['header_frequencies'], plan['degree_mask'],
                                plan['color_code'], plan['residual_code'], plan['header_neurons'], plan['header_hidden'], flags),
             struct.pack('<2f', packed['base_scale'], packed['base_offset'])]
    if plan['payload'] == SH:
        parts.append(struct.pack('<3f', *packed['sh_level_scales']))
    parts += [struct.pack('<3f', *[float(v) for v in center]), struct.pack('<3f', *[float(v) for v in up]), struct.pack('<f', float(distance)),
              struct.pack('<I', cams.shape[0]), cams.astype('<f4').tobytes(), struct.pack('<I', texels.shape[0]), texels.tobytes()]
    host = [packed['splat_words'].cpu().numpy()] + [t.cpu().numpy() for t in packed['textures']]
    size = sum(len(p) for p in parts) + sum(h.nbytes for h in host)
    with open(path, 'wb') as f:
        for p in parts:
            f.write(p)
        for h in host:
            f.write(np.ascontiguousarray(h).astype('<i4', copy=False).tobytes())
    return size


def export_ngsplat(path: str, means: torch.Tensor, scales: torch.Tensor, rotations: torch.Tensor, opacities: torch.Tensor,
                   base_colors: torch.Tensor, residual_params: torch.Tensor, config: dict[str, Any], mlp_params=None,
                   active_degree: int | None = None, proper_antialiasing: bool = False, center=None, up=None, distance=None,
                   test_cameras=None) -> dict[str, Any]:
    """Writes a model to `path` in the .ngsplat format. The tensors are the model's raw parameters on one GPU
    (the checkpoint's _means, _scales (log), _rotations (w, x, y, z), _opacities (logits), appearance._base_colors,
    appearance._residual_params); `config` holds the exporter's appearance keys (appearance_type, base_activation,
    residual_activation, color_activation and, for the neural model, base_input, n_frequencies, sh_degrees,
    n_neurons, n_hidden_layers, hidden_activation); `mlp_params` the flat residual mlp parameters (neural);
    `active_degree` the appearance schedule's state (None = fully enabled); `test_cameras` (M, 18) float32 rows
    of c2w (3 x 4), fx, fy, cx, cy, width, height. Returns a summary of what was written."""
    if mlp_params is not None and hasattr(mlp_params, 'detach'):
        mlp_params = mlp_params.detach().float().cpu().numpy()
    plan = plan_export(config, tuple(residual_params.shape), mlp_params, active_degree)
    packed = pack_textures(means.detach(), scales.detach(), rotations.detach(), opacities.detach(), base_colors.detach(),
                           residual_params.detach(), plan)
    kept_means = means.detach()[packed['source_index'][:packed['n_kept']].long()].cpu().numpy()
    c, u, d = camera_hint(kept_means, test_cameras, center, up, distance)
    size = write_ngsplat(path, plan, packed, c, u, d, test_cameras, proper_antialiasing)
    return dict(path=path, n_splats=packed['n_kept'], n_culled=int(means.shape[0]) - packed['n_kept'], bytes=size,
                baked=bool(plan.get('use_baked', False)), weight_texels=int(plan['weight_texels'].shape[0]),
                payload_textures=len(packed['textures']))
