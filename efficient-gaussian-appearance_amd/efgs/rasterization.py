"""Python interface of the rasterizer, mirroring the reference bindings
(FasterGSVDACudaBackend/FasterGSVDACudaBackend/torch_bindings/rasterization.py:1-251): same function names,
argument meaning and error behaviour, backed by libefgs_hip.so through ctypes.
"""
from __future__ import annotations

import contextlib
import ctypes
from typing import Any, NamedTuple

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from ._lib import check, lib

APPEARANCE_MODEL_IDS = {'sh': 1, 'sv': 2, 'nasg': 3, 'nasgabor': 4, 'neural': 5}  # 0: internal precomputed-colour variant
BASE_ACTIVATION_IDS = {'none': 0, 'exp': 1}
RESIDUAL_ACTIVATION_IDS = {'none': 0, 'tanh': 1, 'softplus': 2}
COLOR_ACTIVATION_IDS = {'none': 0, 'relu': 1, 'softplus': 2, 'sigmoid': 3, 'hardsigmoid': 4, 'satexp': 5}
HIDDEN_ACTIVATION_IDS = {'relu': 1}


class Rasterizer:
    """Owns the native rasterizer state (appearance configuration, specialised kernels)."""

    def __init__(self) -> None:
        h = ctypes.c_void_p()
        check(lib.efgs_rasterizer_create(ctypes.byref(h)))
        self.handle = h

    def __del__(self) -> None:
        if getattr(self, 'handle', None) is not None and lib is not None:
            lib.efgs_rasterizer_destroy(self.handle)
            self.handle = None

    def set_appearance(self, model: int, max_degree: int, base_act: int, residual_act: int, color_act: int, direction_gradient: bool) -> None:
        check(lib.efgs_set_appearance(self.handle, model, max_degree, base_act, residual_act, color_act, int(bool(direction_gradient))))

    def set_residual_mlp(self, n_input_dims: int, n_output_dims: int, n_neurons: int, n_hidden_layers: int, hidden_activation: int,
                         base_input: bool, n_frequencies: int, sh_degree_mask: int) -> None:
        check(lib.efgs_set_residual_mlp(self.handle, n_input_dims, n_output_dims, n_neurons, n_hidden_layers, hidden_activation,
                                        int(bool(base_input)), n_frequencies, sh_degree_mask))

    def mlp_param_count(self) -> int:
        return int(lib.efgs_mlp_param_count(self.handle))

    def precompile(self, arch: str = 'gfx950') -> None:
        check(lib.efgs_precompile(self.handle, arch.encode()))

    def set_stage_timing(self, enable: bool) -> None:
        """Enables (and resets) or disables HIP-event timing of the pipeline stages on their launch stream."""
        check(lib.efgs_set_stage_timing(self.handle, int(bool(enable))))

    def stage_times(self) -> dict[str, tuple[float, int]]:
        """Per stage: (summed milliseconds, timed launches) since timing was enabled; waits for the events."""
        n = len(_lib.STAGES)
        ms = (ctypes.c_double * n)()
        cnt = (ctypes.c_int64 * n)()
        check(lib.efgs_get_stage_times(self.handle, ms, cnt, n))
        return {name: (float(ms[i]), int(cnt[i])) for i, name in enumerate(_lib.STAGES)}


# module-level rasterizer instance owning the specialised kernels (as the reference's _rasterizer)
_rasterizer = Rasterizer()


def initialize_appearance(appearance_model: str, max_degree: int, base_activation: str, residual_activation: str,
                          color_activation: str, direction_gradient: bool) -> None:
    """Configures the rasterizer's runtime-specialised kernels for the given appearance model."""
    _rasterizer.set_appearance(APPEARANCE_MODEL_IDS[appearance_model], max_degree, BASE_ACTIVATION_IDS[base_activation],
                               RESIDUAL_ACTIVATION_IDS[residual_activation], COLOR_ACTIVATION_IDS[color_activation], direction_gradient)


def initialize_residual_mlp(n_input_dims: int, n_output_dims: int, encoding_config: dict[str, Any], network_config: dict[str, Any],
                            base_input: bool, n_frequencies: int, sh_degrees: list[int]) -> None:
    """Creates the residual MLP from a tinycudann-style configuration (requires initialize_appearance('neural', ...) first).

    Supported: encoding 'Identity', network 'FullyFusedMLP' / 'CutlassMLP' with ReLU hidden layers and 'None' output.
    """
    otype = str(encoding_config.get('otype', 'Identity')).lower()
    if otype != 'identity':
        raise RuntimeError(f'efgs: unsupported encoding {encoding_config.get("otype")!r} (only Identity)')
    out_act = str(network_config.get('output_activation', 'None')).lower()
    if out_act != 'none':
        raise RuntimeError(f'efgs: unsupported output activation {network_config.get("output_activation")!r}')
    hidden = str(network_config.get('activation', 'ReLU')).lower()
    if hidden not in HIDDEN_ACTIVATION_IDS:
        raise RuntimeError(f'efgs: unsupported hidden activation {network_config.get("activation")!r}')
    sh_degree_mask = sum(1 << degree for degree in sh_degrees)
    _rasterizer.set_residual_mlp(n_input_dims, n_output_dims, int(network_config['n_neurons']), int(network_config['n_hidden_layers']),
                                 HIDDEN_ACTIVATION_IDS[hidden], base_input, n_frequencies, sh_degree_mask)


class RasterizerSettings(NamedTuple):
    w2c: torch.Tensor  # affine transformation from model/world space to view space
    cam_position: torch.Tensor  # camera position in world space
    bg_color: torch.Tensor  # background color in RGB format
    appearance_degree: int  # appearance degree used for rendering
    width: int  # width of the image plane in pixels
    height: int  # height of the image plane in pixels
    focal_x: float  # focal length in x direction in pixels
    focal_y: float  # focal length in y direction in pixels
    center_x: float  # x coordinate of the image center in pixels (positive -> right)
    center_y: float  # y coordinate of the image center in pixels (positive -> down)
    near_plane: float  # near clipping plane distance
    far_plane: float  # far clipping plane distance
    proper_antialiasing: bool  # whether to use proper antialiasing
    render_base: bool  # whether the view-independent base color contributes to the rendered color
    render_residual: bool  # whether the view-dependent appearance term contributes (if False, the appearance degree is treated as 0)

    def as_tuple(self) -> tuple:
        return tuple(self)


def _ptr(t: torch.Tensor | None) -> int | None:
    return t.data_ptr() if t is not None and t.numel() > 0 else None


def _check_param(name: str, t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.numel() == 0:
        return t
    if t.dtype != torch.float32:
        raise ValueError(f'efgs: {name} must be float32, got {t.dtype}')
    if t.device != device:
        raise ValueError(f'efgs: {name} is on {t.device}, expected {device}')
    if not t.is_contiguous():
        raise ValueError(f'efgs: {name} must be contiguous')
    return t


def _native_settings(s: RasterizerSettings, device: torch.device) -> tuple[_lib.Settings, list[torch.Tensor]]:
    w2c = s.w2c.detach().to(device=device, dtype=torch.float32).contiguous()
    if w2c.numel() < 12:
        raise ValueError('efgs: w2c needs at least 3 rows of 4 entries')
    cam = s.cam_position.detach().to(device=device, dtype=torch.float32).contiguous()
    bg = s.bg_color.detach().to(device=device, dtype=torch.float32).contiguous()
    c = _lib.Settings()
    c.w2c, c.cam_position, c.bg_color = w2c.data_ptr(), cam.data_ptr(), bg.data_ptr()
    c.appearance_degree = int(s.appearance_degree)
    c.width, c.height = int(s.width), int(s.height)
    c.focal_x, c.focal_y, c.center_x, c.center_y = float(s.focal_x), float(s.focal_y), float(s.center_x), float(s.center_y)
    c.near_plane, c.far_plane = float(s.near_plane), float(s.far_plane)
    c.proper_antialiasing = int(bool(s.proper_antialiasing))
    c.render_base = int(bool(s.render_base))
    c.render_residual = int(bool(s.render_residual))
    return c, [w2c, cam, bg]


def _native_primitives(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32):
    p = _lib.Primitives()
    p.n_primitives = int(means.shape[0])
    p.means, p.scales, p.rotations, p.opacities = means.data_ptr(), scales.data_ptr(), rotations.data_ptr(), opacities.data_ptr()
    p.precomputed_colors = _ptr(precomputed_colors)
    p.base_colors = _ptr(base_colors)
    p.residual_params = _ptr(residual_params)
    p.mlp_weights = _ptr(mlp_weights_f32)
    return p


# primitive, visible-primitive, instance and tile counts of the most recent forward (read back by every forward)
last_frame_counts: dict[str, int] = {}


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_inputs(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32) -> torch.device:
    device = means.device
    if device.type != 'cuda':
        raise ValueError('efgs: the rasterizer runs on a GPU device')
    names = ('means', 'scales', 'rotations', 'opacities', 'precomputed_colors', 'base_colors', 'residual_params')
    for name, t in zip(names, (means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params)):
        _check_param(name, t, device)
    if mlp_weights_f32.numel() > 0:
        expected = _rasterizer.mlp_param_count()
        if mlp_weights_f32.numel() != expected or mlp_weights_f32.device != device:
            raise ValueError(f'efgs: mlp_weights must hold {expected} parameters on {device}, got {mlp_weights_f32.numel()}')
    return device


def _forward(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32, settings,
             native=None):
    """native: (settings struct, tensors it points to, primitives struct) already built for these inputs, or None."""
    device = _check_inputs(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32)
    with torch.cuda.device(device):
        if native is not None:
            cs, keep, prims = native
        else:
            cs, keep = _native_settings(settings, device)
            prims = _native_primitives(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32)
        image = torch.empty((3, int(settings.height), int(settings.width)), dtype=torch.float32, device=device)
        alloc = _lib.WorkspaceAllocator(device, 'forward')
        frame = _lib.Frame()
        check(lib.efgs_forward(_rasterizer.handle, ctypes.byref(prims), ctypes.byref(cs), image.data_ptr(), alloc.fn, alloc.ctx,
                               ctypes.byref(frame), _stream(device)))
        alloc.done()
    last_frame_counts.update(n_primitives=int(frame.n_primitives), n_visible=int(frame.n_visible),
                             n_instances=int(frame.n_instances), n_tiles=int(frame.grid_width) * int(frame.grid_height))
    return image, frame, alloc.tensors, keep


class _Rasterize(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights,
                densification_info, rasterizer_settings: RasterizerSettings) -> torch.Tensor:
        mlp_weights_f32 = mlp_weights.detach().float().contiguous() if mlp_weights.numel() > 0 else torch.empty(0, dtype=torch.float32, device=means.device)
        ctx.mlp_numel = mlp_weights.numel()
        # the backward's host-side state is built before the forward launches anything: the host is then still ahead
        # of the GPU (which runs the previous work), and between the forward's counter read and the backward's first
        # launch only autograd's own bookkeeping runs on the host while the GPU finishes the binning and the blend
        prep = _prepare_backward(ctx, means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params,
                                 mlp_weights_f32, densification_info, rasterizer_settings) if any(ctx.needs_input_grad) else None
        ctx.prepared = prep
        image, frame, buffers, _ = _forward(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params,
                                            mlp_weights_f32, rasterizer_settings,
                                            native=(prep.settings, prep.keep, prep.prims) if prep is not None else None)
        ctx.rasterizer_settings = rasterizer_settings
        ctx.frame = frame
        ctx.buffers = buffers
        ctx.save_for_backward(image, means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32)
        ctx.densification_info = densification_info
        ctx.mark_non_differentiable(densification_info)
        return image

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, grad_image: torch.Tensor):
        saved = ctx.saved_tensors  # unpacking checks that no saved tensor was modified in place
        image = saved[0]
        # a second backward of the same graph (retain_graph) gets fresh outputs: the first call's may now be .grad
        prep = ctx.prepared or _prepare_backward(ctx, *saved[1:], ctx.densification_info, ctx.rasterizer_settings)
        ctx.prepared = None
        device = image.device
        grad_image = grad_image.contiguous()
        if grad_image.shape != image.shape or grad_image.dtype != torch.float32 or grad_image.device != device:
            raise ValueError('efgs: the image gradient must be a float32 tensor of the image\'s shape on its device')
        with _on_device(device):
            check(lib.efgs_backward(_rasterizer.handle, ctypes.byref(prep.prims), ctypes.byref(prep.settings), ctypes.byref(ctx.frame),
                                    image.data_ptr(), grad_image.data_ptr(), ctypes.byref(prep.grads), prep.alloc.fn, prep.alloc.ctx,
                                    _stream(device)))
            prep.alloc.done()
        g_means, g_scales, g_rotations, g_opacities, g_pre, g_base, g_res, g_mlp = prep.outputs
        return (g_means, g_scales, g_rotations, g_opacities,
                g_pre if g_pre.numel() > 0 else None,
                g_base if g_base.numel() > 0 else None,
                g_res if g_res.numel() > 0 else None,
                g_mlp if g_mlp.numel() > 0 else None,
                None, None)


class _PreparedBackward(NamedTuple):
    settings: Any       # _lib.Settings
    keep: list          # tensors the settings point to
    prims: Any          # _lib.Primitives
    grads: Any          # _lib.Gradients, pointing into `outputs`
    outputs: tuple      # gradient tensors, views of one allocation
    alloc: Any          # _lib.WorkspaceAllocator of the backward


def _on_device(device: torch.device):
    """torch.cuda.device(device) unless it is already current (entering the context costs host time)."""
    return contextlib.nullcontext() if torch.cuda.current_device() == device.index else torch.cuda.device(device)


def _prepare_backward(ctx, means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32,
                      dinfo, settings) -> _PreparedBackward:
    """Native structs, gradient outputs (every gradient is a view of one allocation, each fully written by the
    backward) and the workspace of the backward of this forward."""
    device = means.device
    n = means.shape[0]
    rows = int(dinfo.shape[0]) if dinfo is not None and dinfo.numel() > 0 else 0
    if rows and (dinfo.dtype != torch.float32 or not dinfo.is_contiguous() or dinfo.shape[-1] != n or dinfo.device != device):
        raise ValueError('efgs: densification_info must be a contiguous float32 (2|3, N) tensor on the rendering device')
    with _on_device(device):
        cs, keep = _native_settings(settings, device)
        prims = _native_primitives(means, scales, rotations, opacities, precomputed_colors, base_colors, residual_params, mlp_weights_f32)
        shapes = [means.shape, scales.shape, rotations.shape, opacities.shape, precomputed_colors.shape, base_colors.shape,
                  residual_params.shape, (ctx.mlp_numel,)]
        sizes = [int(torch.Size(sh).numel()) for sh in shapes]
        flat = torch.empty(sum(sizes), dtype=torch.float32, device=device)
        outputs = tuple(t.view(sh) for t, sh in zip(flat.split(sizes), shapes))
        g_means, g_scales, g_rotations, g_opacities, g_pre, g_base, g_res, g_mlp = outputs
        grads = _lib.Gradients()
        grads.means, grads.scales, grads.rotations, grads.opacities = (g_means.data_ptr(), g_scales.data_ptr(), g_rotations.data_ptr(),
                                                                       g_opacities.data_ptr())
        grads.precomputed_colors = _ptr(g_pre)
        grads.base_colors = _ptr(g_base)
        grads.residual_params = _ptr(g_res)
        grads.mlp_weights = _ptr(g_mlp)
        grads.densification_info = dinfo.data_ptr() if rows else None
        grads.densification_rows = rows
        alloc = _lib.WorkspaceAllocator(device, 'backward')
    return _PreparedBackward(cs, keep, prims, grads, outputs, alloc)


def _empty(device: torch.device, dtype=torch.float32) -> torch.Tensor:
    return torch.empty(0, dtype=dtype, device=device)


def diff_rasterize(means: torch.Tensor, scales: torch.Tensor, rotations: torch.Tensor, opacities: torch.Tensor,
                   densification_info: torch.Tensor, rasterizer_settings: RasterizerSettings,
                   precomputed_colors: torch.Tensor | None = None, base_colors: torch.Tensor | None = None,
                   residual_params: torch.Tensor | None = None, mlp_weights: torch.Tensor | None = None) -> torch.Tensor:
    """Differentiable render (3, H, W); densification_info (0,) or (2|3, N) is updated in place by the backward."""
    d = means.device
    return _Rasterize.apply(means, scales, rotations, opacities,
                            precomputed_colors if precomputed_colors is not None else _empty(d),
                            base_colors if base_colors is not None else _empty(d),
                            residual_params if residual_params is not None else _empty(d),
                            mlp_weights if mlp_weights is not None else _empty(d),
                            densification_info, rasterizer_settings)


@torch.no_grad()
def rasterize(means: torch.Tensor, scales: torch.Tensor, rotations: torch.Tensor, opacities: torch.Tensor,
              rasterizer_settings: RasterizerSettings, to_chw: bool, clamp_output: bool,
              precomputed_colors: torch.Tensor | None = None, base_colors: torch.Tensor | None = None,
              residual_params: torch.Tensor | None = None, mlp_weights: torch.Tensor | None = None) -> torch.Tensor:
    """Inference render (B/torch_bindings/rasterization.py:198-224): (3, H, W) if to_chw else (H, W, 3),
    clamped to [0, 1] if clamp_output; written in that layout by the blend kernel, no backward state."""
    d = means.device
    mlp_f32 = mlp_weights.detach().float().contiguous() if mlp_weights is not None else _empty(d)
    pre = precomputed_colors if precomputed_colors is not None else _empty(d)
    base = base_colors if base_colors is not None else _empty(d)
    res = residual_params if residual_params is not None else _empty(d)
    device = _check_inputs(means, scales, rotations, opacities, pre, base, res, mlp_f32)
    h, w = int(rasterizer_settings.height), int(rasterizer_settings.width)
    with torch.cuda.device(device):
        cs, keep = _native_settings(rasterizer_settings, device)
        prims = _native_primitives(means, scales, rotations, opacities, pre, base, res, mlp_f32)
        image = torch.empty((3, h, w) if to_chw else (h, w, 3), dtype=torch.float32, device=device)
        alloc = _lib.WorkspaceAllocator(device, 'render')
        check(lib.efgs_render(_rasterizer.handle, ctypes.byref(prims), ctypes.byref(cs), image.data_ptr(), int(bool(to_chw)),
                              int(bool(clamp_output)), alloc.fn, alloc.ctx, _stream(device)))
        alloc.done()
    del keep
    return image


class _NeuralDecode(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, features, dirs, mlp_weights, base, degree: int) -> torch.Tensor:
        device = features.device
        mlp_half = mlp_weights.detach().half().contiguous()
        n = int(dirs.shape[0])
        out = torch.empty((n, 3), dtype=torch.float32, device=device)
        with torch.cuda.device(device):
            check(lib.efgs_neural_decode_forward(_rasterizer.handle, n, _ptr(features), _ptr(base), _ptr(dirs), _ptr(mlp_half), int(degree),
                                                 _ptr(out), _stream(device)))
        ctx.degree = int(degree)
        ctx.mlp_numel = mlp_weights.numel()
        ctx.save_for_backward(features, dirs, mlp_half, base)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, grad_out: torch.Tensor):
        features, dirs, mlp_half, base = ctx.saved_tensors
        device = features.device
        n = int(dirs.shape[0])
        grad_out = grad_out.contiguous()
        g_features = torch.empty_like(features)
        g_dirs = torch.empty_like(dirs)
        g_base = torch.empty_like(base)
        g_mlp = torch.empty(ctx.mlp_numel, dtype=torch.float32, device=device)
        with torch.cuda.device(device):
            alloc = _lib.WorkspaceAllocator(device, 'decode')
            check(lib.efgs_neural_decode_backward(_rasterizer.handle, n, _ptr(features), _ptr(base), _ptr(dirs), _ptr(mlp_half), ctx.degree,
                                                  _ptr(grad_out), _ptr(g_features), _ptr(g_base), _ptr(g_dirs), _ptr(g_mlp), alloc.fn,
                                                  alloc.ctx, _stream(device)))
            alloc.done()
        return (g_features if features.numel() > 0 else None, g_dirs, g_mlp, g_base if base.numel() > 0 else None, None)


def neural_decode(features: torch.Tensor, dirs: torch.Tensor, mlp_weights: torch.Tensor, degree: int = 1,
                  base_colors: torch.Tensor | None = None) -> torch.Tensor:
    """Differentiable standalone decode of the configured residual MLP (initialize_residual_mlp): raw outputs
    (N, 3) for features (N, n_features), unit view directions (N, 3) and the tcnn-flat fp32 master weights
    (cast to fp16 per call, as in diff_rasterize); degree gates the direction's SH degrees as the appearance
    degree does in the rasterizer. Gradients flow to the features, the directions, the weights and (with base
    input) the base colours. No counterpart in the reference's Python API: its tiny-cuda-nn MLP runs only inside
    the preprocess kernels."""
    d = features.device
    if d.type != 'cuda':
        raise ValueError('efgs: the neural decode runs on a GPU device')
    base = base_colors if base_colors is not None else _empty(d)
    for name, t in (('features', features), ('dirs', dirs), ('mlp_weights', mlp_weights), ('base_colors', base)):
        _check_param(name, t, d)
    if dirs.dim() != 2 or dirs.shape[1] != 3:
        raise ValueError('efgs: dirs must be (N, 3)')
    if mlp_weights.numel() != _rasterizer.mlp_param_count():
        raise ValueError(f'efgs: mlp_weights must hold {_rasterizer.mlp_param_count()} parameters, got {mlp_weights.numel()}')
    return _NeuralDecode.apply(features, dirs, mlp_weights, base, degree)


@torch.no_grad()
def update_pruning_scores(scores: torch.Tensor, means: torch.Tensor, scales: torch.Tensor, rotations: torch.Tensor,
                          opacities: torch.Tensor, rasterizer_settings: RasterizerSettings,
                          precomputed_colors: torch.Tensor | None = None, base_colors: torch.Tensor | None = None,
                          residual_params: torch.Tensor | None = None, mlp_weights: torch.Tensor | None = None) -> None:
    """Speedy-Splat pruning scores of one view (B/torch_bindings/rasterization.py:226-250): scores (N,) float32
    += per Gaussian the sum over the view's pixels of (o dL/dalpha)^2 for an all-ones image gradient, in place."""
    d = means.device
    mlp_f32 = mlp_weights.detach().float().contiguous() if mlp_weights is not None else _empty(d)
    pre = precomputed_colors if precomputed_colors is not None else _empty(d)
    base = base_colors if base_colors is not None else _empty(d)
    res = residual_params if residual_params is not None else _empty(d)
    device = _check_inputs(means, scales, rotations, opacities, pre, base, res, mlp_f32)
    if scores.dtype != torch.float32 or scores.device != device or not scores.is_contiguous() or scores.numel() != means.shape[0]:
        raise ValueError('efgs: scores must be a contiguous float32 tensor of N entries on the rendering device')
    with torch.cuda.device(device):
        cs, keep = _native_settings(rasterizer_settings, device)
        prims = _native_primitives(means, scales, rotations, opacities, pre, base, res, mlp_f32)
        alloc = _lib.WorkspaceAllocator(device, 'scores')
        check(lib.efgs_update_pruning_scores(_rasterizer.handle, ctypes.byref(prims), ctypes.byref(cs), scores.data_ptr(), alloc.fn,
                                             alloc.ctx, _stream(device)))
        alloc.done()
    del keep


def frame_views(frame: _lib.Frame) -> _lib.FrameViews:
    """Device pointers into a forward frame's buffers (inspection for parity tests)."""
    v = _lib.FrameViews()
    check(lib.efgs_get_frame_views(ctypes.byref(frame), ctypes.byref(v)))
    return v


def forward_with_frame(means, scales, rotations, opacities, rasterizer_settings: RasterizerSettings, precomputed_colors=None,
                       base_colors=None, residual_params=None, mlp_weights=None):
    """Forward pass returning (image, frame, buffers): the frame and the buffers that back it, for inspection."""
    d = means.device
    mlp_f32 = mlp_weights.detach().float().contiguous() if mlp_weights is not None else _empty(d)
    image, frame, buffers, _ = _forward(means, scales, rotations, opacities,
                                        precomputed_colors if precomputed_colors is not None else _empty(d),
                                        base_colors if base_colors is not None else _empty(d),
                                        residual_params if residual_params is not None else _empty(d),
                                        mlp_f32, rasterizer_settings)
    return image, frame, buffers
