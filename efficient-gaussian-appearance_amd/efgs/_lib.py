"""ctypes binding of libefgs_hip.so (the C ABI declared in include/efgs.h).

The library is built in-tree (efficient-gaussian-appearance_amd/build_lib.py) and loaded after torch, so its
libamdhip64 dependency resolves to the HIP runtime torch already has loaded. There is no fallback: importing
this module without the built library raises ImportError.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime first)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, 'libefgs_hip.so')
KERNEL_DIR = os.path.normpath(os.path.join(_HERE, '..', 'csrc', 'rtc'))
CACHE_DIR = os.path.normpath(os.path.join(_HERE, '..', 'rtc_cache'))

if not os.path.exists(LIB_PATH):
    raise ImportError(f'{LIB_PATH} is missing: build it with python efficient-gaussian-appearance_amd/build_lib.py')

_c_float_p = ctypes.POINTER(ctypes.c_float)
ALLOC_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t)


class Settings(ctypes.Structure):
    _fields_ = [('w2c', ctypes.c_void_p), ('cam_position', ctypes.c_void_p), ('bg_color', ctypes.c_void_p),
                ('appearance_degree', ctypes.c_int), ('width', ctypes.c_int), ('height', ctypes.c_int),
                ('focal_x', ctypes.c_float), ('focal_y', ctypes.c_float), ('center_x', ctypes.c_float), ('center_y', ctypes.c_float),
                ('near_plane', ctypes.c_float), ('far_plane', ctypes.c_float),
                ('proper_antialiasing', ctypes.c_int), ('render_base', ctypes.c_int), ('render_residual', ctypes.c_int)]


class Primitives(ctypes.Structure):
    _fields_ = [('n_primitives', ctypes.c_int64), ('means', ctypes.c_void_p), ('scales', ctypes.c_void_p),
                ('rotations', ctypes.c_void_p), ('opacities', ctypes.c_void_p), ('precomputed_colors', ctypes.c_void_p),
                ('base_colors', ctypes.c_void_p), ('residual_params', ctypes.c_void_p), ('mlp_weights', ctypes.c_void_p)]


class Frame(ctypes.Structure):
    _fields_ = [('primitive_buffers', ctypes.c_void_p), ('tile_buffers', ctypes.c_void_p), ('instance_buffers', ctypes.c_void_p),
                ('n_primitives', ctypes.c_int64), ('n_visible', ctypes.c_int64), ('n_instances', ctypes.c_int64),
                ('instance_capacity', ctypes.c_int64), ('grid_width', ctypes.c_int32), ('grid_height', ctypes.c_int32), ('key_bytes', ctypes.c_int32), ('model', ctypes.c_int32)]


class Gradients(ctypes.Structure):
    _fields_ = [('means', ctypes.c_void_p), ('scales', ctypes.c_void_p), ('rotations', ctypes.c_void_p),
                ('opacities', ctypes.c_void_p), ('precomputed_colors', ctypes.c_void_p), ('base_colors', ctypes.c_void_p),
                ('residual_params', ctypes.c_void_p), ('mlp_weights', ctypes.c_void_p), ('densification_info', ctypes.c_void_p),
                ('densification_rows', ctypes.c_int)]


class AdamGroup(ctypes.Structure):
    _fields_ = [('grad', ctypes.c_void_p), ('param', ctypes.c_void_p), ('exp_avg', ctypes.c_void_p),
                ('exp_avg_sq', ctypes.c_void_p), ('n_elements', ctypes.c_int64), ('step', ctypes.c_int64),
                ('n_lrs', ctypes.c_int32), ('pad_', ctypes.c_int32), ('lrs', ctypes.c_double * 7),
                ('beta1', ctypes.c_double), ('beta2', ctypes.c_double), ('eps', ctypes.c_double)]


class Workspace(ctypes.Structure):
    _fields_ = [('base', ctypes.c_void_p), ('capacity', ctypes.c_size_t), ('used', ctypes.c_size_t), ('requested', ctypes.c_size_t),
                ('fallback', ctypes.c_void_p), ('fallback_ctx', ctypes.c_void_p)]


class NgsplatInput(ctypes.Structure):
    _fields_ = [('n', ctypes.c_int64)] + [(name, ctypes.c_void_p) for name in (
        'means', 'raw_scales', 'raw_rotations', 'raw_opacities', 'base_colors', 'residual_params')] + [
        ('residual_row_stride', ctypes.c_int64), ('payload', ctypes.c_int), ('n_items', ctypes.c_int), ('base_input', ctypes.c_int),
        ('n_frequencies', ctypes.c_int), ('n_neurons', ctypes.c_int), ('residual_act', ctypes.c_int), ('color_shift', ctypes.c_float),
        ('bake_matrix', ctypes.c_void_p), ('bake_bias', ctypes.c_void_p)]


class NgsplatOutput(ctypes.Structure):
    _fields_ = [('capacity', ctypes.c_int64), ('splat_words', ctypes.c_void_p), ('params', ctypes.c_void_p), ('source_index', ctypes.c_void_p),
                ('kernel_ms', ctypes.POINTER(ctypes.c_float)), ('n_kept', ctypes.c_int64), ('base_offset', ctypes.c_float), ('base_scale', ctypes.c_float),
                ('sh_level_scale', ctypes.c_float * 3)]


class FrameViews(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        'n_touched', 'depth_keys', 'records', 'visible_prims', 'prim_offset', 'instance_keys', 'instance_primitive',
        'tile_sorted_keys', 'tile_sorted_instances', 'tile_ranges', 'final_transmittance', 'n_contributors', 'counters')]


lib = ctypes.CDLL(LIB_PATH)

EXPORTED = ('efgs_last_error', 'efgs_set_rtc_dirs', 'efgs_rasterizer_create', 'efgs_rasterizer_destroy', 'efgs_set_appearance',
            'efgs_set_residual_mlp', 'efgs_mlp_param_count', 'efgs_forward', 'efgs_backward', 'efgs_adam_step',
            'efgs_get_frame_views', 'efgs_precompile', 'efgs_set_stage_timing', 'efgs_get_stage_times', 'efgs_workspace_alloc',
            'efgs_neural_decode_forward', 'efgs_neural_decode_backward', 'efgs_neural_decode_backward_no_alloc', 'efgs_add_noise', 'efgs_relocation_adjustment', 'efgs_render', 'efgs_update_pruning_scores',
            'efgs_ngsplat_layout', 'efgs_ngsplat_pack')

# stage ids of efgs_get_stage_times, in order (include/efgs.h)
STAGES = ('preprocess_forward', 'compact', 'counter_read', 'create_instances', 'tile_offsets', 'tile_buckets', 'tile_sort',
          'blend_forward', 'blend_backward', 'preprocess_backward', 'mlp_reduce', 'mlp_backward')

lib.efgs_last_error.restype = ctypes.c_char_p
lib.efgs_last_error.argtypes = []
lib.efgs_set_rtc_dirs.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
lib.efgs_rasterizer_create.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
lib.efgs_rasterizer_destroy.restype = None
lib.efgs_rasterizer_destroy.argtypes = [ctypes.c_void_p]
lib.efgs_set_appearance.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 6
lib.efgs_set_residual_mlp.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 8
lib.efgs_mlp_param_count.restype = ctypes.c_int64
lib.efgs_mlp_param_count.argtypes = [ctypes.c_void_p]
lib.efgs_forward.argtypes = [ctypes.c_void_p, ctypes.POINTER(Primitives), ctypes.POINTER(Settings), ctypes.c_void_p, ALLOC_FN,
                             ctypes.c_void_p, ctypes.POINTER(Frame), ctypes.c_void_p]
lib.efgs_backward.argtypes = [ctypes.c_void_p, ctypes.POINTER(Primitives), ctypes.POINTER(Settings), ctypes.POINTER(Frame),
                              ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(Gradients), ALLOC_FN, ctypes.c_void_p, ctypes.c_void_p]
lib.efgs_adam_step.argtypes = [ctypes.POINTER(AdamGroup), ctypes.c_int, ctypes.c_void_p]
lib.efgs_get_frame_views.argtypes = [ctypes.POINTER(Frame), ctypes.POINTER(FrameViews)]
lib.efgs_precompile.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
lib.efgs_set_stage_timing.argtypes = [ctypes.c_void_p, ctypes.c_int]
lib.efgs_workspace_alloc.restype = ctypes.c_void_p
lib.efgs_workspace_alloc.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
WORKSPACE_ALLOC = ctypes.cast(lib.efgs_workspace_alloc, ALLOC_FN)  # C function: no Python per allocation
lib.efgs_get_stage_times.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), ctypes.c_int]
lib.efgs_neural_decode_forward.argtypes = [ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p,
                                                                                                      ctypes.c_void_p]
lib.efgs_neural_decode_backward.argtypes = ([ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_int] +
                                            [ctypes.c_void_p] * 5 + [ALLOC_FN, ctypes.c_void_p, ctypes.c_void_p])
lib.efgs_neural_decode_backward_no_alloc.argtypes = ([ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_int] +
                                                     [ctypes.c_void_p] * 6)
lib.efgs_render.argtypes = [ctypes.c_void_p, ctypes.POINTER(Primitives), ctypes.POINTER(Settings), ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                            ALLOC_FN, ctypes.c_void_p, ctypes.c_void_p]
lib.efgs_update_pruning_scores.argtypes = [ctypes.c_void_p, ctypes.POINTER(Primitives), ctypes.POINTER(Settings), ctypes.c_void_p, ALLOC_FN,
                                           ctypes.c_void_p, ctypes.c_void_p]
lib.efgs_add_noise.argtypes = [ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p]
lib.efgs_relocation_adjustment.argtypes = [ctypes.c_int64] + [ctypes.c_void_p] * 5 + [ctypes.c_void_p]
lib.efgs_ngsplat_layout.argtypes = [ctypes.POINTER(NgsplatInput), ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
lib.efgs_ngsplat_pack.argtypes = [ctypes.POINTER(NgsplatInput), ctypes.POINTER(NgsplatOutput), ALLOC_FN, ctypes.c_void_p, ctypes.c_void_p]


def check(rc: int) -> None:
    """Raises RuntimeError with the library's message for a non-zero status."""
    if rc != 0:
        msg = lib.efgs_last_error()
        raise RuntimeError(f'efgs: {msg.decode() if msg else "error"} (status {rc})')


os.makedirs(CACHE_DIR, exist_ok=True)
check(lib.efgs_set_rtc_dirs(CACHE_DIR.encode(), KERNEL_DIR.encode()))


class WorkspaceAllocator:
    """One torch uint8 device tensor per call, carved by the library's C bump allocator; requests beyond it fall
    back to per-buffer tensors. The region size follows the largest total requested so far (per key), so in
    steady state a call makes a single allocation and no Python callbacks."""

    _sizes: dict = {}

    def __init__(self, device: torch.device, key: str):
        self.key = (key, device)
        capacity = WorkspaceAllocator._sizes.get(self.key, 0)
        self.region = torch.empty(max(capacity, 256), dtype=torch.uint8, device=device)
        self.fallback = TensorAllocator(device)
        self.ws = Workspace(self.region.data_ptr(), capacity, 0, 0, ctypes.cast(self.fallback.fn, ctypes.c_void_p), None)
        self.fn = WORKSPACE_ALLOC
        self.ctx = ctypes.cast(ctypes.pointer(self.ws), ctypes.c_void_p)

    @property
    def tensors(self) -> list:
        """The tensors backing every buffer handed out (keep them alive as long as the buffers are used)."""
        return [self.region] + self.fallback.tensors

    def done(self) -> None:
        """Records the call's total so the next region covers it (with 1/16 headroom)."""
        need = int(self.ws.requested)
        if need > WorkspaceAllocator._sizes.get(self.key, 0):
            WorkspaceAllocator._sizes[self.key] = (need + need // 16 + 255) // 256 * 256


class TensorAllocator:
    """Allocation callback handing out torch uint8 device tensors; keeps them alive in `tensors`."""

    def __init__(self, device: torch.device):
        self.device = device
        self.tensors: list[torch.Tensor] = []
        self.fn = ALLOC_FN(self._alloc)

    def _alloc(self, _ctx, nbytes: int) -> int:
        t = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=self.device)
        self.tensors.append(t)
        return t.data_ptr()
