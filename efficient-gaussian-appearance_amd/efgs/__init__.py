"""efgs -- MI355X-native fused-appearance differentiable Gaussian rasterizer.

Drop-in for the reference package's exports (FasterGSVDACudaBackend/__init__.py:14-23): diff_rasterize,
rasterize, update_pruning_scores, RasterizerSettings, initialize_appearance, initialize_residual_mlp,
FusedAdam, relocation_adjustment, add_noise. `efgs.tcnn` supplies the tiny-cuda-nn network class the appearance plugin
builds its residual MLP with (Appearance/Base.py:23, Appearance/Neural.py:13,40-66). The compute path is libefgs_hip.so
(hand-written HIP kernels for gfx950, hipRTC-specialised preprocess); importing without the built library raises
ImportError.
"""
from .rasterization import (diff_rasterize, rasterize, update_pruning_scores, RasterizerSettings, initialize_appearance,
                            initialize_residual_mlp)
from .adam import FusedAdam
from .densification import relocation_adjustment, add_noise
from . import tcnn

__all__ = ['diff_rasterize', 'rasterize', 'update_pruning_scores', 'RasterizerSettings', 'initialize_appearance',
           'initialize_residual_mlp', 'FusedAdam', 'relocation_adjustment', 'add_noise', 'tcnn']
