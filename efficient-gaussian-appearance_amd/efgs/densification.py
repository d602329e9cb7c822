"""MCMC densification operators, mirroring the reference's bindings
(FasterGSVDACudaBackend/.../torch_bindings/densification.py:6-21, native side
B/densification/src/densification_api.cu:13-72): `relocation_adjustment` and `add_noise` on torch device
tensors, computed by libefgs_hip.so on the current stream.
"""
from __future__ import annotations

import torch

from ._lib import check, lib


def _device_tensor(name: str, t: torch.Tensor, dtype: torch.dtype, device: torch.device | None = None) -> torch.Tensor:
    if t.dtype != dtype:
        raise ValueError(f'efgs: {name} must be {dtype}, got {t.dtype}')
    if t.device.type != 'cuda':
        raise ValueError(f'efgs: {name} must be on a GPU device, got {t.device}')
    if device is not None and t.device != device:
        raise ValueError(f'efgs: {name} is on {t.device}, expected {device}')
    return t


def relocation_adjustment(old_opacities: torch.Tensor, old_scales: torch.Tensor,
                          n_samples_per_primitive: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Opacities (N, 1) and activated scales (N, 3) of Gaussians that are each split into
    n_samples_per_primitive (int64, clamped to 1..50) copies: o' = 1 - (1 - o)^(1/n) and the scales rescaled
    so that the copies keep the original's footprint (3DGS-MCMC, Eq. 9). Inputs: activated opacities (N,) or
    (N, 1), activated scales (N, 3)."""
    device = old_opacities.device
    _device_tensor('old_opacities', old_opacities, torch.float32)
    _device_tensor('old_scales', old_scales, torch.float32, device)
    _device_tensor('n_samples_per_primitive', n_samples_per_primitive, torch.int64, device)
    n = old_opacities.shape[0]
    if old_opacities.numel() != n or old_scales.shape != (n, 3) or n_samples_per_primitive.numel() != n:
        raise ValueError('efgs: relocation_adjustment expects opacities (N, 1), scales (N, 3) and N sample counts')
    o = old_opacities.contiguous()
    s = old_scales.contiguous()
    c = n_samples_per_primitive.contiguous()
    new_opacities = torch.empty((n, 1), dtype=torch.float32, device=device)
    new_scales = torch.empty((n, 3), dtype=torch.float32, device=device)
    if n > 0:
        with torch.cuda.device(device):
            check(lib.efgs_relocation_adjustment(n, o.data_ptr(), s.data_ptr(), c.data_ptr(), new_opacities.data_ptr(),
                                                 new_scales.data_ptr(), torch.cuda.current_stream(device).cuda_stream))
    return new_opacities, new_scales


def add_noise(raw_scales: torch.Tensor, raw_rotations: torch.Tensor, raw_opacities: torch.Tensor, means: torch.Tensor,
              current_lr: float) -> None:
    """Adds 3DGS-MCMC position noise to `means` (N, 3) in place: current_lr * sigmoid(-(100 o - 0.5)) * Sigma z
    with o = sigmoid(raw_opacities), Sigma from the log-scales (N, 3) and unnormalised quaternions (N, 4), and
    z ~ N(0, I) drawn by Philox4x32-10 from the device's default torch generator (its seed, and its offset,
    which advances by 4 per call as the reference's philox_engine_inputs(4))."""
    device = means.device
    for name, t in (('raw_scales', raw_scales), ('raw_rotations', raw_rotations), ('raw_opacities', raw_opacities), ('means', means)):
        _device_tensor(name, t, torch.float32, device)
        if not t.is_contiguous():
            raise ValueError(f'efgs: {name} must be contiguous')
    n = means.shape[0]
    if means.shape != (n, 3) or raw_scales.shape != (n, 3) or raw_rotations.shape != (n, 4) or raw_opacities.numel() != n:
        raise ValueError('efgs: add_noise expects scales (N, 3), rotations (N, 4), opacities (N, 1) and means (N, 3)')
    gen = torch.cuda.default_generators[device.index if device.index is not None else torch.cuda.current_device()]
    seed = gen.initial_seed()
    offset = gen.get_offset()
    gen.set_offset(offset + 4)
    if n == 0:
        return
    with torch.cuda.device(device):
        check(lib.efgs_add_noise(n, raw_scales.data_ptr(), raw_rotations.data_ptr(), raw_opacities.data_ptr(), means.data_ptr(),
                                 float(current_lr), seed, offset, torch.cuda.current_stream(device).cuda_stream))
