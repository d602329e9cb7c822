"""FusedAdam mirroring the reference optimizer (FasterGSVDACudaBackend/.../torch_bindings/adam.py:6-36): a
torch.optim.Adam subclass with one tensor per group, a float or a list of up to 7 learning rates per group
(cycled over the last dimension's columns), and per-group betas and eps. step() updates every group with one
kernel launch.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check, lib


class FusedAdam(torch.optim.Adam):
    def __init__(self, params, lr, eps) -> None:
        super().__init__(params=params, lr=lr, eps=eps)

    @torch.no_grad()
    def step(self) -> None:
        entries = []
        device = None
        for group in self.param_groups:
            assert len(group['params']) == 1, 'more than one tensor in group'
            param = group['params'][0]
            if param.grad is None or param.numel() == 0:
                continue
            state = self.state[param]
            if len(state) == 0:
                state['step'] = 0
                state['exp_avg'] = torch.zeros_like(param)
                state['exp_avg_sq'] = torch.zeros_like(param)
            state['step'] += 1
            lr = group['lr']
            lrs = [float(x) for x in lr] if isinstance(lr, (list, tuple)) else [float(lr)]
            if not 1 <= len(lrs) <= 7:
                raise RuntimeError('between 1 and 7 learning rates are supported')
            grad = param.grad
            for name, t in (('param', param), ('grad', grad)):
                if t.dtype != torch.float32 or not t.is_contiguous() or t.device.type != 'cuda':
                    raise ValueError(f'FusedAdam: {name} must be a contiguous float32 GPU tensor')
            if device is None:
                device = param.device
            elif param.device != device:
                raise ValueError('FusedAdam: all parameters must live on one device')
            g = _lib.AdamGroup()
            g.grad, g.param = grad.data_ptr(), param.data_ptr()
            g.exp_avg, g.exp_avg_sq = state['exp_avg'].data_ptr(), state['exp_avg_sq'].data_ptr()
            g.n_elements = param.numel()
            g.step = int(state['step'])
            g.n_lrs = len(lrs)
            for i, v in enumerate(lrs):
                g.lrs[i] = v
            beta1, beta2 = group['betas']
            g.beta1, g.beta2, g.eps = float(beta1), float(beta2), float(group['eps'])
            entries.append(g)
        if not entries:
            return
        arr = (_lib.AdamGroup * len(entries))(*entries)
        with torch.cuda.device(device):
            check(lib.efgs_adam_step(arr, len(entries), torch.cuda.current_stream(device).cuda_stream))
