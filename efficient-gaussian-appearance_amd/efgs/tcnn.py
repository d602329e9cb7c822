"""The part of tiny-cuda-nn's PyTorch surface that the neural appearance model uses, on this build's fp16 MFMA
MLP: `NetworkWithInputEncoding` (and `Network`, the same without an encoding config).

The reference's appearance plugin imports `Thirdparty.TinyCudaNN as tcnn` (Appearance/Base.py:23,
Appearance/Neural.py:13) and builds its residual MLP as `tcnn.NetworkWithInputEncoding(n_input_dims, 3,
{'otype': 'Identity'}, {'otype': 'FullyFusedMLP', ...})` (Neural.py:40-51). That object
  * owns the fp32 master weights `params` in tcnn's flat layout, which the rasterizer consumes as `mlp_weights`
    (Neural.py:53 zeroes the output rows, :78 hands them to the optimiser, :98-100 to the rasterizer);
  * carries `n_input_dims`, `n_output_dims`, `encoding_config` and `network_config`, which Neural.py:55-66 pass to
    `initialize_residual_mlp`;
  * is called on the encoded (N, n_input_dims) input for the unfused appearance evaluation (Neural.py:102-111) and
    returns (N, n_output_dims) half-precision outputs, differentiable with respect to the input and `params`.
Here the call runs the library's standalone decode (`efgs_neural_decode_forward` / `_backward`) on a rasterizer
handle of the network's own, configured with the identity encoding: the same fp16 MFMA kernels, fp16 rounding
between layers and fp32 accumulation as the rasterizer's fused evaluation, so the unfused and fused colours agree.

Flat layout (as tcnn's FullyFusedMLP): row-major [out x in] matrices, the first layer's input padded to a multiple of
16, hidden layers n_neurons x n_neurons, the output layer padded to 16 rows and stored last. Padded input columns
carry zero. Supported: encoding 'Identity' (optionally with tcnn's `scale` / `offset`), network 'FullyFusedMLP' with
'ReLU' hidden layers, 'None' output activation, 16 / 32 / 64 / 128 neurons, 1..8 hidden layers, 3 outputs and at
most 128 inputs; anything else raises ValueError. Initial weights are Xavier-uniform per matrix (bound
sqrt(6 / (fan_in + fan_out)) over the padded shapes) from a torch generator seeded with `seed`: the distribution of
tcnn's initialisation, not its pcg32 stream (the reference zeroes the output rows right after construction, so no
result depends on those values).
"""
from __future__ import annotations

import math
from typing import Any

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from ._lib import check, lib
from .rasterization import APPEARANCE_MODEL_IDS, HIDDEN_ACTIVATION_IDS, Rasterizer

N_NEURONS = (16, 32, 64, 128)
MAX_INPUT_DIMS = 128
N_OUTPUT_DIMS = 3


def _parse_encoding(encoding_config: dict[str, Any] | None) -> tuple[float, float]:
    cfg = dict(encoding_config or {'otype': 'Identity'})
    if str(cfg.get('otype', 'Identity')).lower() != 'identity':
        raise ValueError(f'efgs.tcnn: unsupported encoding {cfg.get("otype")!r} (only Identity)')
    unknown = set(cfg) - {'otype', 'scale', 'offset'}
    if unknown:
        raise ValueError(f'efgs.tcnn: unsupported Identity encoding options {sorted(unknown)}')
    return float(cfg.get('scale', 1.0)), float(cfg.get('offset', 0.0))


def _parse_network(network_config: dict[str, Any]) -> tuple[int, int]:
    cfg = dict(network_config)
    if str(cfg.get('otype', 'FullyFusedMLP')).lower() != 'fullyfusedmlp':
        raise ValueError(f'efgs.tcnn: unsupported network {cfg.get("otype")!r} (only FullyFusedMLP)')
    if str(cfg.get('activation', 'ReLU')).lower() not in HIDDEN_ACTIVATION_IDS:
        raise ValueError(f'efgs.tcnn: unsupported hidden activation {cfg.get("activation")!r} (only ReLU)')
    if str(cfg.get('output_activation', 'None')).lower() != 'none':
        raise ValueError(f'efgs.tcnn: unsupported output activation {cfg.get("output_activation")!r} (only None)')
    n_neurons, n_hidden = int(cfg['n_neurons']), int(cfg['n_hidden_layers'])
    if n_neurons not in N_NEURONS:
        raise ValueError(f'efgs.tcnn: n_neurons must be one of {N_NEURONS}, got {n_neurons}')
    if not 1 <= n_hidden <= 8:
        raise ValueError(f'efgs.tcnn: n_hidden_layers must be in 1..8, got {n_hidden}')
    return n_neurons, n_hidden


def layer_shapes(n_input_dims: int, n_neurons: int, n_hidden_layers: int, n_output_dims: int = N_OUTPUT_DIMS) -> list[tuple[int, int]]:
    """(rows, cols) of the flat parameter vector's matrices in storage order."""
    n_in = (n_input_dims + 15) // 16 * 16
    n_out = (n_output_dims + 15) // 16 * 16
    return [(n_neurons, n_in)] + [(n_neurons, n_neurons)] * (n_hidden_layers - 1) + [(n_out, n_neurons)]


def initial_params(n_input_dims: int, n_neurons: int, n_hidden_layers: int, seed: int, n_output_dims: int = N_OUTPUT_DIMS) -> torch.Tensor:
    """Xavier-uniform fp32 weights in the flat layout (CPU tensor)."""
    gen = torch.Generator().manual_seed(int(seed))
    parts = []
    for rows, cols in layer_shapes(n_input_dims, n_neurons, n_hidden_layers, n_output_dims):
        bound = math.sqrt(6.0 / (rows + cols))
        parts.append((torch.rand(rows * cols, generator=gen, dtype=torch.float32) * 2.0 - 1.0) * bound)
    return torch.cat(parts)


class _IdentityMLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, net: 'NetworkWithInputEncoding', x: torch.Tensor, params: torch.Tensor) -> torch.Tensor:
        device = params.device
        x32 = x.detach().to(dtype=torch.float32).contiguous()
        w16 = params.detach().to(dtype=torch.float16).contiguous()  # rounded to nearest even, as the rasterizer stages them
        n = int(x32.shape[0])
        out = torch.empty((n, N_OUTPUT_DIMS), dtype=torch.float32, device=device)
        with torch.cuda.device(device):
            check(lib.efgs_neural_decode_forward(net._handle.handle, n, x32.data_ptr() if n else None, None, None, w16.data_ptr(), 0,
                                                 out.data_ptr() if n else None, torch.cuda.current_stream(device).cuda_stream))
        ctx.net = net
        ctx.x_dtype = x.dtype
        ctx.save_for_backward(x32, w16)
        return out.to(dtype=torch.float16)  # (the decode's outputs are fp16 values: exact)

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, grad_out: torch.Tensor):
        x32, w16 = ctx.saved_tensors
        net = ctx.net
        device = w16.device
        n = int(x32.shape[0])
        g = grad_out.to(dtype=torch.float32).contiguous()
        g_x = torch.empty_like(x32)
        g_w = torch.empty(w16.numel(), dtype=torch.float32, device=device)
        with torch.cuda.device(device):
            alloc = _lib.WorkspaceAllocator(device, 'tcnn')
            check(lib.efgs_neural_decode_backward(net._handle.handle, n, x32.data_ptr() if n else None, None, None, w16.data_ptr(), 0,
                                                  g.data_ptr() if n else None, g_x.data_ptr() if n else None, None, None, g_w.data_ptr(),
                                                  alloc.fn, alloc.ctx, torch.cuda.current_stream(device).cuda_stream))
            alloc.done()
        return (None, g_x.to(dtype=ctx.x_dtype) if ctx.needs_input_grad[1] else None,
                g_w if ctx.needs_input_grad[2] else None)


class NetworkWithInputEncoding(torch.nn.Module):
    """tcnn.NetworkWithInputEncoding(n_input_dims, n_output_dims, encoding_config, network_config, seed) with the
    identity encoding: a bias-free fp16 ReLU MLP whose fp32 master weights are `params` (flat tcnn layout).
    `device` (an extension; tcnn uses the current CUDA device) places `params`; calls need a GPU device."""

    def __init__(self, n_input_dims: int, n_output_dims: int, encoding_config: dict[str, Any] | None, network_config: dict[str, Any],
                 seed: int = 1337, device: torch.device | str | None = None) -> None:
        super().__init__()
        n_input_dims, n_output_dims = int(n_input_dims), int(n_output_dims)
        if n_output_dims != N_OUTPUT_DIMS:
            raise ValueError(f'efgs.tcnn: the MLP kernels produce {N_OUTPUT_DIMS} outputs, got n_output_dims={n_output_dims}')
        if not 1 <= n_input_dims <= MAX_INPUT_DIMS:
            raise ValueError(f'efgs.tcnn: n_input_dims must be in 1..{MAX_INPUT_DIMS}, got {n_input_dims}')
        self._scale, self._offset = _parse_encoding(encoding_config)
        n_neurons, n_hidden = _parse_network(network_config)
        self.n_input_dims = n_input_dims
        self.n_output_dims = n_output_dims
        self.encoding_config = dict(encoding_config or {'otype': 'Identity'})
        self.network_config = dict(network_config)
        self.seed = int(seed)
        self.dtype = torch.float16
        self.loss_scale = 128.0  # tcnn's value for half-precision networks (this build scales per launch instead)
        self._n_neurons, self._n_hidden = n_neurons, n_hidden
        self._handle = self._make_handle()
        if device is None:
            device = torch.device('cuda', torch.cuda.current_device()) if torch.cuda.is_available() else torch.device('cpu')
        params = initial_params(n_input_dims, n_neurons, n_hidden, self.seed).to(device=device)
        if params.numel() != self.n_params:
            raise RuntimeError(f'efgs.tcnn: {params.numel()} initial parameters for an MLP of {self.n_params}')
        self.params = torch.nn.Parameter(params, requires_grad=True)

    def _make_handle(self) -> Rasterizer:
        h = Rasterizer()
        h.set_appearance(APPEARANCE_MODEL_IDS['neural'], 0, 0, 0, 0, False)
        # identity encoding: no frequency encoding, no base input, no SH degree values (the inputs as given)
        h.set_residual_mlp(self.n_input_dims, self.n_output_dims, self._n_neurons, self._n_hidden, HIDDEN_ACTIVATION_IDS['relu'], False,
                           0, 0)
        return h

    @property
    def n_params(self) -> int:
        return self._handle.mlp_param_count()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() != 2 or x.shape[1] != self.n_input_dims:
            raise ValueError(f'efgs.tcnn: input must be (batch, {self.n_input_dims}), got {tuple(x.shape)}')
        if not x.is_floating_point():
            raise ValueError(f'efgs.tcnn: input must be floating point, got {x.dtype}')
        if self.params.device.type != 'cuda':
            raise ValueError('efgs.tcnn: the network runs on a GPU device (params are on the CPU)')
        if x.device != self.params.device:
            raise ValueError(f'efgs.tcnn: input is on {x.device}, params on {self.params.device}')
        if self._scale != 1.0 or self._offset != 0.0:
            x = x * self._scale + self._offset
        return _IdentityMLP.apply(self, x, self.params)

    def __getstate__(self):
        state = self.__dict__.copy()
        state.pop('_handle', None)
        return state

    def __setstate__(self, state):
        self.__dict__.update(state)
        self._handle = self._make_handle()

    def extra_repr(self) -> str:
        return (f'n_input_dims={self.n_input_dims}, n_output_dims={self.n_output_dims}, seed={self.seed}, dtype={self.dtype}, '
                f'hyperparams={{"encoding": {self.encoding_config}, "network": {self.network_config}}}')


class Network(NetworkWithInputEncoding):
    """tcnn.Network(n_input_dims, n_output_dims, network_config, seed): the network alone (identity input)."""

    def __init__(self, n_input_dims: int, n_output_dims: int, network_config: dict[str, Any], seed: int = 1337,
                 device: torch.device | str | None = None) -> None:
        super().__init__(n_input_dims, n_output_dims, {'otype': 'Identity'}, network_config, seed, device)


__all__ = ['NetworkWithInputEncoding', 'Network']
