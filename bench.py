#!/usr/bin/env python3
"""Forward + backward benchmark of the fused-appearance rasterizer on one MI355X.

Workload (default, configuration c3): 1M Gaussians, 1920 x 1080, neural appearance (8 latents + SH degree 1
direction -> 64 -> 64 -> 3 fp16 MLP, tanh residual, relu colour), synthetic seeded scene. One step =
the rasterizer's forward + backward (below); the training iteration around it (L1 loss against a seeded
uniform-noise target, one FusedAdam step over all parameter groups: means, scales, rotations, opacities, base
colours, latents, MLP weights) is timed beside it. Inputs are resident in HBM before the timed region.

A timed step is the headline quantity W * H / (t_fwd + t_bwd): diff_rasterize forward (preprocess through blend,
with its counter readback) and backward (blend backward, preprocess backward) with a fixed upstream gradient (the
L1 gradient of the scene's first render). The step first runs untimed for RAMP_S seconds (the GPU's clocks rise
over the first tens of milliseconds of load), then W warm-up steps, then the K timed steps between one pair of HIP
events with device synchronisations on both sides. Output: one JSON line. `value` = W * H / (that time / K) in
Mpix/s (K more steps, each between its own events, give `step_ms_quartiles`); `full_step_*` = one training iteration (forward, L1 loss, backward, FusedAdam over every
group); `inference_ms` / `inference_fps` = `rasterize` as the reference's render_image_benchmark calls it (HWC,
clamped, no autograd). `roofline` covers the step's dominant kernel, timed with HIP events that the library records
around each stage on the stream it launches on; `stages` lists every stage (Adam: events around FusedAdam.step on
the same stream). `cpu_baseline` times the reference's unfused appearance evaluation (restated in torch) on the
host's torch threads; `cpu_port_rasterizer` the C / numpy restatement (oracle/) of one forward + backward of the
same scene on one host thread.

  python bench.py [--steps K] [--warmup W] [--config c3|c1|c4_sv|c4_nasg|c4_nasgabor] [--no-cpu-baseline]
  python bench.py --config c2    # the neural decode alone: 1M primitives, forward + backward (latents, weights)
  python bench.py --config mcmc  # MCMC densification: add_noise and relocation_adjustment of the 1M c3 Gaussians
  python bench.py --config pruning  # Speedy-Splat pruning scores of one c3 view
  python bench.py --copy-calibration    # a plain 1 GiB device copy, for scaling rocprofv3 FETCH/WRITE_SIZE
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, 'efficient-gaussian-appearance_amd')
if PKG not in sys.path:
    sys.path.insert(0, PKG)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
RAMP_S = 0.3                   # untimed clock ramp before the warm-up steps (seconds of the timed step itself)
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'traffic_c3_neural.txt')
KERNELS_FILE = os.path.join(ROOT, 'profiles', 'kernels_c3_neural_train_step.txt')

# kernel names (as rocprofv3 lists them) of each timed stage
STAGE_KERNELS = {
    'preprocess_forward': 'preprocess_forward_<model>',
    # (with the fused emission the scan runs on a first frame only and the compaction not at all: the stage is then
    # not timed, and create_instances_fused_kernel carries the compaction's bytes)
    'compact': 'scan_block_counts_kernel + compact_visible_kernel',
    'create_instances': 'create_instances_fused_kernel',
    'tile_offsets': 'tile_column_scan_kernel',  # (the tile order's runs are placed by an extra block of tile_buckets_kernel)
    'tile_buckets': 'tile_buckets_kernel',
    'tile_sort': 'tile_ranges_kernel',  # (the tiles' runs are sorted by blend_forward_kernel, before its walk)
    'blend_forward': 'blend_forward_kernel',
    'blend_backward': 'blend_backward_kernel',
    'preprocess_backward': 'preprocess_backward_<model>',
    'mlp_backward': 'preprocess_backward_<model>_mlp',
    'mlp_reduce': 'reduce_partials_kernel',
    'adam': 'adam_kernel',
}


def log(msg: str) -> None:
    print(f'bench: {msg}', file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=100)
    p.add_argument('--warmup', type=int, default=10)
    p.add_argument('--config', default='c3')
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--copy-calibration', action='store_true')
    return p.parse_args()


# ---------------------------------------------------------------------------------------------------------
# algorithmic bytes and flops per launch (compulsory traffic: every input read once, every output written
# once; radix-pass re-reads and other design-dependent traffic excluded)
# ---------------------------------------------------------------------------------------------------------

def residual_bytes(model: str, n_units: int) -> int:
    """Residual parameter bytes per primitive: SH3 45 floats, neural 8 latents, SV 7, NASG 8, NASGabor 9
    floats per site / lobe."""
    per_unit = {'sh': 12, 'neural': 4, 'sv': 28, 'nasg': 32, 'nasgabor': 36}[model]
    return per_unit * n_units


def mlp_flops_per_primitive(n_in: int, n_neurons: int, n_hidden: int, n_out: int = 3) -> int:
    """Unpadded forward FLOPs of the bias-free MLP (2 per multiply-add)."""
    return 2 * (n_in * n_neurons + (n_hidden - 1) * n_neurons * n_neurons + n_neurons * n_out)


def algorithmic(stage: str, N: int, V: int, I: int, T: int, P: int, R: int, mlp_fwd_flops: int, adam_elements: int,
                compaction_fused: bool = True):
    """(bytes, flops) of one launch of `stage`. Per-unit figures: preprocess N*(60+R) + V*52 split into the
    preprocess kernel (N*(60+R) + V*44) and the compaction (V*8: visible list and emission offsets); instance
    emission V*40 + I*6 (with the compaction fused into the emission kernel, as on grids whose tile histogram fits
    its LDS: V*48 + I*6 for that one kernel, and no compaction stage), tile ranges T*8; the ordering by (tile, depth) -- the reference's depth sort and
    offset scan (V*24) and tile sort (I*12) -- split into the bucketing (I*6: tile key in, emission index
    out) and the per-tile sort (I*6 + V*24), which the forward blend runs before its walk; the tiles' ranges and
    order T*24 (three words in, two out); blend forward I*48 + P*20 (+ the sort); blend backward P*32 + I*76;
    preprocess backward V*(110+R) + N*(56+R), for the neural model split into the geometry kernel
    (V*110 + N*56 + (N-V)*R: culled primitives' zero latent gradients) and the MLP kernel (V*2R: latents in,
    latent gradients out); Adam 28 B per element. MLP FLOPs: forward V*F, backward (input and weight
    gradients, forward recomputed) 2*V*F, F = unpadded forward FLOPs per primitive."""
    table = {
        'preprocess_forward': (N * (60 + R) + V * 44, V * mlp_fwd_flops),
        'compact': (V * 8, 0),
        'create_instances': (V * (48 if compaction_fused else 40) + I * 6, 0),
        'tile_offsets': (T * 8, 0),
        'tile_buckets': (I * 6, 0),
        'tile_sort': (T * 24, 0),
        'blend_forward': (I * 48 + P * 20 + I * 6 + V * 24, 0),
        'blend_backward': (P * 32 + I * 76, 0),
        'preprocess_backward': ((V * 110 + N * 56 + (N - V) * R, 0) if mlp_fwd_flops
                                else (V * (110 + R) + N * (56 + R), 0)),
        'mlp_backward': (V * 2 * R, 2 * V * mlp_fwd_flops),
        'adam': (28 * adam_elements, 0),
    }
    return table.get(stage, (0, 0))


def read_step_kernel_us():
    """Kernel time of one steady-state c3 step (microseconds) from the committed rocprofv3 kernel-trace summary: its
    line `step_kernels_us <value>`."""
    if not os.path.exists(KERNELS_FILE):
        return None
    with open(KERNELS_FILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 2 and parts[0] == 'step_kernels_us':
                return float(parts[1])
    return None


def read_traffic(kernel: str):
    """L2-to-fabric bytes per launch of `kernel` (read + write) from the committed rocprofv3 TCC summary, if it lists
    the kernel: lines `traffic <kernel> <read_bytes> <write_bytes>`, requests counted by size (128 / 64 / 32 bytes)."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 4 and parts[0] == 'traffic' and parts[1] == kernel:
                return float(parts[2]) + float(parts[3])
    return None


# ---------------------------------------------------------------------------------------------------------
# GPU step
# ---------------------------------------------------------------------------------------------------------

def build_problem(config: str, device):
    import numpy as np
    import torch
    import efgs
    from efgs.synthetic import make_scene, target_image

    sc = make_scene(config)
    cam = sc['camera']
    app = sc['appearance']
    efgs.initialize_appearance(app['model'], app['max_degree'], app['base_act'], app['res_act'], app['color_act'],
                               app['direction_gradient'])
    mlp = app.get('mlp')
    if mlp is not None:
        n_in = mlp['n_feature_dims'] + sum(2 * d + 1 for d in mlp['sh_degrees'])
        efgs.initialize_residual_mlp(n_in, 3, {'otype': 'Identity'},
                                     {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None',
                                      'n_neurons': mlp['n_neurons'], 'n_hidden_layers': mlp['n_hidden_layers']},
                                     mlp['base_input'], mlp['n_frequencies'], list(mlp['sh_degrees']))

    def leaf(a):
        return torch.tensor(np.ascontiguousarray(a, np.float32), device=device).requires_grad_(True)

    params = dict(means=leaf(sc['means']), scales=leaf(sc['scales']), rotations=leaf(sc['rotations']),
                  opacities=leaf(sc['opacities']), base_colors=leaf(sc['base_colors']),
                  residual_params=leaf(sc['residual_params']))
    if sc['mlp_weights'] is not None:
        params['mlp_weights'] = leaf(sc['mlp_weights'])
    degree = app['max_degree'] if app['model'] != 'neural' else 1
    settings = efgs.RasterizerSettings(
        w2c=torch.tensor(cam['w2c'], device=device), cam_position=torch.tensor(cam['position'], device=device),
        bg_color=torch.zeros(3, device=device), appearance_degree=degree, width=cam['width'], height=cam['height'],
        focal_x=cam['focal_x'], focal_y=cam['focal_y'], center_x=cam['center_x'], center_y=cam['center_y'],
        near_plane=cam['near_plane'], far_plane=cam['far_plane'], proper_antialiasing=False, render_base=True,
        render_residual=True)
    target = torch.tensor(target_image(cam['width'], cam['height']), device=device)
    # learning rates of the reference's training configurations (3DGS defaults, means scaled by the extent)
    lrs = dict(means=1.6e-4 * 10.0, scales=5e-3, rotations=1e-3, opacities=2.5e-2, base_colors=2.5e-3,
               residual_params=2.5e-3, mlp_weights=1e-3)
    opt = efgs.FusedAdam([{'params': [t], 'lr': lrs[k], 'name': k} for k, t in params.items()], lr=0.0, eps=1e-15)
    return sc, params, settings, target, opt


def l1_loss_fn():
    """mean |image - target| as one autograd function: forward = difference + one fused L1-norm reduction,
    backward = sign(difference) / numel (4 elementwise/reduction kernels instead of the 7 of
    `(image - target).abs().mean()` and its autograd graph; same value and gradient)."""
    import torch

    class L1Loss(torch.autograd.Function):
        @staticmethod
        def forward(ctx, image, target):
            diff = image - target
            ctx.save_for_backward(diff)
            return torch.linalg.vector_norm(diff, ord=1) / diff.numel()

        @staticmethod
        def backward(ctx, g):
            (diff,) = ctx.saved_tensors
            return torch.sign(diff).mul_(g / diff.numel()), None
    return L1Loss.apply


def _quartiles(xs):
    """min, lower quartile, median, upper quartile, max (nearest-rank)."""
    xs = sorted(xs)
    k = len(xs) - 1
    return [xs[0], xs[k // 4], _median(xs), xs[(3 * k + 3) // 4], xs[-1]]


def _median(xs):
    xs = sorted(xs)
    k = len(xs)
    return xs[k // 2] if k % 2 else 0.5 * (xs[k // 2 - 1] + xs[k // 2])


def gpu_benchmark(args):
    import torch
    import efgs
    from efgs import rasterization as R
    l1_loss = l1_loss_fn()

    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    sc, params, settings, target, opt = build_problem(args.config, device)
    empty = torch.empty(0, device=device)

    def render():
        return efgs.diff_rasterize(params['means'], params['scales'], params['rotations'], params['opacities'], empty, settings,
                                   base_colors=params['base_colors'], residual_params=params['residual_params'],
                                   mlp_weights=params.get('mlp_weights'))

    # the headline step: the rasterizer's forward and backward (t_fwd + t_bwd) with a fixed upstream gradient, the L1
    # gradient of the scene's first render
    with torch.no_grad():
        img0 = render()
        upstream = torch.sign(img0 - target) / img0.numel()
        del img0

    def raster_step():
        img = render()
        img.backward(upstream)
        opt.zero_grad(set_to_none=True)
        return R.last_frame_counts['n_visible'], R.last_frame_counts['n_instances']

    # one training iteration: forward, L1 loss, backward, FusedAdam over every parameter group
    def train_step(events):
        events[0].record()
        img = render()
        loss = l1_loss(img, target)
        loss.backward()
        events[1].record()
        opt.step()
        events[2].record()
        opt.zero_grad(set_to_none=True)

    log(f'scene ready: {sc["means"].shape[0]} Gaussians, {sc["camera"]["width"]}x{sc["camera"]["height"]}, {sc["model"]}')
    # clock ramp: the GPU's clocks rise over the first tens of milliseconds of load (the kernels of the first ~40
    # steps run up to 8 % slower), so the step runs untimed for RAMP_S seconds before the warm-up steps
    ramp_steps = 0
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < RAMP_S:
        raster_step()
        ramp_steps += 1
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        raster_step()
    torch.cuda.synchronize()
    log(f'clock ramp ({ramp_steps} untimed steps, {RAMP_S} s) and {args.warmup} warmup steps done')
    # the K timed steps: one pair of HIP events around all of them, device synchronisations on both sides (no
    # event between steps: a pair per step adds ~10 us of GPU time to every step)
    counts = []
    region = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    region[0].record()
    for _ in range(args.steps):
        counts.append(raster_step())
    region[1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    region_ms = region[0].elapsed_time(region[1]) / args.steps
    # the same K steps again, each between its own pair of events (the per-step spread)
    step_events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for k in range(args.steps):
        step_events[k][0].record()
        raster_step()
        step_events[k][1].record()
    torch.cuda.synchronize()
    step_ms = [e[0].elapsed_time(e[1]) for e in step_events]
    log(f'{args.steps} timed forward + backward steps done: {region_ms:.4f} ms/step (events around the {args.steps} steps), wall '
        f'{wall * 1e3 / args.steps:.4f} ms/step; {args.steps} more between per-step events: median {_median(step_ms):.4f} ms')

    # inference renders as the reference's render_image_benchmark calls them: HWC, clamped, no autograd
    render_events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    with torch.inference_mode():
        for k in range(-2, args.steps):
            if k >= 0:
                render_events[k][0].record()
            efgs.rasterize(params['means'], params['scales'], params['rotations'], params['opacities'], settings, False, True,
                           base_colors=params['base_colors'], residual_params=params['residual_params'],
                           mlp_weights=params.get('mlp_weights'))
            if k >= 0:
                render_events[k][1].record()
    torch.cuda.synchronize()
    render_ms = _median([e[0].elapsed_time(e[1]) for e in render_events])
    log(f'{args.steps} inference renders done: median {render_ms:.4f} ms')
    # per-stage breakdown: the same forward + backward steps on the same scene, in a separate pass because the
    # library's stage events add host work to every launch (the timed steps above run without them)
    R._rasterizer.set_stage_timing(True)
    for _ in range(args.steps):
        raster_step()
    stage_times = R._rasterizer.stage_times()
    R._rasterizer.set_stage_timing(False)
    log(f'{args.steps} steps with stage timing done')

    # full training iterations (loss and Adam included), reported beside the headline; they run last because Adam
    # changes the scene
    for _ in range(max(args.warmup, 2)):
        train_step([torch.cuda.Event(enable_timing=True) for _ in range(3)])
    train_events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for k in range(args.steps):
        train_step(train_events[k])
    torch.cuda.synchronize()
    full_ms = [e[0].elapsed_time(e[2]) for e in train_events]
    fwd_loss_bwd_ms = [e[0].elapsed_time(e[1]) for e in train_events]
    adam_ms = [e[1].elapsed_time(e[2]) for e in train_events]
    log(f'{args.steps} training iterations done: median {_median(full_ms):.4f} ms')

    V = sum(c[0] for c in counts) / len(counts)
    I = sum(c[1] for c in counts) / len(counts)
    cam = sc['camera']
    W, H = cam['width'], cam['height']
    N = sc['means'].shape[0]
    T = math.ceil(W / 16) * math.ceil(H / 12)
    app = sc['appearance']
    model = app['model']
    mlp = app.get('mlp')
    if model == 'neural':
        n_in = mlp['n_feature_dims'] + sum(2 * d + 1 for d in mlp['sh_degrees'])
        F = mlp_flops_per_primitive(n_in, mlp['n_neurons'], mlp['n_hidden_layers'])
        R_bytes = residual_bytes(model, mlp['n_feature_dims'])
    else:
        F = 0
        R_bytes = residual_bytes(model, 15 if model == 'sh' else 8)
    adam_elements = sum(p.numel() for p in params.values())
    per_stage = {name: (ms / max(n, 1), n) for name, (ms, n) in stage_times.items() if n > 0}  # per launch
    fused = 'compact' not in per_stage  # (the compaction stage launches nothing when the emission kernel does it)
    per_stage['adam'] = (_median(adam_ms), args.steps)
    stages = {}
    for name, (ms, n) in per_stage.items():
        b, f = algorithmic(name, N, V, I, T, W * H, R_bytes, F, adam_elements, fused)
        entry = {'ms': round(ms, 5), 'launches': n // args.steps if name != 'adam' else 1}
        if b:
            entry['gb_s'] = round(b / (ms * 1e-3) / 1e9, 1)
            entry['hbm_frac'] = round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        if f:
            entry['tflop_s'] = round(f / (ms * 1e-3) / 1e12, 2)
            entry['mfma_frac'] = round(f / (ms * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4)
        stages[name] = entry

    kernel_stages = [s for s in per_stage if s not in ('counter_read', 'adam')]   # the step's kernels (Adam is reported apart)
    dominant = max(kernel_stages, key=lambda s: per_stage[s][0])
    dms = per_stage[dominant][0]
    b, f = algorithmic(dominant, N, V, I, T, W * H, R_bytes, F, adam_elements, fused)
    hbm_frac = b / (dms * 1e-3) / 1e9 / HBM_PEAK_GBS if b else 0.0
    mfma_frac = f / (dms * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS if f else 0.0
    kernel_name = STAGE_KERNELS.get(dominant, dominant).replace('<model>', model)
    if mfma_frac > hbm_frac:
        roofline = {'bound': 'mfma', 'achieved': round(f / (dms * 1e-3) / 1e12, 3), 'peak': MFMA_FP16_PEAK_TFLOPS,
                    'unit': 'TFLOP/s', 'frac': round(mfma_frac, 5)}
    else:
        roofline = {'bound': 'hbm', 'achieved': round(b / (dms * 1e-3) / 1e9, 2), 'peak': HBM_PEAK_GBS,
                    'unit': 'GB/s', 'frac': round(hbm_frac, 5)}
    # (the committed traffic summary covers the c3 step only)
    roofline['traffic'] = read_traffic(kernel_name) if args.config == 'c3' else None
    roofline.update({'kernel': kernel_name, 'stage': dominant, 'avg_launch_ms': round(dms, 5),
                     'algorithmic_bytes': int(b), 'algorithmic_flops': int(f)})
    return dict(W=W, H=H, N=N, V=V, I=I, model=model, step_ms=step_ms, wall_ms_per_step=wall * 1e3 / args.steps, region_ms=region_ms,
                full_step_ms=_median(full_ms), fwd_loss_bwd_ms=_median(fwd_loss_bwd_ms), adam_ms=_median(adam_ms),
                render_ms=render_ms, roofline=roofline, stages=stages, scene=sc)


# ---------------------------------------------------------------------------------------------------------
# CPU baseline: the C / numpy restatement of the same forward + backward (one iteration, host cores)
# ---------------------------------------------------------------------------------------------------------

def cpu_port_rasterizer(sc: dict) -> dict:
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, 'oracle'))
    import oracle as O
    from threadpoolctl import threadpool_limits

    cam0 = sc['camera']
    app = sc['appearance']
    W, H = cam0['width'], cam0['height']
    cam = O.Camera(w2c=cam0['w2c'], position=cam0['position'], width=W, height=H, focal_x=cam0['focal_x'],
                   focal_y=cam0['focal_y'], center_x=cam0['center_x'], center_y=cam0['center_y'], bg=np.zeros(3, np.float32),
                   degree=app['max_degree'] if app['model'] != 'neural' else 1, near_plane=cam0['near_plane'],
                   far_plane=cam0['far_plane'])
    mlp = O.MLPConfig(**app['mlp']) if app.get('mlp') else None
    scene = O.Scene(means=sc['means'], scales=sc['scales'], rotations=sc['rotations'], opacities=sc['opacities'],
                    base_colors=sc['base_colors'], residual_params=sc['residual_params'], mlp_weights=sc['mlp_weights'])
    oapp = O.Appearance(model=app['model'], base_act=app['base_act'], res_act=app['res_act'], color_act=app['color_act'],
                        direction_gradient=app['direction_gradient'], max_degree=app['max_degree'], mlp=mlp)
    O.build()
    log('cpu baseline: one forward + backward through the CPU restatement')
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        fw = O.render(scene, oapp, cam)
        grad = np.full(fw.image.shape, 1.0 / fw.image.size, np.float32)
        O.backward(scene, oapp, cam, fw, grad)
        seconds = time.perf_counter() - t0
    return {'value': round(W * H / seconds / 1e6, 5), 'unit': 'Mpix/s', 'cores': 1, 'kind': 'port',
            'sample': f'one forward + backward of the full {sc["model"]} scene ({sc["means"].shape[0]} Gaussians, {W}x{H}) '
                      f'through the C/numpy CPU restatement, single thread, no Adam; {seconds:.1f} s'}


def cpu_model() -> str:
    """The host CPU's model name as lscpu reports it (falls back to /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith('model name'):
                return line.split(':', 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_unfused_baseline(sc: dict | None, warmup: int = 3, reps: int = 20) -> dict:
    """The reference's unfused PyTorch appearance evaluation (USE_FUSED_APPEARANCE false: AppearanceModel.forward,
    Appearance/Base.py:83-108 with the per-model residual_colors) on every torch thread of the host, as its
    restatement in oracle/torch_ref.py. BASELINE configuration c0 (10k Gaussians, SH degree 3, colour
    sigmoid(4 (base + residual(dir)))): forward, and forward + backward (autograd with respect to the means, base
    colours and SH coefficients), warm-up `warmup`, median of `reps`. With a neural scene `sc`, also the c3 scene's
    neural appearance forward + backward (1M Gaussians, MLP with fp16-rounded weights; one warm-up, median of 3)."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, 'oracle'))
    import oracle as O
    import torch_ref as TR
    from efgs.synthetic import c0_inputs

    threads = torch.get_num_threads()
    c0 = c0_inputs()
    n0 = c0['means'].shape[0]
    a = c0['appearance']
    app0 = O.Appearance(model='sh', base_act=a['base_act'], res_act=a['res_act'], color_act=a['color_act'], direction_gradient=True,
                        max_degree=3)
    cam0 = torch.tensor(c0['cam_position'])

    def leaves(grad):
        return [torch.tensor(c0[k]).requires_grad_(grad) for k in ('means', 'base_colors', 'residual_params')]

    def timed(fn, grad):
        out = []
        for i in range(warmup + reps):
            m, b, r = leaves(grad)
            t0 = time.perf_counter()
            fn(m, b, r)
            if i >= warmup:
                out.append(time.perf_counter() - t0)
        return _median(out)

    def forward(m, b, r):
        with torch.no_grad():
            TR.appearance_colors(m, cam0, b, r, app0, 3)

    def forward_backward(m, b, r):
        TR.appearance_colors(m, cam0, b, r, app0, 3).sum().backward()

    fwd_s = timed(forward, False)
    fb_s = timed(forward_backward, True)
    model = cpu_model()
    out = {'value': round(n0 / fb_s / 1e6, 4), 'unit': 'Mprim/s', 'cores': threads, 'kind': 'port',
           'sample': f'c0: {n0} Gaussians, SH degree 3 (48 coefficients), colour sigmoid(4x), forward + backward (autograd '
                     f'w.r.t. means, base colours, SH coefficients) of the unfused appearance (torch restatement of '
                     f'Appearance/Base.py:83-108 and SH.py:34-56) on {threads} torch threads, warm-up {warmup}, median of {reps}',
           'cpu_model': model,
           'c0_forward': {'value': round(n0 / fwd_s / 1e6, 4), 'unit': 'Mprim/s', 'ms': round(fwd_s * 1e3, 4)},
           'c0_forward_backward': {'value': round(n0 / fb_s / 1e6, 4), 'unit': 'Mprim/s', 'ms': round(fb_s * 1e3, 4)}}
    if sc is not None and sc['appearance']['model'] == 'neural':
        app = sc['appearance']
        mlp = O.MLPConfig(**app['mlp'])
        oapp = O.Appearance(model='neural', base_act=app['base_act'], res_act=app['res_act'], color_act=app['color_act'],
                            direction_gradient=app['direction_gradient'], max_degree=app['max_degree'], mlp=mlp)
        cam = torch.tensor(sc['camera']['position'])
        times = []
        for i in range(4):
            m = torch.tensor(sc['means'])
            b = torch.tensor(sc['base_colors']).requires_grad_(True)
            r = torch.tensor(sc['residual_params']).requires_grad_(True)
            w = torch.tensor(sc['mlp_weights']).requires_grad_(True)
            t0 = time.perf_counter()
            TR.appearance_colors(m, cam, b, r, oapp, 1, mats=TR.mlp_matrices_torch(w, mlp)).sum().backward()
            if i:
                times.append(time.perf_counter() - t0)
        c3_s = _median(times)
        n3 = sc['means'].shape[0]
        out['c3_neural_forward_backward'] = {
            'value': round(n3 / c3_s / 1e6, 4), 'unit': 'Mprim/s', 'ms': round(c3_s * 1e3, 2),
            'sample': f'{n3} Gaussians of the c3 scene, neural appearance (MLP 11-64-64-3), forward + backward, median of 3'}
    return out


# ---------------------------------------------------------------------------------------------------------
# c2: the neural decode in isolation
# ---------------------------------------------------------------------------------------------------------

def c2_inputs(n: int = 1_000_000, seed: int = 0):
    """Configuration c2: latents N(0, 0.1) (n, 8), directions normalize(N(0, 1)^3), the 11 -> 64 -> 64 -> 3
    Xavier fp16 MLP (tcnn flat layout), upstream gradients N(0, 1) (n, 3); draw order as listed."""
    import numpy as np
    from efgs.synthetic import NEURAL_MLP, xavier_mlp
    rng = np.random.default_rng(seed)
    m = NEURAL_MLP
    n_in = m['n_feature_dims'] + sum(2 * d + 1 for d in m['sh_degrees'])
    feat = rng.normal(0.0, 0.1, size=(n, m['n_feature_dims'])).astype(np.float32)
    d = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    d /= np.maximum(np.linalg.norm(d, axis=1, keepdims=True), 1e-12)
    w = xavier_mlp(rng, n_in, m['n_neurons'], m['n_hidden_layers'])
    dy = rng.normal(0.0, 1.0, size=(n, 3)).astype(np.float32)
    return m, n_in, feat, d.astype(np.float32), w, dy


def decode_benchmark(args) -> None:
    import numpy as np
    import torch
    import efgs
    from efgs.rasterization import neural_decode
    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    m, n_in, feat, d, w, dy = c2_inputs()
    n = feat.shape[0]
    efgs.initialize_appearance('neural', 0, 'none', 'none', 'relu', True)
    efgs.initialize_residual_mlp(n_in, 3, {'otype': 'Identity'},
                                 {'otype': 'FullyFusedMLP', 'activation': 'ReLU', 'output_activation': 'None',
                                  'n_neurons': m['n_neurons'], 'n_hidden_layers': m['n_hidden_layers']},
                                 m['base_input'], m['n_frequencies'], list(m['sh_degrees']))
    tf = torch.tensor(feat, device=device, requires_grad=True)
    td = torch.tensor(d, device=device, requires_grad=True)
    tw = torch.tensor(w, device=device, requires_grad=True)
    tdy = torch.tensor(dy, device=device)

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        out = neural_decode(tf, td, tw, 1)
        if ev is not None:
            ev[1].record()
        out.backward(tdy)
        if ev is not None:
            ev[2].record()
        tf.grad = td.grad = tw.grad = None

    log(f'c2: {n} primitives, MLP {n_in} -> {m["n_neurons"]} x {m["n_hidden_layers"]} -> 3')
    # eager (autograd) steps: the host's launch and autograd work per step (0.1-0.18 ms on these boxes' cores) is
    # as long as the step's kernels, so the eager figure follows the host; it is reported beside the value
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < RAMP_S:
        step()
    for _ in range(args.warmup):
        step()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(events[k])
    torch.cuda.synchronize()
    eager_wall = time.perf_counter() - t0
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in events) / args.steps
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in events) / args.steps
    # the same step (neural_decode and autograd's backward) captured once as a HIP graph and replayed: the step's
    # kernels without the host's per-launch work; the K replays are timed between one pair of events
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = neural_decode(tf, td, tw, 1)
        out.backward(tdy)
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < RAMP_S:
        graph.replay()
    for _ in range(args.warmup):
        graph.replay()
    region = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    region[0].record()
    for _ in range(args.steps):
        graph.replay()
    region[1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = region[0].elapsed_time(region[1]) / args.steps
    F = mlp_flops_per_primitive(n_in, m['n_neurons'], m['n_hidden_layers'])
    flops = 3 * F * n                    # forward + backward (input and weight gradients)
    lat = 4 * m['n_feature_dims']
    # forward: latents + directions in, outputs out; backward: latents + directions + upstream in, latent and
    # direction gradients out (156 B per primitive at c2)
    nbytes = n * ((lat + 12 + 12) + (lat + 12 + 12 + lat + 12))
    line = {
        'metric': 'neural decode fwd+bwd Mprim/s @1M (c2)', 'value': round(n / (ms * 1e-3) / 1e6, 3), 'unit': 'Mprim/s',
        'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(wall * 1e3 / args.steps, 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f16 MFMA, f32 accumulation', 'data': 'synthetic',
        'config': {'workload': f'c2: neural decode of {n} primitives ({n_in} -> {m["n_neurons"]} x {m["n_hidden_layers"]} -> 3), '
                               'forward + backward w.r.t. latents, directions and weights', 'n_primitives': n},
        'timing': (f'HIP events around {args.steps} replays of the step captured as one HIP graph (device synchronisations on '
                   f'both sides), after a {RAMP_S} s untimed ramp of replays and {args.warmup} warm-up replays'),
        'eager_ms_per_step': round(eager_wall * 1e3 / args.steps, 4),
        'eager_forward_ms': round(fwd_ms, 5), 'eager_backward_ms': round(bwd_ms, 5),
        'roofline': {'bound': 'mfma', 'achieved': round(flops / (ms * 1e-3) / 1e12, 3), 'peak': MFMA_FP16_PEAK_TFLOPS,
                     'unit': 'TFLOP/s', 'frac': round(flops / (ms * 1e-3) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 5), 'traffic': None,
                     'kernel': 'neural_decode + neural_decode_backward', 'algorithmic_flops': int(flops),
                     'algorithmic_bytes': int(nbytes), 'hbm_gb_s': round(nbytes / (ms * 1e-3) / 1e9, 1)},
        'cpu_baseline': None if args.no_cpu_baseline else decode_cpu_baseline(m, feat, d, w, dy),
    }
    print(json.dumps(line), flush=True)


def decode_cpu_baseline(m, feat, d, w, dy) -> dict:
    """The numpy statement of the decode (oracle.neural_decode + its backward) on a 100k-primitive sample."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, 'oracle'))
    import oracle as O
    from threadpoolctl import threadpool_limits
    k = 100_000
    mlp = O.MLPConfig(**m)
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        y, acts, mats = O.neural_decode(feat[:k], None, d[:k], w, mlp, 1)
        O.neural_decode_backward(feat[:k], None, d[:k], dy[:k], mats, acts, mlp, 1)
        seconds = time.perf_counter() - t0
    return {'value': round(k / seconds / 1e6, 5), 'unit': 'Mprim/s', 'cores': 1, 'kind': 'port',
            'sample': f'forward + backward of the first {k} c2 primitives through the numpy statement (oracle), one thread; '
                      f'{seconds:.1f} s'}


# ---------------------------------------------------------------------------------------------------------
# mcmc: the densification operators on the c3 scene
# ---------------------------------------------------------------------------------------------------------

def mcmc_benchmark(args) -> None:
    """add_noise over all c3 Gaussians (every step of an MCMC schedule) and relocation_adjustment of all of them
    with 1..5 samples each; HIP events on the launch stream."""
    import numpy as np
    import torch
    import efgs
    from efgs.synthetic import make_scene
    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    torch.cuda.manual_seed(0)
    sc = make_scene('c3')
    n = sc['means'].shape[0]
    scales = torch.tensor(sc['scales'], device=device)
    rotations = torch.tensor(sc['rotations'], device=device)
    opacities = torch.tensor(sc['opacities'], device=device)
    means = torch.tensor(sc['means'], device=device)
    act_o = torch.sigmoid(opacities)
    act_s = torch.exp(scales)
    counts = torch.tensor(np.random.default_rng(0).integers(1, 6, n), dtype=torch.int64, device=device)
    lr = 5e5 * 1.6e-4 * 0.01

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
        for k in range(args.steps):
            ev[k][0].record()
            fn()
            ev[k][1].record()
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in ev) / args.steps

    log(f'mcmc: {n} Gaussians (c3 scene)')
    noise_ms = timed(lambda: efgs.add_noise(scales, rotations, opacities, means, lr))
    reloc_ms = timed(lambda: efgs.relocation_adjustment(act_o, act_s, counts))
    noise_bytes = n * (12 + 16 + 4 + 12 + 12)    # log-scales, quaternion, opacity, mean in; mean out
    reloc_bytes = n * (4 + 12 + 8 + 4 + 12)      # opacity, scales, count in; opacity, scales out
    line = {
        'metric': 'MCMC add_noise Mprim/s @1M Gaussians (c3 scene)', 'value': round(n / (noise_ms * 1e-3) / 1e6, 3), 'unit': 'Mprim/s',
        'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(noise_ms, 5), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32 (Philox4x32-10 u32)', 'data': 'synthetic',
        'config': {'workload': f'mcmc: add_noise and relocation_adjustment (1..5 samples) of the {n} c3 Gaussians', 'n_primitives': n},
        'add_noise_ms': round(noise_ms, 5), 'relocation_ms': round(reloc_ms, 5),
        'relocation_mprim_s': round(n / (reloc_ms * 1e-3) / 1e6, 3),
        'roofline': {'bound': 'hbm', 'achieved': round(noise_bytes / (noise_ms * 1e-3) / 1e9, 2), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(noise_bytes / (noise_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5), 'traffic': None, 'kernel': 'add_noise_kernel',
                     'algorithmic_bytes': int(noise_bytes),
                     'relocation': {'achieved': round(reloc_bytes / (reloc_ms * 1e-3) / 1e9, 2), 'unit': 'GB/s',
                                    'frac': round(reloc_bytes / (reloc_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
                                    'algorithmic_bytes': int(reloc_bytes)}},
        'cpu_baseline': None,
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, 'oracle'))
        import oracle as O
        O.build()
        t0 = time.perf_counter()
        O.add_noise(sc['scales'], sc['rotations'], sc['opacities'].reshape(-1), sc['means'], lr, 1, 0)
        seconds = time.perf_counter() - t0
        line['cpu_baseline'] = {'value': round(n / seconds / 1e6, 5), 'unit': 'Mprim/s', 'cores': 1, 'kind': 'port',
                                'sample': f'add_noise of all {n} Gaussians through the C restatement (oracle), one thread; '
                                          f'{seconds:.2f} s'}
    print(json.dumps(line), flush=True)


# ---------------------------------------------------------------------------------------------------------
# pruning: Speedy-Splat scores of one c3 view
# ---------------------------------------------------------------------------------------------------------

def pruning_benchmark(args) -> None:
    """update_pruning_scores over the c3 scene's view (forward pipeline + score pass), HIP events per call."""
    import torch
    import efgs
    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    sc, params, settings, _, _ = build_problem('c3', device)
    n = sc['means'].shape[0]
    W, H = sc['camera']['width'], sc['camera']['height']
    scores = torch.zeros(n, dtype=torch.float32, device=device)

    def call():
        efgs.update_pruning_scores(scores, params['means'], params['scales'], params['rotations'], params['opacities'], settings,
                                   base_colors=params['base_colors'], residual_params=params['residual_params'],
                                   mlp_weights=params.get('mlp_weights'))

    log(f'pruning: {n} Gaussians, {W}x{H}')
    with torch.no_grad():
        for _ in range(args.warmup):
            call()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
        for k in range(args.steps):
            ev[k][0].record()
            call()
            ev[k][1].record()
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b) for a, b in ev) / args.steps
    line = {
        'metric': 'Speedy-Splat pruning scores Mpix/s @1M Gaussians 1080p (Neural)', 'value': round(W * H / (ms * 1e-3) / 1e6, 3),
        'unit': 'Mpix/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 5), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32 (f16 MFMA MLP)', 'data': 'synthetic',
        'config': {'workload': f'pruning: update_pruning_scores of one view of the c3 scene ({n} Gaussians, {W}x{H}, neural): '
                               'forward pipeline + score pass', 'n_gaussians': n, 'width': W, 'height': H},
        'roofline': None, 'cpu_baseline': None,
    }
    print(json.dumps(line), flush=True)


# ---------------------------------------------------------------------------------------------------------
# .ngsplat export: device packing of a 1M-splat model
# ---------------------------------------------------------------------------------------------------------

def ngsplat_benchmark(args) -> None:
    """efgs_ngsplat_pack over a 1M-splat model in the viewer's default neural configuration (8 features, sin / cos
    encoding, degrees 0..3, 16 neurons: baked layer 0) and in SH degree 3; HIP events around each call on its
    stream (a call is the statistics, combine and pack kernels plus its blocking 32-byte statistics read)."""
    import numpy as np
    import torch
    from efgs import ngsplat as NG
    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    from efgs.synthetic import ngsplat_model as make_case
    n = 1_000_000
    results = {}
    for name in ('baked', 'sh3'):
        m, plan, _ = make_case(name, n=n, seed=9)
        t = {k: torch.tensor(v, device=device) for k, v in m.items()}

        def call(timing=False):
            return NG.pack_textures(t['means'], t['raw_scales'], t['raw_rotations'], t['raw_opacities'], t['base_colors'],
                                    t['residual_params'], plan, timing=timing)
        for _ in range(args.warmup):
            out = call()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
        for k in range(args.steps):
            ev[k][0].record()
            out = call()
            ev[k][1].record()
        torch.cuda.synchronize()
        ms = sum(a.elapsed_time(b) for a, b in ev) / args.steps
        # the kernels alone: HIP events recorded by the library around them, on the launch stream
        kms = [call(timing=True)['kernel_ms'] for _ in range(args.steps)]
        stats_ms = sum(k[0] for k in kms) / len(kms)
        pack_ms = sum(k[1] for k in kms) / len(kms)
        kept = out['n_kept']
        row = m['residual_params'].reshape(n, -1).shape[1] if name == 'sh3' else plan['n_items']
        out_payload = sum(x.shape[1] * 4 for x in out['textures'])
        # compulsory: every input row read once (mean, log-scales, quaternion, opacity, base, the payload's residual
        # parameters), every kept row written once (splat words, payload texels, source index)
        nbytes = n * (12 + 12 + 16 + 4 + 12 + 4 * row) + kept * (16 + out_payload + 4)
        results[name] = dict(ms=ms, kept=kept, bytes=nbytes, m=m, plan=plan, stats_ms=stats_ms, pack_ms=pack_ms)
        log(f'ngsplat {name}: {n} splats, kept {kept}, call {ms:.4f} ms, kernels {stats_ms:.4f} + {pack_ms:.4f} ms')
    r = results['baked']
    line = {
        'metric': '.ngsplat export packing Msplat/s @1M Gaussians (neural, baked layer 0)', 'value': round(n / (r['ms'] * 1e-3) / 1e6, 3),
        'unit': 'Msplat/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(r['ms'], 5),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32 -> u8 / f16 codes', 'data': 'synthetic',
        'config': {'workload': f'ngsplat: cull, quantise and pack {n} splats (viewer default neural model: 8 features, sin/cos, '
                               f'degrees 0-3, 16 neurons) and the same model with SH degree 3', 'n_splats': n},
        'call_note': 'value and ms_per_step time the whole efgs_ngsplat_pack call from Python (ctypes, output allocation, '
                     'three kernels, the blocking statistics read); the roofline times the kernels alone',
        'kernel_ms': {'stats_combine': round(r['stats_ms'], 5), 'pack': round(r['pack_ms'], 5)},
        'sh3_ms': round(results['sh3']['ms'], 5), 'sh3_msplat_s': round(n / (results['sh3']['ms'] * 1e-3) / 1e6, 3),
        'sh3_kernel_ms': {'stats_combine': round(results['sh3']['stats_ms'], 5), 'pack': round(results['sh3']['pack_ms'], 5)},
        'roofline': {'bound': 'hbm', 'achieved': round(r['bytes'] / ((r['stats_ms'] + r['pack_ms']) * 1e-3) / 1e9, 2), 'peak': HBM_PEAK_GBS,
                     'unit': 'GB/s', 'frac': round(r['bytes'] / ((r['stats_ms'] + r['pack_ms']) * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
                     'traffic': None, 'kernel': 'ngsplat_stats_kernel + ngsplat_combine_kernel + ngsplat_pack_kernel (HIP events)',
                     'algorithmic_bytes': int(r['bytes']),
                     'sh3': {'achieved': round(results['sh3']['bytes'] / ((results['sh3']['stats_ms'] + results['sh3']['pack_ms']) * 1e-3) / 1e9, 2),
                             'unit': 'GB/s', 'algorithmic_bytes': int(results['sh3']['bytes']),
                             'frac': round(results['sh3']['bytes'] / ((results['sh3']['stats_ms'] + results['sh3']['pack_ms']) * 1e-3) / 1e9
                                           / HBM_PEAK_GBS, 5)}},
        'cpu_baseline': None,
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, 'oracle'))
        import ngsplat_oracle as ON
        mm, plan = r['m'], r['plan']
        t0 = time.perf_counter()
        ON.export(mm['means'], mm['raw_scales'], mm['raw_rotations'], mm['raw_opacities'], mm['base_colors'], mm['residual_params'], plan)
        seconds = time.perf_counter() - t0
        line['cpu_baseline'] = {'value': round(n / seconds / 1e6, 5), 'unit': 'Msplat/s', 'cores': 1, 'kind': 'port',
                                'sample': f'the numpy restatement of the exporter (oracle/ngsplat_oracle.py) on the same {n}-splat '
                                          f'neural model; {seconds:.2f} s'}
    print(json.dumps(line), flush=True)


def copy_calibration() -> None:
    """A plain device copy of 1 GiB, five times: rocprofv3 FETCH_SIZE / WRITE_SIZE of this command read
    1 GiB each per dispatch when the counters are exact."""
    import torch
    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device='cuda:0')
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_bytes': 4 * n, 'dispatches': 5}))


def main() -> None:
    args = parse_args()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(f'bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); '
              'the rasterizer has no multi-GPU path', file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit('bench.py: --steps must be >= 1 and --warmup >= 0')
    if args.config == 'c2':
        decode_benchmark(args)
        return
    if args.config == 'mcmc':
        mcmc_benchmark(args)
        return
    if args.config == 'pruning':
        pruning_benchmark(args)
        return
    if args.config == 'ngsplat':
        ngsplat_benchmark(args)
        return
    r = gpu_benchmark(args)
    cpu = port = None
    if not args.no_cpu_baseline:
        log('cpu baseline: the unfused appearance on the host threads')
        cpu = cpu_unfused_baseline(r['scene'])
        port = cpu_port_rasterizer(r['scene'])
    print(json.dumps(headline_line(args, r, cpu, port)), flush=True)


def headline_line(args, r: dict, cpu: dict | None, port: dict | None) -> dict:
    """The bench's JSON line. `value` = W * H / t, t = the HIP-event time of the K timed steps (one pair of events
    around all of them, device synchronisations on both sides) divided by K: the rasterizer's forward and backward,
    BASELINE.md's headline; `ms_per_step` = t; `wall_ms_per_step` = host wall time of the same K steps divided by K;
    `step_ms_quartiles` = the spread of K more steps, each between its own pair of events (which adds ~10 us per
    step); `gpu_idle_us_per_step` = t minus the kernel time of one steady-state step of the committed kernel trace of
    this command (no kernel running on the GPU)."""
    W, H = r['W'], r['H']
    ms = r['region_ms']
    # the committed kernel trace and BASELINE's metric name are the c3 step's
    kernel_us = read_step_kernel_us() if args.config == 'c3' else None
    return {
        'metric': ('fwd+bwd Mpix/s @1M Gaussians 1080p (Neural); % HBM/MFMA roofline per kernel' if args.config == 'c3'
                   else f'fwd+bwd Mpix/s ({args.config})'),
        'value': round(W * H / (ms * 1e-3) / 1e6, 3),
        'unit': 'Mpix/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32 (f16 MFMA MLP)' if r['model'] == 'neural' else 'f32',
        'data': 'synthetic',
        'config': {'workload': f'{args.config}: rasterizer forward + backward (t_fwd + t_bwd: preprocess through blend, blend '
                               f'backward, preprocess backward; upstream L1 gradient fixed) of {r["N"]} Gaussians, {W}x{H}, '
                               f'{r["model"]} appearance',
                   'n_gaussians': r['N'], 'width': W, 'height': H, 'appearance': r['model'],
                   'visible': round(r['V']), 'instances': round(r['I'])},
        'timing': (f'HIP events around the {args.steps} timed steps (device synchronisations on both sides), after a {RAMP_S} s '
                   f'untimed clock ramp of the same step and {args.warmup} warm-up steps'),
        'wall_ms_per_step': round(r['wall_ms_per_step'], 4),
        'step_ms_quartiles': [round(q, 4) for q in _quartiles(r['step_ms'])],
        'step_kernels_us_rocprof': kernel_us,
        'gpu_idle_us_per_step': round(ms * 1e3 - kernel_us, 1) if kernel_us is not None else None,
        'full_step_ms': round(r['full_step_ms'], 4),
        'full_step_mpix_s': round(W * H / (r['full_step_ms'] * 1e-3) / 1e6, 3),
        'fwd_loss_bwd_ms': round(r['fwd_loss_bwd_ms'], 4),
        'adam_ms': round(r['adam_ms'], 4),
        'inference_ms': round(r['render_ms'], 4),
        'inference_fps': round(1e3 / r['render_ms'], 1),
        'roofline': r['roofline'],
        'stages': r['stages'],
        'cpu_baseline': cpu,
        'cpu_port_rasterizer': port,
    }


if __name__ == '__main__':
    main()
