"""The C ABI without a GPU: libefgs_hip.so loads, exports every function include/efgs.h declares, and its host-side
validation rejects bad configurations and calls before touching a device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, 'include', 'efgs.h')).read()
    return sorted(set(re.findall(r'\b(efgs_[a-z_]+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    from efgs import _lib
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(_lib.lib, name), name
    assert set(names) == set(_lib.EXPORTED)


def test_struct_sizes_match_header_layout():
    from efgs import _lib
    p = ctypes.sizeof(ctypes.c_void_p)
    assert ctypes.sizeof(_lib.Settings) == 3 * p + 3 * 4 + 6 * 4 + 3 * 4
    assert ctypes.sizeof(_lib.Primitives) == 8 + 8 * p
    assert ctypes.sizeof(_lib.Frame) == 3 * p + 4 * 8 + 4 * 4
    assert ctypes.sizeof(_lib.AdamGroup) == 4 * p + 8 + 8 + 4 + 4 + 7 * 8 + 3 * 8
    assert ctypes.sizeof(_lib.FrameViews) == 13 * p


def test_invalid_ids_raise():
    from efgs import _lib
    from efgs import rasterization as R
    r = R.Rasterizer()
    with pytest.raises(RuntimeError, match='invalid appearance model'):
        r.set_appearance(9, 3, 0, 0, 1, True)
    with pytest.raises(RuntimeError, match='invalid color activation'):
        r.set_appearance(1, 3, 0, 0, 6, True)
    with pytest.raises(RuntimeError, match='invalid residual activation'):
        r.set_appearance(1, 3, 0, 3, 1, True)
    with pytest.raises(KeyError):
        R.initialize_appearance('spherical', 3, 'none', 'none', 'relu', True)


def test_residual_mlp_requires_neural_model():
    from efgs import _lib
    from efgs import rasterization as R
    r = R.Rasterizer()
    with pytest.raises(RuntimeError, match='neural appearance model before set_residual_mlp'):
        r.set_residual_mlp(11, 3, 64, 2, 1, False, 0, 0b10)
    r.set_appearance(5, 0, 0, 1, 1, True)
    with pytest.raises(RuntimeError, match='n_neurons'):
        r.set_residual_mlp(11, 3, 48, 2, 1, False, 0, 0b10)
    r.set_residual_mlp(11, 3, 64, 2, 1, False, 0, 0b10)
    assert r.mlp_param_count() == 64 * 16 + 64 * 64 + 16 * 64


def test_forward_without_appearance_is_rejected_before_device_work():
    """Regression: an unconfigured rasterizer must not fall back to the precomputed-colour variant."""
    from efgs import _lib
    from efgs import _lib
    from efgs import rasterization as R
    r = R.Rasterizer()
    prims = _lib.Primitives()
    prims.n_primitives = 4
    prims.means = prims.scales = prims.rotations = prims.opacities = 0x1000  # never dereferenced
    s = _lib.Settings()
    s.w2c = s.cam_position = s.bg_color = 0x1000
    s.width, s.height = 32, 24
    frame = _lib.Frame()
    alloc = _lib.ALLOC_FN(lambda ctx, n: 0)
    rc = _lib.lib.efgs_forward(r.handle, ctypes.byref(prims), ctypes.byref(s), 0x1000, alloc, None, ctypes.byref(frame), None)
    assert rc == 2
    assert b'not initialized' in _lib.lib.efgs_last_error()


def test_precomputed_variant_requires_colours():
    from efgs import _lib
    from efgs import _lib
    from efgs import rasterization as R
    r = R.Rasterizer()
    r.set_appearance(1, 3, 0, 0, 1, True)
    prims = _lib.Primitives()
    prims.n_primitives = 4
    prims.means = prims.scales = prims.rotations = prims.opacities = 0x1000
    s = _lib.Settings()
    s.w2c = s.cam_position = s.bg_color = 0x1000
    s.width, s.height = 32, 24
    frame = _lib.Frame()
    alloc = _lib.ALLOC_FN(lambda ctx, n: 0)
    rc = _lib.lib.efgs_forward(r.handle, ctypes.byref(prims), ctypes.byref(s), 0x1000, alloc, None, ctypes.byref(frame), None)
    assert rc == 1 and b'base_colors are required' in _lib.lib.efgs_last_error()


def test_adam_validation():
    from efgs import _lib
    g = _lib.AdamGroup()
    g.n_lrs = 8
    g.step = 1
    assert _lib.lib.efgs_adam_step(ctypes.byref(g), 1, None) == 1
    assert b'learning rates' in _lib.lib.efgs_last_error()
    g.n_lrs = 1
    g.step = 0
    assert _lib.lib.efgs_adam_step(ctypes.byref(g), 1, None) == 1


def test_densification_validation():
    """Argument checks of the MCMC entry points happen before any device work: negative counts, null tensors
    and a Philox offset that is not a multiple of 4 are rejected; empty inputs are accepted."""
    from efgs import _lib
    lib = _lib.lib
    fake = ctypes.c_void_p(0x1000)
    assert lib.efgs_add_noise(-1, fake, fake, fake, fake, 0.1, 1, 0, None) == 1
    assert lib.efgs_add_noise(10, None, fake, fake, fake, 0.1, 1, 0, None) == 1
    assert lib.efgs_add_noise(10, fake, fake, fake, fake, 0.1, 1, 2, None) == 1
    assert b'multiple of 4' in lib.efgs_last_error()
    assert lib.efgs_add_noise(0, None, None, None, None, 0.1, 1, 0, None) == 0
    assert lib.efgs_relocation_adjustment(-1, fake, fake, fake, fake, fake, None) == 1
    assert lib.efgs_relocation_adjustment(5, fake, fake, None, fake, fake, None) == 1
    assert lib.efgs_relocation_adjustment(0, None, None, None, None, None, None) == 0


def test_stage_timing_without_launches():
    """Timing can be enabled and read back without any GPU work: every stage reports zero launches."""
    from efgs import _lib
    from efgs import rasterization as R
    r = R.Rasterizer()
    r.set_stage_timing(True)
    times = r.stage_times()
    assert set(times) == set(_lib.STAGES) and len(_lib.STAGES) == 12
    assert all(ms == 0.0 and n == 0 for ms, n in times.values())
    r.set_stage_timing(False)


def test_bench_algorithmic_bytes_match_the_c3_budget():
    """The per-stage algorithmic byte formulas add up to the C3 forward + backward budget (670 MB at
    V = 699,021 and I = 1,420,415; SURVEY's 675 MB also counts the reference's stored MLP outputs)."""
    import sys
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench
    N, V, I, T, P = 1_000_000, 699_021, 1_420_415, 10_800, 1920 * 1080
    F = bench.mlp_flops_per_primitive(11, 64, 2)
    assert F == 9_984
    stages = ['preprocess_forward', 'create_instances', 'tile_offsets', 'tile_buckets', 'tile_sort', 'blend_forward',
              'blend_backward', 'preprocess_backward', 'mlp_backward']
    # the compaction fused into the emission kernel (no compaction stage) or a stage of its own: the same budget
    fused = sum(bench.algorithmic(s, N, V, I, T, P, 32, F, 0, True)[0] for s in stages)
    split = sum(bench.algorithmic(s, N, V, I, T, P, 32, F, 0, False)[0] for s in stages + ['compact'])
    assert abs(fused / 1e6 - 670.0) < 1.0 and fused == split
    assert bench.algorithmic('adam', N, V, I, T, P, 32, F, 22_006_144)[0] == 28 * 22_006_144


def test_workspace_allocator_bumps_aligns_and_falls_back():
    """efgs_workspace_alloc hands out 256-byte-aligned slices of the region in order, sends what does not fit to
    the fallback and counts every request (host-only: no memory is touched)."""
    from efgs import _lib
    calls = []

    def fallback(_ctx, nbytes):
        calls.append(nbytes)
        return 0x900000

    fb = _lib.ALLOC_FN(fallback)
    ws = _lib.Workspace(0x100000, 1100, 0, 0, ctypes.cast(fb, ctypes.c_void_p), None)
    p1 = _lib.lib.efgs_workspace_alloc(ctypes.byref(ws), 10)
    p2 = _lib.lib.efgs_workspace_alloc(ctypes.byref(ws), 300)
    p3 = _lib.lib.efgs_workspace_alloc(ctypes.byref(ws), 600)   # 768 aligned: does not fit after 768 used of 1100
    p4 = _lib.lib.efgs_workspace_alloc(ctypes.byref(ws), 100)   # still fits after p2
    assert (p1, p2, p3, p4) == (0x100000, 0x100100, 0x900000, 0x100300)
    assert calls == [600] and ws.used == 1024
    assert ws.requested == 256 + 512 + 768 + 256
    empty = _lib.Workspace(None, 0, 0, 0, None, None)
    assert _lib.lib.efgs_workspace_alloc(ctypes.byref(empty), 8) is None


def test_ngsplat_layout_validation():
    """efgs_ngsplat_layout plans the payload textures and rejects layouts the pack kernel cannot stage (host-side
    checks: no GPU work)."""
    import ctypes
    from efgs import _lib
    inp = _lib.NgsplatInput()
    n_tex, words = ctypes.c_int(), (ctypes.c_int * 8)()

    def plan(**kw):
        for k, v in kw.items():
            setattr(inp, k, v)
        rc = _lib.lib.efgs_ngsplat_layout(ctypes.byref(inp), ctypes.byref(n_tex), words)
        return rc, n_tex.value, list(words)[:n_tex.value]
    assert plan(payload=2, n_items=15, residual_row_stride=45) == (0, 3, [2, 4, 4])   # SH degree 3: 7 / 8 / 6-bit levels
    assert plan(payload=2, n_items=8, residual_row_stride=45) == (0, 2, [2, 4])
    assert plan(payload=2, n_items=0, residual_row_stride=45) == (0, 0, [])
    assert plan(payload=3, n_items=7, residual_row_stride=49)[:2] == (0, 7)          # SV: 49 fp16 values -> 7 textures
    assert plan(payload=4, n_items=5, residual_row_stride=40)[:2] == (0, 8)          # NASG: 60 values
    assert plan(payload=1, n_items=8, n_frequencies=1, n_neurons=16, residual_row_stride=8)[:2] == (0, 2)
    for bad in (dict(payload=2, n_items=5, residual_row_stride=45),                   # incomplete SH degree
                dict(payload=4, n_items=6, residual_row_stride=48),                   # 72 values > 64
                dict(payload=0, n_items=20, n_frequencies=0, residual_row_stride=20), # stored features > 16
                dict(payload=1, n_items=8, n_frequencies=1, n_neurons=20, residual_row_stride=8),
                dict(payload=3, n_items=7, residual_row_stride=10),                   # stride below the parameters read
                dict(payload=1, n_items=63, n_frequencies=2, n_neurons=16, residual_row_stride=63),  # > 64 KB of LDS
                dict(payload=9, n_items=1, residual_row_stride=1)):
        inp.payload, inp.n_items, inp.n_frequencies, inp.n_neurons, inp.residual_row_stride = 0, 0, 0, 0, 0
        rc, _, _ = plan(**bad)
        assert rc == 1, bad


def test_bench_stage_kernels_exist():
    """Every kernel the bench names for a stage is a kernel of the library's sources (or a hipRTC preprocess kernel)."""
    import glob
    import sys
    sys.path.insert(0, ROOT)
    import bench
    src = ''.join(open(f).read() for f in glob.glob(os.path.join(ROOT, 'efficient-gaussian-appearance_amd', 'csrc', '**', '*.hip'),
                                                      recursive=True))
    kernels = set(re.findall(r'__global__[^;{]*?\bvoid\s+(\w+)\s*\(', src))
    assert 'blend_backward_kernel' in kernels and 'adam_kernel' in kernels
    for stage, names in bench.STAGE_KERNELS.items():
        for name in names.split(' + '):
            if '<model>' in name:
                continue
            assert name in kernels, (stage, name)


def test_bench_line_reports_the_baseline_protocol():
    """The headline line: BASELINE.json's metric, value = W * H / median step time, the step's timing protocol, and a
    CPU baseline that is the unfused appearance on the host's torch threads (c0 forward and forward + backward, the CPU
    model named); the C restatement of the rasterizer stays as an extra key."""
    import json
    import sys
    from types import SimpleNamespace
    import torch
    sys.path.insert(0, ROOT)
    import bench
    cpu = bench.cpu_unfused_baseline(None, warmup=1, reps=3)
    assert cpu['unit'] == 'Mprim/s' and cpu['kind'] == 'port' and cpu['value'] > 0
    assert cpu['cores'] == torch.get_num_threads()
    assert cpu['cpu_model'] and cpu['cpu_model'] != 'unknown'
    assert cpu['c0_forward']['value'] > cpu['c0_forward_backward']['value'] > 0
    assert cpu['value'] == cpu['c0_forward_backward']['value']
    args = SimpleNamespace(steps=5, warmup=2, config='c3')
    r = dict(W=1920, H=1080, N=1_000_000, V=698_000.0, I=1_428_000.0, model='neural', step_ms=[0.61, 0.59, 0.6, 0.62, 0.58],
             wall_ms_per_step=0.605, region_ms=0.6, full_step_ms=0.8, fwd_loss_bwd_ms=0.7, adam_ms=0.1, render_ms=0.22,
             roofline={'bound': 'hbm', 'achieved': 1.0, 'peak': 8000.0, 'unit': 'GB/s', 'frac': 0.1, 'traffic': None}, stages={})
    line = bench.headline_line(args, r, cpu, {'value': 0.27, 'unit': 'Mpix/s', 'cores': 1, 'kind': 'port', 'sample': 'x'})
    baseline = json.load(open(os.path.join(ROOT, 'BASELINE.json')))
    assert line['metric'] == baseline['metric'] and line['unit'] == 'Mpix/s'
    assert line['ms_per_step'] == 0.6 and line['value'] == round(1920 * 1080 / 0.6e-3 / 1e6, 3)
    assert line['steps'] == 5 and line['warmup'] == 2 and line['n_gpus'] == 1 and line['vs_baseline'] is None
    assert 'around the 5 timed steps' in line['timing'] and 'forward + backward' in line['config']['workload']
    assert line['full_step_mpix_s'] == round(1920 * 1080 / 0.8e-3 / 1e6, 3)
    assert line['step_ms_quartiles'] == [0.58, 0.59, 0.6, 0.61, 0.62]
    kernel_us = bench.read_step_kernel_us()
    assert kernel_us is None or line['gpu_idle_us_per_step'] == round(600.0 - kernel_us, 1)
    assert line['cpu_baseline'] is cpu and line['cpu_port_rasterizer']['unit'] == 'Mpix/s'
    json.dumps(line)
    defaults = bench.parse_args.__code__  # defaults: 100 timed steps after 10 warm-up steps
    old = sys.argv
    sys.argv = ['bench.py']
    try:
        a = bench.parse_args()
    finally:
        sys.argv = old
    assert (a.steps, a.warmup) == (100, 10) and defaults is not None
