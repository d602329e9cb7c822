"""CPU oracle of the .ngsplat export (TEST INFRASTRUCTURE: imported only by tests/, smoke() and bench.py's
cpu_baseline, as the checker; the product packs on the GPU through libefgs_hip.so).

A numpy restatement of the per-splat part of the reference's exporter, viewer/export_ngsplat.py, in its float32
numpy expressions (same dtypes, same operation order), plus two readers used to pin it: the file parser of the
WebGL viewer (viewer/utils.js:230-330) and the viewer's decoders (viewer/shaders/splat_decode.glsl, eval_sh.glsl,
eval_neural.glsl).

Each integer code is returned with the value it was rounded from (`*_pre`), so a comparison can tell a code that
sits on a rounding boundary (where a last-bit difference of exp / log / acos / sin flips it) from a real mismatch.
Pins (tests/test_ngsplat_oracle.py): decode round trips within the quantisation steps, the viewer's MLP loop over
the weight texels equal to the matrix product, the baked layer 0 equal to the full evaluation, SH fields decoded
with the shader's shifts, header fields through the viewer's parser, and hand-computed codes for special cases.
"""
from __future__ import annotations

import math
import struct

import numpy as np

SH_C0 = 0.28209479177387814
TEX_WIDTH = 2048
MIN_ALPHA = 1.0 / 255.0
LN_SCALE_MIN = -12.0
LN_SCALE_MAX = 9.0
LN_SCALE_ENCODE = 254.0 / (LN_SCALE_MAX - LN_SCALE_MIN)
SV_SITE_LENGTH_EPS = 1e-12
FP16_SAFE_MAX = 60000.0
COS_LIMIT = 0.999999
SHAPE_LIMIT = 1e4
FREQUENCY_SCALE = 20.0
EPS_NORM = 1e-8
# quantised SH levels: degree, bits per field, u32 words per texel (export_ngsplat.py:539-543)
SH_LEVELS = [(1, 7, 2), (2, 8, 4), (3, 6, 4)]


def f16_bits(x) -> np.ndarray:
    """float32 -> uint32 of the float16 bit pattern (export_ngsplat.py:311-313)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16).astype(np.uint32)


def activated(raw_scales, raw_rotations, raw_opacities):
    """Activated opacities and scales and the normalised (x, y, z, w) quaternions (export_ngsplat.py:1234-1251)."""
    q = np.asarray(raw_rotations, np.float32).copy()
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    opacities = 1.0 / (1.0 + np.exp(-np.asarray(raw_opacities, np.float32).reshape(-1)))
    return opacities, np.exp(np.asarray(raw_scales, np.float32)), q[:, [1, 2, 3, 0]]


def encode_scales(s):
    """8-bit log codes (0 = exact zero) and the values they were rounded from (export_ngsplat.py:320-326)."""
    pre = np.maximum(0.0, (np.log(np.maximum(s, 1e-30)) - LN_SCALE_MIN) * LN_SCALE_ENCODE)
    code = np.minimum(255, np.round(pre) + 1).astype(np.uint32)
    return np.where(s == 0.0, np.uint32(0), code), pre


def encode_quat(q):
    """24-bit folded-octahedral codes (angle << 16 | v << 8 | u) and the pre-round u, v, angle values
    (export_ngsplat.py:329-355). The sign factors are float64 arrays there, which makes u and v float64."""
    q = np.where(q[:, 3:4] < 0.0, -q, q)
    half_theta = np.arccos(np.clip(q[:, 3], -1.0, 1.0))
    theta = 2.0 * half_theta
    s = np.sin(half_theta)
    degenerate = np.abs(s) < 1e-6
    axis = q[:, :3] / np.where(degenerate, 1.0, s)[:, None]
    axis[degenerate] = [1.0, 0.0, 0.0]
    total = np.abs(axis).sum(axis=1)
    pu, pv = axis[:, 0] / total, axis[:, 1] / total
    fold = axis[:, 2] < 0.0
    pu_f = (1.0 - np.abs(pv)) * np.where(pu >= 0.0, 1.0, -1.0)
    pv_f = (1.0 - np.abs(pu)) * np.where(pv >= 0.0, 1.0, -1.0)
    pu, pv = np.where(fold, pu_f, pu), np.where(fold, pv_f, pv)
    pre_u = np.clip((pu * 0.5 + 0.5) * 255.0, 0.0, 255.0)
    pre_v = np.clip((pv * 0.5 + 0.5) * 255.0, 0.0, 255.0)
    pre_a = np.clip(theta / math.pi * 255.0, 0.0, 255.0)
    code = (np.round(pre_a).astype(np.uint32) << 16) | (np.round(pre_v).astype(np.uint32) << 8) | np.round(pre_u).astype(np.uint32)
    return code, np.stack([pre_u, pre_v, pre_a], axis=1)


def residual_activation(raw, act: str):
    """export_ngsplat.py:500-506."""
    if act == 'tanh':
        return np.tanh(raw)
    if act == 'softplus':
        return np.where(raw > 2.0, raw, np.log1p(np.exp(10.0 * np.minimum(raw, 2.0))) / 10.0)
    return raw


def frequency_encode(features, k: int):
    """sin / cos (2^f x) per feature, f < k (export_ngsplat.py:402-411)."""
    if k == 0:
        return features
    scaled = features[..., None] * np.exp2(np.arange(k, dtype=np.float32))
    return np.stack([np.sin(scaled), np.cos(scaled)], axis=-1).reshape(features.shape[0], -1).astype(np.float32)


def sv_values(params, act: str):
    """[N, K * 7]: unit site, clamped exp temperature, activated colour (export_ngsplat.py:624-643)."""
    n = params.shape[0]
    sites = params[..., 0:3]
    lengths = np.maximum(np.linalg.norm(sites, axis=-1, keepdims=True), SV_SITE_LENGTH_EPS)
    tau = np.exp(params[..., 3:4])
    return np.concatenate([sites / lengths, np.minimum(tau, FP16_SAFE_MAX), residual_activation(params[..., 4:7], act)],
                          axis=-1).reshape(n, -1).astype(np.float32)


def lobe_values(lobes, act: str, gabor: bool):
    """[N, L * 12] NASG or [N, L * 13] NASGabor baked lobes (export_ngsplat.py:656-696, :721-765)."""
    n = lobes.shape[0]
    cos = np.clip(np.tanh(lobes[..., 0:3]), -COS_LIMIT, COS_LIMIT)
    sin = np.sqrt(1.0 - cos * cos)
    ct, cp, cu = cos[..., 0], cos[..., 1], cos[..., 2]
    st, sp, su = sin[..., 0], sin[..., 1], sin[..., 2]
    frame_x = np.stack([ct * cp * cu - st * su, st * cp * cu + ct * su, -sp * cu], axis=-1)
    frame_z = np.stack([ct * sp, st * sp, cp], axis=-1)
    lam, a = (np.minimum(np.exp(lobes[..., i]), SHAPE_LIMIT) for i in (3, 4))
    norm = lam * np.sqrt(1.0 + a) / (2.0 * math.pi * (1.0 + EPS_NORM - np.exp(-2.0 * lam)))
    parts = [frame_x, frame_z, (2.0 * lam)[..., None], a[..., None]]
    if gabor:
        parts.append(((np.tanh(lobes[..., 5]) + 1.0) * FREQUENCY_SCALE)[..., None])
    parts += [norm[..., None], residual_activation(lobes[..., -3:], act)]
    return np.concatenate(parts, axis=-1).reshape(n, -1).astype(np.float32)


def pack_half(values, rows: int):
    """[N, V] float32 -> ceil(V / 8) textures [rows, 4] u32, 8 fp16 per texel (export_ngsplat.py:372-386)."""
    n, v = values.shape
    m = (v + 7) // 8
    padded = np.zeros((rows, m * 8), np.float32)
    padded[:n, :v] = values
    bits = f16_bits(padded)
    return [(bits[:, 8 * k:8 * k + 8][:, 0::2] | (bits[:, 8 * k:8 * k + 8][:, 1::2] << 16)).astype(np.uint32) for k in range(m)]


def sh_quantize(coefficients, rows: int):
    """Per present level: signed codes at the level's max |coefficient| scale, bit-packed little-endian
    (export_ngsplat.py:576-611). Returns textures, the three scales (0 = absent) and the pre-round values."""
    n = coefficients.shape[0]
    textures, scales, pres = [], [], []
    offset = 0
    for degree, bits, words in SH_LEVELS:
        width = 2 * degree + 1
        if offset + width > coefficients.shape[1]:
            scales.append(0.0)
            continue
        values = coefficients[:, offset:offset + width, :].reshape(n, -1)
        scale = max(float(np.abs(values).max(initial=0.0)), 1e-8)
        qmax = (1 << (bits - 1)) - 1
        pre = values / scale * qmax
        codes = (np.clip(np.round(pre), -qmax, qmax).astype(np.int32) & ((1 << bits) - 1)).astype(np.uint32)
        out = np.zeros((rows, words), np.uint32)
        for f in range(codes.shape[1]):
            bit = bits * f
            w, shift = bit // 32, bit % 32
            out[:n, w] |= codes[:, f] << np.uint32(shift)
            if shift + bits > 32:
                out[:n, w + 1] |= codes[:, f] >> np.uint32(32 - shift)
        textures.append(out)
        scales.append(scale)
        pres.append(pre)
        offset += width
    return textures, scales, pres


def export(means, raw_scales, raw_rotations, raw_opacities, base_colors, residual_params, plan: dict):
    """The textures and statistics of a model for a plan (payload kind and parameters as efgs.ngsplat.plan_export
    makes them): culling, rgb8 base, a8 opacity and splat words (export_ngsplat.py:1465-1483), then the payload
    (:1487-1530). Returns the kept indices, splat words and textures over P = 2048 ceil(kept / 2048) rows, the
    statistics and the pre-round values of every code."""
    means = np.asarray(means, np.float32)
    opacities, scales, quats = activated(raw_scales, raw_rotations, raw_opacities)
    keep = opacities >= MIN_ALPHA
    kept = np.nonzero(keep)[0]
    means, opacities, scales, quats = means[keep], opacities[keep], scales[keep], quats[keep]
    base_colors = np.asarray(base_colors, np.float32).reshape(-1, 3)[keep]
    residual = np.asarray(residual_params, np.float32)
    residual = residual.reshape(residual.shape[0], *residual.shape[1:])[keep]
    n = means.shape[0]
    rows = -(-n // TEX_WIDTH) * TEX_WIDTH
    base = (plan['color_shift'] + base_colors).astype(np.float32)
    d_min, d_max = (float(base.min()), float(base.max())) if n else (0.0, 0.0)
    d_scale = max(d_max - d_min, 1e-6) / 255.0
    base_pre = (base - d_min) / d_scale
    base_code = np.round(base_pre).clip(0, 255).astype(np.uint32)
    opacity_pre = opacities * 255.0
    opacity8 = np.round(opacity_pre).clip(0, 255).astype(np.uint32)
    scale_code, scale_pre = encode_scales(scales)
    quat_code, quat_pre = encode_quat(quats)
    words = np.zeros((rows, 4), np.uint32)
    words[:n, 0] = base_code[:, 0] | (base_code[:, 1] << 8) | (base_code[:, 2] << 16) | (opacity8 << 24)
    words[:n, 1] = f16_bits(means[:, 0]) | (f16_bits(means[:, 1]) << 16)
    words[:n, 2] = f16_bits(means[:, 2]) | ((quat_code & 0xFF) << 16) | (((quat_code >> 8) & 0xFF) << 24)
    words[:n, 3] = scale_code[:, 0] | (scale_code[:, 1] << 8) | (scale_code[:, 2] << 16) | ((quat_code >> 16) << 24)
    out = dict(kept=kept, n_kept=n, rows=rows, splat_words=words, base_offset=d_min, base_scale=d_scale, sh_level_scales=None,
               base_pre=base_pre, opacity_pre=opacity_pre, scale_pre=scale_pre, quat_pre=quat_pre, values=None, sh_pre=None)
    kind = plan['payload']
    if kind in (0, 1):  # neural: stored encoded features or the baked layer 0
        feats = residual.reshape(n, -1)[:, :plan['n_items']]
        if plan['base_input']:
            feats = np.concatenate([feats, base_colors], axis=-1)
        encoded = frequency_encode(feats, plan['n_frequencies'])
        if kind == 0:
            values = encoded
        else:
            values = encoded @ plan['bake_matrix'].T
            if plan['bake_bias'] is not None:
                values = values + plan['bake_bias']
            out['bake_magnitude'] = np.abs(encoded) @ np.abs(plan['bake_matrix']).T
        out['values'] = values.astype(np.float32)
        out['textures'] = pack_half(out['values'], rows)
    elif kind == 2:
        coefficients = residual.reshape(n, -1, 3)[:, :plan['n_items'], :]
        out['textures'], out['sh_level_scales'], out['sh_pre'] = sh_quantize(coefficients, rows)
    else:
        act = {0: 'none', 1: 'tanh', 2: 'softplus'}[plan['residual_act']]
        if kind == 3:
            values = sv_values(residual.reshape(n, -1, 7)[:, :plan['n_items']], act)
        else:
            width = 9 if kind == 5 else 8
            values = lobe_values(residual.reshape(n, -1, width)[:, :plan['n_items']], act, gabor=kind == 5)
        out['values'] = values
        out['textures'] = pack_half(values, rows)
    return out


def write_file(path: str, plan: dict, packed: dict, center, up, distance: float, test_cameras=None, proper_antialiasing=False):
    """export_ngsplat.py:1581-1623 (without the PPISP block)."""
    n = packed['n_kept']
    cams = np.zeros((0, 18), np.float32) if test_cameras is None else np.asarray(test_cameras, np.float32).reshape(-1, 18)
    with open(path, 'wb') as f:
        f.write(b'NGSPLAT\n')
        f.write(struct.pack('<11I', n, TEX_WIDTH, -(-n // TEX_WIDTH), plan['model_dims'], plan['header_frequencies'], plan['degree_mask'],
                            plan['color_code'], plan['residual_code'], plan['header_neurons'], plan['header_hidden'],
                            plan['flags'] | (1 if proper_antialiasing else 0)))
        f.write(struct.pack('<2f', packed['base_scale'], packed['base_offset']))
        if plan['payload'] == 2:
            f.write(struct.pack('<3f', *packed['sh_level_scales']))
        f.write(struct.pack('<3f', *[float(v) for v in center]))
        f.write(struct.pack('<3f', *[float(v) for v in up]))
        f.write(struct.pack('<f', float(distance)))
        f.write(struct.pack('<I', cams.shape[0]))
        f.write(cams.astype('<f4').tobytes())
        texels = np.asarray(plan['weight_texels'], '<u2')
        f.write(struct.pack('<I', texels.shape[0]))
        f.write(texels.tobytes())
        f.write(packed['splat_words'].astype('<u4').tobytes())
        for t in packed['textures']:
            f.write(t.astype('<u4').tobytes())


APPEARANCE_BY_ID = {0: 'neural', 1: 'sh', 2: 'sv', 3: 'nasg', 4: 'nasgabor'}


def read_file(path_or_bytes):
    """Parser of the WebGL viewer (viewer/utils.js:230-330 and its payload plan), with its validation checks.
    Returns the header fields, the weight texels (uint16 [T, 4]) and the textures as uint32 arrays."""
    data = open(path_or_bytes, 'rb').read() if isinstance(path_or_bytes, str) else bytes(path_or_bytes)
    if data[:8] != b'NGSPLAT\n':
        raise ValueError('Not a .ngsplat file (bad magic)')
    o = 8

    def u32():
        nonlocal o
        v = struct.unpack_from('<I', data, o)[0]
        o += 4
        return v

    def f32():
        nonlocal o
        v = struct.unpack_from('<f', data, o)[0]
        o += 4
        return v

    h = {}
    for key in ('num_splats', 'tex_width', 'tex_height', 'model_dims', 'n_frequencies', 'sh_degree_mask', 'color_activation',
                'residual_activation', 'n_neurons', 'n_hidden_layers', 'flags'):
        h[key] = u32()
    flags = h['flags']
    h['proper_aa'] = bool(flags & 1)
    h['sh0_input'] = not (flags & 2)
    h['baked'] = bool(flags & 4)
    h['appearance'] = APPEARANCE_BY_ID[((flags >> 3) & 3) | (((flags >> 6) & 1) << 2)]
    h['base_exp'] = bool(flags & 32)
    h['base_scale'], h['base_offset'] = f32(), f32()
    h['sh_scales'] = [f32(), f32(), f32()] if h['appearance'] == 'sh' else None
    h['center'] = [f32(), f32(), f32()]
    h['up'] = [f32(), f32(), f32()]
    h['distance'] = f32()
    n_cams = u32()
    h['test_cameras'] = np.frombuffer(data, '<f4', n_cams * 18, o).reshape(n_cams, 18).copy()
    o += 72 * n_cams
    if flags & 128:
        raise ValueError('PPISP blocks are not produced here')
    n_texels = u32()
    if h['tex_width'] != 2048:
        raise ValueError('texWidth must be 2048')
    if h['sh_degree_mask'] & ~0b1111110:
        raise ValueError('shDegreeMask has bits outside degrees 1-6')
    if h['color_activation'] > 5 or h['residual_activation'] > 2:
        raise ValueError('unknown activation code')
    degrees = [d for d in range(1, 7) if h['sh_degree_mask'] & (1 << d)]
    if h['appearance'] == 'neural':
        n_dir = sum(2 * d + 1 for d in degrees)
        nn = h['n_neurons']
        if nn % 4 or nn < 4 or h['n_hidden_layers'] < 1:
            raise ValueError('invalid mlp shape')
        if h['baked']:
            if not n_dir or nn > 16:
                raise ValueError('invalid baked layout')
            l0 = -(-n_dir // 4) * 4
            per_splat = nn
        else:
            if h['model_dims'] < 1 or h['model_dims'] > 16:
                raise ValueError('unsupported featureDim')
            l0 = h['model_dims'] + (1 if h['sh0_input'] else 0) + n_dir
            if l0 % 4:
                raise ValueError('MLP input dim is not a multiple of 4')
            per_splat = h['model_dims']
        expected = (l0 // 4) * nn + (h['n_hidden_layers'] - 1) * (nn // 4) * nn + (nn // 4) * 3
        if n_texels != expected:
            raise ValueError(f'weight texel count {n_texels} != expected {expected}')
        h['l0_in'] = l0
        components = [4] * (-(-per_splat // 8))
    elif h['appearance'] == 'sh':
        if n_texels:
            raise ValueError('sh payload carries no weight stream')
        components = [w for (d, _, w) in SH_LEVELS if h['sh_degree_mask'] & (1 << d)]
    else:
        if n_texels:
            raise ValueError('payload carries no weight stream')
        per = {'sv': 7, 'nasg': 12, 'nasgabor': 13}[h['appearance']]
        components = [4] * (-(-(per * h['model_dims']) // 8))
    texels = np.frombuffer(data, '<u2', n_texels * 4, o).reshape(n_texels, 4).copy()
    o += 8 * n_texels
    rows = h['tex_width'] * h['tex_height']
    splat = np.frombuffer(data, '<u4', rows * 4, o).reshape(rows, 4).copy()
    o += 16 * rows
    textures = []
    for c in components:
        textures.append(np.frombuffer(data, '<u4', rows * c, o).reshape(rows, c).copy())
        o += 4 * rows * c
    if o != len(data):
        raise ValueError(f'{len(data) - o} trailing bytes')
    return h, texels, splat, textures


# ---- viewer decoders (the inverse direction, used to pin the encoders) ----------------------------------------------

def decode_splats(words: np.ndarray):
    """viewer/shaders/splat_decode.glsl: rgba8, fp16 position, log scales, folded-octahedral quaternion (x, y, z, w)."""
    w = words.astype(np.uint32)
    rgba = np.stack([(w[:, 0] >> s) & 0xFF for s in (0, 8, 16, 24)], axis=1).astype(np.float32) / 255.0
    pos = np.stack([(w[:, 1] & 0xFFFF), (w[:, 1] >> 16), (w[:, 2] & 0xFFFF)], axis=1).astype(np.uint16).view(np.float16).astype(np.float32)
    u = np.stack([(w[:, 3] >> s) & 0xFF for s in (0, 8, 16)], axis=1)
    step = (LN_SCALE_MAX - LN_SCALE_MIN) / 254.0
    scales = np.where(u == 0, 0.0, np.exp(LN_SCALE_MIN + (u.astype(np.float64) - 1.0) * step))
    packed = ((w[:, 2] >> 16) & 0xFF) | (((w[:, 2] >> 24) & 0xFF) << 8) | (((w[:, 3] >> 24) & 0xFF) << 16)
    pu = (packed & 0xFF) / 255.0 * 2.0 - 1.0
    pv = ((packed >> 8) & 0xFF) / 255.0 * 2.0 - 1.0
    theta = ((packed >> 16) & 0xFF) / 255.0 * 3.14159265358979
    axis = np.stack([pu, pv, 1.0 - np.abs(pu) - np.abs(pv)], axis=1)
    neg = axis[:, 2] < 0.0
    folded = (1.0 - np.abs(axis[:, [1, 0]])) * np.sign(axis[:, :2])
    axis[neg, :2] = folded[neg]
    axis /= np.linalg.norm(axis, axis=1, keepdims=True)
    quat = np.concatenate([axis * np.sin(theta / 2.0)[:, None], np.cos(theta / 2.0)[:, None]], axis=1)
    return rgba, pos, scales, quat


def decode_sh_field(words: np.ndarray, bits: int, field: int) -> np.ndarray:
    """Signed field `field` of a bit-packed level texel (viewer/shaders/eval_sh.glsl: shift left, arithmetic shift
    right), generalised to any field position."""
    bit = bits * field
    w, shift = bit // 32, bit % 32
    v = words[:, w].astype(np.uint64) >> np.uint64(shift)
    if shift + bits > 32:
        v |= words[:, w + 1].astype(np.uint64) << np.uint64(32 - shift)
    v = (v & np.uint64((1 << bits) - 1)).astype(np.int64)
    return np.where(v >= (1 << (bits - 1)), v - (1 << bits), v)


def shader_mlp(texels: np.ndarray, inputs: np.ndarray, n_neurons: int, n_hidden: int, h0=None) -> np.ndarray:
    """The viewer's MLP loop over the weight texels (viewer/shaders/eval_neural.glsl:146-204): layer 0 accumulates
    input block j times the texels j * N + i .. + 3 (as mat4 columns) into output block i / 4, hidden layers
    likewise after a ReLU, the 3-row output layer reads 3 texels per input block."""
    t = texels.view(np.float16).astype(np.float64)
    n, l0 = inputs.shape
    h = np.zeros((n, n_neurons)) if h0 is None else np.array(h0, np.float64)
    for j in range(l0 // 4):
        b = inputs[:, 4 * j:4 * j + 4]
        for i in range(0, n_neurons, 4):
            m = t[j * n_neurons + i:j * n_neurons + i + 4]  # column c of the mat4 = texel c
            h[:, i:i + 4] += b @ m.T
    base = (l0 // 4) * n_neurons
    for _ in range(1, n_hidden):
        act = np.maximum(h, 0.0)
        h = np.zeros_like(h)
        for j in range(n_neurons // 4):
            for i in range(0, n_neurons, 4):
                m = t[base + j * n_neurons + i:base + j * n_neurons + i + 4]
                h[:, i:i + 4] += act[:, 4 * j:4 * j + 4] @ m.T
        base += (n_neurons // 4) * n_neurons
    out = np.zeros((n, 3))
    for j in range(n_neurons // 4):
        b = np.maximum(h[:, 4 * j:4 * j + 4], 0.0)
        out += b @ t[base + 3 * j:base + 3 * j + 3].T
    return out
