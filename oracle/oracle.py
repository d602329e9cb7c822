"""CPU oracle for the fused-appearance rasterizer -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the product
package never does. It drives the plain-C restatement in efgs_oracle.c (preprocess, instance creation, blend
forward/backward, preprocess backward, Adam) and adds the pieces that are plain numpy:

* compaction of visible primitives in primitive-index order, the 32-bit depth sort and the tile sort as
  numpy stable argsorts, exclusive scans as cumsums, per-tile ranges by searchsorted
  (reference: B/rasterization/src/forward.cu:82-221, B/rasterization/include/kernels_common.cuh:20-157);
* the neural residual MLP (B/rasterization/rtc/appearance_neural.cuh:17-407 with the numpy statement of
  viewer/export_ngsplat.py:485-497 and the tcnn flat layout of viewer/export_ngsplat.py:1013-1029).

"B/" abbreviates FasterGSVDACudaBackend/FasterGSVDACudaBackend/ in the reference repository.

Tie-break: the reference compacts with an atomic counter, so equal depths keep an arbitrary order there.
This oracle (and the HIP path) compacts in primitive-index order and sorts stably, which fixes the order of
equal keys: every key, index and range array is then a deterministic function of the inputs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, '_build', 'libefgs_oracle.so')

TILE_W, TILE_H = 16, 12
MODEL_IDS = {'precomputed': 0, 'sh': 1, 'sv': 2, 'nasg': 3, 'nasgabor': 4, 'neural': 5}
BASE_ACT_IDS = {'none': 0, 'exp': 1}
RES_ACT_IDS = {'none': 0, 'tanh': 1, 'softplus': 2}
COLOR_ACT_IDS = {'none': 0, 'relu': 1, 'softplus': 2, 'sigmoid': 3, 'hardsigmoid': 4, 'satexp': 5}
SH_C0 = 0.28209479177387814


class _Cam(ctypes.Structure):
    _fields_ = [('w2c', ctypes.c_float * 12), ('cam_pos', ctypes.c_float * 3), ('bg', ctypes.c_float * 3),
                ('degree', ctypes.c_int), ('width', ctypes.c_int), ('height', ctypes.c_int),
                ('fx', ctypes.c_float), ('fy', ctypes.c_float), ('cx', ctypes.c_float), ('cy', ctypes.c_float),
                ('near_plane', ctypes.c_float), ('far_plane', ctypes.c_float),
                ('proper_aa', ctypes.c_int), ('render_base', ctypes.c_int)]


class _App(ctypes.Structure):
    _fields_ = [('model', ctypes.c_int), ('base_act', ctypes.c_int), ('res_act', ctypes.c_int),
                ('color_act', ctypes.c_int), ('dir_grad', ctypes.c_int), ('n_units', ctypes.c_int)]


def build() -> str:
    """Compiles the C restatement (gcc) into oracle/_build and returns the library path."""
    subprocess.run(['make', '-s', '-C', _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.ef_expf.restype = ctypes.c_float
        _lib.ef_expf.argtypes = [ctypes.c_float]
        _lib.ef_logf.restype = ctypes.c_float
        _lib.ef_logf.argtypes = [ctypes.c_float]
        _lib.efo_create_instances.restype = ctypes.c_uint32
        _lib.efo_will_primitive_contribute.restype = ctypes.c_int
        _lib.efo_will_primitive_contribute.argtypes = [ctypes.c_float] * 5 + [ctypes.c_uint32] * 2 + [ctypes.c_float]
        _lib.ef_exp2f.restype = ctypes.c_float
        _lib.ef_exp2f.argtypes = [ctypes.c_float]
        _lib.efo_blend_alpha.restype = ctypes.c_float
        _lib.efo_blend_alpha.argtypes = [ctypes.c_float] * 6 + [ctypes.c_int] * 2
        _lib.efo_sh_rest_basis.restype = ctypes.c_int
        _lib.efo_philox4x32_10.argtypes = [ctypes.c_void_p] * 3
        _lib.efo_box_muller.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        _lib.efo_add_noise.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64]
        _lib.efo_relocation_table.argtypes = [ctypes.c_void_p]
        _lib.efo_relocation.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5
        _lib.efo_pruning_scores.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 10
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags['C_CONTIGUOUS'], 'oracle arrays must be C-contiguous'
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ---------------------------------------------------------------------------------------------------------
# configuration objects
# ---------------------------------------------------------------------------------------------------------

@dataclass
class Camera:
    """Pinhole camera and render settings, the fields of RasterizerSettings (B/torch_bindings/rasterization.py:49-83)."""
    w2c: np.ndarray              # (4, 4) or (3, 4) world-to-view, rows 0..2 used
    position: np.ndarray         # (3,)
    width: int
    height: int
    focal_x: float
    focal_y: float
    center_x: float
    center_y: float
    near_plane: float = 0.2
    far_plane: float = 1e4
    bg: np.ndarray = field(default_factory=lambda: np.zeros(3, np.float32))
    degree: int = 3
    proper_aa: bool = False
    render_base: bool = True
    render_residual: bool = True

    def grid(self) -> tuple[int, int]:
        return (self.width + TILE_W - 1) // TILE_W, (self.height + TILE_H - 1) // TILE_H

    def c_struct(self) -> _Cam:
        c = _Cam()
        w = np.asarray(self.w2c, np.float32).reshape(-1, 4)[:3].reshape(-1)
        c.w2c[:] = [float(v) for v in w]
        c.cam_pos[:] = [float(v) for v in np.asarray(self.position, np.float32)]
        c.bg[:] = [float(v) for v in np.asarray(self.bg, np.float32)]
        c.degree = int(self.degree) if self.render_residual else 0
        c.width, c.height = int(self.width), int(self.height)
        c.fx, c.fy, c.cx, c.cy = float(self.focal_x), float(self.focal_y), float(self.center_x), float(self.center_y)
        c.near_plane, c.far_plane = float(self.near_plane), float(self.far_plane)
        c.proper_aa = int(bool(self.proper_aa))
        c.render_base = int(bool(self.render_base))
        return c


@dataclass
class MLPConfig:
    """Residual MLP (tcnn FullyFusedMLP, bias-free, ReLU hidden layers, 'None' output activation)."""
    n_feature_dims: int          # learned per-Gaussian features (FEATURE_DIM minus 3 with base_input)
    n_frequencies: int           # 0: raw features, k>0: sin/cos of 2^f x for f < k
    sh_degrees: tuple            # ascending SH degrees of the direction encoding
    n_neurons: int
    n_hidden_layers: int
    base_input: bool = False

    @property
    def n_raw_feature_dims(self) -> int:
        return self.n_feature_dims + (3 if self.base_input else 0)

    @property
    def n_encoded_feature_dims(self) -> int:
        f = self.n_raw_feature_dims
        return f if self.n_frequencies == 0 else f * 2 * self.n_frequencies

    @property
    def n_sh_dims(self) -> int:
        return sum(2 * d + 1 for d in self.sh_degrees)

    @property
    def n_input_dims(self) -> int:
        return self.n_encoded_feature_dims + self.n_sh_dims

    @property
    def n_input_padded(self) -> int:
        return (self.n_input_dims + 15) // 16 * 16

    @property
    def max_degree(self) -> int:
        return sum(1 for d in self.sh_degrees if d > 0)

    def layer_shapes(self) -> list[tuple[int, int]]:
        """Row-major [out x in] matrices of the flat parameter vector, output layer padded to 16 rows."""
        n = self.n_neurons
        return [(n, self.n_input_padded)] + [(n, n)] * (self.n_hidden_layers - 1) + [(16, n)]

    @property
    def n_params(self) -> int:
        return sum(r * c for r, c in self.layer_shapes())


@dataclass
class Appearance:
    model: str = 'sh'
    base_act: str = 'none'
    res_act: str = 'none'
    color_act: str = 'relu'
    direction_gradient: bool = True
    max_degree: int = 3          # sh degree / sv sites / lobes ; neural: derived from the MLP config
    mlp: MLPConfig | None = None

    def n_units(self) -> int:
        if self.model == 'sh':
            return (self.max_degree + 1) ** 2 - 1
        if self.model in ('sv', 'nasg', 'nasgabor'):
            return self.max_degree
        if self.model == 'neural':
            return self.mlp.n_feature_dims
        return 0

    def params_per_primitive(self) -> int:
        return {'sh': 3, 'sv': 7, 'nasg': 8, 'nasgabor': 9, 'neural': 1}.get(self.model, 0) * self.n_units()

    def c_struct(self) -> _App:
        a = _App()
        a.model = MODEL_IDS[self.model]
        a.base_act = BASE_ACT_IDS[self.base_act]
        a.res_act = RES_ACT_IDS[self.res_act]
        a.color_act = COLOR_ACT_IDS[self.color_act]
        a.dir_grad = int(bool(self.direction_gradient))
        a.n_units = self.n_units()
        return a


@dataclass
class Scene:
    means: np.ndarray            # (N, 3)
    scales: np.ndarray           # (N, 3) log scales
    rotations: np.ndarray        # (N, 4) (w, x, y, z), unnormalized
    opacities: np.ndarray        # (N, 1) logits
    base_colors: np.ndarray | None = None       # (N, 3)
    residual_params: np.ndarray | None = None   # model-specific, (N, ...)
    precomputed_colors: np.ndarray | None = None
    mlp_weights: np.ndarray | None = None       # flat fp32 tcnn layout

    @property
    def n(self) -> int:
        return int(self.means.shape[0])


# ---------------------------------------------------------------------------------------------------------
# activations (numpy statements of B/rasterization/rtc/preprocess_common.cuh:51-142)
# ---------------------------------------------------------------------------------------------------------

def residual_activation(x: np.ndarray, act: str) -> np.ndarray:
    x = x.astype(np.float32)
    if act == 'tanh':
        return np.tanh(x)
    if act == 'softplus':
        bx = 10.0 * x
        return ((np.maximum(bx, 0) + np.log1p(np.exp(-np.abs(bx)))) / 10.0).astype(np.float32)
    return x


def residual_activation_grad(y: np.ndarray, act: str) -> np.ndarray:
    if act == 'tanh':
        return (1.0 - y * y).astype(np.float32)
    if act == 'softplus':
        return (-np.expm1(-10.0 * y)).astype(np.float32)
    return np.ones_like(y, dtype=np.float32)


# ---------------------------------------------------------------------------------------------------------
# neural residual MLP
# ---------------------------------------------------------------------------------------------------------

def sh_degree_encoding(dirs: np.ndarray, sh_degrees, active_degree: int) -> np.ndarray:
    """Direction encoding: degree 0 is never gated, the i-th degree >= 1 is zero unless i < active_degree."""
    cols, rank = [], 0
    for deg in sh_degrees:
        vals = _sh_degree_values(dirs, deg)
        if deg > 0:
            keep = rank < active_degree
            rank += 1
            if not keep:
                vals = [np.zeros_like(v) for v in vals]
        cols += vals
    return np.stack(cols, axis=1).astype(np.float32)


def directions(means: np.ndarray, cam_pos: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    v = (means - cam_pos[None]).astype(np.float32)
    nrm = (np.float32(1.0) / np.sqrt(np.maximum((v * v).sum(1), np.float32(1e-24)))).astype(np.float32)
    return (v * nrm[:, None]).astype(np.float32), nrm


def frequency_encode(feat: np.ndarray, n_freq: int) -> np.ndarray:
    if n_freq == 0:
        return feat.astype(np.float32)
    scaled = feat[..., None] * (2.0 ** np.arange(n_freq, dtype=np.float32))
    return np.stack([np.sin(scaled), np.cos(scaled)], axis=-1).reshape(feat.shape[0], -1).astype(np.float32)


def mlp_inputs(scene: Scene, mlp: MLPConfig, cam: Camera, active_degree: int) -> np.ndarray:
    feats = scene.residual_params.reshape(scene.n, -1).astype(np.float32)
    if mlp.base_input:
        feats = np.concatenate([feats, scene.base_colors.astype(np.float32)], axis=1)
    enc = frequency_encode(feats, mlp.n_frequencies)
    d, _ = directions(scene.means.astype(np.float32), np.asarray(cam.position, np.float32))
    sh = sh_degree_encoding(d, mlp.sh_degrees, active_degree)
    x = np.concatenate([enc, sh], axis=1)
    pad = mlp.n_input_padded - x.shape[1]
    if pad:
        x = np.concatenate([x, np.zeros((x.shape[0], pad), np.float32)], axis=1)
    return x.astype(np.float32)


def mlp_matrices(weights: np.ndarray, mlp: MLPConfig) -> list[np.ndarray]:
    """Flat tcnn parameters -> fp16-rounded row-major [out x in] matrices (viewer/export_ngsplat.py:1013-1029)."""
    w = np.asarray(weights, np.float32).astype(np.float16).astype(np.float32)
    mats, off = [], 0
    for r, c in mlp.layer_shapes():
        mats.append(w[off:off + r * c].reshape(r, c))
        off += r * c
    assert off == w.size, f'mlp weight count {w.size} != {off}'
    return mats


def mlp_forward(x: np.ndarray, mats: list[np.ndarray]) -> tuple[np.ndarray, list[np.ndarray]]:
    """fp16 operands, fp32 accumulation, activations rounded to fp16 between layers; returns the 3 raw
    outputs (fp16-rounded) and the per-layer fp16 activations (inputs of every layer)."""
    h = x.astype(np.float16).astype(np.float32)
    acts = [h]
    for i, w in enumerate(mats):
        h = (h @ w.T).astype(np.float32)
        if i < len(mats) - 1:
            h = np.maximum(h, 0.0)
        h = h.astype(np.float16).astype(np.float32)
        if i < len(mats) - 1:
            acts.append(h)
    return h[:, :3].copy(), acts


def mlp_backward(dy: np.ndarray, mats: list[np.ndarray], acts: list[np.ndarray]) -> tuple[np.ndarray, list[np.ndarray]]:
    """float32 backward of mlp_forward (the fp16 roundings pass gradients straight through); dy (n, 3)."""
    g = np.zeros((dy.shape[0], mats[-1].shape[0]), np.float32)
    g[:, :3] = dy
    grads = [None] * len(mats)
    for i in range(len(mats) - 1, -1, -1):
        grads[i] = (g.T @ acts[i]).astype(np.float32)
        g = (g @ mats[i]).astype(np.float32)
        if i > 0:
            g = g * (acts[i] > 0)
    return g, grads


def sh_degree_encoding_grad(dirs: np.ndarray, dsh: np.ndarray, sh_degrees, active_degree: int) -> np.ndarray:
    """d(loss)/d(direction) through the SH degree values, by central differences of the float64 polynomials
    (exact to ~1e-9 for these degree <= 6 polynomials)."""
    d64 = dirs.astype(np.float64)
    out = np.zeros_like(d64)
    eps = 1e-6
    for k in range(3):
        dp, dm = d64.copy(), d64.copy()
        dp[:, k] += eps
        dm[:, k] -= eps
        fp = _sh_encoding64(dp, sh_degrees, active_degree)
        fm = _sh_encoding64(dm, sh_degrees, active_degree)
        out[:, k] = ((fp - fm) / (2 * eps) * dsh).sum(1)
    return out.astype(np.float32)


def _sh_encoding64(d: np.ndarray, sh_degrees, active_degree: int) -> np.ndarray:
    cols, rank = [], 0
    for deg in sh_degrees:
        vals = _sh_degree_values(d, deg)
        if deg > 0:
            keep = rank < active_degree
            rank += 1
            if not keep:
                vals = [np.zeros_like(v) for v in vals]
        cols += vals
    return np.stack(cols, axis=1)


def _sh_degree_values(d: np.ndarray, degree: int) -> list[np.ndarray]:
    """Real SH basis values of one degree (tcnn sh_enc polynomials, B/rasterization/rtc/appearance_neural.cuh:55-139).
    Python-float constants stay weak under numpy 2 promotion, so float32 input evaluates in float32."""
    x, y, z = d[:, 0], d[:, 1], d[:, 2]
    xy, xz, yz, x2, y2, z2 = x * y, x * z, y * z, x * x, y * y, z * z
    x4, y4, z4 = x2 * x2, y2 * y2, z2 * z2
    x6, y6, z6 = x4 * x2, y4 * y2, z4 * z2
    if degree == 0:
        return [np.full_like(x, SH_C0)]
    if degree == 1:
        return [-0.48860251190291987 * y, 0.48860251190291987 * z, -0.48860251190291987 * x]
    if degree == 2:
        return [1.0925484305920792 * xy, -1.0925484305920792 * yz, 0.94617469575755997 * z2 - 0.31539156525251999,
                -1.0925484305920792 * xz, 0.54627421529603959 * x2 - 0.54627421529603959 * y2]
    if degree == 3:
        return [0.59004358992664352 * y * (-3.0 * x2 + y2), 2.8906114426405538 * xy * z,
                0.45704579946446572 * y * (1.0 - 5.0 * z2), 0.3731763325901154 * z * (5.0 * z2 - 3.0),
                0.45704579946446572 * x * (1.0 - 5.0 * z2), 1.4453057213202769 * z * (x2 - y2),
                0.59004358992664352 * x * (-x2 + 3.0 * y2)]
    if degree == 4:
        return [2.5033429417967046 * xy * (x2 - y2), 1.7701307697799304 * yz * (-3.0 * x2 + y2),
                0.94617469575756008 * xy * (7.0 * z2 - 1.0), 0.66904654355728921 * yz * (3.0 - 7.0 * z2),
                -3.1735664074561294 * z2 + 3.7024941420321507 * z4 + 0.31735664074561293,
                0.66904654355728921 * xz * (3.0 - 7.0 * z2), 0.47308734787878004 * (x2 - y2) * (7.0 * z2 - 1.0),
                1.7701307697799304 * xz * (-x2 + 3.0 * y2),
                -3.7550144126950569 * x2 * y2 + 0.62583573544917614 * x4 + 0.62583573544917614 * y4]
    if degree == 5:
        return [0.65638205684017015 * y * (10.0 * x2 * y2 - 5.0 * x4 - y4), 8.3026492595241645 * xy * z * (x2 - y2),
                -0.48923829943525038 * y * (3.0 * x2 - y2) * (9.0 * z2 - 1.0), 4.7935367849733241 * xy * z * (3.0 * z2 - 1.0),
                0.45294665119569694 * y * (14.0 * z2 - 21.0 * z4 - 1.0), 0.1169503224534236 * z * (-70.0 * z2 + 63.0 * z4 + 15.0),
                0.45294665119569694 * x * (14.0 * z2 - 21.0 * z4 - 1.0), 2.3967683924866621 * z * (x2 - y2) * (3.0 * z2 - 1.0),
                -0.48923829943525038 * x * (x2 - 3.0 * y2) * (9.0 * z2 - 1.0), 2.0756623148810411 * z * (-6.0 * x2 * y2 + x4 + y4),
                0.65638205684017015 * x * (10.0 * x2 * y2 - x4 - 5.0 * y4)]
    if degree == 6:
        return [1.3663682103838286 * xy * (-10.0 * x2 * y2 + 3.0 * x4 + 3.0 * y4),
                2.3666191622317521 * yz * (10.0 * x2 * y2 - 5.0 * x4 - y4),
                2.0182596029148963 * xy * (x2 - y2) * (11.0 * z2 - 1.0),
                -0.92120525951492349 * yz * (3.0 * x2 - y2) * (11.0 * z2 - 3.0),
                0.92120525951492349 * xy * (-18.0 * z2 + 33.0 * z4 + 1.0),
                0.58262136251873131 * yz * (30.0 * z2 - 33.0 * z4 - 5.0),
                6.6747662381009842 * z2 - 20.024298714302954 * z4 + 14.684485723822165 * z6 - 0.31784601133814211,
                0.58262136251873131 * xz * (30.0 * z2 - 33.0 * z4 - 5.0),
                0.46060262975746175 * (x2 - y2) * (11.0 * z2 * (3.0 * z2 - 1.0) - 7.0 * z2 + 1.0),
                -0.92120525951492349 * xz * (x2 - 3.0 * y2) * (11.0 * z2 - 3.0),
                0.50456490072872406 * (11.0 * z2 - 1.0) * (-6.0 * x2 * y2 + x4 + y4),
                2.3666191622317521 * xz * (10.0 * x2 * y2 - x4 - 5.0 * y4),
                10.247761577878714 * x2 * y4 - 10.247761577878714 * x4 * y2 + 0.6831841051919143 * x6 - 0.6831841051919143 * y6]
    raise ValueError(degree)


def frequency_encode_grad(feat: np.ndarray, denc: np.ndarray, n_freq: int) -> np.ndarray:
    """d/d(feature) of frequency_encode (B/rasterization/rtc/appearance_neural.cuh:37-48)."""
    if n_freq == 0:
        return denc.astype(np.float32)
    n, f = feat.shape
    d = denc.reshape(n, f, n_freq, 2)
    scale = (2.0 ** np.arange(n_freq, dtype=np.float32))
    s = feat[..., None] * scale
    return (scale * (np.cos(s) * d[..., 0] - np.sin(s) * d[..., 1])).sum(-1).astype(np.float32)


def decode_inputs(features: np.ndarray, base: np.ndarray | None, dirs: np.ndarray, mlp: MLPConfig,
                  active_degree: int) -> np.ndarray:
    """MLP input rows of the standalone decode: the rasterizer's encoding (mlp_inputs) with the view
    directions given instead of derived from means and camera."""
    n = dirs.shape[0]
    feats = features.reshape(n, -1).astype(np.float32)
    if mlp.base_input:
        feats = np.concatenate([feats, base.astype(np.float32)], axis=1)
    x = np.concatenate([frequency_encode(feats, mlp.n_frequencies),
                        sh_degree_encoding(dirs.astype(np.float32), mlp.sh_degrees, active_degree)], axis=1)
    pad = mlp.n_input_padded - x.shape[1]
    if pad:
        x = np.concatenate([x, np.zeros((n, pad), np.float32)], axis=1)
    return x.astype(np.float32)


def neural_decode(features, base, dirs, weights, mlp: MLPConfig, active_degree: int):
    """Raw MLP outputs (n, 3) of the per-primitive decode (tiny-cuda-nn eval_model as called from
    B/rasterization/rtc/appearance_neural.cuh:308-339), with the per-layer activations and the matrices."""
    mats = mlp_matrices(weights, mlp)
    y, acts = mlp_forward(decode_inputs(features, base, dirs, mlp, active_degree), mats)
    return y, acts, mats


def neural_decode_backward(features, base, dirs, dy, mats, acts, mlp: MLPConfig, active_degree: int) -> dict:
    """Gradients of the decode (backward_eval_model + encoding chain, B/rasterization/rtc/appearance_neural.cuh:348-407):
    features (n, n_feature_dims), base (n, 3) with base input, dirs (n, 3) through the SH degree values, and
    the flat tcnn-layout weight gradients."""
    n = dirs.shape[0]
    dx, dW = mlp_backward(dy.astype(np.float32), mats, acts)
    feats = features.reshape(n, -1).astype(np.float32)
    raw = np.concatenate([feats, base.astype(np.float32)], 1) if mlp.base_input else feats
    dfeat = frequency_encode_grad(raw, dx[:, :mlp.n_encoded_feature_dims], mlp.n_frequencies)
    out = dict(features=dfeat[:, :mlp.n_feature_dims].copy(),
               weights=np.concatenate([g.reshape(-1) for g in dW]).astype(np.float32),
               dirs=sh_degree_encoding_grad(dirs.astype(np.float32), dx[:, mlp.n_encoded_feature_dims:mlp.n_input_dims],
                                            mlp.sh_degrees, active_degree))
    if mlp.base_input:
        out['base'] = dfeat[:, mlp.n_feature_dims:mlp.n_feature_dims + 3].copy()
    return out


# ---------------------------------------------------------------------------------------------------------
# full pipeline
# ---------------------------------------------------------------------------------------------------------

@dataclass
class ForwardState:
    image: np.ndarray
    n_touched: np.ndarray
    depth_key: np.ndarray
    bounds: np.ndarray
    mean2d: np.ndarray
    conic_opacity: np.ndarray
    color: np.ndarray
    visible: np.ndarray          # compacted primitive indices (index order)
    depth_sorted: np.ndarray     # visible primitives in depth order
    offsets: np.ndarray          # exclusive scan of n_touched in depth order
    inst_keys: np.ndarray        # sorted tile keys
    inst_prims: np.ndarray       # sorted primitive indices
    ranges: np.ndarray           # (T, 2)
    final_T: np.ndarray
    n_contrib: np.ndarray
    mlp_out: np.ndarray | None = None
    mlp_acts: list | None = None
    mlp_mats: list | None = None


def preprocess(scene: Scene, app: Appearance, cam: Camera, mlp_out: np.ndarray | None = None) -> dict:
    n = scene.n
    gw, gh = cam.grid()
    out = dict(n_touched=np.zeros(n, np.uint32), depth_key=np.zeros(n, np.uint32),
               bounds=np.zeros((n, 4), np.uint16), mean2d=np.zeros((n, 2), np.float32),
               conic_opacity=np.zeros((n, 4), np.float32), color=np.zeros((n, 3), np.float32))
    c = cam.c_struct()
    a = app.c_struct()
    lib().efo_preprocess_forward(
        ctypes.c_int(n), _p(_f32(scene.means)), _p(_f32(scene.scales)), _p(_f32(scene.rotations)),
        _p(_f32(scene.opacities).reshape(-1)),
        _p(_f32(scene.precomputed_colors)) if scene.precomputed_colors is not None else None,
        _p(_f32(scene.base_colors)) if scene.base_colors is not None else None,
        _p(_f32(scene.residual_params).reshape(n, -1)) if scene.residual_params is not None else None,
        _p(_f32(mlp_out)) if mlp_out is not None else None,
        ctypes.byref(a), ctypes.byref(c), ctypes.c_int(gw), ctypes.c_int(gh),
        _p(out['n_touched']), _p(out['depth_key']), _p(out['bounds']), _p(out['mean2d']),
        _p(out['conic_opacity']), _p(out['color']))
    return out


def neural_outputs(scene: Scene, app: Appearance, cam: Camera):
    deg = cam.degree if cam.render_residual else 0
    mats = mlp_matrices(scene.mlp_weights, app.mlp)
    x = mlp_inputs(scene, app.mlp, cam, deg)
    y, acts = mlp_forward(x, mats)
    if deg == 0:
        y = np.zeros_like(y)
    return y, acts, mats


def sort_stage(pre: dict, cam: Camera) -> dict:
    gw, gh = cam.grid()
    n_touched = pre['n_touched']
    visible = np.nonzero(n_touched > 0)[0].astype(np.uint32)
    keys = pre['depth_key'][visible]
    order = np.argsort(keys, kind='stable')
    depth_sorted = visible[order]
    counts = n_touched[depth_sorted].astype(np.uint64)
    offsets = (np.cumsum(counts) - counts).astype(np.uint32)
    n_inst = int(counts.sum())
    ik = np.zeros(max(n_inst, 1), np.uint32)
    iv = np.zeros(max(n_inst, 1), np.uint32)
    w = lib().efo_create_instances(ctypes.c_int(len(depth_sorted)), _p(np.ascontiguousarray(depth_sorted)),
                                   _p(pre['bounds']), _p(pre['mean2d']), _p(pre['conic_opacity']), ctypes.c_int(gw),
                                   _p(ik), _p(iv))
    assert w == n_inst, f'instance count mismatch {w} != {n_inst}'
    ik, iv = ik[:n_inst], iv[:n_inst]
    torder = np.argsort(ik, kind='stable')
    ik, iv = ik[torder], iv[torder]
    n_tiles = gw * gh
    starts = np.searchsorted(ik, np.arange(n_tiles), side='left')
    ends = np.searchsorted(ik, np.arange(n_tiles), side='right')
    ranges = np.stack([starts, ends], 1).astype(np.uint32)
    ranges[starts == ends] = 0
    return dict(visible=visible, depth_sorted=depth_sorted.astype(np.uint32), offsets=offsets,
                inst_keys=ik.astype(np.uint32), inst_prims=iv.astype(np.uint32), ranges=np.ascontiguousarray(ranges))


def render(scene: Scene, app: Appearance, cam: Camera) -> ForwardState:
    mlp_out = acts = mats = None
    if app.model == 'neural':
        mlp_out, acts, mats = neural_outputs(scene, app, cam)
    pre = preprocess(scene, app, cam, mlp_out)
    st = sort_stage(pre, cam)
    gw, gh = cam.grid()
    W, H = cam.width, cam.height
    image = np.zeros((3, H, W), np.float32)
    final_T = np.zeros(H * W, np.float32)
    n_contrib = np.zeros(H * W, np.uint32)
    lib().efo_blend_forward(ctypes.c_int(W), ctypes.c_int(H), ctypes.c_int(gw), ctypes.c_int(gh), _p(st['ranges']),
                            _p(np.ascontiguousarray(st['inst_prims'])), _p(pre['bounds']), _p(pre['mean2d']),
                            _p(pre['conic_opacity']), _p(pre['color']), _p(_f32(cam.bg)), _p(image), _p(final_T),
                            _p(n_contrib))
    return ForwardState(image=image, final_T=final_T, n_contrib=n_contrib, mlp_out=mlp_out, mlp_acts=acts,
                        mlp_mats=mats, **pre, **st)


def backward(scene: Scene, app: Appearance, cam: Camera, fw: ForwardState, grad_image: np.ndarray,
             densify_rows: int = 0, densification_info: np.ndarray | None = None) -> dict:
    n = scene.n
    gw, gh = cam.grid()
    W, H = cam.width, cam.height
    g_mean2d = np.zeros((n, 2), np.float32)
    g_conic = np.zeros((n, 3), np.float32)
    g_opacity = np.zeros(n, np.float32)
    g_color = np.zeros((n, 3), np.float32)
    g_abs = np.zeros((n, 2), np.float32)
    lib().efo_blend_backward(ctypes.c_int(W), ctypes.c_int(H), ctypes.c_int(gw), ctypes.c_int(gh), _p(fw.ranges),
                             _p(np.ascontiguousarray(fw.inst_prims)), _p(fw.mean2d), _p(fw.conic_opacity), _p(fw.color),
                             _p(_f32(cam.bg)), _p(fw.image), _p(_f32(grad_image)), _p(fw.final_T), _p(fw.n_contrib),
                             ctypes.c_int(int(cam.proper_aa)), ctypes.c_int(n), _p(g_mean2d), _p(g_conic), _p(g_opacity),
                             _p(g_color), _p(g_abs))
    out = dict(g_mean2d=g_mean2d.copy(), g_conic=g_conic.copy(), g_color=g_color.copy(), g_mean2d_abs=g_abs.copy())
    neural_dmean = None
    g_residual = np.zeros((n, max(app.params_per_primitive(), 1)), np.float32)
    g_base_extra = None
    g_mlp = None
    deg = cam.degree if cam.render_residual else 0
    if app.model == 'neural':
        neural_dmean = np.zeros((n, 3), np.float32)
        ca = app.c_struct()
        contrib = fw.n_touched > 0
        dpre = _color_act_grad(fw.color, app.color_act) * g_color
        dpre[~contrib] = 0
        mats = fw.mlp_mats
        g_mlp = np.zeros(app.mlp.n_params, np.float32)
        if deg > 0:
            y = fw.mlp_out
            dy = dpre * residual_activation_grad(residual_activation(y, app.res_act), app.res_act)
            dy[~contrib] = 0
            dx, dW = mlp_backward(dy.astype(np.float32), mats, fw.mlp_acts)
            g_mlp = np.concatenate([g.reshape(-1) for g in dW]).astype(np.float32)
            mlp = app.mlp
            feats = scene.residual_params.reshape(n, -1).astype(np.float32)
            raw = np.concatenate([feats, scene.base_colors.astype(np.float32)], 1) if mlp.base_input else feats
            dfeat = frequency_encode_grad(raw, dx[:, :mlp.n_encoded_feature_dims], mlp.n_frequencies)
            g_residual[:, :mlp.n_feature_dims] = dfeat[:, :mlp.n_feature_dims]
            if mlp.base_input:
                g_base_extra = dfeat[:, mlp.n_feature_dims:mlp.n_feature_dims + 3]
            d, nrm = directions(scene.means.astype(np.float32), np.asarray(cam.position, np.float32))
            dsh = dx[:, mlp.n_encoded_feature_dims:mlp.n_input_dims]
            gd = sh_degree_encoding_grad(d, dsh, mlp.sh_degrees, deg)
            proj = (gd - (gd * d).sum(1, keepdims=True) * d) * nrm[:, None]
            neural_dmean = np.where(contrib[:, None], proj, 0).astype(np.float32)
            g_residual[~contrib] = 0
        del ca
    g_means = np.zeros((n, 3), np.float32)
    g_scales = np.zeros((n, 3), np.float32)
    g_rot = np.zeros((n, 4), np.float32)
    g_pre = np.zeros((n, 3), np.float32)
    g_base = np.zeros((n, 3), np.float32)
    g_res_c = np.zeros_like(g_residual) if app.model != 'neural' else g_residual.copy()
    if densification_info is None:
        densification_info = np.zeros((max(densify_rows, 1), n), np.float32)
    dinfo = np.ascontiguousarray(densification_info.astype(np.float32))
    lib().efo_preprocess_backward(
        ctypes.c_int(n), _p(_f32(scene.means)), _p(_f32(scene.scales)), _p(_f32(scene.rotations)),
        _p(_f32(scene.opacities).reshape(-1)),
        _p(_f32(scene.base_colors)) if scene.base_colors is not None else None,
        _p(_f32(scene.residual_params).reshape(n, -1)) if scene.residual_params is not None else None,
        ctypes.byref(app.c_struct()), ctypes.byref(cam.c_struct()), _p(fw.n_touched), _p(fw.color),
        _p(g_mean2d), _p(g_conic), _p(g_abs), _p(g_color),
        _p(neural_dmean) if neural_dmean is not None else None,
        _p(g_means), _p(g_scales), _p(g_rot), _p(g_opacity), _p(g_pre), _p(g_base), _p(g_res_c), _p(dinfo),
        ctypes.c_int(densify_rows))
    if g_base_extra is not None:
        g_base = g_base + np.where((fw.n_touched > 0)[:, None], g_base_extra, 0)
    out.update(means=g_means, scales=g_scales, rotations=g_rot, opacities=g_opacity.reshape(n, 1),
               precomputed_colors=g_pre, base_colors=g_base, residual_params=g_res_c.reshape(
                   (n,) + tuple(scene.residual_params.shape[1:])) if scene.residual_params is not None else None,
               mlp_weights=g_mlp, densification_info=dinfo)
    return out


def _color_act_grad(y: np.ndarray, act: str) -> np.ndarray:
    if act == 'none':
        return np.ones_like(y)
    if act == 'relu':
        return (y > 0).astype(np.float32)
    if act == 'softplus':
        return (-np.expm1(-10.0 * y)).astype(np.float32)
    if act == 'sigmoid':
        return (4.0 * (y - y * y)).astype(np.float32)
    if act == 'hardsigmoid':
        return np.where((y > 0) & (y < 1), 1.0, 0.0).astype(np.float32)
    if act == 'satexp':
        return (1.0 - y).astype(np.float32)
    raise ValueError(act)


def adam_step(grad, param, m, v, step, lrs, beta1=0.9, beta2=0.999, eps=1e-15):
    """In-place Adam on float32 numpy arrays (B/adam/src/adam.cu:18-87)."""
    lrs = [float(lrs)] if np.isscalar(lrs) else [float(x) for x in lrs]
    arr = (ctypes.c_double * len(lrs))(*lrs)
    for a in (grad, param, m, v):
        assert a.dtype == np.float32 and a.flags['C_CONTIGUOUS']
    lib().efo_adam_step(ctypes.c_int(param.size), _p(grad), _p(param), _p(m), _p(v), ctypes.c_int(step), arr,
                        ctypes.c_int(len(lrs)), ctypes.c_double(beta1), ctypes.c_double(beta2), ctypes.c_double(eps))


def ef_exp(x: float) -> float:
    return lib().ef_expf(ctypes.c_float(x))


def ef_log(x: float) -> float:
    return lib().ef_logf(ctypes.c_float(x))


def ef_exp2(x: float) -> float:
    return lib().ef_exp2f(ctypes.c_float(x))


def blend_alpha(mean2d, conic_opacity, px: int, py: int) -> float:
    co = conic_opacity
    return lib().efo_blend_alpha(float(mean2d[0]), float(mean2d[1]), float(co[0]), float(co[1]), float(co[2]), float(co[3]), px, py)


def sh_rest_basis(direction, degree: int) -> np.ndarray:
    out = np.zeros(15, np.float32)
    d = _f32(direction)
    n = lib().efo_sh_rest_basis(_p(d), ctypes.c_int(degree), _p(out))
    return out[:n]


def quat_to_rot(q) -> tuple[np.ndarray, float]:
    """Rotation matrix of an unnormalised (w, x, y, z) quaternion as the preprocess forms it, and |q|^2."""
    out = np.zeros(9, np.float32)
    nsq = np.zeros(1, np.float32)
    lib().efo_quat_to_rot(_p(_f32(q)), _p(out), _p(nsq))
    return out.reshape(3, 3), float(nsq[0])


def residual(app: 'Appearance', params: np.ndarray, direction, degree: int) -> np.ndarray:
    out = np.zeros(3, np.float32)
    lib().efo_residual(ctypes.byref(app.c_struct()), _p(_f32(params).reshape(-1)), _p(_f32(direction)), ctypes.c_int(degree), _p(out))
    return out


# ---------------------------------------------------------------------------------------------------------
# MCMC densification (B/densification/include/kernels_mcmc.cuh:11-146)
# ---------------------------------------------------------------------------------------------------------

MCMC_MAX_SAMPLES = 50


def philox4x32_10(ctr, key) -> np.ndarray:
    """Philox4x32-10 block (Random123) of the 4-word counter and 2-word key."""
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32))
    out = np.zeros(4, np.uint32)
    lib().efo_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def box_muller(bits_u: int, bits_v: int) -> np.ndarray:
    out = np.zeros(2, np.float32)
    lib().efo_box_muller(ctypes.c_uint32(bits_u), ctypes.c_uint32(bits_v), _p(out))
    return out


def add_noise(raw_scales, raw_rotations, raw_opacities, means, lr: float, seed: int, offset: int) -> np.ndarray:
    """New means after the MCMC noise step (the inputs are not modified)."""
    s, q, o = _f32(raw_scales), _f32(raw_rotations), _f32(raw_opacities)
    m = _f32(means).copy()
    n = m.shape[0]
    lib().efo_add_noise(n, _p(s), _p(q), _p(o), _p(m), ctypes.c_float(lr), ctypes.c_uint64(seed), ctypes.c_uint64(offset))
    return m


def relocation_table() -> np.ndarray:
    t = np.zeros((MCMC_MAX_SAMPLES, MCMC_MAX_SAMPLES), np.float32)
    lib().efo_relocation_table(_p(t))
    return t


def relocation_adjustment(old_opacities, old_scales, n_samples) -> tuple[np.ndarray, np.ndarray]:
    o, s = _f32(old_opacities).reshape(-1), _f32(old_scales)
    c = np.ascontiguousarray(np.asarray(n_samples, dtype=np.int64).reshape(-1))
    n = o.shape[0]
    new_o = np.zeros((n, 1), np.float32)
    new_s = np.zeros((n, 3), np.float32)
    lib().efo_relocation(n, _p(o), _p(s), _p(c), _p(new_o), _p(new_s))
    return new_o, new_s


# ---------------------------------------------------------------------------------------------------------
# pruning scores (Speedy-Splat), B/rasterization/include/kernels_pruning_scores.cuh:11-171
# ---------------------------------------------------------------------------------------------------------

def pruning_scores(cam: Camera, fw: ForwardState, scores: np.ndarray | None = None) -> np.ndarray:
    """scores (n,) plus, per primitive, the sum over pixels of (o dL/dalpha)^2 for the upstream gradient
    (1, 1, 1), from a forward state of `render`."""
    n = fw.n_touched.shape[0]
    out = np.zeros(n, np.float32) if scores is None else _f32(scores).copy()
    gw, gh = cam.grid()
    lib().efo_pruning_scores(cam.width, cam.height, gw, gh, _p(fw.ranges), _p(np.ascontiguousarray(fw.inst_prims)), _p(fw.mean2d),
                             _p(fw.conic_opacity), _p(fw.color), _p(_f32(cam.bg)), _p(fw.image), _p(fw.final_T), _p(fw.n_contrib),
                             _p(out))
    return out
