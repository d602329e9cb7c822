// Device code shared by the hipRTC-specialised preprocess kernels (spliced into their source text) and the
// ahead-of-time kernels (included): rasterizer constants, the deterministic decision-path math, activations,
// the quaternion rotation and the tile-contribution test.
//
// Decision-path rule: everything that decides visibility, screen bounds, touched-tile counts and instance
// emission is written with plain IEEE + - * / sqrt in a fixed order under `#pragma clang fp contract(off)`
// (and the files are compiled with -ffp-contract=off, correctly rounded fp32 divide and sqrt), plus the
// ef_expf / ef_logf below, which are themselves such fixed sequences. Preprocess (hipRTC) and instance
// creation (AOT) therefore evaluate the tile test bit-identically, and so does the CPU oracle.
//
// Reference counterparts: constants B/rasterization/include/rasterization_config.h:10-60, activations and
// quaternion B/rasterization/rtc/preprocess_common.cuh:51-188, tile test
// B/rasterization/include/tile_culling.cuh:13-65 (B/ = FasterGSVDACudaBackend/FasterGSVDACudaBackend/).
#pragma once
#ifndef EFGS_RTC
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

namespace efgs {

constexpr uint32_t tile_width = 16;
constexpr uint32_t tile_height = 12;
constexpr uint32_t tile_pixels = tile_width * tile_height;  // 192 = 3 wave64, one 16x4 row band each
constexpr float dilation = 0.3f;
constexpr float dilation_aa = 0.1f;
constexpr float min_cov2d_det = 1e-6f;
constexpr float one_minus_alpha_eps = 1e-6f;
constexpr float transmittance_threshold = 1e-4f;
constexpr float min_alpha_rcp = 255.0f;
constexpr float min_alpha = 1.0f / 255.0f;

// per-primitive record written by the preprocess for every visible primitive (48 bytes):
//   r0 = (mean2d.x, mean2d.y, conic.x, conic.y)
//   r1 = (conic.z, opacity, color.r, color.g)
//   r2 = (color.b, bits(x_min | x_max << 16), bits(y_min | y_max << 16), bits(first-tiles mask))
// where bit j of the mask (j < 4) records whether tile j of the primitive's tile rectangle (row-major order)
// passes the contribution test, as the preprocess counted it, so instance emission need not test those again
struct PrimRecord {
    float4 r0, r1, r2;
};

// tiles of a primitive's rectangle that the preprocess tests one per lane (and records in the first-tiles mask);
// further tiles are tested wave-cooperatively, by the preprocess and again by instance emission. Eight rather than
// four: a wave's cooperative loop takes one primitive per step, however few tiles it has past the first ones
// (100k SH3 Gaussians at 800x800: emission 37.5 -> 21.4 us, preprocess 24.6 -> 21.4 us; neutral on 1M at 1080p)
constexpr uint32_t n_sequential_tiles = 8;
static_assert(n_sequential_tiles <= 32, "the first-tiles mask is one 32-bit word of the record");
// floats per instance gradient record of the blend backward (dL/dmean2d 2, dL/dconic 3, dL/dopacity, dL/dcolour 3;
// with |dL/dmean2d| for three densification rows: 2 more and a pad)
constexpr uint32_t record_floats = 9;
constexpr uint32_t record_floats_abs = 12;

// ---------------------------------------------------------------------------------------------------------
// deterministic exp / log
// ---------------------------------------------------------------------------------------------------------

__device__ __forceinline__ float ef_pow2i(int k) {  // 2^k, k in [-126, 127]
    return __uint_as_float(static_cast<uint32_t>(k + 127) << 23);
}

// exp(x): Cody-Waite reduction x = k ln2 + r (15-bit ln2 head, so k * head is exact), |r| <= ln2/2, degree-7
// Taylor polynomial of e^r in Horner form, scaling by 2^k in two exact halves.
__device__ inline float ef_expf(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 88.7228394f) return __builtin_inff();
    if (x < -103.972084f) return 0.0f;
    const float kf = __builtin_rintf(x * 1.44269504f);
    const int k = static_cast<int>(kf);
    float r = x - kf * 0.693145752f;
    r = r - kf * 1.42860677e-06f;
    float p = 1.98412698e-04f + r * 2.48015873e-05f;
    p = 1.38888889e-03f + r * p;
    p = 8.33333333e-03f + r * p;
    p = 4.16666667e-02f + r * p;
    p = 1.66666667e-01f + r * p;
    p = 0.5f + r * p;
    p = 1.0f + r * p;
    p = 1.0f + r * p;
    const int k1 = k / 2;
    const int k2 = k - k1;
    return (p * ef_pow2i(k1)) * ef_pow2i(k2);
}

// log(x): x = m 2^e with m in [sqrt(1/2), sqrt(2)), log(m) = 2 atanh(s) with s = (m - 1)/(m + 1), odd series
// through s^11, e ln2 added with the split constant of ef_expf.
__device__ inline float ef_logf(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    int e_adj = 0;
    if (x < 1.17549435e-38f) { x = x * 8388608.0f; e_adj = -23; }
    const uint32_t bits = __float_as_uint(x);
    int e = static_cast<int>((bits >> 23) & 0xffu) - 127 + e_adj;
    float m = __uint_as_float((bits & 0x007fffffu) | 0x3f800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e = e + 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float z = s * s;
    float p = 0.111111111f + z * 0.0909090909f;
    p = 0.142857143f + z * p;
    p = 0.2f + z * p;
    p = 0.333333333f + z * p;
    const float log_m = 2.0f * s + (2.0f * s) * (z * p);
    const float ef = static_cast<float>(e);
    return ef * 0.693145752f + (ef * 1.42860677e-06f + log_m);
}

// 2^x for x in [-127, 0] (the blend's Gaussian factor): x = k + r with k = rint(x) and |r| <= 1/2 (r exact),
// 2^r = 1 + r q(r) with q the degree-5 polynomial of least maximum relative error on [-1/2, 1/2] (Remez
// exchange; 3.9e-9 before float rounding, <= 0.93 ulp overall), Horner form with fused multiply-adds, scaled
// by 2^k built from its exponent bits: k = -127 gives the bits 0 and so the result 0 with no select or branch
// (alpha = opacity * 2^x is far under the 1/255 threshold there).
__device__ __forceinline__ float ef_exp2f_clamped(float x) {
#pragma clang fp contract(off)
    const float k = __builtin_rintf(x);
    const float r = x - k;
    float p = __builtin_fmaf(1.546973217e-04f, r, 1.341000083e-03f);
    p = __builtin_fmaf(p, r, 9.618030861e-03f);
    p = __builtin_fmaf(p, r, 5.550297350e-02f);
    p = __builtin_fmaf(p, r, 2.402265072e-01f);
    p = __builtin_fmaf(p, r, 6.931472421e-01f);
    p = __builtin_fmaf(p, r, 1.0f);
    return p * __uint_as_float(static_cast<uint32_t>(static_cast<int>(k) + 127) << 23);
}

// 2^x for x <= 0: clamped to -127 first (NaN too)
__device__ inline float ef_exp2f(float x) { return ef_exp2f_clamped(__builtin_fmaxf(x, -127.0f)); }

__device__ __forceinline__ float ef_sigmoid(float x) {
#pragma clang fp contract(off)
    return 1.0f / (1.0f + ef_expf(-x));
}

__device__ __forceinline__ float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }
__device__ __forceinline__ float saturatef(float x) { return fminf(fmaxf(x, 0.0f), 1.0f); }

// ---------------------------------------------------------------------------------------------------------
// tile geometry and the tile-contribution test
// ---------------------------------------------------------------------------------------------------------

struct TileRect {
    uint32_t x0, x1, y0, y1;  // half-open tile index ranges
};

__device__ __forceinline__ TileRect screen_to_tile_bounds(uint32_t sx0, uint32_t sx1, uint32_t sy0, uint32_t sy1) {
    return {sx0 / tile_width, (sx1 + tile_width - 1) / tile_width, sy0 / tile_height, (sy1 + tile_height - 1) / tile_height};
}

// Whether the Gaussian (mean shifted by -0.5 to pixel-corner coordinates, conic, ln(255 opacity)) reaches
// alpha >= 1/255 anywhere in tile (tx, ty): the maximum of the Gaussian over the tile's pixel rectangle is at
// the mean when it lies inside, otherwise on the closest edge at the clamped minimiser of the 1-D quadratic.
__device__ inline bool will_primitive_contribute(float mx, float my, float cx, float cy, float cz,
                                                 uint32_t tx, uint32_t ty, float power_threshold) {
#pragma clang fp contract(off)
    const float rminx = static_cast<float>(tx * tile_width);
    const float rminy = static_cast<float>(ty * tile_height);
    const float rmaxx = static_cast<float>((tx + 1) * tile_width - 1);
    const float rmaxy = static_cast<float>((ty + 1) * tile_height - 1);
    const float x_min_diff = rminx - mx;
    const float x_left = static_cast<float>(x_min_diff >= 0.0f);
    const float not_in_x = x_left + static_cast<float>(mx > rmaxx);
    const float y_min_diff = rminy - my;
    const float y_above = static_cast<float>(y_min_diff >= 0.0f);
    const float not_in_y = y_above + static_cast<float>(my > rmaxy);
    if (not_in_y + not_in_x == 0.0f) return true;
    const float ccx = rmaxx + x_left * (rminx - rmaxx);
    const float ccy = rmaxy + y_above * (rminy - rmaxy);
    const float dfx = mx - ccx;
    const float dfy = my - ccy;
    const float dx = __builtin_copysignf(static_cast<float>(tile_width - 1), x_min_diff);
    const float dy = __builtin_copysignf(static_cast<float>(tile_height - 1), y_min_diff);
    const float tx_ = not_in_y * saturatef((dx * cx * dfx + dx * cy * dfy) / (dx * cx * dx));
    const float ty_ = not_in_x * saturatef((dy * cy * dfx + dy * cz * dfy) / (dy * cz * dy));
    const float px = ccx + tx_ * dx;
    const float py = ccy + ty_ * dy;
    const float ddx = mx - px;
    const float ddy = my - py;
    const float max_power = 0.5f * (cx * ddx * ddx + cz * ddy * ddy) + cy * ddx * ddy;
    return max_power <= power_threshold;
}

// alpha-threshold exponent ln(255 opacity) of a stored opacity, shared by preprocess and instance creation
__device__ __forceinline__ float power_threshold_of(float opacity) {
#pragma clang fp contract(off)
    return ef_logf(opacity * min_alpha_rcp);
}

// ---------------------------------------------------------------------------------------------------------
// rotation
// ---------------------------------------------------------------------------------------------------------

struct Mat3 {
    float m11, m12, m13, m21, m22, m23, m31, m32, m33;
};

// rotation matrix of an unnormalised (w, x, y, z) quaternion; norm_sq receives |q|^2
__device__ inline Mat3 quaternion_to_rotation(float r, float x, float y, float z, float& norm_sq) {
#pragma clang fp contract(off)
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float rx = r * x, ry = r * y, rz = r * z;
    norm_sq = r * r + xx + yy + zz;
    const float s = 1.0f / norm_sq;
    return {1.0f - 2.0f * (yy + zz) * s, 2.0f * (xy - rz) * s, 2.0f * (xz + ry) * s,
            2.0f * (xy + rz) * s, 1.0f - 2.0f * (xx + zz) * s, 2.0f * (yz - rx) * s,
            2.0f * (xz - ry) * s, 2.0f * (yz + rx) * s, 1.0f - 2.0f * (xx + yy) * s};
}

// dL/dq for dL/dR of quaternion_to_rotation
__device__ inline float4 quaternion_to_rotation_backward(float r, float x, float y, float z, const Mat3& g) {
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float rx = r * x, ry = r * y, rz = r * z;
    const float s = 1.0f / (r * r + xx + yy + zz);
    const float d_xx = g.m22 + g.m33, d_yy = g.m11 + g.m33, d_zz = g.m11 + g.m22;
    const float d_rz = g.m21 - g.m12, d_xy = g.m21 + g.m12;
    const float d_ry = g.m13 - g.m31, d_xz = g.m13 + g.m31;
    const float d_rx = g.m32 - g.m23, d_yz = g.m32 + g.m23;
    const float t = 2.0f * s;
    const float h = t * (xy * d_xy + xz * d_xz + yz * d_yz + rx * d_rx + ry * d_ry + rz * d_rz - xx * d_xx - yy * d_yy - zz * d_zz);
    return make_float4(t * (x * d_rx + y * d_ry + z * d_rz - r * h),
                       t * (r * d_rx - 2.0f * x * d_xx + y * d_xy + z * d_xz - x * h),
                       t * (r * d_ry + x * d_xy - 2.0f * y * d_yy + z * d_yz - y * h),
                       t * (r * d_rz + x * d_xz + y * d_yz - 2.0f * z * d_zz - z * h));
}

// ---------------------------------------------------------------------------------------------------------
// activations (ids: base 0 none / 1 exp(3x); residual 0 none / 1 tanh / 2 softplus(beta 10);
// color 0 none / 1 relu / 2 softplus / 3 sigmoid(4x) / 4 hardsigmoid / 5 satexp)
// ---------------------------------------------------------------------------------------------------------

__device__ __forceinline__ float softplus10(float x) { return (fmaxf(10.0f * x, 0.0f) + log1pf(expf(-fabsf(10.0f * x)))) / 10.0f; }
__device__ __forceinline__ float softplus10_grad(float y) { return -expm1f(-10.0f * y); }

template <int ACT>
__device__ __forceinline__ float base_activation(float x) { return ACT == 1 ? expf(3.0f * x) : x; }
template <int ACT>
__device__ __forceinline__ float base_activation_grad(float x) { return ACT == 1 ? 3.0f * expf(3.0f * x) : 1.0f; }

// tanh x = 1 - 2 / (e^{2x} + 1) with the hardware exp and reciprocal (absolute error a few 1e-7; saturates
// to +-1 through e^{2x} = inf / 0)
__device__ __forceinline__ float fast_tanh(float x) { return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * x) + 1.0f); }

template <int ACT>
__device__ __forceinline__ float residual_activation(float x) {
    if (ACT == 1) return fast_tanh(x);
    if (ACT == 2) return softplus10(x);
    return x;
}
template <int ACT>
__device__ __forceinline__ float residual_activation_grad(float y) {  // in terms of the output
    if (ACT == 1) return 1.0f - y * y;
    if (ACT == 2) return softplus10_grad(y);
    return 1.0f;
}

template <int ACT>
__device__ __forceinline__ float color_activation(float x) {
    if (ACT == 1) return fmaxf(x + 0.5f, 0.0f);
    if (ACT == 2) return softplus10(x + 0.5f);
    if (ACT == 3) return ef_sigmoid(4.0f * x);
    if (ACT == 4) return clampf(6.0f * x / 6.0f + 0.5f, 0.0f, 1.0f);
    if (ACT == 5) return -expm1f(-x);
    return x + 0.5f;
}
template <int ACT>
__device__ __forceinline__ float color_activation_grad(float y) {  // in terms of the output
    if (ACT == 1) return y > 0.0f ? 1.0f : 0.0f;
    if (ACT == 2) return softplus10_grad(y);
    if (ACT == 3) return 4.0f * (y - y * y);
    if (ACT == 4) return (y > 0.0f && y < 1.0f) ? 1.0f : 0.0f;
    if (ACT == 5) return 1.0f - y;
    return 1.0f;
}

// view direction normalize(mean - cam) and 1/|mean - cam| (clamped like the reference's norm_rcp)
__device__ __forceinline__ float3 view_direction(float3 m, float3 c, float& norm_rcp) {
    const float vx = m.x - c.x, vy = m.y - c.y, vz = m.z - c.z;
    norm_rcp = 1.0f / sqrtf(fmaxf(vx * vx + vy * vy + vz * vz, 1e-24f));
    return make_float3(norm_rcp * vx, norm_rcp * vy, norm_rcp * vz);
}

// tangent-plane projection of a direction gradient, scaled to a mean gradient
__device__ __forceinline__ float3 direction_grad_to_mean(float3 gd, float3 d, float norm_rcp) {
    const float k = gd.x * d.x + gd.y * d.y + gd.z * d.z;
    return make_float3((gd.x - k * d.x) * norm_rcp, (gd.y - k * d.y) * norm_rcp, (gd.z - k * d.z) * norm_rcp);
}

}  // namespace efgs
