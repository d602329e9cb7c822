/*
 * efgs_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C CPU restatement of the reference's fused-appearance rasterizer, used as the parity checker for
 * the HIP product path. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * nothing in the product package links, imports or calls it.
 *
 * Every function follows a reference source (paths relative to the reference repository root,
 * FasterGSVDACudaBackend/FasterGSVDACudaBackend/ abbreviated as "B/"):
 *   constants ............ B/rasterization/include/rasterization_config.h:10-60
 *   activations .......... B/rasterization/rtc/preprocess_common.cuh:51-142
 *   quaternion -> R ...... B/rasterization/rtc/preprocess_common.cuh:144-188
 *   tile culling ......... B/rasterization/include/tile_culling.cuh:13-65
 *   preprocess forward ... B/rasterization/rtc/preprocess_forward.cu:53-277
 *   appearance chunks .... B/rasterization/rtc/appearance_{sh,sv,nasg,nasgabor}.cuh
 *   instance creation .... B/rasterization/include/kernels_common.cuh:33-137
 *   blend forward ........ B/rasterization/include/kernels_forward.cuh:26-166
 *   blend backward ....... B/rasterization/include/kernels_backward.cuh:12-231
 *   preprocess backward .. B/rasterization/rtc/preprocess_backward.cu:78-403
 *   adam ................. B/adam/src/adam.cu:18-87
 *
 * Floating point: built with -ffp-contract=off and without fast-math, so every + - * / sqrt is one IEEE
 * round-to-nearest operation in source order. The decision path (visibility, screen bounds, tile
 * contribution, compaction) uses ef_expf/ef_logf below, a fixed sequence of such operations that the HIP
 * kernels execute identically, which makes keys, counts and tile ranges bit-comparable. The reference
 * itself uses CUDA fast-math intrinsics there (setup.py:130-134), whose exact bits cannot be reproduced
 * off-device; ef_expf/ef_logf are pinned against libm by the tests instead.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define EFO_TILE_W 16
#define EFO_TILE_H 12
#define EFO_SUBTILE_W 8 /* reference warp subtile, kernels_forward.cuh:52-62 */
#define EFO_SUBTILE_H 4

static const float k_dilation = 0.3f;
static const float k_dilation_aa = 0.1f;
static const float k_min_cov2d_det = 1e-6f;
static const float k_one_minus_alpha_eps = 1e-6f;
static const float k_transmittance_threshold = 1e-4f;
static const float k_min_alpha_rcp = 255.0f;
#define K_MIN_ALPHA (1.0f / 255.0f)

/* ------------------------------------------------------------------------------------------------------ */
/* deterministic exp / log (shared algorithm with the HIP decision path)                                  */
/* ------------------------------------------------------------------------------------------------------ */

static float ef_pow2i(int k) { /* 2^k for k in [-126, 127], built from the exponent bits */
    uint32_t bits = (uint32_t)(k + 127) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* exp(x): Cody-Waite reduction x = k ln2 + r with ln2 split in a 15-bit head and a tail, |r| <= ln2/2,
 * degree-7 Taylor polynomial of e^r in Horner form, and scaling by 2^k in two exact halves. */
float ef_expf(float x) {
    if (x != x) return x;
    if (x > 88.7228394f) return INFINITY;
    if (x < -103.972084f) return 0.0f;
    const float kf = rintf(x * 1.44269504f);
    const int k = (int)kf;
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

/* log(x): x = m 2^e with m in [sqrt(1/2), sqrt(2)), log(m) = 2 atanh(s), s = (m - 1)/(m + 1), odd series to
 * s^11, and e ln2 added with the same split constant as ef_expf. */
float ef_logf(float x) {
    if (x != x) return x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (x == INFINITY) return x;
    int e_adj = 0;
    if (x < 1.17549435e-38f) { x = x * 8388608.0f; e_adj = -23; }
    uint32_t bits;
    memcpy(&bits, &x, 4);
    int e = (int)((bits >> 23) & 0xff) - 127 + e_adj;
    uint32_t mbits = (bits & 0x007fffffu) | 0x3f800000u;
    float m;
    memcpy(&m, &mbits, 4);
    if (m > 1.41421354f) { m = m * 0.5f; e = e + 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float z = s * s;
    float p = 0.111111111f + z * 0.0909090909f;
    p = 0.142857143f + z * p;
    p = 0.2f + z * p;
    p = 0.333333333f + z * p;
    const float log_m = 2.0f * s + (2.0f * s) * (z * p);
    const float ef = (float)e;
    return ef * 0.693145752f + (ef * 1.42860677e-06f + log_m);
}

static float ef_sigmoid(float x) { return 1.0f / (1.0f + ef_expf(-x)); }

/* 2^x for x <= 0: x clamped to -127 (NaN too), k = rint(x), r = x - k exact, 2^r = 1 + r q(r) with q the
 * degree-5 minimax polynomial (relative error) on [-1/2, 1/2] in Horner form with fused multiply-adds, scaled
 * by 2^k built from its exponent bits (k = -127 gives 0). */
float ef_exp2f(float x) {
    x = fmaxf(x, -127.0f);
    const float k = rintf(x);
    const float r = x - k;
    float p = fmaf(1.546973217e-04f, r, 1.341000083e-03f);
    p = fmaf(p, r, 9.618030861e-03f);
    p = fmaf(p, r, 5.550297350e-02f);
    p = fmaf(p, r, 2.402265072e-01f);
    p = fmaf(p, r, 6.931472421e-01f);
    p = fmaf(p, r, 1.0f);
    uint32_t bits = (uint32_t)((int)k + 127) << 23;
    float scale;
    memcpy(&scale, &bits, sizeof scale);
    return p * scale;
}

/* exponent of the exp2-scaled conic (ex, ey, ez) at offset (dx, dy): the quadratic form of
 * kernels_forward.cuh:124, ex dx^2 + ey dx dy + ez dy^2, grouped by dy as (ez dy + ey dx) dy + ex dx dx with two
 * fused multiply-adds. The blends evaluate it in this order (the terms in dx alone are shared by the pixels of a
 * column), so host and device agree bit for bit; the reference's grouping differs in the last bits of the exponent. */
static float blend_exponent(float ex, float ey, float ez, float dx, float dy) {
    return fmaf(fmaf(ez, dy, ey * dx), dy, (ex * dx) * dx);
}

/* transmittance after a fragment of opacity alpha, T (1 - alpha) with one rounding (as the blends compute it) */
static float transmit(float T, float alpha) { return fmaf(-T, alpha, T); }


static float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }
static float saturatef(float x) { return fminf(fmaxf(x, 0.0f), 1.0f); }

/* ------------------------------------------------------------------------------------------------------ */
/* settings                                                                                               */
/* ------------------------------------------------------------------------------------------------------ */

typedef struct {
    float w2c[12];     /* rows 0..2 of the world-to-view transform, row-major */
    float cam_pos[3];
    float bg[3];
    int degree;        /* appearance degree used for rendering (0 when the residual is off) */
    int width, height;
    float fx, fy, cx, cy;
    float near_plane, far_plane;
    int proper_aa;
    int render_base;
} efo_cam;

typedef struct {
    int model;         /* 0 precomputed, 1 sh, 2 sv, 3 nasg, 4 nasgabor, 5 neural */
    int base_act;      /* 0 none, 1 exp(3x) */
    int res_act;       /* 0 none, 1 tanh, 2 softplus(beta=10) */
    int color_act;     /* 0 none, 1 relu, 2 softplus, 3 sigmoid(4x), 4 hardsigmoid, 5 satexp */
    int dir_grad;
    int n_units;       /* sh: rest bases (deg+1)^2-1, sv: sites, nasg/nasgabor: lobes, neural: feature dims */
} efo_app;

/* ------------------------------------------------------------------------------------------------------ */
/* activations, B/rasterization/rtc/preprocess_common.cuh:51-142                                          */
/* ------------------------------------------------------------------------------------------------------ */

static float relu(float x) { return fmaxf(x, 0.0f); }
static float softplus(float x, float b) { return (relu(b * x) + log1pf(expf(-fabsf(b * x)))) / b; }
static float softplus_grad(float y, float b) { return -expm1f(-b * y); }

static float base_act(const efo_app* a, float x) { return a->base_act == 1 ? expf(3.0f * x) : x; }
static float base_act_grad(const efo_app* a, float x) { return a->base_act == 1 ? 3.0f * expf(3.0f * x) : 1.0f; }
static float res_act(const efo_app* a, float x) {
    switch (a->res_act) { case 1: return tanhf(x); case 2: return softplus(x, 10.0f); default: return x; }
}
static float res_act_grad(const efo_app* a, float y) {
    switch (a->res_act) { case 1: return 1.0f - y * y; case 2: return softplus_grad(y, 10.0f); default: return 1.0f; }
}
static float color_act(const efo_app* a, float x) {
    switch (a->color_act) {
        case 0: return x + 0.5f;
        case 1: return relu(x + 0.5f);
        case 2: return softplus(x + 0.5f, 10.0f);
        case 3: return ef_sigmoid(4.0f * x);
        case 4: return clampf(6.0f * x / 6.0f + 0.5f, 0.0f, 1.0f);
        case 5: return -expm1f(-x);
    }
    return x;
}
static float color_act_grad(const efo_app* a, float y) {
    switch (a->color_act) {
        case 0: return 1.0f;
        case 1: return y > 0.0f ? 1.0f : 0.0f;
        case 2: return softplus_grad(y, 10.0f);
        case 3: return 4.0f * (y - y * y);
        case 4: return 6.0f * ((y > 0.0f && y < 1.0f) ? (1.0f / 6.0f) : 0.0f);
        case 5: return 1.0f - y;
    }
    return 1.0f;
}

/* ------------------------------------------------------------------------------------------------------ */
/* geometry helpers                                                                                       */
/* ------------------------------------------------------------------------------------------------------ */

typedef struct { float m11, m12, m13, m21, m22, m23, m31, m32, m33; } mat3;

/* B/rasterization/rtc/preprocess_common.cuh:144-159 ; quaternion (w, x, y, z), unnormalized */
static mat3 quat_to_rot(const float* q, float* norm_sq) {
    const float r = q[0], x = q[1], y = q[2], z = q[3];
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float rx = r * x, ry = r * y, rz = r * z;
    *norm_sq = r * r + xx + yy + zz;
    const float s = 1.0f / *norm_sq;
    mat3 R = {
        1.0f - 2.0f * (yy + zz) * s, 2.0f * (xy - rz) * s, 2.0f * (xz + ry) * s,
        2.0f * (xy + rz) * s, 1.0f - 2.0f * (xx + zz) * s, 2.0f * (yz - rx) * s,
        2.0f * (xz - ry) * s, 2.0f * (yz + rx) * s, 1.0f - 2.0f * (xx + yy) * s
    };
    return R;
}

/* B/rasterization/rtc/preprocess_common.cuh:161-188 */
static void quat_to_rot_backward(const float* q, const mat3* g, float* out) {
    const float r = q[0], x = q[1], y = q[2], z = q[3];
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float rx = r * x, ry = r * y, rz = r * z;
    const float norm_sq = r * r + xx + yy + zz;
    const float s = 1.0f / norm_sq;
    const float d_xx = g->m22 + g->m33, d_yy = g->m11 + g->m33, d_zz = g->m11 + g->m22;
    const float d_rz = g->m21 - g->m12, d_xy = g->m21 + g->m12;
    const float d_ry = g->m13 - g->m31, d_xz = g->m13 + g->m31;
    const float d_rx = g->m32 - g->m23, d_yz = g->m32 + g->m23;
    const float t = 2.0f * s;
    const float h = t * (xy * d_xy + xz * d_xz + yz * d_yz + rx * d_rx + ry * d_ry + rz * d_rz - xx * d_xx - yy * d_yy - zz * d_zz);
    out[0] = t * (x * d_rx + y * d_ry + z * d_rz - r * h);
    out[1] = t * (r * d_rx - 2.0f * x * d_xx + y * d_xy + z * d_xz - x * h);
    out[2] = t * (r * d_ry + x * d_xy - 2.0f * y * d_yy + z * d_yz - y * h);
    out[3] = t * (r * d_rz + x * d_xz + y * d_yz - 2.0f * z * d_zz - z * h);
}

/* B/rasterization/include/tile_culling.cuh:23-65 ; mean already shifted by -0.5 */
int efo_will_primitive_contribute(float mx, float my, float cx, float cy, float cz, uint32_t tx, uint32_t ty, float power_threshold) {
    const float rminx = (float)(tx * EFO_TILE_W), rminy = (float)(ty * EFO_TILE_H);
    const float rmaxx = (float)((tx + 1) * EFO_TILE_W - 1), rmaxy = (float)((ty + 1) * EFO_TILE_H - 1);
    const float x_min_diff = rminx - mx;
    const float x_left = (float)(x_min_diff >= 0.0f);
    const float not_in_x = x_left + (float)(mx > rmaxx);
    const float y_min_diff = rminy - my;
    const float y_above = (float)(y_min_diff >= 0.0f);
    const float not_in_y = y_above + (float)(my > rmaxy);
    if (not_in_y + not_in_x == 0.0f) return 1;
    const float ccx = rmaxx + x_left * (rminx - rmaxx);
    const float ccy = rmaxy + y_above * (rminy - rmaxy);
    const float dfx = mx - ccx, dfy = my - ccy;
    const float dx = copysignf((float)(EFO_TILE_W - 1), x_min_diff);
    const float dy = copysignf((float)(EFO_TILE_H - 1), y_min_diff);
    const float tx_ = not_in_y * saturatef((dx * cx * dfx + dx * cy * dfy) / (dx * cx * dx));
    const float ty_ = not_in_x * saturatef((dy * cy * dfx + dy * cz * dfy) / (dy * cz * dy));
    const float px = ccx + tx_ * dx, py = ccy + ty_ * dy;
    const float ddx = mx - px, ddy = my - py;
    const float max_power = 0.5f * (cx * ddx * ddx + cz * ddy * ddy) + cy * ddx * ddy;
    return max_power <= power_threshold;
}

static void dir_from(const float* mean, const float* cam, float* dir, float* norm_rcp) {
    const float v0 = mean[0] - cam[0], v1 = mean[1] - cam[1], v2 = mean[2] - cam[2];
    const float n = 1.0f / sqrtf(fmaxf(v0 * v0 + v1 * v1 + v2 * v2, 1e-24f));
    dir[0] = n * v0; dir[1] = n * v1; dir[2] = n * v2;
    if (norm_rcp) *norm_rcp = n;
}

/* ------------------------------------------------------------------------------------------------------ */
/* appearance chunks (forward)                                                                            */
/* ------------------------------------------------------------------------------------------------------ */

static const float sh_c1 = 0.48860251190291987f;
static const float sh_c2a = 1.0925484305920792f, sh_c2b = 0.94617469575755997f, sh_c2c = 0.31539156525251999f;
static const float sh_c2d = 0.54627421529603959f, sh_c2e = 1.8923493915151202f;
static const float sh_c3a = 0.59004358992664352f, sh_c3b = 1.7701307697799304f, sh_c3c = 2.8906114426405538f;
static const float sh_c3d = 0.45704579946446572f, sh_c3e = 2.2852289973223288f, sh_c3f = 1.865881662950577f;
static const float sh_c3g = 1.1195289977703462f, sh_c3h = 1.4453057213202769f, sh_c3i = 3.5402615395598609f;
static const float sh_c3j = 4.5704579946446566f, sh_c3k = 5.597644988851731f;

/* SH basis values of the rest bands for a unit direction, band order of appearance_sh.cuh:43-61 */
static int sh_rest_basis(const float* d, int degree, float* b) {
    const float x = d[0], y = d[1], z = d[2];
    int n = 0;
    b[n++] = -sh_c1 * y; b[n++] = sh_c1 * z; b[n++] = -sh_c1 * x;
    if (degree > 1) {
        const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, xz = x * z, yz = y * z;
        b[n++] = sh_c2a * xy; b[n++] = -sh_c2a * yz; b[n++] = sh_c2b * zz - sh_c2c;
        b[n++] = -sh_c2a * xz; b[n++] = sh_c2d * (xx - yy);
        if (degree > 2) {
            b[n++] = y * (sh_c3a * yy - sh_c3b * xx); b[n++] = sh_c3c * xy * z;
            b[n++] = y * (sh_c3d - sh_c3e * zz); b[n++] = z * (sh_c3f * zz - sh_c3g);
            b[n++] = x * (sh_c3d - sh_c3e * zz); b[n++] = sh_c3h * z * (xx - yy);
            b[n++] = x * (sh_c3b * yy - sh_c3a * xx);
        }
    }
    return n;
}

/* B/rasterization/rtc/appearance_sh.cuh:30-65 */
static void sh_residual(const efo_app* a, const float* coef, const float* dir, int degree, float* out) {
    out[0] = out[1] = out[2] = 0.0f;
    if (degree == 0) return;
    float b[15];
    const int n = sh_rest_basis(dir, degree, b);
    for (int i = 0; i < n; i++) for (int c = 0; c < 3; c++) out[c] += b[i] * coef[3 * i + c];
    for (int c = 0; c < 3; c++) out[c] = res_act(a, out[c]);
}

/* B/rasterization/rtc/appearance_sv.cuh:26-58 */
static void sv_residual(const efo_app* a, const float* p, const float* dir, int sites, float* out) {
    out[0] = out[1] = out[2] = 0.0f;
    if (sites == 0) return;
    float max_logit = -1e30f, wsum = 0.0f, wc[3] = {0, 0, 0};
    for (int s = 0; s < sites; s++, p += 7) {
        const float len = sqrtf(p[0] * p[0] + p[1] * p[1] + p[2] * p[2]);
        const float inv = 1.0f / fmaxf(len, 1e-12f);
        const float d0 = inv * p[0] - dir[0], d1 = inv * p[1] - dir[1], d2 = inv * p[2] - dir[2];
        const float dist = sqrtf(d0 * d0 + d1 * d1 + d2 * d2);
        const float logit = -expf(p[3]) * dist;
        const float nm = fmaxf(max_logit, logit);
        const float rescale = expf(max_logit - nm);
        const float w = expf(fminf(logit - nm, 0.0f));
        wsum = wsum * rescale + w;
        for (int c = 0; c < 3; c++) wc[c] = wc[c] * rescale + w * res_act(a, p[4 + c]);
        max_logit = nm;
    }
    for (int c = 0; c < 3; c++) out[c] = (1.0f / wsum) * wc[c];
}

typedef struct { float x[3], z[3], ct, cp, cu, st, sp, su; } frame_t;

/* B/rasterization/rtc/appearance_nasg.cuh:180-199 */
static frame_t build_frame(float ct, float cp, float cu) {
    frame_t f;
    f.ct = ct; f.cp = cp; f.cu = cu;
    f.st = sqrtf(1.0f - ct * ct); f.sp = sqrtf(1.0f - cp * cp); f.su = sqrtf(1.0f - cu * cu);
    f.x[0] = ct * cp * cu - f.st * f.su;
    f.x[1] = f.st * cp * cu + ct * f.su;
    f.x[2] = -f.sp * cu;
    f.z[0] = ct * f.sp; f.z[1] = f.st * f.sp; f.z[2] = cp;
    return f;
}

static const float k_two_pi = 6.28318530717958647692f;
static const float k_lobe_eps = 5e-6f, k_lobe_eps_norm = 1e-8f, k_cos_limit = 0.999999f;
static const float k_pole_limit = 0.99999988f, k_shape_limit = 1e4f, k_freq_scale = 20.0f;

/* B/rasterization/rtc/appearance_nasg.cuh:201-235 and appearance_nasgabor.cuh:63-99 (gabor != 0) */
static void lobe_residual(const efo_app* a, const float* p, const float* dir, int lobes, int gabor, float* out) {
    out[0] = out[1] = out[2] = 0.0f;
    const int stride = gabor ? 9 : 8;
    for (int l = 0; l < lobes; l++, p += stride) {
        const frame_t f = build_frame(clampf(tanhf(p[0]), -k_cos_limit, k_cos_limit),
                                      clampf(tanhf(p[1]), -k_cos_limit, k_cos_limit),
                                      clampf(tanhf(p[2]), -k_cos_limit, k_cos_limit));
        const float lambda = fminf(expf(p[3]), k_shape_limit);
        const float an = fminf(expf(p[4]), k_shape_limit);
        const float vz = dir[0] * f.z[0] + dir[1] * f.z[1] + dir[2] * f.z[2];
        const float vx = dir[0] * f.x[0] + dir[1] * f.x[1] + dir[2] * f.x[2];
        const float vzc = clampf(vz, -k_pole_limit, k_pole_limit);
        const float K = 0.5f * (vzc + 1.0f);
        const float Ke = k_lobe_eps + an * vx * vx / (1.0f - vzc * vzc);
        const float E = powf(K, Ke);
        const float N = lambda * sqrtf(1.0f + an) / (k_two_pi * (1.0f + k_lobe_eps_norm - expf(-2.0f * lambda)));
        const float P = expf(2.0f * lambda * (E * K - 1.0f));
        float pdf;
        if (gabor) {
            const float k = (tanhf(p[5]) + 1.0f) * k_freq_scale;
            const float G = 0.5f * (1.0f + cosf(k * vx));
            pdf = vz >= k_pole_limit ? 1.0f : (vz > -k_pole_limit ? P * E * G * N : 0.0f);
        } else {
            pdf = vz >= k_pole_limit ? 1.0f : (vz > -k_pole_limit ? P * E * N : 0.0f);
        }
        const float* w = p + (gabor ? 6 : 5);
        for (int c = 0; c < 3; c++) out[c] += pdf * res_act(a, w[c]);
    }
}

static int residual_param_count(const efo_app* a) {
    switch (a->model) {
        case 1: return 3 * a->n_units;
        case 2: return 7 * a->n_units;
        case 3: return 8 * a->n_units;
        case 4: return 9 * a->n_units;
        case 5: return a->n_units;
    }
    return 0;
}

static int active_residual_param_count(const efo_app* a, int degree) {
    switch (a->model) {
        case 1: return 3 * ((degree + 1) * (degree + 1) - 1);
        case 2: return 7 * degree;
        case 3: return 8 * degree;
        case 4: return 9 * degree;
        case 5: return degree > 0 ? a->n_units : 0;
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------------ */
/* preprocess forward, B/rasterization/rtc/preprocess_forward.cu:53-277                                   */
/* ------------------------------------------------------------------------------------------------------ */

/* Per primitive: n_touched (0 = culled), depth key, screen bounds (x_min, x_max, y_min, y_max), mean2d,
 * conic + opacity, activated color. mlp_out (n, 3) supplies the raw fp16-rounded residual mlp outputs for
 * the neural model, which the numpy part of the oracle evaluates. */
void efo_preprocess_forward(
    int n, const float* means, const float* scales, const float* rotations, const float* opacities,
    const float* precomputed, const float* base, const float* residual, const float* mlp_out,
    const efo_app* app, const efo_cam* cam, int grid_w, int grid_h,
    uint32_t* n_touched, uint32_t* depth_key, uint16_t* bounds, float* mean2d, float* conic_opacity, float* color)
{
    const float* W = cam->w2c;
    const int n_res = residual_param_count(app);
    for (int p = 0; p < n; p++) {
        n_touched[p] = 0;
        depth_key[p] = 0;
        const float* m = means + 3 * p;
        const float depth = W[8] * m[0] + W[9] * m[1] + W[10] * m[2] + W[11];
        if (depth < cam->near_plane || depth > cam->far_plane) continue;
        float opacity = ef_sigmoid(opacities[p]);
        if (opacity < K_MIN_ALPHA) continue;
        const float* s = scales + 3 * p;
        const float var[3] = { ef_expf(2.0f * s[0]), ef_expf(2.0f * s[1]), ef_expf(2.0f * s[2]) };
        float qn;
        const mat3 R = quat_to_rot(rotations + 4 * p, &qn);
        if (qn < 1e-8f) continue;
        const mat3 RSS = { R.m11 * var[0], R.m12 * var[1], R.m13 * var[2],
                           R.m21 * var[0], R.m22 * var[1], R.m23 * var[2],
                           R.m31 * var[0], R.m32 * var[1], R.m33 * var[2] };
        const float c11 = RSS.m11 * R.m11 + RSS.m12 * R.m12 + RSS.m13 * R.m13;
        const float c12 = RSS.m11 * R.m21 + RSS.m12 * R.m22 + RSS.m13 * R.m23;
        const float c13 = RSS.m11 * R.m31 + RSS.m12 * R.m32 + RSS.m13 * R.m33;
        const float c22 = RSS.m21 * R.m21 + RSS.m22 * R.m22 + RSS.m23 * R.m23;
        const float c23 = RSS.m21 * R.m31 + RSS.m22 * R.m32 + RSS.m23 * R.m33;
        const float c33 = RSS.m31 * R.m31 + RSS.m32 * R.m32 + RSS.m33 * R.m33;
        const float x = (W[0] * m[0] + W[1] * m[1] + W[2] * m[2] + W[3]) / depth;
        const float y = (W[4] * m[0] + W[5] * m[1] + W[6] * m[2] + W[7]) / depth;
        const float wf = (float)cam->width, hf = (float)cam->height;
        const float cl = (-0.15f * wf - cam->cx) / cam->fx, cr = (1.15f * wf - cam->cx) / cam->fx;
        const float ct = (-0.15f * hf - cam->cy) / cam->fy, cb = (1.15f * hf - cam->cy) / cam->fy;
        const float xc = clampf(x, cl, cr), yc = clampf(y, ct, cb);
        const float j11 = cam->fx / depth, j13 = -j11 * xc, j22 = cam->fy / depth, j23 = -j22 * yc;
        const float a1x = j11 * W[0] + j13 * W[8], a1y = j11 * W[1] + j13 * W[9], a1z = j11 * W[2] + j13 * W[10];
        const float a2x = j22 * W[4] + j23 * W[8], a2y = j22 * W[5] + j23 * W[9], a2z = j22 * W[6] + j23 * W[10];
        const float b1x = a1x * c11 + a1y * c12 + a1z * c13, b1y = a1x * c12 + a1y * c22 + a1z * c23, b1z = a1x * c13 + a1y * c23 + a1z * c33;
        const float b2x = a2x * c11 + a2y * c12 + a2z * c13, b2y = a2x * c12 + a2y * c22 + a2z * c23, b2z = a2x * c13 + a2y * c23 + a2z * c33;
        float cv_x = b1x * a1x + b1y * a1y + b1z * a1z;
        const float cv_y = b1x * a2x + b1y * a2y + b1z * a2z;
        float cv_z = b2x * a2x + b2y * a2y + b2z * a2z;
        const float det_raw = cv_x * cv_z - cv_y * cv_y;
        const float ks = cam->proper_aa ? k_dilation_aa : k_dilation;
        cv_x += ks;
        cv_z += ks;
        const float det = cv_x * cv_z - cv_y * cv_y;
        if (det < k_min_cov2d_det) continue;
        const float conx = cv_z / det, cony = -cv_y / det, conz = cv_x / det;
        if (cam->proper_aa) {
            opacity *= sqrtf(fmaxf(det_raw / det, 0.0f));
            if (opacity < K_MIN_ALPHA) continue;
        }
        const float m2x = x * cam->fx + cam->cx, m2y = y * cam->fy + cam->cy;
        const float pt = ef_logf(opacity * k_min_alpha_rcp);
        const float cutoff = 2.0f * pt;
        const float ex = fmaxf(sqrtf(cv_x * cutoff) - 0.5f, 0.0f);
        const float ey = fmaxf(sqrtf(cv_z * cutoff) - 0.5f, 0.0f);
        const float pw = (float)(grid_w * EFO_TILE_W), ph = (float)(grid_h * EFO_TILE_H);
        /* equivalent of min(padded, max(0, float2int_rd/ru(v))) with the clamp done before the conversion */
        const int bx0 = (int)floorf(clampf(m2x - ex, -1.0f, pw + 1.0f));
        const int bx1 = (int)ceilf(clampf(m2x + ex, -1.0f, pw + 1.0f));
        const int by0 = (int)floorf(clampf(m2y - ey, -1.0f, ph + 1.0f));
        const int by1 = (int)ceilf(clampf(m2y + ey, -1.0f, ph + 1.0f));
        const uint32_t sb[4] = {
            (uint32_t)(bx0 < 0 ? 0 : (bx0 > (int)pw ? (int)pw : bx0)),
            (uint32_t)(bx1 < 0 ? 0 : (bx1 > (int)pw ? (int)pw : bx1)),
            (uint32_t)(by0 < 0 ? 0 : (by0 > (int)ph ? (int)ph : by0)),
            (uint32_t)(by1 < 0 ? 0 : (by1 > (int)ph ? (int)ph : by1)) };
        const uint32_t tb0 = sb[0] / EFO_TILE_W, tb1 = (sb[1] + EFO_TILE_W - 1) / EFO_TILE_W;
        const uint32_t tb2 = sb[2] / EFO_TILE_H, tb3 = (sb[3] + EFO_TILE_H - 1) / EFO_TILE_H;
        const uint32_t n_max = (tb1 - tb0) * (tb3 - tb2);
        if (n_max == 0) continue;
        uint32_t count = 0;
        const uint32_t bw = tb1 - tb0;
        for (uint32_t i = 0; i < n_max; i++) {
            const uint32_t tx = tb0 + i % bw, ty = tb2 + i / bw;
            count += (uint32_t)efo_will_primitive_contribute(m2x - 0.5f, m2y - 0.5f, conx, cony, conz, tx, ty, pt);
        }
        if (count == 0) continue;
        n_touched[p] = count;
        memcpy(&depth_key[p], &depth, 4);
        for (int k = 0; k < 4; k++) bounds[4 * p + k] = (uint16_t)sb[k];
        mean2d[2 * p] = m2x; mean2d[2 * p + 1] = m2y;
        conic_opacity[4 * p] = conx; conic_opacity[4 * p + 1] = cony; conic_opacity[4 * p + 2] = conz; conic_opacity[4 * p + 3] = opacity;
        float* col = color + 3 * p;
        if (app->model == 0) {
            for (int c = 0; c < 3; c++) col[c] = precomputed[3 * p + c];
            continue;
        }
        float dir[3];
        dir_from(m, cam->cam_pos, dir, NULL);
        float res[3] = {0, 0, 0};
        const float* rp = residual + (size_t)n_res * p;
        switch (app->model) {
            case 1: sh_residual(app, rp, dir, cam->degree, res); break;
            case 2: sv_residual(app, rp, dir, cam->degree, res); break;
            case 3: lobe_residual(app, rp, dir, cam->degree, 0, res); break;
            case 4: lobe_residual(app, rp, dir, cam->degree, 1, res); break;
            case 5:
                if (cam->degree > 0) for (int c = 0; c < 3; c++) res[c] = res_act(app, mlp_out[3 * p + c]);
                break;
        }
        for (int c = 0; c < 3; c++) {
            const float b = base_act(app, base[3 * p + c]);
            float v = color_act(app, b + res[c]);
            if (!cam->render_base) v = fabsf(v - color_act(app, b));
            col[c] = v;
        }
    }
}

/* ------------------------------------------------------------------------------------------------------ */
/* instance creation, B/rasterization/include/kernels_common.cuh:33-137                                   */
/* ------------------------------------------------------------------------------------------------------ */

/* Emits (tile key, primitive) pairs for the visible primitives in depth order; returns the count. Tiles of a
 * primitive are visited in row-major order of its tile bounding rectangle. */
uint32_t efo_create_instances(
    int n_visible, const uint32_t* sorted_prims, const uint16_t* bounds, const float* mean2d,
    const float* conic_opacity, int grid_w, uint32_t* keys, uint32_t* vals)
{
    uint32_t w = 0;
    for (int i = 0; i < n_visible; i++) {
        const uint32_t p = sorted_prims[i];
        const uint16_t* sb = bounds + 4 * p;
        const uint32_t tb0 = sb[0] / EFO_TILE_W, tb1 = (sb[1] + EFO_TILE_W - 1) / EFO_TILE_W;
        const uint32_t tb2 = sb[2] / EFO_TILE_H, tb3 = (sb[3] + EFO_TILE_H - 1) / EFO_TILE_H;
        const uint32_t bw = tb1 - tb0, cnt = bw * (tb3 - tb2);
        const float* co = conic_opacity + 4 * p;
        const float pt = ef_logf(co[3] * k_min_alpha_rcp);
        for (uint32_t k = 0; k < cnt; k++) {
            const uint32_t tx = tb0 + k % bw, ty = tb2 + k / bw;
            if (efo_will_primitive_contribute(mean2d[2 * p] - 0.5f, mean2d[2 * p + 1] - 0.5f, co[0], co[1], co[2], tx, ty, pt)) {
                keys[w] = ty * (uint32_t)grid_w + tx;
                vals[w] = p;
                w++;
            }
        }
    }
    return w;
}

/* ------------------------------------------------------------------------------------------------------ */
/* blend forward, B/rasterization/include/kernels_forward.cuh:26-166                                      */
/* ------------------------------------------------------------------------------------------------------ */

void efo_blend_forward(
    int width, int height, int grid_w, int grid_h, const uint32_t* ranges, const uint32_t* inst_prims,
    const uint16_t* bounds, const float* mean2d, const float* conic_opacity, const float* color, const float* bg,
    float* image, float* final_T, uint32_t* n_contrib)
{
    const float log2e = 1.44269504089f;
    const int n_pixels = width * height;
    for (int ty = 0; ty < grid_h; ty++) for (int tx = 0; tx < grid_w; tx++) {
        const uint32_t t = (uint32_t)(ty * grid_w + tx);
        const uint32_t r0 = ranges[2 * t], r1 = ranges[2 * t + 1];
        for (int ly = 0; ly < EFO_TILE_H; ly++) for (int lx = 0; lx < EFO_TILE_W; lx++) {
            const int px = tx * EFO_TILE_W + lx, py = ty * EFO_TILE_H + ly;
            if (px >= width || py >= height) continue;
            const int sx0 = tx * EFO_TILE_W + (lx / EFO_SUBTILE_W) * EFO_SUBTILE_W;
            const int sy0 = ty * EFO_TILE_H + (ly / EFO_SUBTILE_H) * EFO_SUBTILE_H;
            const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
            float C[3] = {0, 0, 0}, T = 1.0f;
            uint32_t last = 0;
            for (uint32_t i = r0; i < r1; i++) {
                const uint32_t p = inst_prims[i];
                const uint16_t* sb = bounds + 4 * p;
                if (!((int)sb[0] < sx0 + EFO_SUBTILE_W && sx0 < (int)sb[1] && (int)sb[2] < sy0 + EFO_SUBTILE_H && sy0 < (int)sb[3])) continue;
                const float* co = conic_opacity + 4 * p;
                const float ex = -0.5f * log2e * co[0], ey = -log2e * co[1], ez = -0.5f * log2e * co[2];
                const float dx = mean2d[2 * p] - pxf, dy = mean2d[2 * p + 1] - pyf;
                const float g = ef_exp2f(fminf(blend_exponent(ex, ey, ez, dx, dy), 0.0f));
                const float alpha = co[3] * g;
                if (alpha < K_MIN_ALPHA) continue;
                const float w = T * alpha;
                for (int c = 0; c < 3; c++) C[c] = fmaf(w, color[3 * p + c], C[c]);
                T = transmit(T, alpha);
                last = i - r0 + 1;
                if (T < k_transmittance_threshold) break;
            }
            const int pix = py * width + px;
            for (int c = 0; c < 3; c++) image[c * n_pixels + pix] = fmaf(T, bg[c], C[c]);
            final_T[pix] = T;
            n_contrib[pix] = last;
        }
    }
}

/* ------------------------------------------------------------------------------------------------------ */
/* blend backward, B/rasterization/include/kernels_backward.cuh:12-231                                    */
/* ------------------------------------------------------------------------------------------------------ */

/* Accumulates, per primitive, dL/d(mean2d) (n,2), dL/d(conic) (n,3; off-diagonal convention of the
 * reference), dL/d(opacity) (n; times sigmoid' unless proper_aa), dL/d(color) (n,3) and the summed
 * absolute mean2d gradients (n,2). The per-pixel walk is front to back over the pixel's tile list, the
 * same quantities the reference reconstructs per bucket from its checkpoints. */
void efo_blend_backward(
    int width, int height, int grid_w, int grid_h, const uint32_t* ranges, const uint32_t* inst_prims,
    const float* mean2d, const float* conic_opacity, const float* color, const float* bg,
    const float* image, const float* grad_image, const float* final_T, const uint32_t* n_contrib, int proper_aa,
    int n_prims, float* g_mean2d, float* g_conic, float* g_opacity, float* g_color, float* g_mean2d_abs)
{
    const float log2e = 1.44269504089f;
    const int n_pixels = width * height;
    memset(g_mean2d, 0, sizeof(float) * 2 * n_prims);
    memset(g_conic, 0, sizeof(float) * 3 * n_prims);
    memset(g_opacity, 0, sizeof(float) * n_prims);
    memset(g_color, 0, sizeof(float) * 3 * n_prims);
    memset(g_mean2d_abs, 0, sizeof(float) * 2 * n_prims);
    for (int ty = 0; ty < grid_h; ty++) for (int tx = 0; tx < grid_w; tx++) {
        const uint32_t t = (uint32_t)(ty * grid_w + tx);
        const uint32_t r0 = ranges[2 * t];
        for (int ly = 0; ly < EFO_TILE_H; ly++) for (int lx = 0; lx < EFO_TILE_W; lx++) {
            const int px = tx * EFO_TILE_W + lx, py = ty * EFO_TILE_H + ly;
            if (px >= width || py >= height) continue;
            const int pix = py * width + px;
            const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
            const float Tf = final_T[pix];
            float g[3], after[3];
            for (int c = 0; c < 3; c++) {
                g[c] = grad_image[c * n_pixels + pix];
                after[c] = image[c * n_pixels + pix] - Tf * bg[c];
            }
            const float grad_alpha_common = Tf * -(g[0] * bg[0] + g[1] * bg[1] + g[2] * bg[2]);
            float T = 1.0f;
            const uint32_t last = n_contrib[pix];
            for (uint32_t k = 0; k < last; k++) {
                const uint32_t p = inst_prims[r0 + k];
                const float* co = conic_opacity + 4 * p;
                const float ex = -0.5f * log2e * co[0], ey = -log2e * co[1], ez = -0.5f * log2e * co[2];
                const float dx = mean2d[2 * p] - pxf, dy = mean2d[2 * p + 1] - pyf;
                const float G = ef_exp2f(fminf(blend_exponent(ex, ey, ez, dx, dy), 0.0f));
                const float alpha = co[3] * G;
                if (alpha < K_MIN_ALPHA) continue;
                const float w = T * alpha;
                const float* col = color + 3 * p;
                for (int c = 0; c < 3; c++) {
                    g_color[3 * p + c] += w * g[c];
                    after[c] -= w * col[c];
                }
                const float oma = 1.0f - alpha;
                const float rcp = 1.0f / fmaxf(oma, k_one_minus_alpha_eps);
                const float dadc = (T * col[0] - after[0] * rcp) * g[0] + (T * col[1] - after[1] * rcp) * g[1] + (T * col[2] - after[2] * rcp) * g[2];
                const float dalpha = dadc + grad_alpha_common * rcp;
                g_opacity[p] += G * dalpha;
                const float h = -alpha * dalpha;
                g_conic[3 * p] += 0.5f * h * (dx * dx);
                g_conic[3 * p + 1] += 0.5f * h * (dx * dy);
                g_conic[3 * p + 2] += 0.5f * h * (dy * dy);
                const float gmx = h * (co[0] * dx + co[1] * dy), gmy = h * (co[1] * dx + co[2] * dy);
                g_mean2d[2 * p] += gmx;
                g_mean2d[2 * p + 1] += gmy;
                g_mean2d_abs[2 * p] += fabsf(gmx);
                g_mean2d_abs[2 * p + 1] += fabsf(gmy);
                T = transmit(T, alpha);
            }
        }
    }
    if (!proper_aa) {
        for (int p = 0; p < n_prims; p++) {
            const float o = conic_opacity[4 * p + 3];
            g_opacity[p] = (o - o * o) * g_opacity[p];
        }
    }
}

/* ------------------------------------------------------------------------------------------------------ */
/* appearance chunks (backward)                                                                           */
/* ------------------------------------------------------------------------------------------------------ */

static void project_direction_grad(const float* gd, const float* dir, float norm_rcp, float* out) {
    const float d = gd[0] * dir[0] + gd[1] * dir[1] + gd[2] * dir[2];
    for (int c = 0; c < 3; c++) out[c] = (gd[c] - d * dir[c]) * norm_rcp;
}

/* B/rasterization/rtc/appearance_sh.cuh:67-157 */
static void sh_residual_backward(const efo_app* a, const float* coef, const float* gcol, float* gcoef,
                                 const float* mean, const float* cam, int degree, float* dmean) {
    dmean[0] = dmean[1] = dmean[2] = 0.0f;
    if (degree == 0) return;
    float nr, d[3];
    dir_from(mean, cam, d, &nr);
    float res[3];
    sh_residual(a, coef, d, degree, res);
    float ds[3];
    for (int c = 0; c < 3; c++) ds[c] = gcol[c] * res_act_grad(a, res[c]);
    float b[15];
    const int n = sh_rest_basis(d, degree, b);
    for (int i = 0; i < n; i++) for (int c = 0; c < 3; c++) gcoef[3 * i + c] = b[i] * ds[c];
    const float x = d[0], y = d[1], z = d[2];
    float gx[3], gy[3], gz[3];
    const float* C = coef;
#define CF(i, c) C[3 * (i) + (c)]
    for (int c = 0; c < 3; c++) {
        gx[c] = -sh_c1 * CF(2, c);
        gy[c] = -sh_c1 * CF(0, c);
        gz[c] = sh_c1 * CF(1, c);
        if (degree > 1) {
            const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, xz = x * z, yz = y * z;
            gx[c] += sh_c2a * y * CF(3, c) - sh_c2a * z * CF(6, c) + sh_c2a * x * CF(7, c);
            gy[c] += sh_c2a * x * CF(3, c) - sh_c2a * z * CF(4, c) - sh_c2a * y * CF(7, c);
            gz[c] += -sh_c2a * y * CF(4, c) + sh_c2e * z * CF(5, c) - sh_c2a * x * CF(6, c);
            if (degree > 2) {
                gx[c] += -sh_c3i * xy * CF(8, c) + sh_c3c * yz * CF(9, c) + (sh_c3d - sh_c3e * zz) * CF(12, c)
                         + sh_c3c * xz * CF(13, c) + sh_c3b * (yy - xx) * CF(14, c);
                gy[c] += sh_c3b * (yy - xx) * CF(8, c) + sh_c3c * xz * CF(9, c) + (sh_c3d - sh_c3e * zz) * CF(10, c)
                         - sh_c3c * yz * CF(13, c) + sh_c3i * xy * CF(14, c);
                gz[c] += sh_c3c * xy * CF(9, c) - sh_c3j * yz * CF(10, c) + (sh_c3k * zz - sh_c3g) * CF(11, c)
                         - sh_c3j * xz * CF(12, c) + sh_c3h * (xx - yy) * CF(13, c);
            }
        }
    }
#undef CF
    const float gd[3] = { gx[0] * ds[0] + gx[1] * ds[1] + gx[2] * ds[2],
                          gy[0] * ds[0] + gy[1] * ds[1] + gy[2] * ds[2],
                          gz[0] * ds[0] + gz[1] * ds[1] + gz[2] * ds[2] };
    project_direction_grad(gd, d, nr, dmean);
}

/* B/rasterization/rtc/appearance_sv.cuh:60-139 */
static void sv_residual_backward(const efo_app* a, const float* p0, const float* gcol, float* gp,
                                 const float* mean, const float* cam, int sites, float* dmean) {
    dmean[0] = dmean[1] = dmean[2] = 0.0f;
    if (sites == 0) return;
    float nr, d[3];
    dir_from(mean, cam, d, &nr);
    float max_logit = -1e30f, wsum = 0.0f, wc[3] = {0, 0, 0};
    const float* p = p0;
    for (int s = 0; s < sites; s++, p += 7) {
        const float inv = 1.0f / fmaxf(sqrtf(p[0] * p[0] + p[1] * p[1] + p[2] * p[2]), 1e-12f);
        const float d0 = inv * p[0] - d[0], d1 = inv * p[1] - d[1], d2 = inv * p[2] - d[2];
        const float dist = sqrtf(d0 * d0 + d1 * d1 + d2 * d2);
        const float logit = -expf(p[3]) * dist;
        const float nm = fmaxf(max_logit, logit);
        const float rescale = expf(max_logit - nm);
        const float w = expf(fminf(logit - nm, 0.0f));
        wsum = wsum * rescale + w;
        for (int c = 0; c < 3; c++) wc[c] = wc[c] * rescale + w * res_act(a, p[4 + c]);
        max_logit = nm;
    }
    const float wr = 1.0f / wsum;
    const float gmean = gcol[0] * (wr * wc[0]) + gcol[1] * (wr * wc[1]) + gcol[2] * (wr * wc[2]);
    float gd[3] = {0, 0, 0};
    p = p0;
    float* g = gp;
    for (int s = 0; s < sites; s++, p += 7, g += 7) {
        const float lr = 1.0f / fmaxf(sqrtf(p[0] * p[0] + p[1] * p[1] + p[2] * p[2]), 1e-12f);
        const float site[3] = { lr * p[0], lr * p[1], lr * p[2] };
        const float sd[3] = { site[0] - d[0], site[1] - d[1], site[2] - d[2] };
        const float dist = sqrtf(sd[0] * sd[0] + sd[1] * sd[1] + sd[2] * sd[2]);
        const float tau = expf(p[3]);
        const float w = expf(fminf(-tau * dist - max_logit, 0.0f)) * wr;
        float col[3];
        for (int c = 0; c < 3; c++) {
            col[c] = res_act(a, p[4 + c]);
            g[4 + c] = w * gcol[c] * res_act_grad(a, col[c]);
        }
        const float glogit = w * ((gcol[0] * col[0] + gcol[1] * col[1] + gcol[2] * col[2]) - gmean);
        g[3] = -dist * tau * glogit;
        const float gdist = -tau * glogit;
        const float f = gdist / fmaxf(dist, 1e-12f);
        const float gsd[3] = { f * sd[0], f * sd[1], f * sd[2] };
        const float dd = gsd[0] * site[0] + gsd[1] * site[1] + gsd[2] * site[2];
        for (int c = 0; c < 3; c++) {
            g[c] = (gsd[c] - dd * site[c]) * lr;
            gd[c] -= gsd[c];
        }
    }
    project_direction_grad(gd, d, nr, dmean);
}

/* B/rasterization/rtc/appearance_nasg.cuh:237-350 and appearance_nasgabor.cuh:101-223 (gabor != 0) */
static void lobe_residual_backward(const efo_app* a, const float* p, const float* gcol, float* g,
                                   const float* mean, const float* cam, int lobes, int gabor, float* dmean) {
    dmean[0] = dmean[1] = dmean[2] = 0.0f;
    if (lobes == 0) return;
    const int stride = gabor ? 9 : 8;
    float nr, d[3];
    dir_from(mean, cam, d, &nr);
    float gd[3] = {0, 0, 0};
    for (int l = 0; l < lobes; l++, p += stride, g += stride) {
        const float th = tanhf(p[0]), tp = tanhf(p[1]), tu = tanhf(p[2]);
        const frame_t f = build_frame(clampf(th, -k_cos_limit, k_cos_limit), clampf(tp, -k_cos_limit, k_cos_limit),
                                      clampf(tu, -k_cos_limit, k_cos_limit));
        const float lu = expf(p[3]), au = expf(p[4]);
        const float lambda = fminf(lu, k_shape_limit), an = fminf(au, k_shape_limit);
        float tk = 0.0f, k = 0.0f;
        if (gabor) { tk = tanhf(p[5]); k = (tk + 1.0f) * k_freq_scale; }
        const float* wr = p + (gabor ? 6 : 5);
        const float w[3] = { res_act(a, wr[0]), res_act(a, wr[1]), res_act(a, wr[2]) };
        const float vz = d[0] * f.z[0] + d[1] * f.z[1] + d[2] * f.z[2];
        const float vx = d[0] * f.x[0] + d[1] * f.x[1] + d[2] * f.x[2];
        const float vzc = clampf(vz, -k_pole_limit, k_pole_limit);
        const float K = 0.5f * (vzc + 1.0f);
        const float om = 1.0f - vzc * vzc;
        const float Ke = k_lobe_eps + an * vx * vx / om;
        const float E = powf(K, Ke);
        const float nd = k_two_pi * (1.0f + k_lobe_eps_norm - expf(-2.0f * lambda));
        const float N = lambda * sqrtf(1.0f + an) / nd;
        const float G = gabor ? 0.5f * (1.0f + cosf(k * vx)) : 1.0f;
        const float P = expf(2.0f * lambda * (E * K - 1.0f));
        const float logK = logf(K);
        const int valid = fabsf(vz) < k_pole_limit;
        const float pdf = vz >= k_pole_limit ? 1.0f : (valid ? P * E * G * N : 0.0f);
        const int wo = gabor ? 6 : 5;
        for (int c = 0; c < 3; c++) g[wo + c] = gcol[c] * pdf * res_act_grad(a, w[c]);
        const float gpdf = valid ? (gcol[0] * w[0] + gcol[1] * w[1] + gcol[2] * w[2]) : 0.0f;
        const float dP_dl = P * 2.0f * (E * K - 1.0f);
        const float s1a = sqrtf(1.0f + an);
        const float dN_dl = (s1a * nd - lambda * s1a * 2.0f * k_two_pi * expf(-2.0f * lambda)) / (nd * nd);
        const float dpdf_dl = dP_dl * E * G * N + P * E * G * dN_dl;
        g[3] = lu >= k_shape_limit ? 0.0f : gpdf * dpdf_dl * lambda;
        const float dE_da = E * logK * (vx * vx / om);
        const float dP_da = P * 2.0f * lambda * K * dE_da;
        const float dN_da = (lambda / (2.0f * s1a)) / nd;
        const float dpdf_da = dP_da * E * G * N + P * dE_da * G * N + P * E * G * dN_da;
        g[4] = au >= k_shape_limit ? 0.0f : gpdf * dpdf_da * an;
        float dG_dvx = 0.0f;
        if (gabor) {
            const float skv = sinf(k * vx);
            const float dpdf_dk = P * E * (-0.5f * skv * vx) * N;
            g[5] = gpdf * dpdf_dk * k_freq_scale * (1.0f - tk * tk);
            dG_dvx = -0.5f * skv * k;
        }
        const float dE_dvx = E * logK * (2.0f * an * vx / om);
        const float dP_dvx = P * 2.0f * lambda * K * dE_dvx;
        const float gvx = gpdf * (dP_dvx * E * G * N + P * dE_dvx * G * N + P * E * dG_dvx * N);
        const float dKe_dvz = an * vx * vx * 2.0f * vz / (om * om);
        const float dE_dvz = E * (Ke / K) * 0.5f + E * logK * dKe_dvz;
        const float dP_dvz = P * 2.0f * lambda * (K * dE_dvz + E * 0.5f);
        const float gvz = gpdf * (dP_dvz * E * G * N + P * dE_dvz * G * N);
        const float gxv[3] = { gvx * d[0], gvx * d[1], gvx * d[2] };
        const float gzv[3] = { gvz * d[0], gvz * d[1], gvz * d[2] };
        for (int c = 0; c < 3; c++) gd[c] += gvx * f.x[c] + gvz * f.z[c];
        const float dst = -f.ct / f.st, dsp = -f.cp / f.sp, dsu = -f.cu / f.su;
        const float gct = gxv[0] * (f.cp * f.cu - dst * f.su) + gxv[1] * (dst * f.cp * f.cu + f.su)
                          + gzv[0] * f.sp + gzv[1] * dst * f.sp;
        const float gcp = gxv[0] * f.ct * f.cu + gxv[1] * f.st * f.cu - gxv[2] * dsp * f.cu
                          + gzv[0] * f.ct * dsp + gzv[1] * f.st * dsp + gzv[2];
        const float gcu = gxv[0] * (f.ct * f.cp - f.st * dsu) + gxv[1] * (f.st * f.cp + f.ct * dsu) - gxv[2] * f.sp;
        g[0] = fabsf(th) >= k_cos_limit ? 0.0f : gct * (1.0f - th * th);
        g[1] = fabsf(tp) >= k_cos_limit ? 0.0f : gcp * (1.0f - tp * tp);
        g[2] = fabsf(tu) >= k_cos_limit ? 0.0f : gcu * (1.0f - tu * tu);
    }
    project_direction_grad(gd, d, nr, dmean);
}

/* ------------------------------------------------------------------------------------------------------ */
/* preprocess backward, B/rasterization/rtc/preprocess_backward.cu:78-403                                 */
/* ------------------------------------------------------------------------------------------------------ */

/* g_opacity enters as the blend backward's output and leaves as dL/d(opacity logit). For the neural model
 * the residual chunk is evaluated by the numpy part of the oracle: neural_dmean supplies its direction
 * gradient (n,3) and its residual/base contributions are added there. densification_info has
 * densify_rows (0, 2 or 3) rows of n entries. */
void efo_preprocess_backward(
    int n, const float* means, const float* scales, const float* rotations, const float* opacities,
    const float* base, const float* residual, const efo_app* app, const efo_cam* cam,
    const uint32_t* n_touched, const float* color,
    const float* g_mean2d, const float* g_conic, const float* g_mean2d_abs, const float* g_color,
    const float* neural_dmean,
    float* g_means, float* g_scales, float* g_rotations, float* g_opacity,
    float* g_precomputed, float* g_base, float* g_residual, float* densification_info, int densify_rows)
{
    const float* W = cam->w2c;
    const int n_res = residual_param_count(app);
    const int n_act = active_residual_param_count(app, cam->degree);
    for (int p = 0; p < n; p++) {
        const int contributes = n_touched[p] > 0;
        float* gm = g_means + 3 * p;
        float* gs = g_scales + 3 * p;
        float* gr = g_rotations + 4 * p;
        if (!contributes) {
            memset(gm, 0, 12); memset(gs, 0, 12); memset(gr, 0, 16);
            if (app->model == 0) memset(g_precomputed + 3 * p, 0, 12);
            else {
                memset(g_base + 3 * p, 0, 12);
                if (n_res > 0) memset(g_residual + (size_t)n_res * p, 0, sizeof(float) * n_res);
            }
            continue;
        }
        const float* m = means + 3 * p;
        float dm_color[3] = {0, 0, 0};
        if (app->model == 0) {
            for (int c = 0; c < 3; c++) g_precomputed[3 * p + c] = g_color[3 * p + c];
        } else {
            float dpre[3];
            for (int c = 0; c < 3; c++) {
                dpre[c] = color_act_grad(app, color[3 * p + c]) * g_color[3 * p + c];
                g_base[3 * p + c] = cam->render_base ? base_act_grad(app, base[3 * p + c]) * dpre[c] : 0.0f;
            }
            float* grp = g_residual + (size_t)n_res * p;
            const float* rp = residual + (size_t)n_res * p;
            switch (app->model) {
                case 1: sh_residual_backward(app, rp, dpre, grp, m, cam->cam_pos, cam->degree, dm_color); break;
                case 2: sv_residual_backward(app, rp, dpre, grp, m, cam->cam_pos, cam->degree, dm_color); break;
                case 3: lobe_residual_backward(app, rp, dpre, grp, m, cam->cam_pos, cam->degree, 0, dm_color); break;
                case 4: lobe_residual_backward(app, rp, dpre, grp, m, cam->cam_pos, cam->degree, 1, dm_color); break;
                case 5: for (int c = 0; c < 3; c++) dm_color[c] = neural_dmean[3 * p + c]; break;
            }
            if (app->model != 5) for (int i = n_act; i < n_res; i++) grp[i] = 0.0f;
        }
        const float depth = W[8] * m[0] + W[9] * m[1] + W[10] * m[2] + W[11];
        const float x = (W[0] * m[0] + W[1] * m[1] + W[2] * m[2] + W[3]) / depth;
        const float y = (W[4] * m[0] + W[5] * m[1] + W[6] * m[2] + W[7]) / depth;
        const float* s = scales + 3 * p;
        const float var[3] = { ef_expf(2.0f * s[0]), ef_expf(2.0f * s[1]), ef_expf(2.0f * s[2]) };
        float qn;
        const float* q = rotations + 4 * p;
        const mat3 R = quat_to_rot(q, &qn);
        const mat3 RSS = { R.m11 * var[0], R.m12 * var[1], R.m13 * var[2],
                           R.m21 * var[0], R.m22 * var[1], R.m23 * var[2],
                           R.m31 * var[0], R.m32 * var[1], R.m33 * var[2] };
        const float c11 = RSS.m11 * R.m11 + RSS.m12 * R.m12 + RSS.m13 * R.m13;
        const float c12 = RSS.m11 * R.m21 + RSS.m12 * R.m22 + RSS.m13 * R.m23;
        const float c13 = RSS.m11 * R.m31 + RSS.m12 * R.m32 + RSS.m13 * R.m33;
        const float c22 = RSS.m21 * R.m21 + RSS.m22 * R.m22 + RSS.m23 * R.m23;
        const float c23 = RSS.m21 * R.m31 + RSS.m22 * R.m32 + RSS.m23 * R.m33;
        const float c33 = RSS.m31 * R.m31 + RSS.m32 * R.m32 + RSS.m33 * R.m33;
        const float wf = (float)cam->width, hf = (float)cam->height;
        const float cl = (-0.15f * wf - cam->cx) / cam->fx, cr = (1.15f * wf - cam->cx) / cam->fx;
        const float ct = (-0.15f * hf - cam->cy) / cam->fy, cb = (1.15f * hf - cam->cy) / cam->fy;
        const float xc = clampf(x, cl, cr), yc = clampf(y, ct, cb);
        const float j11 = cam->fx / depth, j13 = -j11 * xc, j22 = cam->fy / depth, j23 = -j22 * yc;
        const float a1x = j11 * W[0] + j13 * W[8], a1y = j11 * W[1] + j13 * W[9], a1z = j11 * W[2] + j13 * W[10];
        const float a2x = j22 * W[4] + j23 * W[8], a2y = j22 * W[5] + j23 * W[9], a2z = j22 * W[6] + j23 * W[10];
        const float b1x = a1x * c11 + a1y * c12 + a1z * c13, b1y = a1x * c12 + a1y * c22 + a1z * c23, b1z = a1x * c13 + a1y * c23 + a1z * c33;
        const float b2x = a2x * c11 + a2y * c12 + a2z * c13, b2y = a2x * c12 + a2y * c22 + a2z * c23, b2z = a2x * c13 + a2y * c23 + a2z * c33;
        const float a_raw = b1x * a1x + b1y * a1y + b1z * a1z;
        const float bb_ = b1x * a2x + b1y * a2y + b1z * a2z;
        const float c_raw = b2x * a2x + b2y * a2y + b2z * a2z;
        const float ks = cam->proper_aa ? k_dilation_aa : k_dilation;
        const float A = a_raw + ks, Cc = c_raw + ks, B = bb_;
        const float aa = A * A, bb = B * B, cc = Cc * Cc, ac = A * Cc, ab = A * B, bc = B * Cc;
        const float det = ac - bb;
        const float det_rcp_sq = 1.0f / (det * det);
        const float* gc = g_conic + 3 * p;
        float dcx = det_rcp_sq * (2.0f * bc * gc[1] - cc * gc[0] - bb * gc[2]);
        float dcy = det_rcp_sq * (bc * gc[0] - (ac + bb) * gc[1] + ab * gc[2]);
        float dcz = det_rcp_sq * (2.0f * ab * gc[1] - bb * gc[0] - aa * gc[2]);
        if (cam->proper_aa) {
            const float o = ef_sigmoid(opacities[p]);
            const float gconv = g_opacity[p];
            const float det_raw = a_raw * c_raw - bb;
            const float rad = fmaxf(det_raw / det, 0.0f);
            g_opacity[p] = gconv * sqrtf(rad) * o * (1.0f - o);
        }
        const float d11 = a1x * a1x * dcx + 2.0f * a1x * a2x * dcy + a2x * a2x * dcz;
        const float d12 = a1x * a1y * dcx + (a1x * a2y + a1y * a2x) * dcy + a2x * a2y * dcz;
        const float d13 = a1x * a1z * dcx + (a1x * a2z + a1z * a2x) * dcy + a2x * a2z * dcz;
        const float d22 = a1y * a1y * dcx + 2.0f * a1y * a2y * dcy + a2y * a2y * dcz;
        const float d23 = a1y * a1z * dcx + (a1y * a2z + a1z * a2y) * dcy + a2y * a2z * dcz;
        const float d33 = a1z * a1z * dcx + 2.0f * a1z * a2z * dcy + a2z * a2z * dcz;
        const float g1x = 2.0f * (b1x * dcx + b2x * dcy), g1y = 2.0f * (b1y * dcx + b2y * dcy), g1z = 2.0f * (b1z * dcx + b2z * dcy);
        const float g2x = 2.0f * (b1x * dcy + b2x * dcz), g2y = 2.0f * (b1y * dcy + b2y * dcz), g2z = 2.0f * (b1z * dcy + b2z * dcz);
        const float dj11 = W[0] * g1x + W[1] * g1y + W[2] * g1z;
        const float dj22 = W[4] * g2x + W[5] * g2y + W[6] * g2z;
        const float dj13 = W[8] * g1x + W[9] * g1y + W[10] * g1z;
        const float dj23 = W[8] * g2x + W[9] * g2y + W[10] * g2z;
        const float gmx = g_mean2d[2 * p], gmy = g_mean2d[2 * p + 1];
        if (densify_rows > 0) {
            densification_info[p] += 1.0f;
            const float nx = 0.5f * (gmx * wf), ny = 0.5f * (gmy * hf);
            densification_info[n + p] += sqrtf(nx * nx + ny * ny);
            if (densify_rows > 2) {
                const float ax = 0.5f * (g_mean2d_abs[2 * p] * wf), ay = 0.5f * (g_mean2d_abs[2 * p + 1] * hf);
                densification_info[2 * n + p] += sqrtf(ax * ax + ay * ay);
            }
        }
        float mcx = j11 * gmx, mcy = j22 * gmy, mcz = -j11 * x * gmx - j22 * y * gmy;
        const int vx = x >= cl && x <= cr, vy = y >= ct && y <= cb;
        if (vx) mcx -= j11 * dj13 / depth;
        if (vy) mcy -= j22 * dj23 / depth;
        const float fxv = 1.0f + (float)vx, fyv = 1.0f + (float)vy;
        mcz += (j11 * (fxv * xc * dj13 - dj11) + j22 * (fyv * yc * dj23 - dj22)) / depth;
        const float sx = W[0] * mcx + W[4] * mcy + W[8] * mcz;
        const float sy = W[1] * mcx + W[5] * mcy + W[9] * mcz;
        const float sz = W[2] * mcx + W[6] * mcy + W[10] * mcz;
        if (app->dir_grad) { gm[0] = sx + dm_color[0]; gm[1] = sy + dm_color[1]; gm[2] = sz + dm_color[2]; }
        else { gm[0] = sx; gm[1] = sy; gm[2] = sz; }
        const float dv0 = R.m11 * R.m11 * d11 + R.m21 * R.m21 * d22 + R.m31 * R.m31 * d33 + 2.0f * (R.m11 * R.m21 * d12 + R.m11 * R.m31 * d13 + R.m21 * R.m31 * d23);
        const float dv1 = R.m12 * R.m12 * d11 + R.m22 * R.m22 * d22 + R.m32 * R.m32 * d33 + 2.0f * (R.m12 * R.m22 * d12 + R.m12 * R.m32 * d13 + R.m22 * R.m32 * d23);
        const float dv2 = R.m13 * R.m13 * d11 + R.m23 * R.m23 * d22 + R.m33 * R.m33 * d33 + 2.0f * (R.m13 * R.m23 * d12 + R.m13 * R.m33 * d13 + R.m23 * R.m33 * d23);
        gs[0] = 2.0f * var[0] * dv0; gs[1] = 2.0f * var[1] * dv1; gs[2] = 2.0f * var[2] * dv2;
        const mat3 dR = {
            2.0f * (RSS.m11 * d11 + RSS.m21 * d12 + RSS.m31 * d13), 2.0f * (RSS.m12 * d11 + RSS.m22 * d12 + RSS.m32 * d13), 2.0f * (RSS.m13 * d11 + RSS.m23 * d12 + RSS.m33 * d13),
            2.0f * (RSS.m11 * d12 + RSS.m21 * d22 + RSS.m31 * d23), 2.0f * (RSS.m12 * d12 + RSS.m22 * d22 + RSS.m32 * d23), 2.0f * (RSS.m13 * d12 + RSS.m23 * d22 + RSS.m33 * d23),
            2.0f * (RSS.m11 * d13 + RSS.m21 * d23 + RSS.m31 * d33), 2.0f * (RSS.m12 * d13 + RSS.m22 * d23 + RSS.m32 * d33), 2.0f * (RSS.m13 * d13 + RSS.m23 * d23 + RSS.m33 * d33) };
        quat_to_rot_backward(q, &dR, gr);
    }
}

/* ------------------------------------------------------------------------------------------------------ */
/* adam, B/adam/src/adam.cu:18-87                                                                          */
/* ------------------------------------------------------------------------------------------------------ */

/* lrs: n_lrs per-column learning rates cycled by element index; step counts from 1. The denominator is
 * one fused multiply-add, the contraction nvcc applies to adam.cu:325 by default. */
void efo_adam_step(int n, const float* grad, float* param, float* m, float* v, int step,
                   const double* lrs, int n_lrs, double beta1, double beta2, double eps)
{
    const double bc1_rcp = 1.0 / (1.0 - pow(beta1, step));
    const double bc2_rcp = 1.0 / sqrt(1.0 - pow(beta2, step));
    float steps[8];
    for (int i = 0; i < n_lrs; i++) steps[i] = (float)(lrs[i] * bc1_rcp);
    const float b1 = (float)beta1, b2 = (float)beta2, e = (float)eps, c2 = (float)bc2_rcp;
    for (int i = 0; i < n; i++) {
        const float g = grad[i];
        const float g2 = g * g;
        const float m1 = fmaf(b1, m[i] - g, g);
        const float m2 = fmaf(b2, v[i] - g2, g2);
        const float denom = fmaf(sqrtf(m2), c2, e);
        param[i] -= steps[i % n_lrs] * m1 / denom;
        m[i] = m1;
        v[i] = m2;
    }
}

/* ------------------------------------------------------------------------------------------------------ */
/* helpers exposed for closed-form tests                                                                  */
/* ------------------------------------------------------------------------------------------------------ */

/* rest-band SH basis values (15) of a unit direction, band order of appearance_sh.cuh:43-61 */
int efo_sh_rest_basis(const float* dir, int degree, float* out) { return sh_rest_basis(dir, degree, out); }

/* rotation matrix (row-major 3x3) of an unnormalised (w, x, y, z) quaternion as preprocess forms it, and |q|^2 */
void efo_quat_to_rot(const float* q, float* out, float* norm_sq) {
    const mat3 R = quat_to_rot(q, norm_sq);
    memcpy(out, &R, sizeof(R));
}

/* activated residual colour of one primitive for the SH / SV / NASG / NASGabor models */
void efo_residual(const efo_app* a, const float* params, const float* dir, int degree, float* out) {
    switch (a->model) {
        case 1: sh_residual(a, params, dir, degree, out); break;
        case 2: sv_residual(a, params, dir, degree, out); break;
        case 3: lobe_residual(a, params, dir, degree, 0, out); break;
        case 4: lobe_residual(a, params, dir, degree, 1, out); break;
        default: out[0] = out[1] = out[2] = 0.0f;
    }
}

/* alpha of a Gaussian (mean2d, conic, opacity) at pixel centre (px + 0.5, py + 0.5), as the blend computes it */
float efo_blend_alpha(float mx, float my, float cx, float cy, float cz, float opacity, int px, int py) {
    const float log2e = 1.44269504089f;
    const float ex = -0.5f * log2e * cx, ey = -log2e * cy, ez = -0.5f * log2e * cz;
    const float dx = mx - ((float)px + 0.5f), dy = my - ((float)py + 0.5f);
    return opacity * ef_exp2f(fminf(blend_exponent(ex, ey, ez, dx, dy), 0.0f));
}

/* ------------------------------------------------------------------------------------------------------ */
/* MCMC densification, B/densification/include/kernels_mcmc.cuh:11-146                                    */
/* ------------------------------------------------------------------------------------------------------ */

/* Philox4x32-10: Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC 2011), the
   Random123 philox4x32 generator with 10 rounds. Round: (c0, c1, c2, c3) -> (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2),
   hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)); the key is bumped by the Weyl constants before every round but the first. */
void efo_philox4x32_10(const uint32_t* ctr, const uint32_t* key, uint32_t* out) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* two standard normal samples from two 32-bit words: u = (bits_u + 1/2) 2^-32 in (0, 1], angle bits_v 2 pi 2^-32
   (kernels_mcmc.cuh:70-77) */
void efo_box_muller(uint32_t bits_u, uint32_t bits_v, float* z) {
    const float u = fmaf((float)bits_u, 2.3283064e-10f, 1.1641532e-10f);
    const float radius = sqrtf(-2.0f * logf(u));
    const float angle = (float)bits_v * 1.4629181e-9f;
    z[0] = radius * cosf(angle);
    z[1] = radius * sinf(angle);
}

/* means[i] += lr sigmoid(-(100 sigmoid(raw_opacity) - 0.5)) Sigma z (kernels_mcmc.cuh:79-144): Sigma = R diag(e^{2 s})
   R^T of the normalised quaternion, z from the Philox block with counter (offset / 4, i, 0) and key seed */
void efo_add_noise(int n, const float* raw_scales, const float* raw_rotations, const float* raw_opacities, float* means, float lr,
                   uint64_t seed, uint64_t offset) {
    const uint64_t counter = offset / 4;
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int i = 0; i < n; i++) {
        const float* q = raw_rotations + 4 * i;
        const float w = q[0], x = q[1], y = q[2], z = q[3];
        const float norm_sq = w * w + x * x + y * y + z * z;
        if (norm_sq < 1e-8f) continue;
        const float inv = 1.0f / norm_sq;
        const float R[3][3] = {{1.0f - 2.0f * (y * y + z * z) * inv, 2.0f * (x * y - w * z) * inv, 2.0f * (x * z + w * y) * inv},
                               {2.0f * (x * y + w * z) * inv, 1.0f - 2.0f * (x * x + z * z) * inv, 2.0f * (y * z - w * x) * inv},
                               {2.0f * (x * z - w * y) * inv, 2.0f * (y * z + w * x) * inv, 1.0f - 2.0f * (x * x + y * y) * inv}};
        const float v[3] = {expf(2.0f * raw_scales[3 * i]), expf(2.0f * raw_scales[3 * i + 1]), expf(2.0f * raw_scales[3 * i + 2])};
        float S[3][3];
        for (int a = 0; a < 3; a++)
            for (int b = 0; b < 3; b++) S[a][b] = R[a][0] * v[0] * R[b][0] + R[a][1] * v[1] * R[b][1] + R[a][2] * v[2] * R[b][2];
        const uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32), (uint32_t)i, 0u};
        uint32_t bits[4];
        efo_philox4x32_10(ctr, key, bits);
        float zxy[2], zz[2];
        efo_box_muller(bits[0], bits[1], zxy);
        efo_box_muller(bits[2], bits[3], zz);
        const float zv[3] = {zxy[0], zxy[1], zz[0]};
        const float o = 1.0f / (1.0f + expf(-raw_opacities[i]));
        const float f = lr * (1.0f / (1.0f + expf(100.0f * o - 0.5f)));
        for (int a = 0; a < 3; a++) means[3 * i + a] += f * (S[a][0] * zv[0] + S[a][1] * zv[1] + S[a][2] * zv[2]);
    }
}

#define EFO_MCMC_MAX_SAMPLES 50

/* c[m][k] = C(m, k) (-1)^k / sqrt(k + 1) in double, rounded to float (kernels_mcmc.cuh:13-26) */
void efo_relocation_table(float* table) {
    for (int m = 0; m < EFO_MCMC_MAX_SAMPLES; m++) {
        double binom = 1.0, sign = 1.0;
        for (int k = 0; k < EFO_MCMC_MAX_SAMPLES; k++) {
            if (k > m) {
                table[m * EFO_MCMC_MAX_SAMPLES + k] = 0.0f;
                continue;
            }
            table[m * EFO_MCMC_MAX_SAMPLES + k] = (float)(binom * sign * (1.0 / sqrt((double)(k + 1))));
            binom *= (double)(m - k) / (double)(k + 1);
            sign = -sign;
        }
    }
}

/* kernels_mcmc.cuh:28-56: o' = 1 - (1 - o)^(1/n), scales times o / sum_{m<n} sum_{k<=m} c[m][k] o'^(k+1) */
void efo_relocation(int n, const float* old_opacities, const float* old_scales, const int64_t* n_samples, float* new_opacities,
                    float* new_scales) {
    float table[EFO_MCMC_MAX_SAMPLES * EFO_MCMC_MAX_SAMPLES];
    efo_relocation_table(table);
    for (int i = 0; i < n; i++) {
        const float o = old_opacities[i];
        const int64_t s = n_samples[i];
        const int ns = s < 1 ? 1 : (s > EFO_MCMC_MAX_SAMPLES ? EFO_MCMC_MAX_SAMPLES : (int)s);
        const float o_new = 1.0f - powf(1.0f - o, 1.0f / (float)ns);
        new_opacities[i] = o_new;
        float denominator = 0.0f;
        for (int m = 0; m < ns; m++) {
            float p = o_new;
            for (int k = 0; k <= m; k++, p *= o_new) denominator += table[m * EFO_MCMC_MAX_SAMPLES + k] * p;
        }
        const float factor = o / denominator;
        for (int a = 0; a < 3; a++) new_scales[3 * i + a] = factor * old_scales[3 * i + a];
    }
}

/* ------------------------------------------------------------------------------------------------------ */
/* pruning scores (Speedy-Splat), B/rasterization/include/kernels_pruning_scores.cuh:11-171               */
/* ------------------------------------------------------------------------------------------------------ */

/* scores[p] += sum over pixels of (o_p dL/dalpha_p)^2 for the upstream gradient (1, 1, 1): the second pass of
   the reference replays each pixel's walk with the colour still to come and the final transmittance of the
   first (here: the forward's image, final T and last contributor). Accumulated in pixel order. */
void efo_pruning_scores(
    int width, int height, int grid_w, int grid_h, const uint32_t* ranges, const uint32_t* inst_prims,
    const float* mean2d, const float* conic_opacity, const float* color, const float* bg,
    const float* image, const float* final_T, const uint32_t* n_contrib, float* scores)
{
    const float log2e = 1.44269504089f;
    const int n_pixels = width * height;
    for (int ty = 0; ty < grid_h; ty++) for (int tx = 0; tx < grid_w; tx++) {
        const uint32_t t = (uint32_t)(ty * grid_w + tx);
        const uint32_t r0 = ranges[2 * t];
        for (int ly = 0; ly < EFO_TILE_H; ly++) for (int lx = 0; lx < EFO_TILE_W; lx++) {
            const int px = tx * EFO_TILE_W + lx, py = ty * EFO_TILE_H + ly;
            if (px >= width || py >= height) continue;
            const int pix = py * width + px;
            const float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
            const float Tf = final_T[pix];
            float after[3];
            for (int c = 0; c < 3; c++) after[c] = image[c * n_pixels + pix] - Tf * bg[c];
            const float grad_alpha_common = Tf * -(bg[0] + bg[1] + bg[2]);
            float T = 1.0f;
            const uint32_t last = n_contrib[pix];
            for (uint32_t k = 0; k < last; k++) {
                const uint32_t p = inst_prims[r0 + k];
                const float* co = conic_opacity + 4 * p;
                const float ex = -0.5f * log2e * co[0], ey = -log2e * co[1], ez = -0.5f * log2e * co[2];
                const float dx = mean2d[2 * p] - pxf, dy = mean2d[2 * p + 1] - pyf;
                const float G = ef_exp2f(fminf(blend_exponent(ex, ey, ez, dx, dy), 0.0f));
                const float alpha = co[3] * G;
                if (alpha < K_MIN_ALPHA) continue;
                const float* col = color + 3 * p;
                for (int c = 0; c < 3; c++) after[c] -= T * alpha * col[c];
                const float oma = 1.0f - alpha;
                const float rcp = 1.0f / fmaxf(oma, k_one_minus_alpha_eps);
                const float dalpha = (T * col[0] - after[0] * rcp) + (T * col[1] - after[1] * rcp) + (T * col[2] - after[2] * rcp) +
                                     grad_alpha_common * rcp;
                const float dg = co[3] * dalpha;
                scores[p] += dg * dg;
                T = transmit(T, alpha);
            }
        }
    }
}
