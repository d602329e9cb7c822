// Normalised anisotropic spherical Gaussian lobes: NASG (EFGS_MODEL == 3, 8 raw parameters per lobe) and
// NASGabor (EFGS_MODEL == 4, 9 per lobe, an extra Gabor factor (1 + cos(k v_x)) / 2).
//   raw [0..2] -> tanh -> cos(theta), cos(phi), cos(tau) of the lobe frame
//   raw [3]    -> exp  -> sharpness lambda (<= 1e4)       raw [4] -> exp -> anisotropy a (<= 1e4)
//   NASGabor raw [5] -> k = 20 (tanh + 1)                 last 3 -> residual activation -> rgb amplitude
//   K = (v.z + 1)/2, K_e = eps + a (v.x)^2 / (1 - (v.z)^2), E = K^K_e,
//   N = lambda sqrt(1 + a) / (2 pi (1 + eps_n - exp(-2 lambda))), pdf = exp(2 lambda (E K - 1)) E [G] N
// Reference: B/rasterization/rtc/appearance_nasg.cuh:164-350, appearance_nasgabor.cuh:25-223.
#pragma once

namespace efgs {

constexpr float lobe_two_pi = 6.28318530717958647692f;
constexpr float lobe_eps = 5e-6f;
constexpr float lobe_eps_norm = 1e-8f;
constexpr float lobe_cos_limit = 0.999999f;
constexpr float lobe_pole_limit = 0.99999988f;
constexpr float lobe_shape_limit = 1e4f;
constexpr float lobe_freq_scale = 20.0f;

struct LobeFrame {
    float3 x, z;
    float ct, cp, cu, st, sp, su;
};

__device__ __forceinline__ LobeFrame build_lobe_frame(float ct, float cp, float cu) {
    LobeFrame f;
    f.ct = ct; f.cp = cp; f.cu = cu;
    f.st = sqrtf(1.0f - ct * ct);
    f.sp = sqrtf(1.0f - cp * cp);
    f.su = sqrtf(1.0f - cu * cu);
    f.x = make_float3(ct * cp * cu - f.st * f.su, f.st * cp * cu + ct * f.su, -f.sp * cu);
    f.z = make_float3(ct * f.sp, f.st * f.sp, cp);
    return f;
}

template <int RES_ACT, bool GABOR>
__device__ inline float3 lobe_residual(const float* p, float3 d, uint32_t lobes) {
    constexpr int stride = GABOR ? 9 : 8;
    constexpr int wo = GABOR ? 6 : 5;
    float r = 0.0f, g = 0.0f, b = 0.0f;
    for (uint32_t l = 0; l < lobes; l++, p += stride) {
        const LobeFrame f = build_lobe_frame(clampf(tanhf(p[0]), -lobe_cos_limit, lobe_cos_limit),
                                             clampf(tanhf(p[1]), -lobe_cos_limit, lobe_cos_limit),
                                             clampf(tanhf(p[2]), -lobe_cos_limit, lobe_cos_limit));
        const float lambda = fminf(expf(p[3]), lobe_shape_limit);
        const float an = fminf(expf(p[4]), lobe_shape_limit);
        const float vz = d.x * f.z.x + d.y * f.z.y + d.z * f.z.z;
        const float vx = d.x * f.x.x + d.y * f.x.y + d.z * f.x.z;
        const float vzc = clampf(vz, -lobe_pole_limit, lobe_pole_limit);
        const float K = 0.5f * (vzc + 1.0f);
        const float Ke = lobe_eps + an * vx * vx / (1.0f - vzc * vzc);
        const float E = expf(Ke * logf(K));  // K^Ke (K in (0, 1], Ke > 0)
        const float N = lambda * sqrtf(1.0f + an) / (lobe_two_pi * (1.0f + lobe_eps_norm - expf(-2.0f * lambda)));
        const float P = expf(2.0f * lambda * (E * K - 1.0f));
        float G = 1.0f;
        if (GABOR) G = 0.5f * (1.0f + cosf((tanhf(p[5]) + 1.0f) * lobe_freq_scale * vx));
        const float pdf = vz >= lobe_pole_limit ? 1.0f : (vz > -lobe_pole_limit ? (GABOR ? P * E * G * N : P * E * N) : 0.0f);
        r += pdf * residual_activation<RES_ACT>(p[wo]);
        g += pdf * residual_activation<RES_ACT>(p[wo + 1]);
        b += pdf * residual_activation<RES_ACT>(p[wo + 2]);
    }
    return make_float3(r, g, b);
}

template <int RES_ACT, bool GABOR>
__device__ inline float3 lobe_residual_backward(const float* p, float3 gc, float* gp, float3 d, float norm_rcp, uint32_t lobes) {
    constexpr int stride = GABOR ? 9 : 8;
    constexpr int wo = GABOR ? 6 : 5;
    float3 gd = make_float3(0.0f, 0.0f, 0.0f);
    for (uint32_t l = 0; l < lobes; l++, p += stride, gp += stride) {
        const float th = tanhf(p[0]), tp = tanhf(p[1]), tu = tanhf(p[2]);
        const LobeFrame f = build_lobe_frame(clampf(th, -lobe_cos_limit, lobe_cos_limit), clampf(tp, -lobe_cos_limit, lobe_cos_limit),
                                             clampf(tu, -lobe_cos_limit, lobe_cos_limit));
        const float lu = expf(p[3]), au = expf(p[4]);
        const float lambda = fminf(lu, lobe_shape_limit), an = fminf(au, lobe_shape_limit);
        float tk = 0.0f, k = 0.0f;
        if (GABOR) { tk = tanhf(p[5]); k = (tk + 1.0f) * lobe_freq_scale; }
        const float w0 = residual_activation<RES_ACT>(p[wo]);
        const float w1 = residual_activation<RES_ACT>(p[wo + 1]);
        const float w2 = residual_activation<RES_ACT>(p[wo + 2]);
        const float vz = d.x * f.z.x + d.y * f.z.y + d.z * f.z.z;
        const float vx = d.x * f.x.x + d.y * f.x.y + d.z * f.x.z;
        const float vzc = clampf(vz, -lobe_pole_limit, lobe_pole_limit);
        const float K = 0.5f * (vzc + 1.0f);
        const float om = 1.0f - vzc * vzc;
        const float rom = 1.0f / om;
        const float Ke = lobe_eps + an * vx * vx * rom;
        const float logK = logf(K);
        const float E = expf(Ke * logK);  // K^Ke (K in (0, 1], Ke > 0)
        const float em2l = expf(-2.0f * lambda);
        const float nd = lobe_two_pi * (1.0f + lobe_eps_norm - em2l);
        const float rnd = 1.0f / nd;
        const float s1a = sqrtf(1.0f + an);
        const float N = lambda * s1a * rnd;
        float skv = 0.0f, ckv = 1.0f;
        if (GABOR) sincosf(k * vx, &skv, &ckv);
        const float G = GABOR ? 0.5f * (1.0f + ckv) : 1.0f;
        const float P = expf(2.0f * lambda * (E * K - 1.0f));
        const bool valid = fabsf(vz) < lobe_pole_limit;
        const float pdf = vz >= lobe_pole_limit ? 1.0f : (valid ? P * E * G * N : 0.0f);
        gp[wo] = gc.x * pdf * residual_activation_grad<RES_ACT>(w0);
        gp[wo + 1] = gc.y * pdf * residual_activation_grad<RES_ACT>(w1);
        gp[wo + 2] = gc.z * pdf * residual_activation_grad<RES_ACT>(w2);
        const float gpdf = valid ? (gc.x * w0 + gc.y * w1 + gc.z * w2) : 0.0f;
        const float dP_dl = P * 2.0f * (E * K - 1.0f);
        const float dN_dl = (s1a * nd - lambda * s1a * 2.0f * lobe_two_pi * em2l) * (rnd * rnd);
        gp[3] = lu >= lobe_shape_limit ? 0.0f : gpdf * (dP_dl * E * G * N + P * E * G * dN_dl) * lambda;
        const float dE_da = E * logK * (vx * vx * rom);
        const float dP_da = P * 2.0f * lambda * K * dE_da;
        const float dN_da = lambda * rnd / (2.0f * s1a);
        gp[4] = au >= lobe_shape_limit ? 0.0f : gpdf * (dP_da * E * G * N + P * dE_da * G * N + P * E * G * dN_da) * an;
        float dG_dvx = 0.0f;
        if (GABOR) {
            gp[5] = gpdf * (P * E * (-0.5f * skv * vx) * N) * lobe_freq_scale * (1.0f - tk * tk);
            dG_dvx = -0.5f * skv * k;
        }
        const float dE_dvx = E * logK * (2.0f * an * vx * rom);
        const float dP_dvx = P * 2.0f * lambda * K * dE_dvx;
        const float gvx = gpdf * (dP_dvx * E * G * N + P * dE_dvx * G * N + P * E * dG_dvx * N);
        const float dKe_dvz = an * vx * vx * 2.0f * vz * (rom * rom);
        const float dE_dvz = E * (Ke / K) * 0.5f + E * logK * dKe_dvz;
        const float dP_dvz = P * 2.0f * lambda * (K * dE_dvz + E * 0.5f);
        const float gvz = gpdf * (dP_dvz * E * G * N + P * dE_dvz * G * N);
        const float3 gx = make_float3(gvx * d.x, gvx * d.y, gvx * d.z);
        const float3 gz = make_float3(gvz * d.x, gvz * d.y, gvz * d.z);
        gd.x += gvx * f.x.x + gvz * f.z.x;
        gd.y += gvx * f.x.y + gvz * f.z.y;
        gd.z += gvx * f.x.z + gvz * f.z.z;
        const float dst = -f.ct / f.st, dsp = -f.cp / f.sp, dsu = -f.cu / f.su;
        const float gct = gx.x * (f.cp * f.cu - dst * f.su) + gx.y * (dst * f.cp * f.cu + f.su) + gz.x * f.sp + gz.y * dst * f.sp;
        const float gcp = gx.x * f.ct * f.cu + gx.y * f.st * f.cu - gx.z * dsp * f.cu + gz.x * f.ct * dsp + gz.y * f.st * dsp + gz.z;
        const float gcu = gx.x * (f.ct * f.cp - f.st * dsu) + gx.y * (f.st * f.cp + f.ct * dsu) - gx.z * f.sp;
        gp[0] = fabsf(th) >= lobe_cos_limit ? 0.0f : gct * (1.0f - th * th);
        gp[1] = fabsf(tp) >= lobe_cos_limit ? 0.0f : gcp * (1.0f - tp * tp);
        gp[2] = fabsf(tu) >= lobe_cos_limit ? 0.0f : gcu * (1.0f - tu * tu);
    }
    return direction_grad_to_mean(gd, d, norm_rcp);
}

}  // namespace efgs
