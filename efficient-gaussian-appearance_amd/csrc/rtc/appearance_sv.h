// Soft spherical-Voronoi residual (EFGS_MODEL == 2): R(v) = sum_k softmax_k(-tau_k |site_k - v|) c_k with
// 7 raw parameters per site [site xyz | log tau | rgb], evaluated as a single-pass online softmax.
// Reference: B/rasterization/rtc/appearance_sv.cuh:26-139.
#pragma once

namespace efgs {

constexpr float sv_eps = 1e-12f;

template <int RES_ACT>
__device__ inline float3 sv_residual(const float* p, float3 d, uint32_t sites) {
    if (sites == 0) return make_float3(0.0f, 0.0f, 0.0f);
    float max_logit = -1e30f, wsum = 0.0f, r = 0.0f, g = 0.0f, b = 0.0f;
    for (uint32_t s = 0; s < sites; s++, p += 7) {
        const float inv = 1.0f / fmaxf(sqrtf(p[0] * p[0] + p[1] * p[1] + p[2] * p[2]), sv_eps);
        const float d0 = inv * p[0] - d.x, d1 = inv * p[1] - d.y, d2 = inv * p[2] - d.z;
        const float dist = sqrtf(d0 * d0 + d1 * d1 + d2 * d2);
        const float logit = -expf(p[3]) * dist;
        const float nm = fmaxf(max_logit, logit);
        const float rescale = expf(max_logit - nm);
        const float w = expf(fminf(logit - nm, 0.0f));
        wsum = wsum * rescale + w;
        r = r * rescale + w * residual_activation<RES_ACT>(p[4]);
        g = g * rescale + w * residual_activation<RES_ACT>(p[5]);
        b = b * rescale + w * residual_activation<RES_ACT>(p[6]);
        max_logit = nm;
    }
    const float wr = 1.0f / wsum;
    return make_float3(wr * r, wr * g, wr * b);
}

// writes dL/d(site parameters) of the active sites and returns dL/dmean through the view direction. A site's
// parameters are read before its gradients are written, and no later step reads them, so gp may be p0 itself.
template <int RES_ACT>
__device__ inline float3 sv_residual_backward(const float* p0, float3 gc, float* gp, float3 d, float norm_rcp, uint32_t sites) {
    if (sites == 0) return make_float3(0.0f, 0.0f, 0.0f);
    float max_logit = -1e30f, wsum = 0.0f, r = 0.0f, g = 0.0f, b = 0.0f;
    const float* p = p0;
    for (uint32_t s = 0; s < sites; s++, p += 7) {
        const float inv = 1.0f / fmaxf(sqrtf(p[0] * p[0] + p[1] * p[1] + p[2] * p[2]), sv_eps);
        const float d0 = inv * p[0] - d.x, d1 = inv * p[1] - d.y, d2 = inv * p[2] - d.z;
        const float dist = sqrtf(d0 * d0 + d1 * d1 + d2 * d2);
        const float logit = -expf(p[3]) * dist;
        const float nm = fmaxf(max_logit, logit);
        const float rescale = expf(max_logit - nm);
        const float w = expf(fminf(logit - nm, 0.0f));
        wsum = wsum * rescale + w;
        r = r * rescale + w * residual_activation<RES_ACT>(p[4]);
        g = g * rescale + w * residual_activation<RES_ACT>(p[5]);
        b = b * rescale + w * residual_activation<RES_ACT>(p[6]);
        max_logit = nm;
    }
    const float wr = 1.0f / wsum;
    const float gmean = gc.x * (wr * r) + gc.y * (wr * g) + gc.z * (wr * b);
    float3 gd = make_float3(0.0f, 0.0f, 0.0f);
    p = p0;
    for (uint32_t s = 0; s < sites; s++, p += 7, gp += 7) {
        const float lr = 1.0f / fmaxf(sqrtf(p[0] * p[0] + p[1] * p[1] + p[2] * p[2]), sv_eps);
        const float3 site = make_float3(lr * p[0], lr * p[1], lr * p[2]);
        const float3 sd = make_float3(site.x - d.x, site.y - d.y, site.z - d.z);
        const float dist = sqrtf(sd.x * sd.x + sd.y * sd.y + sd.z * sd.z);
        const float tau = expf(p[3]);
        const float w = expf(fminf(-tau * dist - max_logit, 0.0f)) * wr;
        const float cr = residual_activation<RES_ACT>(p[4]);
        const float cg = residual_activation<RES_ACT>(p[5]);
        const float cb = residual_activation<RES_ACT>(p[6]);
        gp[4] = w * gc.x * residual_activation_grad<RES_ACT>(cr);
        gp[5] = w * gc.y * residual_activation_grad<RES_ACT>(cg);
        gp[6] = w * gc.z * residual_activation_grad<RES_ACT>(cb);
        const float glogit = w * ((gc.x * cr + gc.y * cg + gc.z * cb) - gmean);
        gp[3] = -dist * tau * glogit;
        const float f = (-tau * glogit) / fmaxf(dist, sv_eps);
        const float3 gsd = make_float3(f * sd.x, f * sd.y, f * sd.z);
        const float dd = gsd.x * site.x + gsd.y * site.y + gsd.z * site.z;
        gp[0] = (gsd.x - dd * site.x) * lr;
        gp[1] = (gsd.y - dd * site.y) * lr;
        gp[2] = (gsd.z - dd * site.z) * lr;
        gd.x -= gsd.x;
        gd.y -= gsd.y;
        gd.z -= gsd.z;
    }
    return direction_grad_to_mean(gd, d, norm_rcp);
}

}  // namespace efgs
