// Spherical-harmonics residual (EFGS_MODEL == 1): band sum of degrees 1..degree over EFGS_N_UNITS rgb
// coefficients per primitive, residual activation applied to the sum.
// Reference: B/rasterization/rtc/appearance_sh.cuh:30-157 (constants are the real SH normalisations).
#pragma once

namespace efgs {

constexpr float sh_c1 = 0.48860251190291987f;
constexpr float sh_c2a = 1.0925484305920792f, sh_c2b = 0.94617469575755997f, sh_c2c = 0.31539156525251999f;
constexpr float sh_c2d = 0.54627421529603959f, sh_c2e = 1.8923493915151202f;
constexpr float sh_c3a = 0.59004358992664352f, sh_c3b = 1.7701307697799304f, sh_c3c = 2.8906114426405538f;
constexpr float sh_c3d = 0.45704579946446572f, sh_c3e = 2.2852289973223288f, sh_c3f = 1.865881662950577f;
constexpr float sh_c3g = 1.1195289977703462f, sh_c3h = 1.4453057213202769f, sh_c3i = 3.5402615395598609f;
constexpr float sh_c3j = 4.5704579946446566f, sh_c3k = 5.597644988851731f;

// rest-band basis values b[0..14] (degree-gated entries beyond the active degree are left unwritten)
__device__ __forceinline__ void sh_rest_basis(float x, float y, float z, uint32_t degree, float* b) {
    b[0] = -sh_c1 * y; b[1] = sh_c1 * z; b[2] = -sh_c1 * x;
    if (degree > 1) {
        const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, xz = x * z, yz = y * z;
        b[3] = sh_c2a * xy; b[4] = -sh_c2a * yz; b[5] = sh_c2b * zz - sh_c2c; b[6] = -sh_c2a * xz; b[7] = sh_c2d * (xx - yy);
        if (degree > 2) {
            b[8] = y * (sh_c3a * yy - sh_c3b * xx); b[9] = sh_c3c * xy * z; b[10] = y * (sh_c3d - sh_c3e * zz);
            b[11] = z * (sh_c3f * zz - sh_c3g); b[12] = x * (sh_c3d - sh_c3e * zz); b[13] = sh_c3h * z * (xx - yy);
            b[14] = x * (sh_c3b * yy - sh_c3a * xx);
        }
    }
}

__device__ __forceinline__ uint32_t sh_bases_of_degree(uint32_t degree) { return (degree + 1) * (degree + 1) - 1; }

template <int RES_ACT>
__device__ inline float3 sh_residual(const float* coef, float3 d, uint32_t degree) {
    if (degree == 0) return make_float3(0.0f, 0.0f, 0.0f);
    float b[15];
    sh_rest_basis(d.x, d.y, d.z, degree, b);
    const uint32_t nb = sh_bases_of_degree(degree);
    float r = 0.0f, g = 0.0f, bl = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < 15; i++) {
        if (i < nb) {
            r += b[i] * coef[3 * i];
            g += b[i] * coef[3 * i + 1];
            bl += b[i] * coef[3 * i + 2];
        }
    }
    return make_float3(residual_activation<RES_ACT>(r), residual_activation<RES_ACT>(g), residual_activation<RES_ACT>(bl));
}

// writes dL/dcoef for the active bases and returns dL/dmean through the view direction. Every coefficient is read
// before the first gradient is written, so gcoef may be coef itself (the gradients replace the coefficients).
template <int RES_ACT>
__device__ inline float3 sh_residual_backward(const float* coef, float3 dpre, float* gcoef, float3 d, float norm_rcp, uint32_t degree) {
    if (degree == 0) return make_float3(0.0f, 0.0f, 0.0f);
    const float3 res = sh_residual<RES_ACT>(coef, d, degree);
    const float3 ds = make_float3(dpre.x * residual_activation_grad<RES_ACT>(res.x), dpre.y * residual_activation_grad<RES_ACT>(res.y),
                                  dpre.z * residual_activation_grad<RES_ACT>(res.z));
    const float x = d.x, y = d.y, z = d.z;
    float gx[3], gy[3], gz[3];
#pragma unroll
    for (int c = 0; c < 3; c++) {
        gx[c] = -sh_c1 * coef[3 * 2 + c];
        gy[c] = -sh_c1 * coef[3 * 0 + c];
        gz[c] = sh_c1 * coef[3 * 1 + c];
        if (degree > 1) {
            const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, xz = x * z, yz = y * z;
            gx[c] += sh_c2a * y * coef[9 + c] - sh_c2a * z * coef[18 + c] + sh_c2a * x * coef[21 + c];
            gy[c] += sh_c2a * x * coef[9 + c] - sh_c2a * z * coef[12 + c] - sh_c2a * y * coef[21 + c];
            gz[c] += -sh_c2a * y * coef[12 + c] + sh_c2e * z * coef[15 + c] - sh_c2a * x * coef[18 + c];
            if (degree > 2) {
                gx[c] += -sh_c3i * xy * coef[24 + c] + sh_c3c * yz * coef[27 + c] + (sh_c3d - sh_c3e * zz) * coef[36 + c]
                         + sh_c3c * xz * coef[39 + c] + sh_c3b * (yy - xx) * coef[42 + c];
                gy[c] += sh_c3b * (yy - xx) * coef[24 + c] + sh_c3c * xz * coef[27 + c] + (sh_c3d - sh_c3e * zz) * coef[30 + c]
                         - sh_c3c * yz * coef[39 + c] + sh_c3i * xy * coef[42 + c];
                gz[c] += sh_c3c * xy * coef[27 + c] - sh_c3j * yz * coef[30 + c] + (sh_c3k * zz - sh_c3g) * coef[33 + c]
                         - sh_c3j * xz * coef[36 + c] + sh_c3h * (xx - yy) * coef[39 + c];
            }
        }
    }
    const float3 gd = make_float3(gx[0] * ds.x + gx[1] * ds.y + gx[2] * ds.z, gy[0] * ds.x + gy[1] * ds.y + gy[2] * ds.z,
                                  gz[0] * ds.x + gz[1] * ds.y + gz[2] * ds.z);
    float b[15];
    sh_rest_basis(d.x, d.y, d.z, degree, b);
    const uint32_t nb = sh_bases_of_degree(degree);
#pragma unroll
    for (uint32_t i = 0; i < 15; i++) {
        if (i < nb) {
            gcoef[3 * i] = b[i] * ds.x;
            gcoef[3 * i + 1] = b[i] * ds.y;
            gcoef[3 * i + 2] = b[i] * ds.z;
        }
    }
    return direction_grad_to_mean(gd, d, norm_rcp);
}

}  // namespace efgs
