// MCMC densification kernels (3DGS-MCMC), one thread per primitive.
//
//   relocation_kernel   opacity and scale of a Gaussian split into n samples: o' = 1 - (1 - o)^(1/n), scales
//                       times o / sum_{m<n} sum_{k<=m} c[m][k] o'^(k+1) with c[m][k] = C(m, k) (-1)^k / sqrt(k + 1)
//                       (Eq. 9 of the paper; the table is built in double on the host, once per device)
//   add_noise_kernel    means += lr sigmoid(-(100 sigmoid(raw_opacity) - 0.5)) Sigma z, Sigma = R S^2 R^T from the
//                       log-scales and the unnormalised quaternion, z ~ N(0, I) from one Philox4x32-10 block per
//                       primitive (counter = (offset / 4, primitive index, 0), key = seed) and two Box-Muller
//                       transforms; quaternions with |q|^2 < 1e-8 leave their mean unchanged
//
// Philox4x32-10 is the counter-based generator of Salmon, Moraes, Dror and Shaw ("Parallel random numbers: as
// easy as 1, 2, 3", SC 2011; Random123): ten rounds of two 32x32 -> 64-bit multiplications (0xD2511F53,
// 0xCD9E8D57) with the key bumped by the Weyl constants (0x9E3779B9, 0xBB67AE85) between rounds.
//
// Reference: B/densification/include/kernels_mcmc.cuh:11-146, B/densification/src/mcmc.cu:1-56,
// B/densification/src/densification_api.cu:13-72.
#include "internal.h"

#include <cmath>
#include <mutex>

namespace efgs {

namespace {

constexpr uint32_t densify_block = 256;

__constant__ float c_relocation[mcmc_max_samples * mcmc_max_samples];

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        if (r > 0) {
            k.x += 0x9E3779B9u;
            k.y += 0xBB67AE85u;
        }
        const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
        const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
        c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
    }
    return c;
}

// two standard normal samples from two uniform 32-bit words: u = (bits_u + 1/2) 2^-32 in (0, 1], angle =
// bits_v 2 pi 2^-32
__device__ __forceinline__ float2 box_muller(uint32_t bits_u, uint32_t bits_v) {
    const float u = fmaf(static_cast<float>(bits_u), 2.3283064e-10f, 1.1641532e-10f);
    const float radius = sqrtf(-2.0f * logf(u));
    float s, c;
    sincosf(static_cast<float>(bits_v) * 1.4629181e-9f, &s, &c);
    return make_float2(radius * c, radius * s);
}

__global__ __launch_bounds__(densify_block) void add_noise_kernel(const float* __restrict__ raw_scales, const float4* __restrict__ raw_rotations,
                                                                  const float* __restrict__ raw_opacities, float* __restrict__ means,
                                                                  uint32_t n, float lr, uint64_t seed, uint64_t offset) {
    const uint32_t i = blockIdx.x * densify_block + threadIdx.x;
    if (i >= n) return;
    const float4 q = raw_rotations[i];
    const float w = q.x, x = q.y, y = q.z, z = q.w;
    const float norm_sq = w * w + x * x + y * y + z * z;
    if (norm_sq < 1e-8f) return;
    const float inv = 1.0f / norm_sq;
    // rotation of the normalised quaternion
    const float r11 = 1.0f - 2.0f * (y * y + z * z) * inv, r12 = 2.0f * (x * y - w * z) * inv, r13 = 2.0f * (x * z + w * y) * inv;
    const float r21 = 2.0f * (x * y + w * z) * inv, r22 = 1.0f - 2.0f * (x * x + z * z) * inv, r23 = 2.0f * (y * z - w * x) * inv;
    const float r31 = 2.0f * (x * z - w * y) * inv, r32 = 2.0f * (y * z + w * x) * inv, r33 = 1.0f - 2.0f * (x * x + y * y) * inv;
    const float v0 = expf(2.0f * raw_scales[3 * i]), v1 = expf(2.0f * raw_scales[3 * i + 1]), v2 = expf(2.0f * raw_scales[3 * i + 2]);
    // Sigma = (R diag(v)) R^T, upper triangle
    const float a11 = r11 * v0, a12 = r12 * v1, a13 = r13 * v2;
    const float a21 = r21 * v0, a22 = r22 * v1, a23 = r23 * v2;
    const float a31 = r31 * v0, a32 = r32 * v1, a33 = r33 * v2;
    const float s11 = a11 * r11 + a12 * r12 + a13 * r13, s12 = a11 * r21 + a12 * r22 + a13 * r23, s13 = a11 * r31 + a12 * r32 + a13 * r33;
    const float s22 = a21 * r21 + a22 * r22 + a23 * r23, s23 = a21 * r31 + a22 * r32 + a23 * r33;
    const float s33 = a31 * r31 + a32 * r32 + a33 * r33;
    const uint64_t counter = offset / 4;
    const uint4 bits = philox4x32_10(make_uint4(static_cast<uint32_t>(counter), static_cast<uint32_t>(counter >> 32), i, 0u),
                                     make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
    const float2 zxy = box_muller(bits.x, bits.y);
    const float zz = box_muller(bits.z, bits.w).x;
    const float o = 1.0f / (1.0f + expf(-raw_opacities[i]));
    const float f = lr * (1.0f / (1.0f + expf(100.0f * o - 0.5f)));
    means[3 * i] += f * (s11 * zxy.x + s12 * zxy.y + s13 * zz);
    means[3 * i + 1] += f * (s12 * zxy.x + s22 * zxy.y + s23 * zz);
    means[3 * i + 2] += f * (s13 * zxy.x + s23 * zxy.y + s33 * zz);
}

__global__ __launch_bounds__(densify_block) void relocation_kernel(const float* __restrict__ old_opacities, const float* __restrict__ old_scales,
                                                                   const int64_t* __restrict__ n_samples, float* __restrict__ new_opacities,
                                                                   float* __restrict__ new_scales, uint32_t n) {
    const uint32_t i = blockIdx.x * densify_block + threadIdx.x;
    if (i >= n) return;
    const float o = old_opacities[i];
    const int64_t s = n_samples[i];
    const int m_samples = s < 1 ? 1 : (s > static_cast<int64_t>(mcmc_max_samples) ? static_cast<int>(mcmc_max_samples) : static_cast<int>(s));
    const float o_new = 1.0f - powf(1.0f - o, 1.0f / static_cast<float>(m_samples));
    new_opacities[i] = o_new;
    float denominator = 0.0f;
    for (int m = 0; m < m_samples; m++) {
        float p = o_new;
        for (int k = 0; k <= m; k++, p *= o_new) denominator += c_relocation[m * mcmc_max_samples + k] * p;
    }
    const float factor = o / denominator;
    new_scales[3 * i] = factor * old_scales[3 * i];
    new_scales[3 * i + 1] = factor * old_scales[3 * i + 1];
    new_scales[3 * i + 2] = factor * old_scales[3 * i + 2];
}

// C(m, k) (-1)^k / sqrt(k + 1) in double, rounded to float (row m, column k <= m; zero above the diagonal)
void relocation_table(float* table) {
    for (uint32_t m = 0; m < mcmc_max_samples; m++) {
        double binom = 1.0, sign = 1.0;
        for (uint32_t k = 0; k < mcmc_max_samples; k++) {
            if (k > m) {
                table[m * mcmc_max_samples + k] = 0.0f;
                continue;
            }
            table[m * mcmc_max_samples + k] = static_cast<float>(binom * sign * (1.0 / std::sqrt(static_cast<double>(k + 1))));
            binom *= static_cast<double>(m - k) / static_cast<double>(k + 1);
            sign = -sign;
        }
    }
}

// uploads the table to the current device once per process
bool ensure_relocation_table() {
    static std::mutex mutex;
    static bool uploaded[64] = {};
    int device = 0;
    EFGS_HIP_CHECK(hipGetDevice(&device));
    if (device < 0 || device >= 64) {
        set_error("device index out of range for the relocation table");
        return false;
    }
    std::lock_guard<std::mutex> lock(mutex);
    if (uploaded[device]) return true;
    static float table[mcmc_max_samples * mcmc_max_samples];
    relocation_table(table);
    EFGS_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(c_relocation), table, sizeof(table)));
    uploaded[device] = true;
    return true;
}

}  // namespace

bool launch_add_noise(const float* raw_scales, const float* raw_rotations, const float* raw_opacities, float* means, uint32_t n, float lr,
                      uint64_t seed, uint64_t offset, hipStream_t s) {
    if (n == 0) return true;
    add_noise_kernel<<<div_up(n, densify_block), densify_block, 0, s>>>(raw_scales, reinterpret_cast<const float4*>(raw_rotations),
                                                                        raw_opacities, means, n, lr, seed, offset);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_relocation(const float* old_opacities, const float* old_scales, const int64_t* n_samples, float* new_opacities, float* new_scales,
                       uint32_t n, hipStream_t s) {
    if (n == 0) return true;
    if (!ensure_relocation_table()) return false;
    relocation_kernel<<<div_up(n, densify_block), densify_block, 0, s>>>(old_opacities, old_scales, n_samples, new_opacities, new_scales, n);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
