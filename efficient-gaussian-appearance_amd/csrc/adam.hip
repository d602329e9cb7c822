// Fused Adam over several parameter groups in one launch. Blocks are assigned to groups by a prefix of
// per-group block counts (first_block); each thread updates 4 strided elements per block tile.
// Per element (PyTorch formulation with the bias correction of the first moment folded into the step size):
//   m = beta1 (m - g) + g, v = beta2 (v - g^2) + g^2 (fused multiply-adds)
//   p -= lr_k / (1 - beta1^t) * m / (sqrt(v) / sqrt(1 - beta2^t) + eps), lr_k cycled by element index
// Reference: B/adam/src/adam.cu:18-87, B/torch_bindings/adam.py:10-36.
#include "internal.h"

namespace efgs {

namespace {

constexpr uint32_t adam_block = 256;
constexpr uint32_t adam_items = 4;

struct AdamLaunch {
    AdamGroupDevice groups[adam_max_groups];
    int n_groups;
};

__global__ __launch_bounds__(adam_block) void adam_kernel(AdamLaunch L) {
    int g = 0;
    for (int k = 1; k < L.n_groups; k++)
        if (L.groups[k].first_block <= blockIdx.x) g = k;
    const AdamGroupDevice& G = L.groups[g];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x - G.first_block) * adam_block * adam_items + threadIdx.x;
#pragma unroll
    for (uint32_t k = 0; k < adam_items; k++) {
        const uint64_t i = base + k * adam_block;
        if (i >= G.n) break;
        const float grad = G.grad[i];
        const float m = G.m[i];
        const float v = G.v[i];
        const float g2 = grad * grad;
        const float m1 = __builtin_fmaf(G.beta1, m - grad, grad);
        const float m2 = __builtin_fmaf(G.beta2, v - g2, g2);
        const float denom = __builtin_fmaf(sqrtf(m2), G.bc2_sqrt_rcp, G.eps);
        const float step = G.n_lrs == 1 ? G.step_sizes[0] : G.step_sizes[i % static_cast<uint64_t>(G.n_lrs)];  // uniform branch
        G.param[i] -= step * m1 / denom;
        G.m[i] = m1;
        G.v[i] = m2;
    }
}

}  // namespace

bool launch_adam(const AdamGroupDevice* groups, int n_groups, hipStream_t s) {
    for (int g0 = 0; g0 < n_groups; g0 += adam_max_groups) {
        AdamLaunch L;
        L.n_groups = 0;
        uint32_t blocks = 0;
        for (int g = g0; g < n_groups && g < g0 + adam_max_groups; g++) {
            if (groups[g].n == 0) continue;
            L.groups[L.n_groups] = groups[g];
            L.groups[L.n_groups].first_block = blocks;
            blocks += div_up(groups[g].n, static_cast<uint64_t>(adam_block) * adam_items);
            L.n_groups++;
        }
        if (blocks == 0) continue;
        adam_kernel<<<blocks, adam_block, 0, s>>>(L);
        EFGS_HIP_CHECK(hipGetLastError());
    }
    return true;
}

}  // namespace efgs
