// .ngsplat packing: the per-splat textures of the WebGL viewer's file format, built from a model resident in HBM.
//
//   ngsplat_stats_kernel    one block per 256 splats: kept count (sigmoid(raw opacity) >= 1/255), min / max of the
//                           shifted base colour over the kept splats, and for the SH payload max |coefficient| of
//                           each quantised level over the kept splats (coefficients read as one flat coalesced
//                           sweep over the block's rows)
//   ngsplat_combine_kernel  one block: exclusive scan of the block counts (each block's first output row) and the
//                           global reductions -> base offset / scale and the SH level scales
//   ngsplat_pack_kernel     one block per 256 splats (= 256 output rows): the block's residual rows are staged in
//                           LDS with a coalesced copy, the kept splats are compacted in source order (wave ballot
//                           + block prefix) and each writes its row: the RGBA32UI splat words (rgb8 base + a8
//                           opacity, fp16 position, 24-bit folded-octahedral rotation, 8-bit log scales) and its
//                           payload texels; rows from the kept count to the capacity are written as zeros
//
// The arithmetic follows the exporter's float32 numpy expressions operation by operation (compiled without FP
// contraction): the quantisation codes and fp16 values are those the exporter computes, up to the last-bit
// differences of the transcendental functions (exp, log, acos, sin, cos, tanh, log1p) and, for the baked layer 0,
// the summation order of a dot product.
//
// Reference: viewer/export_ngsplat.py:311-400 (packing helpers), :545-611 (SH levels), :624-643 / :656-696 /
// :721-765 (SV / NASG / NASGabor payloads), :1465-1530 (culling, base quantisation, layer-0 bake), :1234-1251
// (activated opacity / scales, normalised quaternion).
#include "internal.h"

#include <hip/hip_fp16.h>

#include <cmath>

namespace efgs {

namespace {

constexpr float ng_min_alpha = static_cast<float>(1.0 / 255.0);
constexpr float ng_ln_scale_min = -12.0f;
constexpr float ng_ln_scale_encode = static_cast<float>(254.0 / (9.0 - -12.0));
constexpr float ng_pi = static_cast<float>(3.14159265358979323846);
constexpr float ng_two_pi = static_cast<float>(2.0 * 3.14159265358979323846);
constexpr float ng_fp16_safe_max = 60000.0f;
constexpr float ng_cos_limit = 0.999999f;
constexpr float ng_shape_limit = 1e4f;
constexpr float ng_frequency_scale = 20.0f;

// quantised SH levels (degrees 1..3): first coefficient, coefficient count, bits per field, u32 words per texel
constexpr int ng_level_offset[3] = {0, 3, 8};
constexpr int ng_level_width[3] = {3, 5, 7};
constexpr int ng_level_bits[3] = {7, 8, 6};
constexpr int ng_level_words[3] = {2, 4, 4};

__device__ __forceinline__ float ng_opacity(float raw) { return 1.0f / (1.0f + expf(-raw)); }

__device__ __forceinline__ uint32_t ng_half_bits(float x) { return static_cast<uint32_t>(__half_as_ushort(__float2half_rn(x))); }

__device__ __forceinline__ float ng_round_clip(float v, float hi) { return fminf(fmaxf(rintf(v), 0.0f), hi); }

// residual activation of the exporter (0 none, 1 tanh, 2 softplus with beta 10 in its overflow-safe form)
__device__ __forceinline__ float ng_residual(float x, int act) {
    if (act == 1) return tanhf(x);
    if (act == 2) return x > 2.0f ? x : log1pf(expf(10.0f * fminf(x, 2.0f))) / 10.0f;
    return x;
}

// 8-bit log-scale code of exp(raw) (0 = exactly zero)
__device__ __forceinline__ uint32_t ng_scale_code(float raw) {
    const float s = expf(raw);
    if (s == 0.0f) return 0u;
    const float c = rintf(fmaxf(0.0f, (logf(fmaxf(s, 1e-30f)) - ng_ln_scale_min) * ng_ln_scale_encode)) + 1.0f;
    return static_cast<uint32_t>(fminf(255.0f, c));
}

// 24-bit folded-octahedral code (angle << 16 | v << 8 | u) of the normalised quaternion (w, x, y, z)
__device__ __forceinline__ uint32_t ng_quat_code(float4 q) {
    const float norm = sqrtf(((q.x * q.x + q.y * q.y) + q.z * q.z) + q.w * q.w);  // (w, x, y, z) in .x .. .w
    float w = q.x / norm, x = q.y / norm, y = q.z / norm, z = q.w / norm;
    if (w < 0.0f) {
        w = -w;
        x = -x;
        y = -y;
        z = -z;
    }
    const float half_theta = acosf(fminf(fmaxf(w, -1.0f), 1.0f));
    const float theta = 2.0f * half_theta;
    const float s = sinf(half_theta);
    float ax = 1.0f, ay = 0.0f, az = 0.0f;
    if (!(fabsf(s) < 1e-6f)) {
        ax = x / s;
        ay = y / s;
        az = z / s;
    }
    const float total = (fabsf(ax) + fabsf(ay)) + fabsf(az);
    float pu = ax / total, pv = ay / total;
    if (az < 0.0f) {
        const float fu = (1.0f - fabsf(pv)) * (pu >= 0.0f ? 1.0f : -1.0f);
        const float fv = (1.0f - fabsf(pu)) * (pv >= 0.0f ? 1.0f : -1.0f);
        pu = fu;
        pv = fv;
    }
    // the exporter's sign factors are float64 arrays, so its u / v quantisation runs in double
    const uint32_t qu = static_cast<uint32_t>(rint(fmin(fmax((static_cast<double>(pu) * 0.5 + 0.5) * 255.0, 0.0), 255.0)));
    const uint32_t qv = static_cast<uint32_t>(rint(fmin(fmax((static_cast<double>(pv) * 0.5 + 0.5) * 255.0, 0.0), 255.0)));
    const uint32_t angle = static_cast<uint32_t>(rintf(fminf(fmaxf(theta / ng_pi * 255.0f, 0.0f), 255.0f)));
    return (angle << 16) | (qv << 8) | qu;
}

// Wave reductions and scans without LDS permutes (every lane takes part). Reduction: four DPP row rotations,
// then two lane swaps across the rows, the result in every lane. Inclusive scan: DPP row shifts (zero filled),
// then lane 15 of rows 0, 2 into rows 1, 3 and lane 31 into rows 2, 3 (row broadcasts).
template <typename OP>
__device__ __forceinline__ float wave_reduce_f(float x, OP op) {
    int v = __float_as_int(x);
    v = __float_as_int(op(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false))));  // row_ror:1
    v = __float_as_int(op(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false))));  // row_ror:2
    v = __float_as_int(op(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false))));  // row_ror:4
    v = __float_as_int(op(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false))));  // row_ror:8
    const auto a = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
    const float w = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(w), __float_as_uint(w), false, false);
    return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float wave_min(float v) { return wave_reduce_f(v, [](float x, float y) { return fminf(x, y); }); }
__device__ __forceinline__ float wave_max(float v) { return wave_reduce_f(v, [](float x, float y) { return fmaxf(x, y); }); }
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, true));  // row_shr:1
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, true));  // row_shr:2
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, true));  // row_shr:4
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, true));  // row_shr:8
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
    return v;
}

// partial record per block: [0] kept count, [1] base min, [2] base max, [3..5] SH level max |coefficient|
constexpr int ng_partial_words = 8;

__global__ __launch_bounds__(ng_block) void ngsplat_stats_kernel(NgsplatArgs a, uint32_t* partials) {
    __shared__ uint32_t s_keep[ng_block];
    __shared__ float s_red[ng_block / 64][6];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t i0 = blockIdx.x * ng_block, i = i0 + tid;
    bool keep = false;
    float mn = INFINITY, mx = -INFINITY;
    if (i < a.n) {
        keep = ng_opacity(a.raw_opacities[i]) >= ng_min_alpha;
        if (keep) {
#pragma unroll
            for (int c = 0; c < 3; c++) {
                const float b = a.color_shift + a.base_colors[3 * static_cast<size_t>(i) + c];
                mn = fminf(mn, b);
                mx = fmaxf(mx, b);
            }
        }
    }
    float level[3] = {0.0f, 0.0f, 0.0f};
    if (a.payload == ng_sh && i0 < a.n && a.row_used == a.row_stride && (reinterpret_cast<uintptr_t>(a.residual_params) & 15u) == 0 &&
        a.row_used >= 4) {
        // whole rows, 16-byte aligned: the block's rows are one contiguous run read as float4 (element k of a float4
        // at flat position p belongs to row (p + k) / used, column (p + k) % used)
        s_keep[tid] = keep ? 1u : 0u;
        __syncthreads();
        const uint32_t rows = min(ng_block, a.n - i0);
        const uint32_t used = a.row_used, total = rows * used;
        const float* src = a.residual_params + static_cast<size_t>(i0) * used;
        const uint32_t step = 4 * ng_block, dr = step / used, dc = step - dr * used;
        uint32_t r = (4 * tid) / used, col = 4 * tid - r * used;
#pragma unroll 4
        for (uint32_t p = 4 * tid; p < total; p += step) {
            float4 v4;
            if (p + 4 <= total) {
                v4 = *reinterpret_cast<const float4*>(src + p);
            } else {
                v4.x = src[p];
                v4.y = p + 1 < total ? src[p + 1] : 0.0f;
                v4.z = p + 2 < total ? src[p + 2] : 0.0f;
                v4.w = 0.0f;
            }
            const float vals[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t ck = col + k, wrap = ck >= used ? 1u : 0u;
                const uint32_t cc = ck - wrap * used, rr = r + wrap;
                const float v = rr < rows && s_keep[rr] ? fabsf(vals[k]) : 0.0f;
                const uint32_t c = cc / 3;
                level[0] = c < 3 ? fmaxf(level[0], v) : level[0];
                level[1] = c >= 3 && c < 8 ? fmaxf(level[1], v) : level[1];
                level[2] = c >= 8 ? fmaxf(level[2], v) : level[2];
            }
            col += dc;
            r += dr;
            const bool wrap = col >= used;
            col = wrap ? col - used : col;
            r = wrap ? r + 1 : r;
        }
    } else if (a.payload == ng_sh && i0 < a.n) {
        s_keep[tid] = keep ? 1u : 0u;
        __syncthreads();
        const uint32_t rows = min(ng_block, a.n - i0);
        const uint32_t used = a.row_used;
        const float* src = a.residual_params + static_cast<size_t>(i0) * a.row_stride;
        // flat sweep over the rows' first `used` floats (branch-free, unrolled: several loads in flight)
        const uint32_t total = rows * used, dr = ng_block / used, dc = ng_block - dr * used;
        uint32_t r = tid / used, col = tid - r * used;
#pragma unroll 8
        for (uint32_t p = tid; p < total; p += ng_block) {
            const float v = s_keep[r] ? fabsf(src[static_cast<size_t>(r) * a.row_stride + col]) : 0.0f;
            const uint32_t c = col / 3;
            level[0] = c < 3 ? fmaxf(level[0], v) : level[0];
            level[1] = c >= 3 && c < 8 ? fmaxf(level[1], v) : level[1];
            level[2] = c >= 8 ? fmaxf(level[2], v) : level[2];
            col += dc;
            r += dr;
            const bool wrap = col >= used;
            col = wrap ? col - used : col;
            r = wrap ? r + 1 : r;
        }
    }
    const uint32_t count = static_cast<uint32_t>(__popcll(__ballot(keep)));
    mn = wave_min(mn);
    mx = wave_max(mx);
#pragma unroll
    for (int l = 0; l < 3; l++) level[l] = wave_max(level[l]);
    if (lane == 0) {
        s_red[wave][0] = __uint_as_float(count);
        s_red[wave][1] = mn;
        s_red[wave][2] = mx;
        s_red[wave][3] = level[0];
        s_red[wave][4] = level[1];
        s_red[wave][5] = level[2];
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t total = 0;
        float bmn = INFINITY, bmx = -INFINITY, l0 = 0.0f, l1 = 0.0f, l2 = 0.0f;
        for (uint32_t w = 0; w < ng_block / 64; w++) {
            total += __float_as_uint(s_red[w][0]);
            bmn = fminf(bmn, s_red[w][1]);
            bmx = fmaxf(bmx, s_red[w][2]);
            l0 = fmaxf(l0, s_red[w][3]);
            l1 = fmaxf(l1, s_red[w][4]);
            l2 = fmaxf(l2, s_red[w][5]);
        }
        uint32_t* p = partials + static_cast<size_t>(blockIdx.x) * ng_partial_words;
        p[0] = total;
        p[1] = __float_as_uint(bmn);
        p[2] = __float_as_uint(bmx);
        p[3] = __float_as_uint(l0);
        p[4] = __float_as_uint(l1);
        p[5] = __float_as_uint(l2);
    }
}

// One block of 1024 threads; thread t owns a contiguous run of blocks. Writes each block's first output row into
// partials[b * 8 + 6] and the statistics.
__global__ __launch_bounds__(1024) void ngsplat_combine_kernel(uint32_t* partials, uint32_t n_blocks, NgsplatStats* stats) {
    __shared__ uint32_t s_wave_sum[16];
    __shared__ float s_red[16][5];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t per = (n_blocks + 1023) / 1024;
    const uint32_t b0 = min(n_blocks, tid * per), b1 = min(n_blocks, b0 + per);
    uint32_t sum = 0;
    float mn = INFINITY, mx = -INFINITY, l0 = 0.0f, l1 = 0.0f, l2 = 0.0f;
    for (uint32_t b = b0; b < b1; b++) {
        const uint32_t* p = partials + static_cast<size_t>(b) * ng_partial_words;
        sum += p[0];
        mn = fminf(mn, __uint_as_float(p[1]));
        mx = fmaxf(mx, __uint_as_float(p[2]));
        l0 = fmaxf(l0, __uint_as_float(p[3]));
        l1 = fmaxf(l1, __uint_as_float(p[4]));
        l2 = fmaxf(l2, __uint_as_float(p[5]));
    }
    // inclusive scan of the per-thread sums within the wave, then over the 16 wave totals
    const uint32_t incl = wave_inclusive_sum(sum);
    mn = wave_min(mn);
    mx = wave_max(mx);
    l0 = wave_max(l0);
    l1 = wave_max(l1);
    l2 = wave_max(l2);
    if (lane == 63) s_wave_sum[wave] = incl;
    if (lane == 0) {
        s_red[wave][0] = mn;
        s_red[wave][1] = mx;
        s_red[wave][2] = l0;
        s_red[wave][3] = l1;
        s_red[wave][4] = l2;
    }
    __syncthreads();
    uint32_t before = 0, total = 0;
    for (uint32_t w = 0; w < 16; w++) {
        before += w < wave ? s_wave_sum[w] : 0u;
        total += s_wave_sum[w];
    }
    uint32_t run = before + incl - sum;
    for (uint32_t b = b0; b < b1; b++) {
        uint32_t* p = partials + static_cast<size_t>(b) * ng_partial_words;
        p[6] = run;
        run += p[0];
    }
    if (tid == 0) {
        float gmn = INFINITY, gmx = -INFINITY, g0 = 0.0f, g1 = 0.0f, g2 = 0.0f;
        for (int w = 0; w < 16; w++) {
            gmn = fminf(gmn, s_red[w][0]);
            gmx = fmaxf(gmx, s_red[w][1]);
            g0 = fmaxf(g0, s_red[w][2]);
            g1 = fmaxf(g1, s_red[w][3]);
            g2 = fmaxf(g2, s_red[w][4]);
        }
        NgsplatStats st;
        st.n_kept = total;
        if (total == 0) {
            gmn = 0.0f;
            gmx = 0.0f;
        }
        // d_scale = max(d_max - d_min, 1e-6) / 255 and the level scales max(max |c|, 1e-8) in double, as the
        // exporter's Python floats, then used (and stored) as float32
        st.base_offset = gmn;
        st.base_scale = static_cast<float>(fmax(static_cast<double>(gmx) - static_cast<double>(gmn), 1e-6) / 255.0);
        st.level_scale[0] = static_cast<float>(fmax(static_cast<double>(g0), 1e-8));
        st.level_scale[1] = static_cast<float>(fmax(static_cast<double>(g1), 1e-8));
        st.level_scale[2] = static_cast<float>(fmax(static_cast<double>(g2), 1e-8));
        *stats = st;
    }
}

// neural layer-0 input j (frequency encoded: feature j / 2k at frequency (j mod 2k) / 2, sin for even j, cos for odd)
__device__ __forceinline__ float ng_encoded(const float* row, float3 base, int n_features, int k, int j) {
    const int f = k ? j / (2 * k) : j;
    const int b = f - n_features;
    const float x = b < 0 ? row[f] : (b == 0 ? base.x : (b == 1 ? base.y : base.z));
    if (!k) return x;
    const float s = ldexpf(x, (j % (2 * k)) >> 1);
    return (j & 1) ? cosf(s) : sinf(s);
}

// fp16 payload values of one splat (neural features / baked layer 0, SV sites, NASG / NASGabor lobes)
template <int PAYLOAD>
__device__ __forceinline__ void ng_values(const NgsplatArgs& a, const float* row, float3 base, const float* bake, float (&v)[ng_max_values]) {
    if (PAYLOAD == ng_neural_features) {
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (j < a.n_values) v[j] = ng_encoded(row, base, a.n_items, a.n_frequencies, j);
    } else if (PAYLOAD == ng_neural_baked) {
        float h[ng_max_baked];
#pragma unroll
        for (int o = 0; o < static_cast<int>(ng_max_baked); o++) h[o] = 0.0f;
        for (int j = 0; j < a.n_encoded; j++) {
            const float e = ng_encoded(row, base, a.n_items, a.n_frequencies, j);
            const float4* m = reinterpret_cast<const float4*>(bake + j * ng_max_baked);
#pragma unroll
            for (int q = 0; q < static_cast<int>(ng_max_baked) / 4; q++) {
                const float4 w = m[q];
                h[4 * q + 0] = fmaf(e, w.x, h[4 * q + 0]);
                h[4 * q + 1] = fmaf(e, w.y, h[4 * q + 1]);
                h[4 * q + 2] = fmaf(e, w.z, h[4 * q + 2]);
                h[4 * q + 3] = fmaf(e, w.w, h[4 * q + 3]);
            }
        }
#pragma unroll
        for (int o = 0; o < static_cast<int>(ng_max_baked); o++)
            if (o < a.n_values) v[o] = a.bake_bias ? h[o] + a.bake_bias[o] : h[o];
    } else if (PAYLOAD == ng_sv) {
#pragma unroll
        for (int s = 0; s < 9; s++) {
            if (s >= a.n_items) continue;
            const float* x = row + 7 * s;
            const float len = fmaxf(sqrtf((x[0] * x[0] + x[1] * x[1]) + x[2] * x[2]), 1e-12f);
            v[7 * s + 0] = x[0] / len;
            v[7 * s + 1] = x[1] / len;
            v[7 * s + 2] = x[2] / len;
            v[7 * s + 3] = fminf(expf(x[3]), ng_fp16_safe_max);
            v[7 * s + 4] = ng_residual(x[4], a.residual_act);
            v[7 * s + 5] = ng_residual(x[5], a.residual_act);
            v[7 * s + 6] = ng_residual(x[6], a.residual_act);
        }
    } else {
        constexpr bool gabor = PAYLOAD == ng_nasgabor;
        constexpr int in_w = gabor ? 9 : 8, out_w = gabor ? 13 : 12, max_lobes = gabor ? 4 : 5;
#pragma unroll
        for (int l = 0; l < max_lobes; l++) {
            if (l >= a.n_items) continue;
            const float* x = row + in_w * l;
            const float ct = fminf(fmaxf(tanhf(x[0]), -ng_cos_limit), ng_cos_limit);
            const float cp = fminf(fmaxf(tanhf(x[1]), -ng_cos_limit), ng_cos_limit);
            const float cu = fminf(fmaxf(tanhf(x[2]), -ng_cos_limit), ng_cos_limit);
            const float st = sqrtf(1.0f - ct * ct), sp = sqrtf(1.0f - cp * cp), su = sqrtf(1.0f - cu * cu);
            const float lam = fminf(expf(x[3]), ng_shape_limit), an = fminf(expf(x[4]), ng_shape_limit);
            // the exporter's 1 + 1e-8 rounds to 1 in float32
            const float norm = lam * sqrtf(1.0f + an) / (ng_two_pi * (1.0f - expf(-2.0f * lam)));
            float* o = v + out_w * l;
            o[0] = ct * cp * cu - st * su;
            o[1] = st * cp * cu + ct * su;
            o[2] = -sp * cu;
            o[3] = ct * sp;
            o[4] = st * sp;
            o[5] = cp;
            o[6] = 2.0f * lam;
            o[7] = an;
            if (gabor) {
                o[8] = (tanhf(x[5]) + 1.0f) * ng_frequency_scale;
                o[9] = norm;
            } else {
                o[8] = norm;
            }
            o[out_w - 3] = ng_residual(x[in_w - 3], a.residual_act);
            o[out_w - 2] = ng_residual(x[in_w - 2], a.residual_act);
            o[out_w - 1] = ng_residual(x[in_w - 1], a.residual_act);
        }
    }
}

template <int PAYLOAD>
__global__ __launch_bounds__(ng_block) void ngsplat_pack_kernel(NgsplatArgs a, NgsplatTextures t, const uint32_t* partials,
                                                                 const NgsplatStats* stats) {
    extern __shared__ float s_rows[];  // ng_block rows of (row_used | 1) floats
    __shared__ uint32_t s_wave[ng_block / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t i0 = blockIdx.x * ng_block, i = i0 + tid;
    const NgsplatStats st = *stats;

    // rows past the kept count are zero (the format pads every texture to whole texture rows)
    if (i >= st.n_kept) {
        reinterpret_cast<uint4*>(t.splat_words)[i] = make_uint4(0u, 0u, 0u, 0u);
        for (int k = 0; k < t.n_textures; k++) {
            uint32_t* dst = t.params + t.texture_offset[k] + static_cast<size_t>(i) * t.texel_words[k];
            if (t.texel_words[k] == 4) *reinterpret_cast<uint4*>(dst) = make_uint4(0u, 0u, 0u, 0u);
            else *reinterpret_cast<uint2*>(dst) = make_uint2(0u, 0u);
        }
        if (t.source_index) t.source_index[i] = -1;
    }

    const bool keep = i < a.n && ng_opacity(a.raw_opacities[i]) >= ng_min_alpha;
    const uint64_t ballot = __ballot(keep);
    if (lane == 0) s_wave[wave] = static_cast<uint32_t>(__popcll(ballot));
    // the block's residual rows into LDS (stride row_used | 1 keeps consecutive rows in different banks)
    const uint32_t used = a.row_used, ld = used | 1u;
    if (used && i0 < a.n) {
        const uint32_t rows = min(ng_block, a.n - i0);
        const float* src = a.residual_params + static_cast<size_t>(i0) * a.row_stride;
        const uint32_t total = rows * used, dr = ng_block / used, dc = ng_block - dr * used;
        uint32_t r = tid / used, col = tid - r * used;
#pragma unroll 8
        for (uint32_t p = tid; p < total; p += ng_block) {
            s_rows[r * ld + col] = src[static_cast<size_t>(r) * a.row_stride + col];
            col += dc;
            r += dr;
            const bool wrap = col >= used;
            col = wrap ? col - used : col;
            r = wrap ? r + 1 : r;
        }
    }
    // baked layer 0: the matrix transposed into LDS after the rows (column j of all neurons is 16 consecutive floats)
    float* s_bake = s_rows + (used ? ng_block * ld : 0u);
    if (PAYLOAD == ng_neural_baked) {
        for (uint32_t p = tid; p < static_cast<uint32_t>(a.n_encoded) * ng_max_baked; p += ng_block) {
            const uint32_t j = p / ng_max_baked, o = p % ng_max_baked;
            s_bake[p] = o < static_cast<uint32_t>(a.n_values) ? a.bake_matrix[o * a.n_encoded + j] : 0.0f;
        }
    }
    __syncthreads();
    if (!keep) return;

    uint32_t row = partials[static_cast<size_t>(blockIdx.x) * ng_partial_words + 6] +
                   __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ballot >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(ballot), 0u));
    for (uint32_t w = 0; w < wave; w++) row += s_wave[w];
    if (t.source_index) t.source_index[row] = static_cast<int32_t>(i);

    // splat words
    const size_t i3 = 3 * static_cast<size_t>(i);
    float base[3];
    uint32_t base_code[3];
#pragma unroll
    for (int c = 0; c < 3; c++) {
        base[c] = a.base_colors[i3 + c];
        const float b = a.color_shift + base[c];
        base_code[c] = static_cast<uint32_t>(ng_round_clip((b - st.base_offset) / st.base_scale, 255.0f));
    }
    const uint32_t opacity_code = static_cast<uint32_t>(ng_round_clip(ng_opacity(a.raw_opacities[i]) * 255.0f, 255.0f));
    const float mx = a.means[i3], my = a.means[i3 + 1], mz = a.means[i3 + 2];
    const float* rq = a.raw_rotations + 4 * static_cast<size_t>(i);
    const uint32_t q = ng_quat_code(make_float4(rq[0], rq[1], rq[2], rq[3]));
    const uint32_t s0 = ng_scale_code(a.raw_scales[i3]), s1 = ng_scale_code(a.raw_scales[i3 + 1]), s2 = ng_scale_code(a.raw_scales[i3 + 2]);
    uint4 words;
    words.x = base_code[0] | (base_code[1] << 8) | (base_code[2] << 16) | (opacity_code << 24);
    words.y = ng_half_bits(mx) | (ng_half_bits(my) << 16);
    words.z = ng_half_bits(mz) | ((q & 0xFFu) << 16) | (((q >> 8) & 0xFFu) << 24);
    words.w = s0 | (s1 << 8) | (s2 << 16) | ((q >> 16) << 24);
    reinterpret_cast<uint4*>(t.splat_words)[row] = words;

    const float* x = s_rows + tid * ld;
    if (PAYLOAD == ng_sh) {
        // per present level: signed codes clip(round(c / scale * qmax)) bit-packed little-endian, coefficient-major rgb
#pragma unroll
        for (int l = 0; l < 3; l++) {
            if (ng_level_offset[l] + ng_level_width[l] > a.n_items) break;
            const int bits = ng_level_bits[l];
            const float qmax = static_cast<float>((1 << (bits - 1)) - 1);
            const uint32_t mask = (1u << bits) - 1u;
            const float scale = st.level_scale[l];
            // c / scale correctly rounded from the correctly rounded reciprocal and one FMA correction (Markstein)
            const float inv = 1.0f / scale;
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int f = 0; f < 3 * ng_level_width[l]; f++) {
                const float c0 = x[3 * ng_level_offset[l] + f];
                const float q0 = c0 * inv;
                const float quot = fmaf(fmaf(-q0, scale, c0), inv, q0);
                const float c = fminf(fmaxf(rintf(quot * qmax), -qmax), qmax);
                const uint32_t code = static_cast<uint32_t>(static_cast<int32_t>(c)) & mask;
                const int bit = bits * f, word = bit >> 5, shift = bit & 31;
                w[word] |= code << shift;
                if (shift + bits > 32) w[word + 1] |= code >> (32 - shift);
            }
            uint32_t* dst = t.params + t.texture_offset[l] + static_cast<size_t>(row) * ng_level_words[l];
            if (ng_level_words[l] == 4) *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
            else *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
        }
    } else {
        float v[ng_max_values];
#pragma unroll
        for (int j = 0; j < static_cast<int>(ng_max_values); j++) v[j] = 0.0f;
        ng_values<PAYLOAD>(a, x, make_float3(base[0], base[1], base[2]), s_bake, v);
#pragma unroll
        for (int k = 0; k < static_cast<int>(ng_max_textures); k++) {
            if (k >= t.n_textures) break;
            uint4 w;
            w.x = ng_half_bits(v[8 * k + 0]) | (ng_half_bits(v[8 * k + 1]) << 16);
            w.y = ng_half_bits(v[8 * k + 2]) | (ng_half_bits(v[8 * k + 3]) << 16);
            w.z = ng_half_bits(v[8 * k + 4]) | (ng_half_bits(v[8 * k + 5]) << 16);
            w.w = ng_half_bits(v[8 * k + 6]) | (ng_half_bits(v[8 * k + 7]) << 16);
            *reinterpret_cast<uint4*>(t.params + t.texture_offset[k] + static_cast<size_t>(row) * 4) = w;
        }
    }
}

}  // namespace

int ngsplat_texture_plan(int payload, int n_items, int n_values, uint32_t* texel_words) {
    if (payload == ng_sh) {
        int n = 0;
        for (int l = 0; l < 3; l++)
            if (ng_level_offset[l] + ng_level_width[l] <= n_items) texel_words[n++] = static_cast<uint32_t>(ng_level_words[l]);
        return n;
    }
    const int n = (n_values + 7) / 8;
    for (int k = 0; k < n; k++) texel_words[k] = 4;
    return n;
}

bool launch_ngsplat_pack(const NgsplatArgs& a, const NgsplatTextures& t, uint32_t* partials, NgsplatStats* stats, hipEvent_t* events,
                         hipStream_t s) {
    const uint32_t blocks = t.capacity / ng_block;
    if (events) EFGS_HIP_CHECK(hipEventRecord(events[0], s));
    ngsplat_stats_kernel<<<blocks, ng_block, 0, s>>>(a, partials);
    EFGS_HIP_CHECK(hipGetLastError());
    ngsplat_combine_kernel<<<1, 1024, 0, s>>>(partials, blocks, stats);
    EFGS_HIP_CHECK(hipGetLastError());
    if (events) EFGS_HIP_CHECK(hipEventRecord(events[1], s));
    const size_t lds = sizeof(float) * (a.row_used ? ng_block * (a.row_used | 1u) : 0) +
                       (a.payload == ng_neural_baked ? sizeof(float) * a.n_encoded * ng_max_baked : 0);
    switch (a.payload) {
    case ng_neural_features: ngsplat_pack_kernel<ng_neural_features><<<blocks, ng_block, lds, s>>>(a, t, partials, stats); break;
    case ng_neural_baked: ngsplat_pack_kernel<ng_neural_baked><<<blocks, ng_block, lds, s>>>(a, t, partials, stats); break;
    case ng_sh: ngsplat_pack_kernel<ng_sh><<<blocks, ng_block, lds, s>>>(a, t, partials, stats); break;
    case ng_sv: ngsplat_pack_kernel<ng_sv><<<blocks, ng_block, lds, s>>>(a, t, partials, stats); break;
    case ng_nasg: ngsplat_pack_kernel<ng_nasg><<<blocks, ng_block, lds, s>>>(a, t, partials, stats); break;
    case ng_nasgabor: ngsplat_pack_kernel<ng_nasgabor><<<blocks, ng_block, lds, s>>>(a, t, partials, stats); break;
    default: set_error("unknown ngsplat payload"); return false;
    }
    EFGS_HIP_CHECK(hipGetLastError());
    if (events) EFGS_HIP_CHECK(hipEventRecord(events[2], s));
    return true;
}

}  // namespace efgs
