// Alpha blending per 16x12 tile: 192 threads = 3 wave64, wave w owns pixel rows 4w..4w+3 (a 16x4 band),
// one pixel per lane. Gaussians of the tile are staged 192 at a time in LDS; each wave culls a 64-Gaussian
// chunk against its band with one 64-bit ballot and walks the surviving bits.
//
// Forward: front-to-back compositing, alpha = o exp2(min(q, 0)) with the conic pre-scaled by -log2(e)/2 and
// exp2 from ef_exp2f (a fixed operation sequence, so alpha, T and the image are reproducible bit for bit),
// alpha < 1/255 skipped, stop at T < 1e-4; stores the image, final T and last-contributor index per pixel and
// the per-tile maximum. No per-bucket checkpoints.
//
// Backward: every pixel replays its forward walk (the evaluation below is shared and compiled with
// -ffp-contract=off, so T and every skip decision are reproduced bit-exactly) and forms the reference's
// per-pixel terms; the 9 per-Gaussian values (11 with the |dL/dmean2d| pair) are summed over the wave
// (lanes = pixels) with DPP row operations, each wave keeps its own LDS slot per Gaussian, and the three band
// sums are added in a fixed order into one 48-byte record per instance at its emission slot. No float
// atomics; the result is run-to-run deterministic.
//
// Reference: B/rasterization/include/kernels_forward.cuh:26-166, kernels_backward.cuh:12-231.
#include "internal.h"

namespace efgs {

namespace {

constexpr float log2e = 1.44269504089f;

struct Staged {
    float2 xy;
    float4 co;  // exp2-scaled conic (x, y, z) and opacity
};

__device__ __forceinline__ float4 scale_conic_for_exp2(float cx, float cy, float cz, float opacity) {
    return make_float4(-0.5f * log2e * cx, -log2e * cy, -0.5f * log2e * cz, opacity);
}

// alpha of a staged Gaussian at a pixel centre; G receives the Gaussian factor
// exponent clamped to [-127, 0] with one median-of-three (the same value as min(q, 0) then max(-127) for
// every finite q)
__device__ __forceinline__ float eval_alpha(float4 xy, float4 co, float pxf, float pyf, float& dx, float& dy, float& G) {
    dx = xy.x - pxf;
    dy = xy.y - pyf;
    const float q = __builtin_fmaf(dx, __builtin_fmaf(co.x, dx, co.y * dy), co.z * dy * dy);
    G = ef_exp2f_clamped(__builtin_amdgcn_fmed3f(q, -127.0f, 0.0f));
    return co.w * G;
}

__device__ __forceinline__ uint2 rect_of(float4 xy) { return make_uint2(__float_as_uint(xy.z), __float_as_uint(xy.w)); }

__device__ __forceinline__ bool band_overlap(uint2 b, uint32_t bx0, uint32_t bx1, uint32_t by0, uint32_t by1) {
    return (b.x & 0xffffu) < bx1 && bx0 < (b.x >> 16) && (b.y & 0xffffu) < by1 && by0 < (b.y >> 16);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, o)));
    return v;
}

__global__ __launch_bounds__(tile_pixels) void blend_forward_kernel(BlendForwardArgs a) {
    // (x, y, packed pixel rectangle): the 16-byte stride of s_co and s_col, so the pair loads share one address
    __shared__ float4 s_xy[tile_pixels];
    __shared__ float4 s_co[tile_pixels];
    __shared__ float4 s_col[tile_pixels];
    __shared__ uint32_t s_max[tile_pixels / 64];

    const uint32_t tile = blockIdx.x;
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t px = tx * tile_width + (lane & 15u);
    const uint32_t py = ty * tile_height + wave * 4u + (lane >> 4);
    const bool inside = px < a.width && py < a.height;
    const float pxf = static_cast<float>(px) + 0.5f, pyf = static_cast<float>(py) + 0.5f;
    const uint32_t bx0 = tx * tile_width, bx1 = bx0 + tile_width;
    const uint32_t by0 = ty * tile_height + wave * 4u, by1 = by0 + 4u;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;

    float cr = 0.0f, cg = 0.0f, cb = 0.0f, T = 1.0f;
    uint32_t last = 0;
    bool done = !inside;
    for (uint32_t start = 0; start < n_total; start += tile_pixels) {
        if (__syncthreads_and(done)) break;
        if (start + tid < n_total) {
            const uint32_t e = a.sorted_inst[range.x + start + tid];
            const PrimRecord rec = a.records[a.inst_prim[e]];
            s_xy[tid] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            s_co[tid] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_col[tid] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
        }
        __syncthreads();
        const uint32_t batch_n = min(tile_pixels, n_total - start);
        for (uint32_t c0 = 0; c0 < batch_n; c0 += 64) {
            const uint32_t j = c0 + lane;
            const bool ov = j < batch_n && band_overlap(rect_of(s_xy[j]), bx0, bx1, by0, by1);
            uint64_t mask = __ballot(ov);
            while (mask != 0) {
                const uint32_t jj = c0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(mask)) - 1);
                mask &= mask - 1;
                // branch-free: a skipped Gaussian gets weight 0, which leaves C and T bit for bit unchanged
                float dx, dy, G;
                const float alpha = eval_alpha(s_xy[jj], s_co[jj], pxf, pyf, dx, dy, G);
                const bool take = !done && alpha >= min_alpha;
                const float a_t = take ? alpha : 0.0f;
                const float w = T * a_t;
                const float4 col = s_col[jj];
                cr = __builtin_fmaf(w, col.x, cr);
                cg = __builtin_fmaf(w, col.y, cg);
                cb = __builtin_fmaf(w, col.z, cb);
                T = T * (1.0f - a_t);
                last = take ? start + jj + 1 : last;
                done = done || (take && T < transmittance_threshold);
            }
        }
    }
    const uint32_t slot = tile * tile_pixels + tid;
    if (inside) {
        const uint32_t pix = py * a.width + px;
        const uint32_t np = a.width * a.height;
        a.image[pix] = __builtin_fmaf(T, a.bg[0], cr);
        a.image[np + pix] = __builtin_fmaf(T, a.bg[1], cg);
        a.image[2 * np + pix] = __builtin_fmaf(T, a.bg[2], cb);
    }
    a.final_T[slot] = T;
    a.n_contrib[slot] = last;
    const uint32_t wm = wave_max_u32(last);
    if (lane == 0) s_max[wave] = wm;
    __syncthreads();
    if (tid == 0) a.tile_max[tile] = max(max(s_max[0], s_max[1]), s_max[2]);
}

// Wave sums of several per-lane values at once ("transposing" reductions). Each exchange step swaps half of
// the values between lane groups so that every lane keeps fewer values, each summed over more lanes:
//   permlane32 swap: lanes l and l + 32 exchange, a pair of registers becomes one register holding value
//                    a in lanes 0-31 and value b in lanes 32-63 (sums over 2 lanes);
//   permlane16 swap: 16-lane rows 1, 3 of the first register exchange with rows 0, 2 of the second; two such
//                    registers become one holding four values, one per row (sums over 4 lanes);
//   row_ror:8      : the two 8-lane halves of a row exchange, two registers become one holding eight
//                    values, one per half-row (sums over 8 lanes);
// and plain DPP adds (quad permutations, row_shr) finish the remaining lanes. Every step is a full-rate
// VALU operation and the order is fixed, so the sums are reproducible.
template <int CTRL, int ROW_MASK, bool BOUND_CTRL>
__device__ __forceinline__ float dpp(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xf, BOUND_CTRL));
}

// v32 + swapped partner; returns a register with a's pair sums in lanes 0-31 and b's in lanes 32-63
__device__ __forceinline__ float swap32_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// rows (0, 1, 2, 3) of the result: a rows 0+1, b rows 0+1, a rows 2+3, b rows 2+3
__device__ __forceinline__ float swap16_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Eight values -> lanes 8m + 7 (m = 0..7) hold complete sums; value index of lane l: see reduced8_index.
__device__ __forceinline__ float transpose_reduce8(const float* v, uint32_t lane) {
    const float w0 = swap32_add(v[0], v[1]), w1 = swap32_add(v[2], v[3]);
    const float w2 = swap32_add(v[4], v[5]), w3 = swap32_add(v[6], v[7]);
    // rows of x0: v0, v2, v1, v3; rows of x1: v4, v6, v5, v7 (each summed over the 4 lanes equal mod 16)
    const float x0 = swap16_add(w0, w1), x1 = swap16_add(w2, w3);
    const bool hi = (lane & 8u) != 0;
    const float keep = hi ? x1 : x0, send = hi ? x0 : x1;
    float y = keep + dpp<0x128, 0xf, false>(0.0f, send);  // row_ror:8
    y += dpp<0xB1, 0xf, false>(0.0f, y);                    // quad_perm [1, 0, 3, 2]
    y += dpp<0x4E, 0xf, false>(0.0f, y);                    // quad_perm [2, 3, 0, 1]
    y += dpp<0x114, 0xf, true>(0.0f, y);                    // row_shr:4; lanes 4-7 / 12-15 of a row complete
    return y;
}

__device__ __forceinline__ uint32_t reduced8_index(uint32_t lane) {
    const uint32_t row = lane >> 4, half = (lane >> 3) & 1u;
    return 4u * half + ((row & 1u) << 1) + (row >> 1);  // rows 0..3 hold values 0, 2, 1, 3 of the half
}

// Sixteen values -> every lane of the quad (4 lanes) that holds value k has its complete sum; value index of
// lane l: see reduced16_index. The eight-value steps, then row_half_mirror (lane i of a half-row exchanges
// with lane 7 - i) splits each half-row into two quads and two quad permutations finish.
__device__ __forceinline__ float transpose_reduce16(const float* v, uint32_t lane) {
    float w[8];
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = swap32_add(v[2 * i], v[2 * i + 1]);
    // rows of x[k]: v[4k], v[4k + 2], v[4k + 1], v[4k + 3]
    float x[4];
#pragma unroll
    for (int k = 0; k < 4; k++) x[k] = swap16_add(w[2 * k], w[2 * k + 1]);
    const bool hi = (lane & 8u) != 0;  // half-row h of y0 holds x[h], of y1 holds x[2 + h]
    const float y0 = (hi ? x[1] : x[0]) + dpp<0x128, 0xf, false>(0.0f, hi ? x[0] : x[1]);  // row_ror:8
    const float y1 = (hi ? x[3] : x[2]) + dpp<0x128, 0xf, false>(0.0f, hi ? x[2] : x[3]);
    const bool q = (lane & 4u) != 0;  // quad q of each half-row holds y_q
    float z = (q ? y1 : y0) + dpp<0x141, 0xf, false>(0.0f, q ? y0 : y1);  // row_half_mirror
    z += dpp<0xB1, 0xf, false>(0.0f, z);  // quad_perm [1, 0, 3, 2]
    z += dpp<0x4E, 0xf, false>(0.0f, z);  // quad_perm [2, 3, 0, 1]
    return z;
}

__device__ __forceinline__ uint32_t reduced16_index(uint32_t lane) {
    const uint32_t row = lane >> 4, half = (lane >> 3) & 1u, quad = (lane >> 2) & 1u;
    return 4u * (half + 2u * quad) + ((row & 1u) << 1) + (row >> 1);
}

// Two values -> lanes 15, 31 hold the complete sum of a, lanes 47, 63 that of b.
__device__ __forceinline__ float transpose_reduce2(float a, float b) {
    const float w = swap32_add(a, b);  // a in lanes 0-31, b in lanes 32-63
    float x = swap16_add(w, w);        // rows 0, 1: a; rows 2, 3: b
    x += dpp<0x111, 0xf, true>(0.0f, x);  // row_shr:1
    x += dpp<0x112, 0xf, true>(0.0f, x);  // row_shr:2
    x += dpp<0x114, 0xf, true>(0.0f, x);  // row_shr:4
    x += dpp<0x118, 0xf, true>(0.0f, x);  // row_shr:8; lane 15 of each row complete
    return x;
}

// Per pixel: the nine (eleven with ABS) gradient terms of one Gaussian, zero where the pixel skips it, and the
// pixel's transmittance and remaining-colour state advanced past it (unchanged bit for bit when skipped).
template <bool ABS>
__device__ __forceinline__ void pair_terms(bool contrib, float alpha, float G, float dx, float dy, float4 col, float4 craw,
                                           float gr, float gg, float gb, float gbg, float& T, float& A, float* v,
                                           float& wgb, float& e1, float& e2) {
    const float ae = contrib ? alpha : 0.0f;
    const float Ge = contrib ? G : 0.0f;
    const float w = T * ae;
    const float oma = 1.0f - ae;
    const float rcp = __builtin_amdgcn_rcpf(fmaxf(oma, one_minus_alpha_eps));
    const float cg = __builtin_fmaf(col.z, gb, __builtin_fmaf(col.y, gg, col.x * gr));
    A = __builtin_fmaf(-w, cg, A);
    const float dalpha = __builtin_fmaf(T, cg, -rcp * (A - gbg));
    const float h = -ae * dalpha;
    const float hdx = h * dx, hdy = h * dy;
    v[0] = hdx; v[1] = hdy; v[2] = hdx * dx; v[3] = hdx * dy; v[4] = hdy * dy;
    v[5] = Ge * dalpha; v[6] = w * gr; v[7] = w * gg;
    wgb = w * gb;
    if (ABS) {
        e1 = fabsf(__builtin_fmaf(craw.x, hdx, craw.y * hdy));
        e2 = fabsf(__builtin_fmaf(craw.y, hdx, craw.z * hdy));
    }
    T = T * oma;
}

// ABS: also reduce |dL/dmean2d| per pixel (needed only for the third densification row).
//
// Only alpha has to reproduce the forward bit for bit (it decides which Gaussians a pixel skips); T and the
// gradient terms use fused multiply-adds and the hardware reciprocal. Per pixel and Gaussian the kernel
// forms, branch-free (zero for pixels that skip the Gaussian),
//   h = -alpha dL/dalpha,  dL/dalpha = T (c . g) - (A - g_bg) / max(1 - alpha, eps)
// with A = (colour still to come) . g, and the wave sums
//   h dx, h dy, h dx^2, h dx dy, h dy^2, G dL/dalpha, w g_r, w g_g, w g_b   (w = T alpha)
// from which the instance's record is dL/dmean2d = (C h d summed), dL/dconic = 0.5 (h d d^T summed),
// dL/dopacity-term = sum G dL/dalpha, dL/dcolour = sum w g.
template <bool ABS>
__global__ __launch_bounds__(tile_pixels) void blend_backward_kernel(BlendBackwardArgs a) {
    constexpr uint32_t n_values = ABS ? 11u : 9u;
    constexpr uint32_t n_waves = tile_pixels / 64;
    // (x, y, packed pixel rectangle): the 16-byte stride of s_co and s_col, so the pair loads share one address
    __shared__ float4 s_xy[tile_pixels];
    __shared__ float4 s_co[tile_pixels];    // exp2-scaled conic (x, y, z), opacity
    __shared__ float4 s_col[tile_pixels];
    __shared__ float4 s_craw[ABS ? tile_pixels : 1];  // raw conic, for the per-pixel |dL/dmean2d|
    // per wave and value one row of the batch's 192 instances, rows 200 floats apart (8 mod the 64 LDS banks):
    // the 16 lanes that store a pair's values for instances a and b hit distinct banks
    constexpr uint32_t grad_row = tile_pixels + 8;
    __shared__ float4 s_grad4[n_waves * n_values * grad_row / 4];
    float (*s_grad)[n_values][grad_row] = reinterpret_cast<float (*)[n_values][grad_row]>(s_grad4);

    const uint32_t tile = blockIdx.x;
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t px = tx * tile_width + (lane & 15u);
    const uint32_t py = ty * tile_height + wave * 4u + (lane >> 4);
    const bool inside = px < a.width && py < a.height;
    const float pxf = static_cast<float>(px) + 0.5f, pyf = static_cast<float>(py) + 0.5f;
    const uint32_t bx0 = tx * tile_width, bx1 = bx0 + tile_width;
    const uint32_t by0 = ty * tile_height + wave * 4u, by1 = by0 + 4u;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;
    const uint32_t n_proc = min(n_total, a.tile_max[tile]);

    // pixel state: upstream gradient, (colour still to come) . g, background term
    float gr = 0.0f, gg = 0.0f, gb = 0.0f, A = 0.0f, gbg = 0.0f;
    uint32_t last = 0;
    if (inside) {
        const uint32_t pix = py * a.width + px;
        const uint32_t np = a.width * a.height;
        const uint32_t slot = tile * tile_pixels + tid;
        const float Tf = a.final_T[slot];
        last = a.n_contrib[slot];
        gr = a.grad_image[pix]; gg = a.grad_image[np + pix]; gb = a.grad_image[2 * np + pix];
        const float ar = a.image[pix] - Tf * a.bg[0];
        const float ag = a.image[np + pix] - Tf * a.bg[1];
        const float ab = a.image[2 * np + pix] - Tf * a.bg[2];
        A = __builtin_fmaf(ab, gb, __builtin_fmaf(ag, gg, ar * gr));
        gbg = Tf * -(gr * a.bg[0] + gg * a.bg[1] + gb * a.bg[2]);
    }
    const uint32_t wave_last = wave_max_u32(last);  // no pixel of the band uses instances at or after this
    float T = 1.0f;

    uint32_t covered = 0;
    for (uint32_t start = 0; start < n_proc; start += tile_pixels) {
        __syncthreads();
        const bool own = start + tid < n_total;
        uint32_t e_own = 0;
        float4 craw = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (own) {
            e_own = a.sorted_inst[range.x + start + tid];
            const PrimRecord rec = a.records[a.inst_prim[e_own]];
            craw = make_float4(rec.r0.z, rec.r0.w, rec.r1.x, 0.0f);
            s_xy[tid] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            s_co[tid] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_col[tid] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
            if (ABS) s_craw[tid] = craw;
        }
        for (uint32_t k = tid; k < n_waves * n_values * grad_row / 4; k += tile_pixels) s_grad4[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        __syncthreads();
        const uint32_t batch_n = min(tile_pixels, n_total - start);
        const uint32_t batch_wave = wave_last > start ? min(min(tile_pixels, n_proc - start), wave_last - start) : 0u;
        for (uint32_t c0 = 0; c0 < batch_wave; c0 += 64) {
            const uint32_t j = c0 + lane;
            const bool ov = j < batch_wave && band_overlap(rect_of(s_xy[j]), bx0, bx1, by0, by1);
            uint64_t mask = __ballot(ov);
            // two Gaussians (a, b) per step share the transposing reductions; with an odd count the last b is
            // a = b again, skipped by every pixel and not written
            while (mask != 0) {
                const uint32_t ja = c0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(mask)) - 1);
                mask &= mask - 1;
                const bool has_b = mask != 0;
                const uint32_t jb = has_b ? c0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(mask)) - 1) : ja;
                mask &= mask - 1;
                float dxa, dya, Ga, dxb, dyb, Gb;
                const float alpha_a = eval_alpha(s_xy[ja], s_co[ja], pxf, pyf, dxa, dya, Ga);
                const float alpha_b = eval_alpha(s_xy[jb], s_co[jb], pxf, pyf, dxb, dyb, Gb);
                const bool contrib_a = start + ja < last && alpha_a >= min_alpha;
                const bool contrib_b = has_b && start + jb < last && alpha_b >= min_alpha;
                if (__ballot(contrib_a || contrib_b) == 0) continue;
                float v[16], wgb_a, wgb_b, e1a = 0.0f, e2a = 0.0f, e1b = 0.0f, e2b = 0.0f;
                const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                pair_terms<ABS>(contrib_a, alpha_a, Ga, dxa, dya, s_col[ja], ABS ? s_craw[ja] : zero4, gr, gg, gb, gbg, T, A,
                                v, wgb_a, e1a, e2a);
                pair_terms<ABS>(contrib_b, alpha_b, Gb, dxb, dyb, s_col[jb], ABS ? s_craw[jb] : zero4, gr, gg, gb, gbg, T, A,
                                v + 8, wgb_b, e1b, e2b);
                const float s16 = transpose_reduce16(v, lane);
                const uint32_t k16 = reduced16_index(lane);
                if ((lane & 3u) == 3u && (k16 < 8u || has_b)) s_grad[wave][k16 & 7u][k16 < 8u ? ja : jb] = s16;
                if (ABS) {
                    const float u[8] = {wgb_a, e1a, e2a, wgb_b, e1b, e2b, 0.0f, 0.0f};
                    const float s8 = transpose_reduce8(u, lane);
                    const uint32_t k8 = reduced8_index(lane);  // 0-2: values 8-10 of a, 3-5: of b
                    if ((lane & 7u) == 7u && (k8 < 3u || (k8 < 6u && has_b)))
                        s_grad[wave][8u + (k8 < 3u ? k8 : k8 - 3u)][k8 < 3u ? ja : jb] = s8;
                } else {
                    const float s2 = transpose_reduce2(wgb_a, wgb_b);
                    if ((lane & 31u) == 15u && (lane < 32u || has_b)) s_grad[wave][8][lane < 32u ? ja : jb] = s2;
                }
            }
        }
        __syncthreads();
        if (tid < batch_n) {
            float r[11];
#pragma unroll
            for (uint32_t c = 0; c < n_values; c++) r[c] = (s_grad[0][c][tid] + s_grad[1][c][tid]) + s_grad[2][c][tid];
            if (!ABS) r[9] = r[10] = 0.0f;
            const float gmx = __builtin_fmaf(craw.x, r[0], craw.y * r[1]);
            const float gmy = __builtin_fmaf(craw.y, r[0], craw.z * r[1]);
            float4* out = reinterpret_cast<float4*>(a.inst_grads) + 3 * static_cast<size_t>(e_own);
            out[0] = make_float4(gmx, gmy, 0.5f * r[2], 0.5f * r[3]);
            out[1] = make_float4(0.5f * r[4], r[5], r[6], r[7]);
            out[2] = make_float4(r[8], r[9], r[10], 0.0f);
        }
        covered = min(n_total, start + tile_pixels);
    }
    // instances the tile never reached (after every pixel's last contributor) get zero records
    for (uint32_t k = covered + tid; k < n_total; k += tile_pixels) {
        const uint32_t e = a.sorted_inst[range.x + k];
        float4* out = reinterpret_cast<float4*>(a.inst_grads) + 3 * static_cast<size_t>(e);
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        out[0] = z;
        out[1] = z;
        out[2] = z;
    }
}

}  // namespace

bool launch_blend_forward(const BlendForwardArgs& a, hipStream_t s) {
    if (a.n_tiles == 0) return true;
    blend_forward_kernel<<<a.n_tiles, tile_pixels, 0, s>>>(a);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_blend_backward(const BlendBackwardArgs& a, hipStream_t s) {
    if (a.n_tiles == 0) return true;
    if (a.abs_grads)
        blend_backward_kernel<true><<<a.n_tiles, tile_pixels, 0, s>>>(a);
    else
        blend_backward_kernel<false><<<a.n_tiles, tile_pixels, 0, s>>>(a);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
