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
// per-pixel terms; the 11 per-Gaussian values are summed over the wave (lanes = pixels), each wave keeps
// its own LDS slot per Gaussian, and the three band sums are added in a fixed order into one 48-byte record
// per instance at its emission slot. No float atomics; the result is run-to-run deterministic.
//
// Reference: B/rasterization/include/kernels_forward.cuh:26-166, kernels_backward.cuh:12-231.
#include "internal.h"

namespace efgs {

namespace {

constexpr float log2e = 1.44269504089f;
constexpr uint32_t grad_values = 11;

struct Staged {
    float2 xy;
    float4 co;  // exp2-scaled conic (x, y, z) and opacity
};

__device__ __forceinline__ float4 scale_conic_for_exp2(float cx, float cy, float cz, float opacity) {
    return make_float4(-0.5f * log2e * cx, -log2e * cy, -0.5f * log2e * cz, opacity);
}

// alpha of a staged Gaussian at a pixel centre; G receives the Gaussian factor
__device__ __forceinline__ float eval_alpha(float2 xy, float4 co, float pxf, float pyf, float& dx, float& dy, float& G) {
    dx = xy.x - pxf;
    dy = xy.y - pyf;
    const float q = __builtin_fmaf(dx, __builtin_fmaf(co.x, dx, co.y * dy), co.z * dy * dy);
    G = ef_exp2f(fminf(q, 0.0f));
    return co.w * G;
}

__device__ __forceinline__ bool band_overlap(uint2 b, uint32_t bx0, uint32_t bx1, uint32_t by0, uint32_t by1) {
    return (b.x & 0xffffu) < bx1 && bx0 < (b.x >> 16) && (b.y & 0xffffu) < by1 && by0 < (b.y >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, o)));
    return v;
}

__global__ __launch_bounds__(tile_pixels) void blend_forward_kernel(BlendForwardArgs a) {
    __shared__ float2 s_xy[tile_pixels];
    __shared__ float4 s_co[tile_pixels];
    __shared__ float4 s_col[tile_pixels];
    __shared__ uint2 s_b[tile_pixels];
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
            s_xy[tid] = make_float2(rec.r0.x, rec.r0.y);
            s_co[tid] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_col[tid] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
            s_b[tid] = make_uint2(__float_as_uint(rec.r2.y), __float_as_uint(rec.r2.z));
        }
        __syncthreads();
        const uint32_t batch_n = min(tile_pixels, n_total - start);
        for (uint32_t c0 = 0; c0 < batch_n; c0 += 64) {
            const uint32_t j = c0 + lane;
            const bool ov = j < batch_n && band_overlap(s_b[j], bx0, bx1, by0, by1);
            uint64_t mask = __ballot(ov);
            while (mask != 0) {
                const uint32_t jj = c0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(mask)) - 1);
                mask &= mask - 1;
                if (done) continue;
                float dx, dy, G;
                const float alpha = eval_alpha(s_xy[jj], s_co[jj], pxf, pyf, dx, dy, G);
                if (alpha < min_alpha) continue;
                const float w = T * alpha;
                const float4 col = s_col[jj];
                cr = __builtin_fmaf(w, col.x, cr);
                cg = __builtin_fmaf(w, col.y, cg);
                cb = __builtin_fmaf(w, col.z, cb);
                T = T * (1.0f - alpha);
                last = start + jj + 1;
                if (T < transmittance_threshold) done = true;
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

__global__ __launch_bounds__(tile_pixels) void blend_backward_kernel(BlendBackwardArgs a) {
    __shared__ float2 s_xy[tile_pixels];
    __shared__ float4 s_co[tile_pixels];
    __shared__ float4 s_craw[tile_pixels];
    __shared__ float4 s_col[tile_pixels];
    __shared__ uint2 s_b[tile_pixels];
    __shared__ float s_grad[tile_pixels / 64][tile_pixels][grad_values];

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

    // pixel state: upstream gradient, colour still to come after each Gaussian, background term
    float gr = 0.0f, gg = 0.0f, gb = 0.0f, ar = 0.0f, ag = 0.0f, ab = 0.0f, gac = 0.0f;
    uint32_t last = 0;
    if (inside) {
        const uint32_t pix = py * a.width + px;
        const uint32_t np = a.width * a.height;
        const uint32_t slot = tile * tile_pixels + tid;
        const float Tf = a.final_T[slot];
        last = a.n_contrib[slot];
        gr = a.grad_image[pix]; gg = a.grad_image[np + pix]; gb = a.grad_image[2 * np + pix];
        ar = a.image[pix] - Tf * a.bg[0];
        ag = a.image[np + pix] - Tf * a.bg[1];
        ab = a.image[2 * np + pix] - Tf * a.bg[2];
        gac = Tf * -(gr * a.bg[0] + gg * a.bg[1] + gb * a.bg[2]);
    }
    float T = 1.0f;

    uint32_t covered = 0;
    for (uint32_t start = 0; start < n_proc; start += tile_pixels) {
        __syncthreads();
        const bool own = start + tid < n_total;
        uint32_t e_own = 0;
        if (own) {
            e_own = a.sorted_inst[range.x + start + tid];
            const PrimRecord rec = a.records[a.inst_prim[e_own]];
            s_xy[tid] = make_float2(rec.r0.x, rec.r0.y);
            s_co[tid] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_craw[tid] = make_float4(rec.r0.z, rec.r0.w, rec.r1.x, 0.0f);
            s_col[tid] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
            s_b[tid] = make_uint2(__float_as_uint(rec.r2.y), __float_as_uint(rec.r2.z));
        }
#pragma unroll
        for (uint32_t w = 0; w < tile_pixels / 64; w++)
#pragma unroll
            for (uint32_t c = 0; c < grad_values; c++) s_grad[w][tid][c] = 0.0f;
        __syncthreads();
        const uint32_t batch_n = min(tile_pixels, n_total - start);
        const uint32_t batch_proc = min(tile_pixels, n_proc - start);
        for (uint32_t c0 = 0; c0 < batch_proc; c0 += 64) {
            const uint32_t j = c0 + lane;
            const bool ov = j < batch_proc && band_overlap(s_b[j], bx0, bx1, by0, by1);
            uint64_t mask = __ballot(ov);
            while (mask != 0) {
                const uint32_t jj = c0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(mask)) - 1);
                mask &= mask - 1;
                float v[grad_values];
#pragma unroll
                for (uint32_t c = 0; c < grad_values; c++) v[c] = 0.0f;
                bool contrib = false;
                if (start + jj < last) {
                    float dx, dy, G;
                    const float alpha = eval_alpha(s_xy[jj], s_co[jj], pxf, pyf, dx, dy, G);
                    if (alpha >= min_alpha) {
                        contrib = true;
                        const float4 col = s_col[jj];
                        const float4 cr = s_craw[jj];
                        const float w = T * alpha;
                        v[6] = w * gr; v[7] = w * gg; v[8] = w * gb;
                        ar -= w * col.x; ag -= w * col.y; ab -= w * col.z;
                        const float oma = 1.0f - alpha;
                        const float rcp = 1.0f / fmaxf(oma, one_minus_alpha_eps);
                        const float dadc = (T * col.x - ar * rcp) * gr + (T * col.y - ag * rcp) * gg + (T * col.z - ab * rcp) * gb;
                        const float dalpha = dadc + gac * rcp;
                        v[5] = G * dalpha;
                        const float h = -alpha * dalpha;
                        v[2] = 0.5f * h * (dx * dx);
                        v[3] = 0.5f * h * (dx * dy);
                        v[4] = 0.5f * h * (dy * dy);
                        v[0] = h * (cr.x * dx + cr.y * dy);
                        v[1] = h * (cr.y * dx + cr.z * dy);
                        v[9] = fabsf(v[0]);
                        v[10] = fabsf(v[1]);
                        T = T * oma;
                    }
                }
                if (__ballot(contrib) != 0) {
#pragma unroll
                    for (uint32_t c = 0; c < grad_values; c++) {
                        const float s = wave_sum(v[c]);
                        if (lane == 0) s_grad[wave][jj][c] = s;
                    }
                }
            }
        }
        __syncthreads();
        if (tid < batch_n) {
            float g[grad_values];
#pragma unroll
            for (uint32_t c = 0; c < grad_values; c++) g[c] = (s_grad[0][tid][c] + s_grad[1][tid][c]) + s_grad[2][tid][c];
            float4* out = reinterpret_cast<float4*>(a.inst_grads) + 3 * static_cast<size_t>(e_own);
            out[0] = make_float4(g[0], g[1], g[2], g[3]);
            out[1] = make_float4(g[4], g[5], g[6], g[7]);
            out[2] = make_float4(g[8], g[9], g[10], 0.0f);
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
    blend_backward_kernel<<<a.n_tiles, tile_pixels, 0, s>>>(a);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
