// Alpha blending per 16x12 tile: 192 threads = 3 wave64, wave w owns pixel rows 4w..4w+3 (a 16x4 band),
// one pixel per lane (lane l: x = l & 15, y = 4w + (l >> 4)). Each band is split into four 4x4 pixel groups:
// group g = (l >> 2) & 3 holds lanes 4g..4g+3 of every 16-lane row. Gaussians of the tile are staged in LDS;
// a 64-Gaussian chunk is culled against the four group rectangles with four 64-bit ballots, and every group
// walks its own surviving list, in order, one Gaussian per loop step (four Gaussians per wave instruction).
// Small Gaussians cover few pixels: a 4x4 group wastes far fewer lanes than a 16x4 band would.
//
// Forward: front-to-back compositing, alpha = o exp2(min(q, 0)) with the conic pre-scaled by -log2(e)/2 and
// the hardware exp2 (v_exp_f32, as the reference's fast-math exp2f), alpha < 1/255 skipped, stop at
// T < 1e-4; stores the image, final T and last-contributor index per pixel and the per-tile maximum (an
// inference render stores only the image, in CHW or HWC layout, optionally clamped). No per-bucket checkpoints.
//
// Backward: every pixel replays its forward walk (the evaluation below is shared and compiled with
// -ffp-contract=off, so T and every skip decision are reproduced bit-exactly) and forms the reference's
// per-pixel terms; the 9 per-Gaussian values (11 with the |dL/dmean2d| pair) are summed over each 16-lane
// group with two permlane swaps and two quad DPP steps, each (wave, group) keeps its own LDS slot per
// Gaussian, and the twelve group sums are added in a fixed order into one 48-byte record per instance at its
// emission slot. No float atomics; the result is run-to-run deterministic.
//
// Reference: B/rasterization/include/kernels_forward.cuh:26-166, kernels_backward.cuh:12-231.
#include "internal.h"

namespace efgs {

namespace {

constexpr float log2e = 1.44269504089f;

typedef float native_float4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(3))) char lds_char;
typedef const __attribute__((address_space(3))) native_float4 lds_float4;

struct Staged {
    float2 xy;
    float4 co;  // exp2-scaled conic (x, y, z) and opacity
};

__device__ __forceinline__ float4 scale_conic_for_exp2(float cx, float cy, float cz, float opacity) {
    return make_float4(-0.5f * log2e * cx, -log2e * cy, -0.5f * log2e * cz, opacity);
}

// alpha of a staged Gaussian at a pixel centre; G receives the Gaussian factor. v_exp_f32 (a quarter-rate
// instruction: 4 issue slots) replaces an 11-operation polynomial; its result is a fixed function of q, so
// the backward's replay reproduces the forward's alpha, T and decisions bit for bit.
__device__ __forceinline__ float eval_alpha(float4 xy, float4 co, float pxf, float pyf, float& dx, float& dy, float& G) {
    dx = xy.x - pxf;
    dy = xy.y - pyf;
    const float q = __builtin_fmaf(dx, __builtin_fmaf(co.x, dx, co.y * dy), co.z * dy * dy);
    G = __builtin_amdgcn_exp2f(fminf(q, 0.0f));
    return co.w * G;
}

__device__ __forceinline__ uint2 rect_of(float4 xy) { return make_uint2(__float_as_uint(xy.z), __float_as_uint(xy.w)); }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, o)));
    return v;
}

// Culls lane's Gaussian (rectangle `rect`, `in` = exists) against the four 4x4 groups of the band whose pixel
// columns start at bx0 and rows span [by0, by1); m[g] receives the wave's ballot for group g.
__device__ __forceinline__ void cull_groups(uint2 rect, bool in, uint32_t bx0, uint32_t by0, uint32_t by1, uint64_t (&m)[4]) {
    const uint32_t rx0 = rect.x & 0xffffu, rx1 = rect.x >> 16, ry0 = rect.y & 0xffffu, ry1 = rect.y >> 16;
    const bool yov = in && ry0 < by1 && by0 < ry1;
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        const uint32_t gx0 = bx0 + 4u * k;
        m[k] = __ballot(yov && rx0 < gx0 + 4u && gx0 < rx1);
    }
}

// the value of the lane's own group among four wave-uniform ones
__device__ __forceinline__ uint32_t pick_group(uint32_t g, uint32_t j0, uint32_t j1, uint32_t j2, uint32_t j3) {
    return (g & 2u) ? ((g & 1u) ? j3 : j2) : ((g & 1u) ? j1 : j0);
}

// Writes each group's surviving Gaussians of the chunk, in order, to list[k * list_len + 0 .. n[k]) (entry:
// (base + lane) << shift for the Gaussian, a batch index or, shifted, a byte offset into 16-byte staged arrays);
// n[k] = popcount(m[k]). A group then walks its list with one LDS read per step instead of scanning a 64-bit
// mask per lane.
__device__ __forceinline__ void build_group_lists(const uint64_t (&m)[4], uint32_t lane, uint32_t base, uint32_t* list,
                                                  uint32_t list_len, uint32_t (&n)[4], uint32_t shift = 0) {
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        const uint32_t lo = static_cast<uint32_t>(m[k]), hi = static_cast<uint32_t>(m[k] >> 32);
        if ((m[k] >> lane) & 1u) list[k * list_len + __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u))] = (base + lane) << shift;
        n[k] = static_cast<uint32_t>(__popcll(m[k]));
    }
}

// orders a wave's LDS accesses around its list writes (lanes read entries other lanes wrote)
__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

__global__ __launch_bounds__(tile_pixels) void blend_forward_kernel(BlendForwardArgs a) {
    if (a.overflow && *a.overflow != 0) return;  // the binning was skipped: the host re-runs the frame
    constexpr uint32_t list_len = 64;
    // (x, y, packed pixel rectangle): the 16-byte stride of s_co and s_col, so the pair loads share one address
    __shared__ float4 s_xy[tile_pixels];
    __shared__ float4 s_co[tile_pixels];
    __shared__ float4 s_col[tile_pixels];
    __shared__ uint32_t s_list[tile_pixels / 64][4][list_len];  // per wave and group: batch indices to walk
    __shared__ uint32_t s_max[tile_pixels / 64];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tile = a.order ? a.order[blockIdx.x] : blockIdx.x;  // heaviest tiles first
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t g = (lane >> 2) & 3u;
    const uint32_t px = tx * tile_width + (lane & 15u);
    const uint32_t py = ty * tile_height + wave * 4u + (lane >> 4);
    const bool inside = px < a.width && py < a.height;
    const float pxf = static_cast<float>(px) + 0.5f, pyf = static_cast<float>(py) + 0.5f;
    const uint32_t bx0 = tx * tile_width;
    const uint32_t by0 = ty * tile_height + wave * 4u, by1 = by0 + 4u;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;
    const uint32_t* const my_list = &s_list[wave][g][0];
    // list entries past a group's count are read (and skipped): keep them valid batch indices
    for (uint32_t k = tid; k < tile_pixels / 64 * 4 * list_len; k += tile_pixels) (&s_list[0][0][0])[k] = 0;

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
        // byte offset of the last Gaussian of this batch the pixel took (~0: none); the last-contributor index
        // start + offset / 16 + 1 is formed once per batch
        uint32_t last_off = ~0u;
        for (uint32_t c0 = 0; c0 < batch_n; c0 += 64) {
            uint64_t m[4];
            cull_groups(rect_of(s_xy[c0 + lane]), c0 + lane < batch_n, bx0, by0, by1, m);
            uint32_t n[4];
            build_group_lists(m, lane, c0, &s_list[wave][0][0], list_len, n, 4u);  // entries: byte offsets of the staged float4s
            wave_lds_fence();
            const uint32_t n_max = max(max(n[0], n[1]), max(n[2], n[3]));
            const uint32_t my_n = pick_group(g, n[0], n[1], n[2], n[3]);
            // two Gaussians of the group's list per step (list_len is even, so entry k + 1 exists; past the
            // group's count it is a stale entry, skipped)
            const auto walk = [&](uint32_t k, uint32_t off) {
                const auto at = [off](const float4* arr) { return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(arr) + off); };
                // branch-free: a skipped Gaussian gets weight 0, which leaves C and T bit for bit unchanged
                float dx, dy, G;
                const float alpha = eval_alpha(at(s_xy), at(s_co), pxf, pyf, dx, dy, G);
                const bool take = k < my_n && !done && alpha >= min_alpha;
                const float a_t = take ? alpha : 0.0f;
                const float w = T * a_t;
                const float4 col = at(s_col);
                cr = __builtin_fmaf(w, col.x, cr);
                cg = __builtin_fmaf(w, col.y, cg);
                cb = __builtin_fmaf(w, col.z, cb);
                T = T * (1.0f - a_t);
                last_off = take ? off : last_off;
                done = done || (take && T < transmittance_threshold);
            };
            for (uint32_t k = 0; k < n_max; k += 2) {
                const uint2 jab = *reinterpret_cast<const uint2*>(my_list + k);
                walk(k, jab.x);
                walk(k + 1, jab.y);
            }
            wave_lds_fence();
        }
        if (last_off != ~0u) last = start + (last_off >> 4) + 1u;
    }
    const uint32_t slot = tile * tile_pixels + tid;
    if (inside) {
        const uint32_t pix = py * a.width + px;
        float c[3] = {__builtin_fmaf(T, a.bg[0], cr), __builtin_fmaf(T, a.bg[1], cg), __builtin_fmaf(T, a.bg[2], cb)};
        if (a.clamp) {
#pragma unroll
            for (int k = 0; k < 3; k++) c[k] = fminf(fmaxf(c[k], 0.0f), 1.0f);
        }
        if (a.hwc) {
#pragma unroll
            for (int k = 0; k < 3; k++) a.image[3 * pix + k] = c[k];
        } else {
            const uint32_t np = a.width * a.height;
#pragma unroll
            for (int k = 0; k < 3; k++) a.image[k * np + pix] = c[k];
        }
    }
    if (!a.final_T) return;  // inference render: no backward state (uniform over the block)
    a.final_T[slot] = T;
    a.n_contrib[slot] = last;
    const uint32_t wm = wave_max_u32(last);
    if (lane == 0) s_max[wave] = wm;
    __syncthreads();
    if (tid == 0) a.tile_max[tile] = max(max(s_max[0], s_max[1]), s_max[2]);
}

// Sums of several per-lane values over each 4x4 pixel group at once ("transposing" reductions). A group's
// 16 lanes are lanes 4g..4g+3 of the four 16-lane rows. Each exchange step swaps half of the values between
// lanes so that every lane keeps fewer values, each summed over more lanes of its group:
//   permlane32 swap: lanes l and l + 32 exchange, a pair of registers becomes one register holding value
//                    a in rows 0, 1 and value b in rows 2, 3 (sums over 2 rows);
//   permlane16 swap: rows 1, 3 of the first register exchange with rows 0, 2 of the second; two such
//                    registers become one holding four values, one per row (sums over the 4 rows);
//   quad_perm      : lanes i and i ^ 2 of a row quad exchange, then i and i ^ 1 add (sums over the quad).
// Every step is a full-rate VALU operation and the order is fixed, so the sums are reproducible.
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

// Eight values -> lane (r, i) of a group (row r, quad position i) holds the group sum of value
// 4 (i >> 1) + {0, 2, 1, 3}[r].
__device__ __forceinline__ float group_reduce8(const float* v, uint32_t lane) {
    const float w0 = swap32_add(v[0], v[1]), w1 = swap32_add(v[2], v[3]);
    const float w2 = swap32_add(v[4], v[5]), w3 = swap32_add(v[6], v[7]);
    const float x0 = swap16_add(w0, w1), x1 = swap16_add(w2, w3);  // rows: v0, v2, v1, v3 / v4, v6, v5, v7
    const bool hi = (lane & 2u) != 0;
    float y = (hi ? x1 : x0) + dpp<0x4E, 0xf, true>(0.0f, hi ? x0 : x1);  // quad_perm [2, 3, 0, 1]
    y += dpp<0xB1, 0xf, true>(0.0f, y);                                     // quad_perm [1, 0, 3, 2]
    return y;
}

__device__ __forceinline__ uint32_t group_reduced8_index(uint32_t lane) {
    const uint32_t r = lane >> 4;
    return 4u * ((lane >> 1) & 1u) + ((r & 1u) << 1) + (r >> 1);
}

// Sixteen values -> lane (r, i) of a group holds the group sum of value 4 m + {0, 2, 1, 3}[r] with
// m = {0, 2, 1, 3}[i]: values 0-7 on even quad positions, 8-15 on odd ones.
__device__ __forceinline__ float group_reduce16(const float* v, uint32_t lane) {
    float w[8];
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = swap32_add(v[2 * i], v[2 * i + 1]);
    float x[4];  // rows of x[m]: v[4m], v[4m + 2], v[4m + 1], v[4m + 3]
#pragma unroll
    for (int m = 0; m < 4; m++) x[m] = swap16_add(w[2 * m], w[2 * m + 1]);
    const bool h2 = (lane & 2u) != 0;  // quad positions 2, 3 keep x[1] and x[3]
    const float y0 = (h2 ? x[1] : x[0]) + dpp<0x4E, 0xf, true>(0.0f, h2 ? x[0] : x[1]);  // quad_perm [2, 3, 0, 1]
    const float y1 = (h2 ? x[3] : x[2]) + dpp<0x4E, 0xf, true>(0.0f, h2 ? x[2] : x[3]);
    const bool h1 = (lane & 1u) != 0;  // odd positions keep y1
    return (h1 ? y1 : y0) + dpp<0xB1, 0xf, true>(0.0f, h1 ? y0 : y1);                  // quad_perm [1, 0, 3, 2]
}

__device__ __forceinline__ uint32_t group_reduced16_index(uint32_t lane) {
    const uint32_t r = lane >> 4, i = lane & 3u;
    return 4u * (2u * (i & 1u) + (i >> 1)) + ((r & 1u) << 1) + (r >> 1);
}

// Two values -> rows 0, 1 of a group hold the group sum of a, rows 2, 3 that of b.
__device__ __forceinline__ float group_reduce2(float a, float b) {
    float w = swap32_add(a, b);
    w = swap16_add(w, w);
    w += dpp<0x4E, 0xf, true>(0.0f, w);
    w += dpp<0xB1, 0xf, true>(0.0f, w);
    return w;
}

// Per pixel: the nine (eleven with ABS) gradient terms of one Gaussian, zero where the pixel skips it, and the
// pixel's transmittance and remaining-colour state advanced past it (unchanged bit for bit when skipped).
template <bool ABS>
__device__ __forceinline__ void pair_terms(bool contrib, float alpha, float dx, float dy, float4 col, float4 conic,
                                           float gr, float gg, float gb, float gbg, float& T, float& A, float* v,
                                           float& wgb, float& e1, float& e2) {
    const float ae = contrib ? alpha : 0.0f;
    const float w = T * ae;
    const float oma = 1.0f - ae;
    const float rcp = __builtin_amdgcn_rcpf(fmaxf(oma, one_minus_alpha_eps));
    const float cg = __builtin_fmaf(col.z, gb, __builtin_fmaf(col.y, gg, col.x * gr));
    A = __builtin_fmaf(-w, cg, A);
    const float dalpha = __builtin_fmaf(T, cg, -rcp * (A - gbg));
    const float h = -ae * dalpha;
    const float hdx = h * dx, hdy = h * dy;
    v[0] = hdx; v[1] = hdy; v[2] = hdx * dx; v[3] = hdx * dy; v[4] = hdy * dy;
    v[5] = h; v[6] = w * gr; v[7] = w * gg;
    wgb = w * gb;
    if (ABS) {  // |dL/dmean2d| of the pixel: the raw conic times h d (the exp2-scaled conic divided back)
        e1 = fabsf(__builtin_fmaf(conic.x, hdx, conic.y * hdy));
        e2 = fabsf(__builtin_fmaf(conic.y, hdx, conic.z * hdy));
    }
    T = T * oma;
}

// raw conic (x, y, z) of an exp2-scaled one (scale_conic_for_exp2 inverted)
__device__ __forceinline__ float4 raw_conic_of(float4 co) {
    constexpr float ln2 = 0.69314718055994531f;
    return make_float4(-2.0f * ln2 * co.x, -ln2 * co.y, -2.0f * ln2 * co.z, 0.0f);
}

// ABS: also reduce |dL/dmean2d| per pixel (needed only for the third densification row).
//
// Only alpha has to reproduce the forward bit for bit (it decides which Gaussians a pixel skips); T and the
// gradient terms use fused multiply-adds and the hardware reciprocal. Per pixel and Gaussian the kernel
// forms, branch-free (zero for pixels that skip the Gaussian),
//   h = -alpha dL/dalpha,  dL/dalpha = T (c . g) - (A - g_bg) / max(1 - alpha, eps)
// with A = (colour still to come) . g, and the group sums
//   h dx, h dy, h dx^2, h dx dy, h dy^2, h, w g_r, w g_g, w g_b   (w = T alpha)
// from which the instance's record is dL/dmean2d = (C h d summed), dL/dconic = 0.5 (h d d^T summed),
// dL/dopacity-term = sum G dL/dalpha = -(sum h) / o, dL/dcolour = sum w g.
//
// Each group walks two Gaussians (a, b) of its list per step, so their first eight values share one
// 16-value reduction and their ninth values a 2-value one; every (wave, group) stores its sums in its own
// LDS slot per Gaussian (a group visits a Gaussian at most once per batch). Gaussians are staged BATCH at a
// time (double-buffered, the next batch's records fetched into registers while the current one is walked):
// one block barrier before the walk, one before the combine, which adds the twelve slots of each value in a
// fixed order and clears them for the next batch. The groups' lists are padded to an even length with a staged
// dummy of opacity 0 (index BATCH: its alpha is 0, it is never taken, and its sums land in the slots' spare
// column), so the walk needs no per-entry bounds. No atomics: the result is run-to-run deterministic.
constexpr uint32_t blend_backward_batch = 32;

template <bool ABS, uint32_t BATCH>
__global__ __launch_bounds__(tile_pixels) void blend_backward_kernel(BlendBackwardArgs a) {
    constexpr uint32_t n_values = ABS ? 11u : 9u;
    constexpr uint32_t n_waves = tile_pixels / 64;
    constexpr uint32_t list_len = BATCH;
    constexpr uint32_t n_slots = n_waves * 4;  // (wave, group) pairs
    constexpr uint32_t dummy = BATCH;          // staged Gaussian of opacity 0 and slot column past the batch
    // slots [wave][group][value][instance]; value rows BATCH + 1 floats apart
    constexpr uint32_t value_stride = BATCH + 1;
    constexpr uint32_t slot_stride = n_values * value_stride;
    constexpr uint32_t n_parts = 6;  // 8-byte parts of the 48-byte record written by the combine
    static_assert(BATCH <= 64 && BATCH % 2 == 0, "a batch is culled by one wave ballot");
    // staged per Gaussian: (x, y, packed rect), exp2-scaled conic + opacity, colour
    __shared__ float4 s_stage[2][BATCH + 1][3];
    __shared__ uint32_t s_emit[2][BATCH];
    __shared__ uint32_t s_list[n_waves][4][list_len];
    __shared__ float s_part[n_slots * slot_stride];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tile = a.order ? a.order[blockIdx.x] : blockIdx.x;  // heaviest tiles first
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t g = (lane >> 2) & 3u;
    const uint32_t px = tx * tile_width + (lane & 15u);
    const uint32_t py = ty * tile_height + wave * 4u + (lane >> 4);
    const bool inside = px < a.width && py < a.height;
    const float pxf = static_cast<float>(px) + 0.5f, pyf = static_cast<float>(py) + 0.5f;
    const uint32_t bx0 = tx * tile_width;
    const uint32_t by0 = ty * tile_height + wave * 4u;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;
    const uint32_t n_proc = min(n_total, a.tile_max[tile]);
    const uint32_t* const my_list = &s_list[wave][g][0];
    for (uint32_t k = tid; k < n_slots * slot_stride; k += tile_pixels) s_part[k] = 0.0f;
    if (tid < 6) (&s_stage[tid / 3u][dummy][0])[tid % 3u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    // where this lane stores after the reductions: every lane one of the 16 main values (even quad positions
    // Gaussian a, odd ones b); a few lanes one of the extra values (value 8, with ABS also 9 and 10)
    const uint32_t row = lane >> 4, qpos = lane & 3u;
    const uint32_t main_b = qpos & 1u;
    float* const slot = s_part + (wave * 4u + g) * slot_stride;
    float* const part_main = slot + (group_reduced16_index(lane) & 7u) * value_stride;
    bool extra_lane;
    uint32_t extra_b, extra_k;
    if (ABS) {  // group_reduce8 of (wgb, e1, e2) of a then b: value u = 4 (i >> 1) + {0, 2, 1, 3}[r]
        const uint32_t u = group_reduced8_index(lane);
        extra_lane = (qpos & 1u) == 0 && u < 6u;
        extra_b = u >= 3u ? 1u : 0u;
        extra_k = 8u + (u >= 3u ? u - 3u : u);
    } else {    // group_reduce2: rows 0, 1 hold a, rows 2, 3 hold b
        extra_lane = qpos == 0 && (row == 0 || row == 2);
        extra_b = row == 2 ? 1u : 0u;
        extra_k = 8u;
    }
    float* const part_extra = slot + extra_k * value_stride;

    // pixel state: upstream gradient, (colour still to come) . g, background term
    float gr = 0.0f, gg = 0.0f, gb = 0.0f, A = 0.0f, gbg = 0.0f;
    uint32_t last = 0;
    if (inside) {
        const uint32_t pix = py * a.width + px;
        const uint32_t np = a.width * a.height;
        const uint32_t pslot = tile * tile_pixels + tid;
        const float Tf = a.final_T[pslot];
        last = a.n_contrib[pslot];
        gr = a.grad_image[pix]; gg = a.grad_image[np + pix]; gb = a.grad_image[2 * np + pix];
        const float ar = a.image[pix] - Tf * a.bg[0];
        const float ag = a.image[np + pix] - Tf * a.bg[1];
        const float ab = a.image[2 * np + pix] - Tf * a.bg[2];
        A = __builtin_fmaf(ab, gb, __builtin_fmaf(ag, gg, ar * gr));
        gbg = Tf * -(gr * a.bg[0] + gg * a.bg[1] + gb * a.bg[2]);
    }
    const uint32_t wave_last = wave_max_u32(last);  // no pixel of the band uses instances at or after this
    float T = 1.0f;

    // staging threads (the first BATCH threads) fetch the record of their instance one batch ahead
    uint32_t e_next = 0;
    PrimRecord rec_next{};
    const auto fetch = [&](uint32_t s) {
        if (tid < BATCH && s + tid < n_total) {
            e_next = a.sorted_inst[range.x + s + tid];
            rec_next = a.records[a.inst_prim[e_next]];
        }
    };
    const auto stage = [&](uint32_t s, uint32_t buf) {
        if (tid < BATCH && s + tid < n_total) {
            const PrimRecord& rec = rec_next;
            float4* st = s_stage[buf][tid];
            const float4 co = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            st[0] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            st[1] = co;
            st[2] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
            s_emit[buf][tid] = e_next;
        }
    };
    if (n_proc > 0) {
        fetch(0);
        stage(0, 0);
        fetch(BATCH);
    }

    uint32_t covered = 0;
    uint32_t buf = 0;
    for (uint32_t start = 0; start < n_proc; start += BATCH, buf ^= 1u) {
        __syncthreads();  // batch staged; the previous combine has read and cleared the slots
        const uint32_t batch_wave = wave_last > start ? min(min(BATCH, n_proc - start), wave_last - start) : 0u;
        const float4(*const stg)[3] = s_stage[buf];
        uint64_t m[4];
        cull_groups(rect_of(stg[lane < BATCH ? lane : dummy][0]), lane < batch_wave, bx0, by0, by0 + 4u, m);
        uint32_t n[4];
        build_group_lists(m, lane, 0u, &s_list[wave][0][0], list_len, n);
        const uint32_t n_max = __builtin_amdgcn_readfirstlane(max(max(n[0], n[1]), max(n[2], n[3])));
        const uint32_t n_steps = (n_max + 1u) & ~1u;
        // pad every list to the even step count with the dummy
#pragma unroll
        for (uint32_t k = 0; k < 4; k++)
            if (lane >= n[k] && lane < n_steps) s_list[wave][k][lane] = dummy;
        wave_lds_fence();
        const uint32_t last_rel = last > start ? last - start : 0u;  // Gaussians j < last_rel are before `last`
        for (uint32_t k = 0; k < n_steps; k += 2) {
            const uint2 jab = *reinterpret_cast<const uint2*>(my_list + k);
            const uint32_t ja = jab.x, jb = jab.y;
            // staged float4 c of instance j, addressed in the LDS address space (32-bit offsets, 24-bit product)
            const auto at = [stg](uint32_t j, uint32_t c) {
                lds_char* base = (lds_char*)(stg);
                const native_float4 v = *reinterpret_cast<lds_float4*>(base + __umul24(j, static_cast<uint32_t>(sizeof(stg[0]))) + 16u * c);
                return make_float4(v.x, v.y, v.z, v.w);
            };
            float dxa, dya, Ga, dxb, dyb, Gb;
            const float alpha_a = eval_alpha(at(ja, 0), at(ja, 1), pxf, pyf, dxa, dya, Ga);
            const float alpha_b = eval_alpha(at(jb, 0), at(jb, 1), pxf, pyf, dxb, dyb, Gb);
            const bool ca = ja < last_rel && alpha_a >= min_alpha;
            const bool cb = jb < last_rel && alpha_b >= min_alpha;
            float v[16], wgb_a, wgb_b, e1a = 0.0f, e2a = 0.0f, e1b = 0.0f, e2b = 0.0f;
            const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            pair_terms<ABS>(ca, alpha_a, dxa, dya, at(ja, 2), ABS ? raw_conic_of(at(ja, 1)) : zero4, gr, gg, gb, gbg, T, A, v, wgb_a, e1a, e2a);
            pair_terms<ABS>(cb, alpha_b, dxb, dyb, at(jb, 2), ABS ? raw_conic_of(at(jb, 1)) : zero4, gr, gg, gb, gbg, T, A, v + 8, wgb_b, e1b, e2b);
            part_main[main_b ? jb : ja] = group_reduce16(v, lane);
            float sx;
            if (ABS) {
                const float u[8] = {wgb_a, e1a, e2a, wgb_b, e1b, e2b, 0.0f, 0.0f};
                sx = group_reduce8(u, lane);
            } else {
                sx = group_reduce2(wgb_a, wgb_b);
            }
            if (extra_lane) part_extra[extra_b ? jb : ja] = sx;
        }
        wave_lds_fence();
        __syncthreads();  // every group's sums are in its slots
        // combine: item (part p, instance j) adds the twelve slots of its two values in a fixed order, clears
        // them, and writes its 8 bytes of the 48-byte record
        const uint32_t batch_n = min(BATCH, n_total - start);
        for (uint32_t item = tid; item < n_parts * BATCH; item += tile_pixels) {
            const uint32_t j = item % BATCH, p = item / BATCH;  // p = 0..5: values 2p, 2p + 1
            if (j >= batch_n) continue;
            float r[2] = {0.0f, 0.0f};
#pragma unroll
            for (uint32_t c = 0; c < 2; c++) {
                const uint32_t k = 2u * p + c;
                if (k < n_values) {
                    float* src = s_part + k * value_stride + j;
                    float acc = 0.0f;
#pragma unroll
                    for (uint32_t q = 0; q < n_slots; q++) {
                        acc += src[q * slot_stride];
                        src[q * slot_stride] = 0.0f;
                    }
                    r[c] = acc;
                }
            }
            float2* out = reinterpret_cast<float2*>(a.inst_grads) + 6 * static_cast<size_t>(s_emit[buf][j]) + p;
            float2 o;
            if (p == 0) {
                const float4 craw = raw_conic_of(s_stage[buf][j][1]);
                o = make_float2(__builtin_fmaf(craw.x, r[0], craw.y * r[1]), __builtin_fmaf(craw.y, r[0], craw.z * r[1]));
            } else if (p == 1) {
                o = make_float2(0.5f * r[0], 0.5f * r[1]);
            } else if (p == 2) {
                o = make_float2(0.5f * r[0], -r[1] / s_stage[buf][j][1].w);   // sum of G dL/dalpha = -(sum of h) / o
            } else {
                o = make_float2(r[0], r[1]);  // zero past the last value
            }
            *out = o;
        }
        covered = min(n_total, start + BATCH);
        // stage the next batch into the other buffer (its last readers finished before this batch's first
        // barrier) and fetch the one after it
        if (start + BATCH < n_proc) {
            stage(start + BATCH, buf ^ 1u);
            fetch(start + 2 * BATCH);
        }
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

// Speedy-Splat pruning scores: per pixel and contributing Gaussian (o dL/dalpha)^2 for the upstream gradient
// (1, 1, 1), with dL/dalpha formed as in the backward: T (c . 1) - (A - g_bg) / max(1 - alpha, eps), A = (colour
// still to come) . 1, g_bg = -T_final (bg . 1). Same replay, 4x4 groups and lists as the backward; each group
// walks two Gaussians per step and sums their scores over its 16 lanes with one two-value reduction; per batch
// the twelve (wave, group) slots are added in a fixed order into one float per instance at its emission slot
// (instances after every pixel's last contributor get 0). No atomics (the reference adds per pixel with float
// atomics). Reference: B/rasterization/include/kernels_pruning_scores.cuh:11-171.
__global__ __launch_bounds__(tile_pixels) void blend_scores_kernel(BlendBackwardArgs a) {
    constexpr uint32_t n_waves = tile_pixels / 64;
    constexpr uint32_t batch = 32;
    constexpr uint32_t list_len = batch;
    constexpr uint32_t n_slots = n_waves * 4;
    __shared__ float4 s_stage[batch][3];  // (x, y, packed rect), exp2-scaled conic + opacity, colour
    __shared__ uint32_t s_emit[batch];
    __shared__ uint32_t s_list[n_waves][4][list_len];
    __shared__ float s_part[n_slots][batch + 1];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tile = a.order ? a.order[blockIdx.x] : blockIdx.x;  // heaviest tiles first
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t g = (lane >> 2) & 3u;
    const uint32_t px = tx * tile_width + (lane & 15u);
    const uint32_t py = ty * tile_height + wave * 4u + (lane >> 4);
    const bool inside = px < a.width && py < a.height;
    const float pxf = static_cast<float>(px) + 0.5f, pyf = static_cast<float>(py) + 0.5f;
    const uint32_t bx0 = tx * tile_width;
    const uint32_t by0 = ty * tile_height + wave * 4u, by1 = by0 + 4u;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;
    const uint32_t n_proc = min(n_total, a.tile_max[tile]);
    const uint32_t* const my_list = &s_list[wave][g][0];
    for (uint32_t k = tid; k < n_waves * 4 * list_len; k += tile_pixels) (&s_list[0][0][0])[k] = 0;
    for (uint32_t k = tid; k < n_slots * (batch + 1); k += tile_pixels) (&s_part[0][0])[k] = 0.0f;
    // group_reduce2 leaves Gaussian a's sum in rows 0, 1 and b's in rows 2, 3: lane 4g of rows 0 and 2 store
    const uint32_t row = lane >> 4;
    const bool store_lane = (lane & 3u) == 0 && (row == 0 || row == 2);
    const uint32_t store_b = row == 2 ? 1u : 0u;
    float* const slot = &s_part[wave * 4u + g][0];

    float A = 0.0f, gbg = 0.0f;
    uint32_t last = 0;
    if (inside) {
        const uint32_t pix = py * a.width + px;
        const uint32_t np = a.width * a.height;
        const uint32_t pslot = tile * tile_pixels + tid;
        const float Tf = a.final_T[pslot];
        last = a.n_contrib[pslot];
        A = (a.image[pix] - Tf * a.bg[0]) + (a.image[np + pix] - Tf * a.bg[1]) + (a.image[2 * np + pix] - Tf * a.bg[2]);
        gbg = Tf * -(a.bg[0] + a.bg[1] + a.bg[2]);
    }
    const uint32_t wave_last = wave_max_u32(last);
    float T = 1.0f;

    uint32_t covered = 0;
    for (uint32_t start = 0; start < n_proc; start += batch) {
        __syncthreads();  // the previous batch's combine has read the stage and cleared the slots
        if (tid < batch && start + tid < n_total) {
            const uint32_t e = a.sorted_inst[range.x + start + tid];
            const PrimRecord rec = a.records[a.inst_prim[e]];
            s_stage[tid][0] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            s_stage[tid][1] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_stage[tid][2] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
            s_emit[tid] = e;
        }
        __syncthreads();
        const uint32_t batch_wave = wave_last > start ? min(min(batch, n_proc - start), wave_last - start) : 0u;
        uint64_t m[4];
        cull_groups(rect_of(s_stage[lane & (batch - 1)][0]), lane < batch_wave, bx0, by0, by1, m);
        uint32_t n[4];
        build_group_lists(m, lane, 0u, &s_list[wave][0][0], list_len, n);
        wave_lds_fence();
        const uint32_t n_max = __builtin_amdgcn_readfirstlane(max(max(n[0], n[1]), max(n[2], n[3])));
        const uint32_t my_n = pick_group(g, n[0], n[1], n[2], n[3]);
        const uint32_t n_store = store_lane && my_n > store_b ? my_n - store_b : 0u;
        const uint32_t last_rel = last > start ? last - start : 0u;
        for (uint32_t k = 0; k < n_max; k += 2) {
            const uint2 jab = *reinterpret_cast<const uint2*>(my_list + k);  // past the count: stale, skipped
            float sc[2];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                const uint32_t j = h ? jab.y : jab.x;
                float dx, dy, G;
                const float4 co = s_stage[j][1];
                const float alpha = eval_alpha(s_stage[j][0], co, pxf, pyf, dx, dy, G);
                const bool contrib = k + h < my_n && j < last_rel && alpha >= min_alpha;
                const float ae = contrib ? alpha : 0.0f;
                const float4 col = s_stage[j][2];
                const float cg = col.x + col.y + col.z;
                const float oma = 1.0f - ae;
                const float rcp = __builtin_amdgcn_rcpf(fmaxf(oma, one_minus_alpha_eps));
                A = __builtin_fmaf(-T * ae, cg, A);
                const float dg = co.w * __builtin_fmaf(T, cg, -rcp * (A - gbg));
                sc[h] = contrib ? dg * dg : 0.0f;
                T = T * oma;
            }
            const float sx = group_reduce2(sc[0], sc[1]);
            if (k < n_store) slot[store_b ? jab.y : jab.x] = sx;
        }
        wave_lds_fence();
        __syncthreads();  // every group's sums are in its slots
        const uint32_t batch_n = min(batch, n_total - start);
        if (tid < batch_n) {
            float acc = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < n_slots; q++) {
                acc += s_part[q][tid];
                s_part[q][tid] = 0.0f;
            }
            a.inst_grads[s_emit[tid]] = acc;
        }
        covered = min(n_total, start + batch);
    }
    for (uint32_t k = covered + tid; k < n_total; k += tile_pixels) a.inst_grads[a.sorted_inst[range.x + k]] = 0.0f;
}

// scores[p] += the primitive's per-instance scores, in emission order (contiguous slots from prim_offset)
__global__ __launch_bounds__(256) void accumulate_scores_kernel(const uint32_t* n_touched, const uint32_t* prim_offset, const float* inst_scores,
                                                               float* scores, uint32_t n) {
    const uint32_t p = blockIdx.x * 256u + threadIdx.x;
    if (p >= n) return;
    const uint32_t touched = n_touched[p];
    if (touched == 0) return;
    const float* src = inst_scores + prim_offset[p];
    float sum = 0.0f;
    for (uint32_t k = 0; k < touched; k++) sum += src[k];
    scores[p] += sum;
}

}  // namespace

bool launch_blend_forward(const BlendForwardArgs& a, hipStream_t s) {
    if (a.n_tiles == 0) return true;
    blend_forward_kernel<<<a.n_tiles, tile_pixels, 0, s>>>(a);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_pruning_scores(const BlendBackwardArgs& a, const uint32_t* n_touched, const uint32_t* prim_offset, float* scores, uint32_t n,
                           hipStream_t s) {
    if (a.n_tiles > 0) {
        blend_scores_kernel<<<a.n_tiles, tile_pixels, 0, s>>>(a);
        EFGS_HIP_CHECK(hipGetLastError());
    }
    if (n > 0) {
        accumulate_scores_kernel<<<div_up(n, 256), 256, 0, s>>>(n_touched, prim_offset, a.inst_grads, scores, n);
        EFGS_HIP_CHECK(hipGetLastError());
    }
    return true;
}

bool launch_blend_backward(const BlendBackwardArgs& a, hipStream_t s) {
    if (a.n_tiles == 0) return true;
    if (a.abs_grads)
        blend_backward_kernel<true, blend_backward_batch><<<a.n_tiles, tile_pixels, 0, s>>>(a);
    else
        blend_backward_kernel<false, blend_backward_batch><<<a.n_tiles, tile_pixels, 0, s>>>(a);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
