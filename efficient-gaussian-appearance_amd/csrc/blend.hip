// Alpha blending per 16x12 tile.
//
// Forward: one wave per tile, sixteen 4x3 pixel groups, three pixels per lane (lane l: group i = l & 15, column
// k = l >> 4 of the group, rows 3 (i >> 2) + 0..2; see blend_forward_kernel). Gaussians are staged in LDS 32 at a
// time into a ring of two chunks, culled against the sixteen group rectangles, and every group walks its own hits
// in order, one Gaussian per wave step (sixteen per wave instruction), running ahead into the next chunk while
// another group finishes the current one. A lane's three pixels share the Gaussian's LDS reads and its terms in dx.
// Front-to-back compositing, alpha = o exp2(min(q, 0)) with the conic pre-scaled by -log2(e)/2 and the hardware
// exp2 (v_exp_f32, as the reference's fast-math exp2f), alpha < 1/255 skipped, stop at T < 1e-4; stores the image,
// final T and last-contributor index per pixel and the per-tile maximum (an inference render stores only the
// image, in CHW or HWC layout, optionally clamped). No per-bucket checkpoints.
//
// Backward: one wave per tile, sixteen 4x3 pixel groups, three pixels per lane (see blend_backward_kernel). Every
// pixel replays its forward walk (the evaluation is shared and compiled with -ffp-contract=off, so T and every
// skip decision are reproduced bit-exactly; which pixels evaluate a Gaussian differs from the forward only where
// its alpha is below 1/255, outside its screen rectangle) and forms the reference's per-pixel terms; the
// per-Gaussian sums of each group are added in a fixed order into one 36-byte record per instance at its emission
// slot. No float atomics; the result is run-to-run deterministic.
//
// Reference: B/rasterization/include/kernels_forward.cuh:26-166, kernels_backward.cuh:12-231.
#include "internal.h"
#include "tile_sort.h"

namespace efgs {

namespace {

constexpr float log2e = 1.44269504089f;

typedef float native_float4 __attribute__((ext_vector_type(4)));
typedef float native_float3 __attribute__((ext_vector_type(3)));
typedef float native_float2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(3))) char lds_char;
typedef const __attribute__((address_space(3))) native_float4 lds_float4;
typedef const __attribute__((address_space(3))) native_float3 lds_float3;
typedef const __attribute__((address_space(3))) native_float2 lds_float2;

struct Staged {
    float2 xy;
    float4 co;  // exp2-scaled conic (x, y, z) and opacity
};

__device__ __forceinline__ float4 scale_conic_for_exp2(float cx, float cy, float cz, float opacity) {
    return make_float4(-0.5f * log2e * cx, -log2e * cy, -0.5f * log2e * cz, opacity);
}

// The exponent q = cx dx^2 + cy dx dy + cz dy^2 of an exp2-scaled conic at offset (dx, dy), grouped by dy:
// (cz dy + cy dx) dy + (cx dx) dx, two fused multiply-adds after the terms in dx alone, which the backward's three
// pixels of a column share (dx_terms); every blend evaluates it in this order, so the backward's replay reproduces
// the forward's alpha, T and decisions bit for bit.
struct DxTerms {
    float dx, ydx, xdxdx;  // dx, cy dx, (cx dx) dx
};
__device__ __forceinline__ DxTerms dx_terms(float4 xy, float4 co, float pxf) {
    const float dx = xy.x - pxf;
    return DxTerms{dx, co.y * dx, (co.x * dx) * dx};
}
// alpha at the pixel row pyf of a column's dx terms; G receives the Gaussian factor. v_exp_f32 (a quarter-rate
// instruction: 4 issue slots) replaces an 11-operation polynomial; its result is a fixed function of q. exp2(min(q,
// 0)) is taken as exp2(q) clamped to [0, 1] (equal for every q that is not NaN), which the exp instruction applies
// as its output modifier: one instruction fewer per pixel and Gaussian.
__device__ __forceinline__ float eval_alpha_row(const DxTerms& t, float4 xy, float4 co, float pyf, float& dy, float& G) {
    dy = xy.y - pyf;
    const float q = __builtin_fmaf(__builtin_fmaf(co.z, dy, t.ydx), dy, t.xdxdx);
    G = fminf(fmaxf(__builtin_amdgcn_exp2f(q), 0.0f), 1.0f);  // exp2(min(q, 0)): the clamp is the exp's output modifier
    return co.w * G;
}
__device__ __forceinline__ float eval_alpha(float4 xy, float4 co, float pxf, float pyf, float& dx, float& dy, float& G) {
    const DxTerms t = dx_terms(xy, co, pxf);
    dx = t.dx;
    return eval_alpha_row(t, xy, co, pyf, dy, G);
}

// transmittance after a fragment of opacity a: T (1 - a) with one rounding (one instruction, where T * (1 - a) took
// two; a = 0 leaves T bit for bit)
__device__ __forceinline__ float transmit(float T, float a) { return __builtin_fmaf(-T, a, T); }

__device__ __forceinline__ uint2 rect_of(float4 xy) { return make_uint2(__float_as_uint(xy.z), __float_as_uint(xy.w)); }

// the maximum over the wave, in every lane: four row rotations (DPP), then two lane swaps across the rows
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xf, 0xf, false)));  // row_ror:1
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xf, 0xf, false)));  // row_ror:2
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xf, 0xf, false)));  // row_ror:4
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false)));  // row_ror:8
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = max(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return max(b[0], b[1]);
}

// Writes each group's surviving Gaussians of the chunk, in order, to list[k * list_len + 0 .. n[k]) (entry:
// (base + lane) << shift for the Gaussian, a batch index or, shifted, a byte offset into 16-byte staged arrays);
// n[k] = popcount(m[k]). A group then walks its list with one LDS read per step instead of scanning a 64-bit
// mask per lane. hit[k] is the lane's own bit of m[k]: a lane mask as it stands, so the store's branch and the
// rank (the bits of m[k] below the lane) take no per-lane test of m[k].
template <uint32_t N>
__device__ __forceinline__ void build_group_lists(const uint64_t (&m)[N], const bool (&hit)[N], uint32_t lane, uint32_t base,
                                                  uint32_t* list, uint32_t list_len, uint32_t (&n)[N], uint32_t shift = 0) {
#pragma unroll
    for (uint32_t k = 0; k < N; k++) {
        const uint32_t lo = static_cast<uint32_t>(m[k]), hi = static_cast<uint32_t>(m[k] >> 32);
        if (hit[k]) list[k * list_len + __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u))] = (base + lane) << shift;
        n[k] = static_cast<uint32_t>(__popcll(m[k]));
    }
}

// The lanes (of those active) where a < b, as a lane mask: the compare's own result, which the compiler shares
// with a bool of the same compare (a ballot of the bool would turn it into a value and back: two instructions).
__device__ __forceinline__ uint64_t lanes_lt(uint32_t a, uint32_t b) { return __builtin_amdgcn_uicmp(a, b, 36); }  // unsigned <

// Culls lane's Gaussian (number idx of count) against the eight 4x2 groups of the 16x4 band whose pixel columns
// start at bx0 and rows at by0: hit[4h + g] is the lane's test for columns 4g .. 4g + 3, band rows 2h and 2h + 1,
// and m[4h + g] the wave's ballot of it.
__device__ __forceinline__ void cull_groups8(uint2 rect, uint32_t idx, uint32_t count, uint32_t bx0, uint32_t by0, uint64_t (&m)[8], bool (&hit)[8]) {
    const uint32_t rx0 = rect.x & 0xffffu, rx1 = rect.x >> 16, ry0 = rect.y & 0xffffu, ry1 = rect.y >> 16;
    const bool in = idx < count;
    const uint64_t in_m = lanes_lt(idx, count);
    bool xov[4];
    uint64_t xov_m[4];
#pragma unroll
    for (uint32_t g = 0; g < 4; g++) {
        const uint32_t gx0 = bx0 + 4u * g;
        xov[g] = rx0 < gx0 + 4u && gx0 < rx1;
        xov_m[g] = lanes_lt(rx0, gx0 + 4u) & lanes_lt(gx0, rx1);
    }
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        const uint32_t y0 = by0 + 2u * h;
        const bool yov = in && ry0 < y0 + 2u && y0 < ry1;
        const uint64_t yov_m = in_m & lanes_lt(ry0, y0 + 2u) & lanes_lt(y0, ry1);
#pragma unroll
        for (uint32_t g = 0; g < 4; g++) {
            hit[4 * h + g] = yov && xov[g];
            m[4 * h + g] = yov_m & xov_m[g];
        }
    }
}


// Sums of several per-lane values over the four 16-lane rows (and, in the 4x4 groups of the score kernel, over
// a row quad) at once ("transposing" reductions). Each exchange step swaps half of the values between lanes so
// that every lane keeps fewer values, each summed over more lanes:
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

// raw conic (x, y, z) of an exp2-scaled one (scale_conic_for_exp2 inverted)
__device__ __forceinline__ float4 raw_conic_of(float4 co) {
    constexpr float ln2 = 0.69314718055994531f;
    return make_float4(-2.0f * ln2 * co.x, -ln2 * co.y, -2.0f * ln2 * co.z, 0.0f);
}

// Four values summed over the four lane rows (lanes l, l + 16, l + 32, l + 48): row k of the result holds the
// sum of value {0, 2, 1, 3}[k].
__device__ __forceinline__ float rows_reduce4(float v0, float v1, float v2, float v3) {
    return swap16_add(swap32_add(v0, v1), swap32_add(v2, v3));
}

// The maximum over the lane's 16-lane row, in every lane of it (four row rotations).
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xf, 0xf, false)));  // row_ror:1
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xf, 0xf, false)));  // row_ror:2
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xf, 0xf, false)));  // row_ror:4
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false)));  // row_ror:8
    return v;
}

// Two values summed over the four lane rows: rows 0 and 1 of the result hold the sum of a, rows 2 and 3 that of b
// (each sum in the order of rows_reduce1).
__device__ __forceinline__ float rows_reduce2(float a, float b) {
    const float w = swap32_add(a, b);
    return swap16_add(w, w);
}

// The sum of one value over the four lane rows, in every row.
__device__ __forceinline__ float rows_reduce1(float v) {
    const float w = swap32_add(v, v);
    return swap16_add(w, w);
}

// Backward, one wave per tile. Lane l serves column k = l >> 4 of pixel group i = l & 15, a 4x3 block of the tile
// (columns 4 (i & 3) + 0..3, rows 3 (i >> 2) + 0..2), and that column's three pixels. Every pixel replays its forward
// walk (alpha bit-identical, the decisions are the forward's) and forms, branch-free (zero where it skips the
// Gaussian), h = -alpha dL/dalpha with dL/dalpha = T (c . g) - (A - g_bg) / max(1 - alpha, eps), A = (colour still
// to come) . g, and the Gaussian's group sums
//   h dx, h dy, h dx^2, h dx dy, h dy^2, h, w g_r, w g_g, w g_b   (w = T alpha; with ABS also |dL/dmean2d|)
// from which the instance's record is dL/dmean2d = (C h d summed), dL/dconic = 0.5 (h d d^T summed),
// dL/dopacity-term = sum G dL/dalpha = -(sum h) / o, dL/dcolour = sum w g. A lane's three pixels share dx, so it
// accumulates h, h dy, h dy^2 and the colour terms over its rows and forms the dx terms once; the group's four
// columns are then summed with two permlane swaps per four values (a lane row ends holding one of every four
// sums), no selects: the three pixels per lane amortise the cross-lane work that a pixel per lane paid alone.
//
// Gaussians are staged 32 at a time (a chunk). Each of a group's four lanes tests a quarter of the chunk against
// the group's rectangle, and two lane swaps give every lane of the group the group's 32-bit hit mask. The chunk
// is then walked in sub-batches: a sub-batch ends before the first Gaussian that would give some group more than
// LIST hits (or at the chunk's end), so each takes at most LIST wave steps while covering as many Gaussians as
// the busiest group allows. A group walks its hits in the sub-batch in Gaussian order, one per step (the next
// one is the mask's lowest set bit; past its hits it walks a staged Gaussian of opacity 0), sixteen different
// Gaussians per wave instruction, and stores step s's sums at position s of its slot row of each value. The
// combine then gives two lanes to each Gaussian of the sub-batch; they add the sixteen groups' slots in group
// order (a per-group byte table holds the Gaussian's position in the group's walk, or an always-zero slot when
// the group did not walk it) and write the 36-byte record at the instance's emission slot. A single wave needs
// no block barrier: LDS accesses of a wave complete in order, and a wavefront fence keeps the compiler from
// reordering them around the table and slot exchanges. No atomics: the result is run-to-run deterministic.
// LIST trades walk steps against LDS (the records take (8 + extra) x 16 x LIST floats; at most 10 KB per wave
// keeps four waves per SIMD: LIST 14, or 11 with the three extra values of ABS). Against fixed batches of 12
// Gaussians per walk (each group's list padded to the batch's longest), sub-batches of LIST 14 take 17 % fewer
// wave steps and 44 % as many combines on the 1M-Gaussian 1080p scene; LIST 12 / 13 / 14 measured 148.6 / 146.4 /
// 145.2 us there (fixed batches: 176 us).
#ifndef EFGS_BACKWARD_LIST
#define EFGS_BACKWARD_LIST 14
#endif
#ifndef EFGS_BACKWARD_WAVES
#define EFGS_BACKWARD_WAVES 4
#endif
constexpr uint32_t backward_list = EFGS_BACKWARD_LIST;
constexpr uint32_t backward_list_abs = EFGS_BACKWARD_LIST < 11 ? EFGS_BACKWARD_LIST : 11;
constexpr uint32_t backward_groups = 16;
constexpr uint32_t backward_chunk = 32;

// Instance gradient records: dL/dmean2d (x, y), dL/dconic (x, y, z), dL/dopacity, dL/dcolour (r, g, b), then with the
// absolute-gradient variant |dL/dmean2d| (x, y) and a pad: 9 floats (36 bytes), or 12. A record starts at a 4-byte
// aligned address, which its 16-byte stores need (dword-aligned vector accesses to global memory).
struct __attribute__((aligned(4))) Float4A4 {
    float x, y, z, w;
};
__device__ __forceinline__ void store_record4(float* p, float4 v) { *reinterpret_cast<Float4A4*>(p) = Float4A4{v.x, v.y, v.z, v.w}; }

// The bitwise OR of one value over the four lane rows, in every row.
__device__ __forceinline__ uint32_t rows_or(uint32_t v) {
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = a[0] | a[1];
    const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return b[0] | b[1];
}

// The minimum over the lane's 16-lane row, in every lane of it (four row rotations).
__device__ __forceinline__ uint32_t row_min_u32(uint32_t v) {
    v = min(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xf, 0xf, false)));  // row_ror:1
    v = min(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xf, 0xf, false)));  // row_ror:2
    v = min(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xf, 0xf, false)));  // row_ror:4
    v = min(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false)));  // row_ror:8
    return v;
}

// Forward, one wave per tile, with the backward's lanes and pixel groups: lane l serves column k = l >> 4 of the
// 4x3 group i = l & 15 and that column's three pixels. The walk runs over a window of two staged 32-Gaussian
// chunks (a ring of 64 LDS entries, chunk c in half c & 1): a group's hits in the window (Gaussians whose screen
// rectangle overlaps its 4x3 pixels) form a 64-bit mask held by its four lanes, chunk c in the low word. Each wave
// step every group walks its next hit (sixteen Gaussians per wave instruction), and a group that has finished
// chunk c goes on into c + 1 while the others are still in c; after as many steps as the busiest group had hits
// left in c, chunk c + 2 is staged into c's half and culled. A step lasts as long as its busiest group, so groups
// wait for each other only where one would run a whole chunk ahead (435k wave steps on the 1M-Gaussian 1080p scene,
// against 536k with the chunks in lockstep and 434k for sixteen unsynchronised walks). A group past its hits walks
// ring entry RING, a Gaussian of opacity 0. A lane's three pixels share the Gaussian's LDS reads and its terms in dx.
// The wave stops at a chunk boundary once every pixel is done. (Against the three waves of eight 4x2 groups, one
// pixel per lane, that this replaced: 14 % fewer VALU instructions and a third of the LDS reads per pixel, at the
// same time, 70.6 against 70.5 us on the 1M-Gaussian 1080p scene: both waited on the gather chain emission index
// -> primitive -> record; with the primitives read from the sorted array it takes 57 us.)
template <typename KeyT>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(7))) void blend_forward_kernel(BlendForwardArgs a) {
    if (a.overflow && *a.overflow != 0) return;  // the binning was skipped: the host re-runs the frame
    constexpr uint32_t CHUNK = 32;
    constexpr uint32_t RING = 2 * CHUNK;
    // The sort's slab (wave_slab keys), which the stage reuses for the walk: ring entry r (x, y, packed pixel
    // rectangle), exp2-scaled conic + opacity, colour; entry RING: opacity 0.
    __shared__ __align__(16) uint64_t s_slab[wave_slab];
    float4 (*const s_stage)[3] = reinterpret_cast<float4 (*)[3]>(s_slab);
    static_assert(sizeof(s_slab) >= (RING + 1) * 3 * sizeof(float4), "the stage fits the slab");
    __shared__ uint32_t s_sorted_prim[forward_sort_max];  // a register-sorted run's primitives in sorted order

    const uint32_t lane = threadIdx.x;
    const uint32_t tile = a.order ? a.order[blockIdx.x] : blockIdx.x;  // heaviest tiles first
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t i = lane & 15u, k = lane >> 4;
    const uint32_t lx = 4u * (i & 3u) + k, ly0 = 3u * (i >> 2);        // tile-local column, first row
    const uint32_t bx0 = tx * tile_width, by0 = ty * tile_height;
    const uint32_t px = bx0 + lx;
    const float pxf = static_cast<float>(px) + 0.5f;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;
    // The tile's run is sorted here: the emission indices, primitives and tile keys in (depth, primitive) order for
    // the backward; a run that fits the register networks also leaves its primitives in LDS for the walk, a longer
    // one (LDS slab, chunks) is read back from the sorted array.
    const bool in_regs = n_total <= forward_sort_max;  // (wave-uniform)
    if (n_total > 0) {
        if (in_regs) {
            const SortedOut<KeyT> o{a.sorted_inst + range.x, a.sorted_prim + range.x, static_cast<KeyT*>(a.sorted_keys) + range.x,
                                    a.inst_prim, tile, s_sorted_prim};
            const bool packed = a.counters[1] < (1u << 24) - 1u;  // every emission index fits 24 bits (and no key packs to all ones)
            sort_small_run(a.bucket + range.x, n_total, o, lane, packed, s_slab);
        } else {
            sort_big_run(a.bucket, range, n_total, tile, a.sorted_inst, static_cast<KeyT*>(a.sorted_keys), a.inst_prim, a.sorted_prim, lane,
                         s_slab);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");  // the wave reads back the primitives its lanes wrote
        }
        wave_lds_fence();
    }
    if (lane < 3) s_stage[RING][lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    // A pixel is done (takes no further Gaussian) exactly when T < transmittance_threshold: T changes only when a
    // Gaussian is taken and starts at 1; pixels outside the image start at 0, done from the start.
    float pyf[3], T[3], cr[3], cg[3], cb[3];
    uint32_t last[3];  // 1-based index in the tile's list of the pixel's last Gaussian taken (0: none)
    bool inside[3];
#pragma unroll
    for (uint32_t r = 0; r < 3; r++) {
        const uint32_t py = by0 + ly0 + r;
        pyf[r] = static_cast<float>(py) + 0.5f;
        inside[r] = px < a.width && py < a.height;
        T[r] = inside[r] ? 1.0f : 0.0f;
        cr[r] = cg[r] = cb[r] = 0.0f;
        last[r] = 0u;
    }

    // The records of a chunk's instances are gathered through a two-stage pipeline over the chunks: while chunk c
    // is walked, the primitive indices of chunk c + 3 (from LDS, or the sorted array: coalesced) and the records of
    // chunk c + 2 are loaded (indices clamped to the tile's last instance; lanes past CHUNK repeat lane CHUNK - 1).
    const uint32_t gather_lane = min(lane, CHUNK - 1u);
    const uint32_t last_inst = n_total > 0 ? n_total - 1u : 0u;
    const uint32_t* const prim_src = in_regs ? s_sorted_prim : a.sorted_prim + range.x;
    const auto load_p = [&](uint32_t s) { return prim_src[min(s + gather_lane, last_inst)]; };
    const auto stage = [&](uint32_t half, uint32_t s, const PrimRecord& rec) {
        if (lane < CHUNK && s + lane < n_total) {
            float4* const d = s_stage[half * CHUNK + lane];
            d[0] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            d[1] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            d[2] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
        }
    };
    // the group's hits among the first n Gaussians of the chunk in ring half `half` (bit j: Gaussian j overlaps the
    // group's rectangle): lane row k tests Gaussians 8k .. 8k + 7, and the mask then sits in all four lanes
    const uint32_t gx0 = bx0 + 4u * (i & 3u), gy0 = by0 + ly0;
    const auto cull = [&](uint32_t half, uint32_t n) {
        constexpr uint32_t Q = CHUNK / 4;
        uint32_t hits = 0;
        uint2 rects[Q];
#pragma unroll
        for (uint32_t t = 0; t < Q; t++) rects[t] = rect_of(s_stage[half * CHUNK + k * Q + t][0]);  // (all reads in flight at once)
#pragma unroll
        for (uint32_t t = 0; t < Q; t++) {
            const uint2 rect = rects[t];
            const uint32_t rx0 = rect.x & 0xffffu, rx1 = rect.x >> 16, ry0 = rect.y & 0xffffu, ry1 = rect.y >> 16;
            const bool hit = (rx0 < gx0 + 4u) & (gx0 < rx1) & (ry0 < gy0 + 3u) & (gy0 < ry1);
            hits |= hit ? 1u << t : 0u;
        }
        // (entries past the chunk's count hold stale rectangles: masked off)
        const uint32_t n_own = n > Q * k ? min(n - Q * k, Q) : 0u;
        return rows_or((hits & ((1u << n_own) - 1u)) << (Q * k));
    };

    uint64_t M = 0;        // the group's unwalked hits: chunk c in bits 0..31, chunk c + 1 in bits 32..63
    uint32_t p_next = 0;   // primitive indices of chunk c + 2
    if (n_total > 0) {
        const uint32_t p0 = load_p(0), p1 = load_p(CHUNK);
        p_next = load_p(2 * CHUNK);
        const PrimRecord rec0 = a.records[p0], rec1 = a.records[p1];
        stage(0, 0, rec0);
        stage(1, CHUNK, rec1);
        wave_lds_fence();
        const uint32_t m0 = cull(0, min(CHUNK, n_total));
        const uint32_t m1 = cull(1, n_total > CHUNK ? min(CHUNK, n_total - CHUNK) : 0u);
        M = (static_cast<uint64_t>(m1) << 32) | m0;
    }
    for (uint32_t c = 0, base = 0; base < n_total; c++, base += CHUNK) {
        // every pixel of the tile done: the rest of the list changes nothing
        if (__builtin_amdgcn_ballot_w64(T[0] >= transmittance_threshold || T[1] >= transmittance_threshold ||
                                        T[2] >= transmittance_threshold) == 0)
            break;
        const uint32_t half = c & 1u, flip = half * CHUNK;  // (wave-uniform) ring index of window position j: j ^ flip
        const PrimRecord rec_n = a.records[p_next];          // chunk c + 2
        p_next = load_p(base + 3 * CHUNK);                   // chunk c + 3
        // the busiest group's hits left in chunk c (rows hold the same masks)
        const uint32_t n_steps = __builtin_amdgcn_readfirstlane(row_max_u32(static_cast<uint32_t>(__popc(static_cast<uint32_t>(M)))));
        const auto peek = [&]() {  // the lowest unwalked hit's window position (all ones: none)
            uint32_t lo, hi;
            asm("v_ffbl_b32 %0, %1" : "=v"(lo) : "v"(static_cast<uint32_t>(M)));
            asm("v_ffbl_b32 %0, %1" : "=v"(hi) : "v"(static_cast<uint32_t>(M >> 32)));
            return min(lo, hi | CHUNK);
        };
        const auto ring = [&](uint32_t j) { return min(j ^ flip, RING); };
        // staged float4 c4 of ring entry r, read only as far as the walk uses it (LDS address space, 32-bit offsets)
        const auto at = [&](uint32_t r, uint32_t c4) {
            lds_char* const p = (lds_char*)(&s_stage[0][0]) + __umul24(r, static_cast<uint32_t>(sizeof(s_stage[0]))) + 16u * c4;
            if (c4 == 0) {
                const native_float2 v = *reinterpret_cast<lds_float2*>(p);
                return make_float4(v.x, v.y, 0.0f, 0.0f);
            }
            if (c4 == 2) {
                const native_float3 v = *reinterpret_cast<lds_float3*>(p);
                return make_float4(v.x, v.y, v.z, 0.0f);
            }
            const native_float4 v = *reinterpret_cast<lds_float4*>(p);
            return make_float4(v.x, v.y, v.z, v.w);
        };
        // branch-free: a skipped Gaussian gets weight 0, which leaves C and T bit for bit unchanged
        const auto walk = [&](uint32_t j, float4 xy, float4 co, float4 col) {
            const DxTerms xt = dx_terms(xy, co, pxf);  // (the lane's three pixels share their column)
            const uint32_t pos = base + j + 1u;
#pragma unroll
            for (uint32_t r = 0; r < 3; r++) {
                float dy, G;
                const float alpha = eval_alpha_row(xt, xy, co, pyf[r], dy, G);
                const bool take = T[r] >= transmittance_threshold && alpha >= min_alpha;
                const float a_t = take ? alpha : 0.0f;
                const float w = T[r] * a_t;
                cr[r] = __builtin_fmaf(w, col.x, cr[r]);
                cg[r] = __builtin_fmaf(w, col.y, cg[r]);
                cb[r] = __builtin_fmaf(w, col.z, cb[r]);
                T[r] = transmit(T[r], a_t);
                last[r] = take ? pos : last[r];
            }
        };
        // the next step's Gaussian is read from LDS before the current one is evaluated (two register sets, the
        // loop unrolled by two); a hit leaves M when its step starts, so M keeps every hit not yet walked
        if (n_steps > 0) {
            uint32_t ja = peek(), ra = ring(ja);
            float4 xya = at(ra, 0), coa = at(ra, 1), cola = at(ra, 2);
            for (uint32_t s = 0; s < n_steps; s += 2) {
                M &= M - 1u;
                const uint32_t jb = peek(), rb = ring(jb);
                const float4 xyb = at(rb, 0), cob = at(rb, 1), colb = at(rb, 2);
                walk(ja, xya, coa, cola);
                if (s + 1 >= n_steps) break;
                M &= M - 1u;
                ja = peek();
                ra = ring(ja);
                xya = at(ra, 0);
                coa = at(ra, 1);
                cola = at(ra, 2);
                walk(jb, xyb, cob, colb);
            }
        }
        wave_lds_fence();  // the walk has read chunk c's entries
        // chunk c + 2 into chunk c's half; the window moves on by a chunk
        const uint32_t nb = base + 2 * CHUNK;
        uint32_t m2 = 0;
        if (nb < n_total) {
            stage(half, nb, rec_n);
            wave_lds_fence();
            m2 = cull(half, min(CHUNK, n_total - nb));
        }
        M = (M >> 32) | (static_cast<uint64_t>(m2) << 32);
    }

    const uint32_t np = a.width * a.height;
#pragma unroll
    for (uint32_t r = 0; r < 3; r++) {
        if (!inside[r]) continue;
        const uint32_t pix = (by0 + ly0 + r) * a.width + px;
        float c[3] = {__builtin_fmaf(T[r], a.bg[0], cr[r]), __builtin_fmaf(T[r], a.bg[1], cg[r]), __builtin_fmaf(T[r], a.bg[2], cb[r])};
        if (a.clamp) {
#pragma unroll
            for (int q = 0; q < 3; q++) c[q] = fminf(fmaxf(c[q], 0.0f), 1.0f);
        }
        if (a.hwc) {
#pragma unroll
            for (int q = 0; q < 3; q++) a.image[3 * pix + q] = c[q];
        } else {
#pragma unroll
            for (int q = 0; q < 3; q++) a.image[q * np + pix] = c[q];
        }
    }
    if (!a.final_T) return;  // inference render: no backward state (uniform over the wave)
#pragma unroll
    for (uint32_t r = 0; r < 3; r++) {
        const uint32_t pslot = tile * tile_pixels + (ly0 + r) * tile_width + lx;
        a.final_T[pslot] = T[r];
        a.n_contrib[pslot] = last[r];
    }
    const uint32_t wm = wave_max_u32(max(max(last[0], last[1]), last[2]));
    if (lane == 0) a.tile_max[tile] = wm;
}

template <bool ABS, uint32_t LIST>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(EFGS_BACKWARD_WAVES))) void blend_backward_kernel(BlendBackwardArgs a) {
    constexpr uint32_t CHUNK = backward_chunk;
    constexpr uint32_t NX = ABS ? 3u : 1u;                 // values after the first eight (w g_b; |dL/dmean2d|)
    constexpr uint32_t n_values = NX + 8u;
    // One record of VS floats (values 0..7, then the extras) per group and walk step: group g's step s at record
    // g LIST + s, then one record never written (zero_rec, zeros) and padding that the second combine lane's
    // reads of the extras' offsets reach past it. VS is odd: a wave step's 64 stores (four values of sixteen
    // records) and a combine read (sixteen steps of one group, two values four apart) hit distinct banks.
    constexpr uint32_t VS = n_values;
    constexpr uint32_t RECORD = ABS ? record_floats_abs : record_floats;  // floats per instance gradient record
    constexpr uint32_t zero_rec = backward_groups * LIST;
    static_assert(LIST >= 1 && zero_rec < 256u && (VS & 1u), "record indices fit a byte");
    // (x, y, packed rect), exp2-scaled conic + opacity, colour + the instance's emission index (bits): Gaussian j
    // of the chunk at entry j + 1, entry 0 a Gaussian of opacity 0 that a group walks past its hits
    __shared__ float4 s_stage[CHUNK + 1][3];
    __shared__ __align__(8) uint8_t s_pos[backward_groups][CHUNK];  // per group and Gaussian: its record (g LIST + step) or zero_rec
    __shared__ float s_part[(zero_rec + 1) * VS + 4];

    const uint32_t lane = threadIdx.x;
    const uint32_t tile = a.order ? a.order[blockIdx.x] : blockIdx.x;  // heaviest tiles first
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t i = lane & 15u, k = lane >> 4;
    const uint32_t lx = 4u * (i & 3u) + k, ly0 = 3u * (i >> 2);        // tile-local column, first row
    const uint32_t bx0 = tx * tile_width, by0 = ty * tile_height;
    const uint32_t px = bx0 + lx;
    const float pxf = static_cast<float>(px) + 0.5f;
    const uint2 range = a.ranges[tile];
    const uint32_t n_total = range.y - range.x;
    const uint32_t n_proc = min(n_total, a.tile_max[tile]);
    if (lane < VS) s_part[zero_rec * VS + lane] = 0.0f;
    if (lane < 3) s_stage[0][lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    // pixel state of the lane's three rows: upstream gradient and Ab = (colour still to come) . g - g_bg, the
    // background term g_bg = -T_final (bg . g) folded in. The loads are unconditional (clamped to the image) so
    // that all of them are in flight together.
    float pyf[3], T[3], Ab[3], gr[3], gg[3], gb[3];
    uint32_t last[3];
    {
        const uint32_t np = a.width * a.height;
        const uint32_t pxc = min(px, a.width - 1u);
        float Tf[3], im[3][3];
        uint32_t nc[3];
        bool inside[3];
#pragma unroll
        for (uint32_t r = 0; r < 3; r++) {
            const uint32_t py = by0 + ly0 + r;
            pyf[r] = static_cast<float>(py) + 0.5f;
            inside[r] = px < a.width && py < a.height;
            const uint32_t pix = min(py, a.height - 1u) * a.width + pxc;
            const uint32_t pslot = tile * tile_pixels + (ly0 + r) * tile_width + lx;
            Tf[r] = a.final_T[pslot];
            nc[r] = a.n_contrib[pslot];
            gr[r] = a.grad_image[pix]; gg[r] = a.grad_image[np + pix]; gb[r] = a.grad_image[2 * np + pix];
            im[r][0] = a.image[pix]; im[r][1] = a.image[np + pix]; im[r][2] = a.image[2 * np + pix];
        }
        const float bg0 = a.bg[0], bg1 = a.bg[1], bg2 = a.bg[2];
#pragma unroll
        for (uint32_t r = 0; r < 3; r++) {
            T[r] = 1.0f;
            last[r] = inside[r] ? nc[r] : 0u;
            gr[r] = inside[r] ? gr[r] : 0.0f;
            gg[r] = inside[r] ? gg[r] : 0.0f;
            gb[r] = inside[r] ? gb[r] : 0.0f;
            const float ar = im[r][0] - Tf[r] * bg0;
            const float ag = im[r][1] - Tf[r] * bg1;
            const float ab = im[r][2] - Tf[r] * bg2;
            const float A = __builtin_fmaf(ab, gb[r], __builtin_fmaf(ag, gg[r], ar * gr[r]));
            const float gbg = Tf[r] * -(gr[r] * bg0 + gg[r] * bg1 + gb[r] * bg2);
            Ab[r] = inside[r] ? A - gbg : 0.0f;
        }
    }

    // where the lane stores its sums: value 4m + {0, 2, 1, 3}[k] of group i (m = 0, 1; the extras: 8 + the same),
    // in the record of the walk step
    const uint32_t vk = (k & 1u) * 2u + (k >> 1);
    float* const slot0 = s_part + i * LIST * VS + vk;
    // the combine's lanes: Gaussian cj of the chunk, half ch (values 0..3 and the extras; values 4..7)
    const uint32_t cj = lane & (CHUNK - 1u), ch = lane / CHUNK;
    const uint32_t below8k = (1u << (8u * k)) - 1u;  // the chunk's Gaussians before the lane's eight

    // The records of a chunk's instances are gathered through a two-stage pipeline over the chunks: while chunk b
    // is walked, the primitive indices of chunk b + 2 (the sorted array: coalesced) and the records and emission
    // indices of chunk b + 1 are loaded, so no load is waited on in the chunk that issues it. The loads are
    // unconditional (indices clamped to the tile's last instance; lanes past CHUNK repeat lane CHUNK - 1), so the
    // compiler places each wait at the value's use.
    const uint32_t gather_lane = min(lane, CHUNK - 1u);
    const uint32_t last_inst = n_total > 0 ? n_total - 1u : 0u;
    const auto load_e = [&](uint32_t s) { return a.sorted_inst[range.x + min(s + gather_lane, last_inst)]; };
    const auto load_p = [&](uint32_t s) { return a.sorted_prim[range.x + min(s + gather_lane, last_inst)]; };
    const auto stage = [&](uint32_t s, const PrimRecord& rec, uint32_t e) {
        if (lane < CHUNK && s + lane < n_total) {
            s_stage[lane + 1][0] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            s_stage[lane + 1][1] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_stage[lane + 1][2] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, __uint_as_float(e));
        }
    };
    // The loads of a chunk's top have their consumers a whole chunk later (the staging at the end of the chunk,
    // the next chunk's top), and no loaded value is copied between loop-carried registers (a copy would make the
    // loop wait for the load).
    uint32_t p_next = 0;  // primitive indices of chunk b + 1
    if (n_proc > 0) {
        const uint32_t e0 = load_e(0), p0 = load_p(0);
        p_next = load_p(CHUNK);
        const PrimRecord rec0 = a.records[p0];
        stage(0, rec0, e0);
    }
    const uint32_t gx0 = bx0 + 4u * (i & 3u), gy0 = by0 + ly0;  // the lane's group rectangle: 4 x 3 pixels
    for (uint32_t base = 0; base < n_proc; base += CHUNK) {
        // advance the gather pipeline: records and emission indices of chunk b + 1, primitive indices of b + 2
        const PrimRecord rec_n = a.records[p_next];
        const uint32_t e_n = load_e(base + CHUNK);
        p_next = load_p(base + 2 * CHUNK);
        wave_lds_fence();  // the chunk is staged
        const uint32_t n_chunk = min(CHUNK, n_proc - base);
        uint32_t last_rel[3];
#pragma unroll
        for (uint32_t r = 0; r < 3; r++) last_rel[r] = last[r] > base ? last[r] - base : 0u;

        // cull: lane row k tests Gaussians 8k .. 8k + 7 against the group's rectangle; the group's mask (bit j:
        // Gaussian j overlaps the group) then sits in all four of its lanes
        uint32_t R;
        {
            constexpr uint32_t Q = CHUNK / 4;
            uint32_t hits = 0;
            uint2 rects[Q];
#pragma unroll
            for (uint32_t t = 0; t < Q; t++) rects[t] = rect_of(s_stage[k * Q + t + 1][0]);  // (all reads in flight at once)
#pragma unroll
            for (uint32_t t = 0; t < Q; t++) {
                const uint2 rect = rects[t];
                const uint32_t rx0 = rect.x & 0xffffu, rx1 = rect.x >> 16, ry0 = rect.y & 0xffffu, ry1 = rect.y >> 16;
                const bool hit = (rx0 < gx0 + 4u) & (gx0 < rx1) & (ry0 < gy0 + 3u) & (gy0 < ry1);
                hits |= hit ? 1u << t : 0u;
            }
            // (Gaussians past the chunk's count hold stale rectangles: masked off)
            const uint32_t n_own = n_chunk > Q * k ? min(n_chunk - Q * k, Q) : 0u;
            R = rows_or((hits & ((1u << n_own) - 1u)) << (Q * k));
        }

        for (uint32_t pos0 = 0;;) {
            // the sub-batch: Gaussians pos0 .. cut - 1, cut the position of the first Gaussian that would be some
            // group's (LIST + 1)-th hit (the chunk's end if there is none); every group then has at most LIST hits
            const uint32_t tot = static_cast<uint32_t>(__popc(R));
            const bool over = __ballot(tot > LIST) != 0;  // (wave-uniform)
            uint32_t cut = CHUNK, n_steps = LIST;
            if (over) {
                uint32_t m = R;
#pragma unroll
                for (uint32_t n = 0; n < LIST; n++) m &= m - 1u;  // the group's hits after its first LIST
                const uint32_t cand = tot > LIST ? static_cast<uint32_t>(__ffs(m) - 1) : CHUNK;
                cut = __builtin_amdgcn_readfirstlane(row_min_u32(cand));  // rows hold the same values
            } else {
                n_steps = __builtin_amdgcn_readfirstlane(row_max_u32(tot));
            }
            const uint32_t sel = cut < 32u ? R & ((1u << cut) - 1u) : R;
            R ^= sel;
            // the combine's table: for this lane's eight Gaussians, the record the group stores them in, or zero_rec.
            // Per four Gaussians: their bits spread to bytes (b0 + b1 2^8 + ...: one 24-bit product), the bits
            // below each byte (another product, shifted by a byte), plus the first record in every byte, and a
            // byte select against zero_rec.
            {
                constexpr uint32_t Q = CHUNK / 4;
                const uint32_t own = (sel >> (Q * k)) & 0xffu;
                const uint32_t r0 = static_cast<uint32_t>(__popc(sel & below8k)) + i * LIST;  // the first hit's record
                const uint32_t lo = own & 15u, hi = own >> 4;
                const uint32_t bl = __umul24(lo, 0x00204081u) & 0x01010101u, bh = __umul24(hi, 0x00204081u) & 0x01010101u;
                const uint32_t rl = (__umul24(bl, 0x010101u) << 8) + __builtin_amdgcn_perm(0u, r0, 0u);
                const uint32_t rh = (__umul24(bh, 0x010101u) << 8) + __builtin_amdgcn_perm(0u, r0 + static_cast<uint32_t>(__popc(lo)), 0u);
                const uint32_t ml = (bl << 8) - bl, mh = (bh << 8) - bh;  // 0xff in the bytes of hits
                constexpr uint32_t zb = zero_rec * 0x01010101u;
                *reinterpret_cast<uint2*>(&s_pos[i][Q * k]) = make_uint2((rl & ml) | (zb & ~ml), (rh & mh) | (zb & ~mh));
            }
            wave_lds_fence();

            // step s walks the group's s-th hit (after the last: j = all ones, staged entry 0, which also fails every
            // j < last test); the next step's Gaussian is read from LDS before the current one is evaluated (two
            // register sets, the loop unrolled by two)
            uint32_t M = sel;
            const auto next = [&]() {
                uint32_t j;
                asm("v_ffbl_b32 %0, %1" : "=v"(j) : "v"(M));  // lowest set bit, all ones for 0 (no select around it)
                M &= M - 1u;
                return j;
            };
            // the staged float4 c of Gaussian j, addressed in the LDS address space (32-bit offsets, one signed 24-bit
            // multiply-add: j = all ones is -1 in 24 bits, entry 0), read only as far as the walk uses it: (x, y), the
            // conic and opacity, the colour. (An unused component read along would be a register the compiler reuses
            // at once, waiting for the read to land.)
            const auto at = [&](uint32_t j, uint32_t c) {
                lds_char* const p = (lds_char*)(&s_stage[1][0]) + __mul24(static_cast<int>(j), static_cast<int>(sizeof(s_stage[0]))) + 16u * c;
                if (c == 0) {
                    const native_float2 v = *reinterpret_cast<lds_float2*>(p);
                    return make_float4(v.x, v.y, 0.0f, 0.0f);
                }
                if (c == 2) {
                    const native_float3 v = *reinterpret_cast<lds_float3*>(p);
                    return make_float4(v.x, v.y, v.z, 0.0f);
                }
                const native_float4 v = *reinterpret_cast<lds_float4*>(p);
                return make_float4(v.x, v.y, v.z, v.w);
            };
            // (without ABS the step's w g_b sum is returned in swb and reduced with the next step's)
            const auto walk = [&](uint32_t j, uint32_t s, float4 xy, float4 co, float4 col, float& swb) {
                float sh, shdy, shdyy, swr, swg, e1 = 0.0f, e2 = 0.0f;
                const float4 craw = ABS ? raw_conic_of(co) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                const DxTerms xt = dx_terms(xy, co, pxf);  // (the lane's three pixels share their column)
                const float dx = xt.dx;
#pragma unroll
                for (uint32_t r = 0; r < 3; r++) {
                    float dy, G;
                    const float alpha = eval_alpha_row(xt, xy, co, pyf[r], dy, G);
                    const bool contrib = j < last_rel[r] && alpha >= min_alpha;
                    const float ae = contrib ? alpha : 0.0f;
                    const float w = T[r] * ae;
                    const float oma = 1.0f - ae;
                    const float rcp = __builtin_amdgcn_rcpf(fmaxf(oma, one_minus_alpha_eps));
                    const float cg = __builtin_fmaf(col.z, gb[r], __builtin_fmaf(col.y, gg[r], col.x * gr[r]));
                    Ab[r] = __builtin_fmaf(-w, cg, Ab[r]);
                    const float dalpha = __builtin_fmaf(T[r], cg, -rcp * Ab[r]);
                    const float h = -ae * dalpha;
                    const float hdy = h * dy;
                    if (r == 0) {
                        sh = h;
                        shdy = hdy;
                        shdyy = hdy * dy;
                        swr = w * gr[r];
                        swg = w * gg[r];
                        swb = w * gb[r];
                    } else {
                        sh += h;
                        shdy += hdy;
                        shdyy = __builtin_fmaf(hdy, dy, shdyy);
                        swr = __builtin_fmaf(w, gr[r], swr);
                        swg = __builtin_fmaf(w, gg[r], swg);
                        swb = __builtin_fmaf(w, gb[r], swb);
                    }
                    if (ABS) {  // |dL/dmean2d| of the pixel: the raw conic times h d
                        const float hdx = h * dx;
                        e1 += fabsf(__builtin_fmaf(craw.x, hdx, craw.y * hdy));
                        e2 += fabsf(__builtin_fmaf(craw.y, hdx, craw.z * hdy));
                    }
                    T[r] = transmit(T[r], ae);
                }
                const float shdx = dx * sh;
                float* const sw = slot0 + s * VS;
                sw[0] = rows_reduce4(shdx, shdy, dx * shdx, dx * shdy);           // h dx, h dy, h dx^2, h dx dy
                sw[4] = rows_reduce4(shdyy, sh, swr, swg);                         // h dy^2, h, w g_r, w g_g
                if (ABS) {
                    const float x2 = rows_reduce4(swb, e1, e2, 0.0f);              // w g_b, |.|_x, |.|_y
                    if (vk < 3u) sw[8] = x2;
                }
            };
            {
                // w g_b of a pair of steps in one reduction: rows 0 and 2 store the first and the second step's sum
                // (row 2's lanes have vk = 1: their value-8 slot of the next record is VS + 7 floats on)
                float* const b8 = slot0 + (k == 2u ? VS + 7u : 8u);
                const bool store8 = (k & 1u) == 0u;
                uint32_t ja = next();
                float4 xya = at(ja, 0), coa = at(ja, 1), cola = at(ja, 2);
                for (uint32_t s = 0; s < n_steps; s += 2) {
                    const uint32_t jb = next();
                    const float4 xyb = at(jb, 0), cob = at(jb, 1), colb = at(jb, 2);
                    float swb_a, swb_b;
                    walk(ja, s, xya, coa, cola, swb_a);
                    if (s + 1 >= n_steps) {
                        if (!ABS) {
                            const float x = rows_reduce1(swb_a);
                            if (k == 0u) slot0[s * VS + 8u] = x;
                        }
                        break;
                    }
                    ja = next();
                    xya = at(ja, 0);
                    coa = at(ja, 1);
                    cola = at(ja, 2);
                    walk(jb, s + 1, xyb, cob, colb, swb_b);
                    if (!ABS) {
                        const float x = rows_reduce2(swb_a, swb_b);
                        if (store8) b8[s * VS] = x;
                    }
                }
            }
            wave_lds_fence();  // every group's sums are in its slots

            // combine: the two lanes of Gaussian cj (of this sub-batch) add its sixteen group slots in group order
            // (values 0..3 and the extras, resp. values 4..7: the second lane reads four floats on, and its reads
            // of the extras' offsets land in the next record, unused) and write the instance's record (36 bytes, 48 with ABS):
            // dL/dmean2d = C (sum h d), 0.5 (sum h dx^2, sum h dx dy); 0.5 sum h dy^2, sum G dL/dalpha = -(sum of
            // h) / o, colour r, g; colour b, |dL/dmean2d| (x, y), 0. Gaussians that no group walked get zeros.
            const uint32_t cend = over ? cut : n_chunk;
            if (cj >= pos0 && cj < cend) {
                const float* const cb = s_part + ch * 4u;
                float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ax[NX];
#pragma unroll
                for (uint32_t x = 0; x < NX; x++) ax[x] = 0.0f;
#pragma unroll
                for (uint32_t g = 0; g < backward_groups; g++) {
                    const float* const b = cb + s_pos[g][cj] * VS;
#pragma unroll
                    for (uint32_t c = 0; c < 4; c++) acc[c] += b[c];
#pragma unroll
                    for (uint32_t x = 0; x < NX; x++) ax[x] += b[8 + x];
                }
                // (the extras' sums are formed here in both halves, with the reads of the group loop: otherwise the
                // compiler moves their reads into the first half's branch, recomputing every address)
#pragma unroll
                for (uint32_t x = 0; x < NX; x++) asm volatile("" : "+v"(ax[x]));
                const float4 co = s_stage[cj + 1][1];
                // the record at the instance's emission slot (a 64-bit offset: 36 e passes 2^32 from e = 119,304,648 on)
                float* const out = a.inst_grads + RECORD * static_cast<uint64_t>(__float_as_uint(s_stage[cj + 1][2].w));
                // first half: floats 0..3 (and the extras from float 8), second half: floats 4..7, formed by selects so
                // that both halves run one store path
                const float4 craw = raw_conic_of(co);
                const float q1y = -acc[1] * __builtin_amdgcn_rcpf(co.w);
                const bool first = ch == 0u;
                store_record4(out + 4u * ch, make_float4(first ? __builtin_fmaf(craw.x, acc[0], craw.y * acc[1]) : 0.5f * acc[0],
                                                        first ? __builtin_fmaf(craw.y, acc[0], craw.z * acc[1]) : q1y,
                                                        first ? 0.5f * acc[2] : acc[2], first ? 0.5f * acc[3] : acc[3]));
                if (first) {
                    if (ABS) store_record4(out + 8, make_float4(ax[0], ax[NX > 1 ? 1 : 0], ax[NX > 2 ? 2 : 0], 0.0f));
                    else out[8] = ax[0];
                }
            }
            if (!over) break;
            pos0 = cend;
            wave_lds_fence();  // the combine has read the table before the next sub-batch rewrites it
        }
        wave_lds_fence();  // the combine has read the stage
        if (base + CHUNK < n_proc) stage(base + CHUNK, rec_n, e_n);  // the next chunk
    }
    // instances the tile never reached (after every pixel's last contributor) get zero records
    for (uint32_t q = n_proc + lane; q < n_total; q += 64) {
        const uint32_t e = a.sorted_inst[range.x + q];
        float* const out = a.inst_grads + RECORD * static_cast<uint64_t>(e);
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        store_record4(out, z);
        store_record4(out + 4, z);
        if (ABS) store_record4(out + 8, z);
        else out[8] = 0.0f;
    }
}

// Speedy-Splat pruning scores: per pixel and contributing Gaussian (o dL/dalpha)^2 for the upstream gradient
// (1, 1, 1), with dL/dalpha formed as in the backward: T (c . 1) - (A - g_bg) / max(1 - alpha, eps), A = (colour
// still to come) . 1, g_bg = -T_final (bg . 1). Three waves per tile, wave w owning pixel rows 4w..4w+3, each
// split into eight 4x2 groups of one pixel per lane (the lists padded with a staged Gaussian of opacity 0): one
// value per Gaussian gains nothing from three pixels per lane. Each group walks two Gaussians per step and sums their
// scores over its 8 lanes with one row-pair swap and two quad additions; per batch the 24 (wave, group) slots
// are added in a fixed order into one float per instance at its emission slot (instances after every pixel's
// last contributor get 0). No atomics (the reference adds per pixel with float atomics).
// Reference: B/rasterization/include/kernels_pruning_scores.cuh:11-171.
__global__ __launch_bounds__(tile_pixels) void blend_scores_kernel(BlendBackwardArgs a) {
    constexpr uint32_t n_waves = tile_pixels / 64;
    constexpr uint32_t batch = 32;
    constexpr uint32_t list_len = batch;
    constexpr uint32_t n_groups = 8;
    constexpr uint32_t n_slots = n_waves * n_groups;
    constexpr uint32_t dummy = batch;  // staged Gaussian of opacity 0 (its slot column is never read)
    __shared__ float4 s_stage[batch + 1][3];  // (x, y, packed rect), exp2-scaled conic + opacity, colour
    __shared__ uint32_t s_emit[batch];
    __shared__ __align__(16) uint32_t s_list[n_waves][n_groups][list_len];
    __shared__ float s_part[n_slots][batch + 1];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tile = a.order ? a.order[blockIdx.x] : blockIdx.x;  // heaviest tiles first
    const uint32_t tx = tile % a.grid_w, ty = tile / a.grid_w;
    const uint32_t g = ((lane >> 2) & 3u) + 4u * (lane >> 5);  // the lane's 4x2 group within the wave's band
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
    for (uint32_t k = tid; k < n_slots * (batch + 1); k += tile_pixels) (&s_part[0][0])[k] = 0.0f;
    if (tid < 3) s_stage[dummy][tid] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // after the reduction lane row r holds the group sum of Gaussian a (rows 0, 2) or b (rows 1, 3) of the
    // group of rows r & 2, r | 1: the first lane of each quad stores it
    const uint32_t row = lane >> 4;
    const bool store_lane = (lane & 3u) == 0;
    const bool store_b = (row & 1u) != 0;
    float* const slot = &s_part[wave * n_groups + g][0];

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
            const PrimRecord rec = a.records[a.sorted_prim[range.x + start + tid]];
            s_stage[tid][0] = make_float4(rec.r0.x, rec.r0.y, rec.r2.y, rec.r2.z);
            s_stage[tid][1] = scale_conic_for_exp2(rec.r0.z, rec.r0.w, rec.r1.x, rec.r1.y);
            s_stage[tid][2] = make_float4(rec.r1.z, rec.r1.w, rec.r2.x, 0.0f);
            s_emit[tid] = e;
        }
        __syncthreads();
        const uint32_t batch_wave = wave_last > start ? min(min(batch, n_proc - start), wave_last - start) : 0u;
        {
            static_assert(n_groups * list_len == 4 * 64, "one 16-byte store per lane pads the wave's lists");
            const uint4 pad = make_uint4(dummy, dummy, dummy, dummy);
            reinterpret_cast<uint4*>(&s_list[wave][0][0])[lane] = pad;
        }
        wave_lds_fence();
        uint64_t m[n_groups];
        bool hit[n_groups];
        cull_groups8(rect_of(s_stage[lane & (batch - 1)][0]), lane, batch_wave, bx0, by0, m, hit);
        uint32_t n[n_groups];
        build_group_lists(m, hit, lane, 0u, &s_list[wave][0][0], list_len, n);
        wave_lds_fence();
        uint32_t n_max = n[0];
#pragma unroll
        for (uint32_t q = 1; q < n_groups; q++) n_max = max(n_max, n[q]);
        n_max = __builtin_amdgcn_readfirstlane(n_max);
        const uint32_t last_rel = last > start ? last - start : 0u;
        for (uint32_t k = 0; k < n_max; k += 2) {
            const uint2 jab = *reinterpret_cast<const uint2*>(my_list + k);  // past the count: the opacity-0 entry
            float sc[2];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                const uint32_t j = h ? jab.y : jab.x;
                float dx, dy, G;
                const float4 co = s_stage[j][1];
                const float alpha = eval_alpha(s_stage[j][0], co, pxf, pyf, dx, dy, G);
                const bool contrib = j < last_rel && alpha >= min_alpha;
                const float ae = contrib ? alpha : 0.0f;
                const float4 col = s_stage[j][2];
                const float cg = col.x + col.y + col.z;
                const float oma = 1.0f - ae;
                const float rcp = __builtin_amdgcn_rcpf(fmaxf(oma, one_minus_alpha_eps));
                A = __builtin_fmaf(-T * ae, cg, A);
                const float dg = co.w * __builtin_fmaf(T, cg, -rcp * (A - gbg));
                sc[h] = contrib ? dg * dg : 0.0f;
                T = transmit(T, ae);
            }
            // rows 0 + 1 and 2 + 3 (a and b of the upper group, a and b of the lower), then over the quad
            float sx = swap16_add(sc[0], sc[1]);
            sx += dpp<0x4E, 0xf, true>(0.0f, sx);
            sx += dpp<0xB1, 0xf, true>(0.0f, sx);
            if (store_lane) slot[store_b ? jab.y : jab.x] = sx;
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
    if (a.key_bytes == 2)
        blend_forward_kernel<uint16_t><<<a.n_tiles, 64, 0, s>>>(a);
    else
        blend_forward_kernel<uint32_t><<<a.n_tiles, 64, 0, s>>>(a);
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
        blend_backward_kernel<true, backward_list_abs><<<a.n_tiles, 64, 0, s>>>(a);
    else
        blend_backward_kernel<false, backward_list><<<a.n_tiles, 64, 0, s>>>(a);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
