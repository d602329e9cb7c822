// Forward preprocess, runtime-specialised with hipRTC. The loader prepends a token preamble
// (EFGS_KERNEL_NAME, EFGS_MODEL, EFGS_BASE_ACT, EFGS_RES_ACT, EFGS_COLOR_ACT, EFGS_N_UNITS, neural MLP shape
// tokens), efgs_common.h, efgs_args.h and the selected appearance header.
//
// One thread per primitive, 256 threads = 4 wave64 per block. Per primitive: view-depth cull, opacity cull,
// 3D covariance from log-scales and quaternion, EWA projection with the 1.15x clip, dilation and determinant
// cull, conic, screen bounds clamped to the padded tile grid, exact touched-tile count (first 8 tiles per
// lane, larger footprints wave-cooperatively 64 tiles per step), activated colour, and the 48-byte record.
// Each 256-primitive chunk also records its visible and instance counts, which a scan turns into
// deterministic (primitive-index ordered) compaction offsets. No global atomics. The neural variant runs a
// persistent grid (chunks strided by the grid size) so its MLP weights are staged into LDS once per block, and
// evaluates the MLP only for the chunk's visible primitives, compacted into as few waves as they fill.
//
// Reference: B/rasterization/rtc/preprocess_forward.cu:12-278, preprocess_common.cuh:190-252.

namespace efgs {

constexpr uint32_t preprocess_block = 256;

struct Projected {
    float mean2d_x, mean2d_y, conic_x, conic_y, conic_z, opacity, power_threshold, depth;
    uint32_t sx0, sx1, sy0, sy1;
    TileRect tiles;
    bool visible;
};

__device__ inline Projected project(const PreprocessForwardArgs& a, uint32_t p, bool active) {
#pragma clang fp contract(off)
    Projected r;
    r.visible = false;
    r.sx0 = r.sx1 = r.sy0 = r.sy1 = 0;
    r.tiles = {0, 0, 0, 0};
    const float* W = a.cam.w2c;
    // every raw input is loaded before the first cull (p is a valid index for inactive lanes too): the loads are
    // in flight together, one memory round trip instead of one per cull and per special-cased exp
    float mx = a.means[3 * p], my = a.means[3 * p + 1], mz = a.means[3 * p + 2];
    float raw_opacity = a.opacities[p];
    float ls0 = a.scales[3 * p], ls1 = a.scales[3 * p + 1], ls2 = a.scales[3 * p + 2];
    float q0 = a.rotations[4 * p], q1 = a.rotations[4 * p + 1], q2 = a.rotations[4 * p + 2], q3 = a.rotations[4 * p + 3];
    asm volatile("" : "+v"(mx), "+v"(my), "+v"(mz), "+v"(raw_opacity), "+v"(ls0), "+v"(ls1), "+v"(ls2), "+v"(q0), "+v"(q1), "+v"(q2),
                 "+v"(q3));
    const float depth = W[8] * mx + W[9] * my + W[10] * mz + W[11];
    r.depth = depth;
    if (!active || depth < a.cam.near_plane || depth > a.cam.far_plane) return r;
    float opacity = ef_sigmoid(raw_opacity);
    if (opacity < min_alpha) return r;
    const float v0 = ef_expf(2.0f * ls0);
    const float v1 = ef_expf(2.0f * ls1);
    const float v2 = ef_expf(2.0f * ls2);
    float qn;
    const Mat3 R = quaternion_to_rotation(q0, q1, q2, q3, qn);
    if (qn < 1e-8f) return r;
    const Mat3 S = {R.m11 * v0, R.m12 * v1, R.m13 * v2, R.m21 * v0, R.m22 * v1, R.m23 * v2, R.m31 * v0, R.m32 * v1, R.m33 * v2};
    const float c11 = S.m11 * R.m11 + S.m12 * R.m12 + S.m13 * R.m13;
    const float c12 = S.m11 * R.m21 + S.m12 * R.m22 + S.m13 * R.m23;
    const float c13 = S.m11 * R.m31 + S.m12 * R.m32 + S.m13 * R.m33;
    const float c22 = S.m21 * R.m21 + S.m22 * R.m22 + S.m23 * R.m23;
    const float c23 = S.m21 * R.m31 + S.m22 * R.m32 + S.m23 * R.m33;
    const float c33 = S.m31 * R.m31 + S.m32 * R.m32 + S.m33 * R.m33;
    const float x = (W[0] * mx + W[1] * my + W[2] * mz + W[3]) / depth;
    const float y = (W[4] * mx + W[5] * my + W[6] * mz + W[7]) / depth;
    const float fx = a.cam.focal_x, fy = a.cam.focal_y, cx = a.cam.center_x, cy = a.cam.center_y;
    const float xc = clampf(x, a.cam.clip_left, a.cam.clip_right), yc = clampf(y, a.cam.clip_top, a.cam.clip_bottom);
    const float j11 = fx / depth, j13 = -j11 * xc, j22 = fy / depth, j23 = -j22 * yc;
    const float a1x = j11 * W[0] + j13 * W[8], a1y = j11 * W[1] + j13 * W[9], a1z = j11 * W[2] + j13 * W[10];
    const float a2x = j22 * W[4] + j23 * W[8], a2y = j22 * W[5] + j23 * W[9], a2z = j22 * W[6] + j23 * W[10];
    const float b1x = a1x * c11 + a1y * c12 + a1z * c13, b1y = a1x * c12 + a1y * c22 + a1z * c23, b1z = a1x * c13 + a1y * c23 + a1z * c33;
    const float b2x = a2x * c11 + a2y * c12 + a2z * c13, b2y = a2x * c12 + a2y * c22 + a2z * c23, b2z = a2x * c13 + a2y * c23 + a2z * c33;
    float vx = b1x * a1x + b1y * a1y + b1z * a1z;
    const float vy = b1x * a2x + b1y * a2y + b1z * a2z;
    float vz = b2x * a2x + b2y * a2y + b2z * a2z;
    const float det_raw = vx * vz - vy * vy;
    const float ks = a.cam.proper_aa ? dilation_aa : dilation;
    vx += ks;
    vz += ks;
    const float det = vx * vz - vy * vy;
    if (det < min_cov2d_det) return r;
    r.conic_x = vz / det;
    r.conic_y = -vy / det;
    r.conic_z = vx / det;
    if (a.cam.proper_aa) {
        opacity *= sqrtf(fmaxf(det_raw / det, 0.0f));
        if (opacity < min_alpha) return r;
    }
    r.opacity = opacity;
    r.mean2d_x = x * fx + cx;
    r.mean2d_y = y * fy + cy;
    const float pt = power_threshold_of(opacity);
    r.power_threshold = pt;
    const float cutoff = 2.0f * pt;
    const float ex = fmaxf(sqrtf(vx * cutoff) - 0.5f, 0.0f);
    const float ey = fmaxf(sqrtf(vz * cutoff) - 0.5f, 0.0f);
    const float pw = static_cast<float>(a.cam.grid_w * tile_width), ph = static_cast<float>(a.cam.grid_h * tile_height);
    // min(padded, max(0, round_down/up(v))) with the clamp applied before the float-to-int conversion
    const int bx0 = static_cast<int>(floorf(clampf(r.mean2d_x - ex, -1.0f, pw + 1.0f)));
    const int bx1 = static_cast<int>(ceilf(clampf(r.mean2d_x + ex, -1.0f, pw + 1.0f)));
    const int by0 = static_cast<int>(floorf(clampf(r.mean2d_y - ey, -1.0f, ph + 1.0f)));
    const int by1 = static_cast<int>(ceilf(clampf(r.mean2d_y + ey, -1.0f, ph + 1.0f)));
    const int ipw = static_cast<int>(a.cam.grid_w * tile_width), iph = static_cast<int>(a.cam.grid_h * tile_height);
    r.sx0 = static_cast<uint32_t>(min(ipw, max(0, bx0)));
    r.sx1 = static_cast<uint32_t>(min(ipw, max(0, bx1)));
    r.sy0 = static_cast<uint32_t>(min(iph, max(0, by0)));
    r.sy1 = static_cast<uint32_t>(min(iph, max(0, by1)));
    r.tiles = screen_to_tile_bounds(r.sx0, r.sx1, r.sy0, r.sy1);
    r.visible = (r.tiles.x1 - r.tiles.x0) * (r.tiles.y1 - r.tiles.y0) > 0;
    return r;
}

// exact number of tiles in the tile rectangle that the primitive reaches; first_tiles receives the test results of
// the rectangle's first n_sequential_tiles tiles (bit i: tile i, row-major). Every lane of the wave must call it.
__device__ inline uint32_t count_touched_tiles(const Projected& pr, uint32_t lane, uint32_t& first_tiles) {
#pragma clang fp contract(off)
    const uint32_t bw = pr.tiles.x1 - pr.tiles.x0;
    const uint32_t cnt = pr.visible ? bw * (pr.tiles.y1 - pr.tiles.y0) : 0u;
    const float smx = pr.mean2d_x - 0.5f, smy = pr.mean2d_y - 0.5f;
    uint32_t touched = 0;
    first_tiles = 0;
    for (uint32_t i = 0; i < cnt && i < n_sequential_tiles; i++) {
        const uint32_t tx = pr.tiles.x0 + i % bw, ty = pr.tiles.y0 + i / bw;
        const bool hit = will_primitive_contribute(smx, smy, pr.conic_x, pr.conic_y, pr.conic_z, tx, ty, pr.power_threshold);
        touched += hit ? 1u : 0u;
        first_tiles |= (hit ? 1u : 0u) << i;
    }
    uint64_t coop = __ballot(cnt > n_sequential_tiles);
    while (coop != 0) {
        // (the source lane is wave-uniform: its values come by readlane, no LDS permute)
        const int src = static_cast<int>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(__ffsll(static_cast<long long>(coop)) - 1)));
        coop &= coop - 1;
        const auto lane_u = [src](uint32_t v) { return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), src)); };
        const auto lane_f = [src](float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src)); };
        const uint32_t c_x0 = lane_u(pr.tiles.x0), c_y0 = lane_u(pr.tiles.y0);
        const uint32_t c_bw = lane_u(bw), c_cnt = lane_u(cnt);
        const float c_mx = lane_f(smx), c_my = lane_f(smy);
        const float c_cx = lane_f(pr.conic_x), c_cy = lane_f(pr.conic_y), c_cz = lane_f(pr.conic_z);
        const float c_pt = lane_f(pr.power_threshold);
        uint32_t hits = 0;
        for (uint32_t base = n_sequential_tiles; base < c_cnt; base += 64) {
            const uint32_t i = base + lane;
            const bool hit = i < c_cnt && will_primitive_contribute(c_mx, c_my, c_cx, c_cy, c_cz, c_x0 + i % c_bw, c_y0 + i / c_bw, c_pt);
            hits += static_cast<uint32_t>(__popcll(__ballot(hit)));
        }
        if (lane == static_cast<uint32_t>(src)) touched += hits;
    }
    return touched;
}

// Reductions over the wave, the result in every lane, without LDS round trips: four row rotations (DPP) give
// every lane its 16-lane row's result, then two lane swaps (rows 0 <-> 2 and 1 <-> 3, then 0 <-> 1 and 2 <-> 3)
// combine the rows. Every lane of the wave must take part.
template <typename OP>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, OP op) {
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xf, 0xf, false)));  // row_ror:1
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xf, 0xf, false)));  // row_ror:2
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xf, 0xf, false)));  // row_ror:4
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false)));  // row_ror:8
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return op(b[0], b[1]);
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    return wave_reduce_u32(v, [](uint32_t x, uint32_t y) { return x + y; });
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    return wave_reduce_u32(v, [](uint32_t x, uint32_t y) { return min(x, y); });
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return wave_reduce_u32(v, [](uint32_t x, uint32_t y) { return max(x, y); });
}

}  // namespace efgs

// four waves per SIMD (128 VGPRs): the neural variant's LDS admits four blocks per CU as well
extern "C" __global__ __launch_bounds__(256, 4) void EFGS_KERNEL_NAME(efgs::PreprocessForwardArgs a) {
    using namespace efgs;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    __shared__ uint32_t wave_counts[4 * (preprocess_block / 64)];
#if EFGS_MODEL >= 1 && EFGS_MODEL <= 4
    // the forward stages its rows only for the lobe models: SH and SV read each row once and keep more waves per
    // SIMD without the LDS
    constexpr bool staged_forward = ForwardRows::staged && (EFGS_MODEL == 3 || EFGS_MODEL == 4);
    constexpr uint32_t row_ld = ForwardRows::row_ld, pass_units = ForwardRows::pass_units, n_passes = ForwardRows::n_passes;
    __shared__ float s_rows[staged_forward ? preprocess_block * row_ld : 1];
#endif
#if EFGS_MODEL == 5
    // residual MLP weights staged once per block (padded rows); staging rows of the MLP inputs (64 per wave)
    extern __shared__ __align__(16) unsigned char smem[];
    const _Float16* WL = reinterpret_cast<const _Float16*>(smem);
    _Float16* stage = reinterpret_cast<_Float16*>(smem + nn::WEIGHT_BYTES);
    nn::load_weights<preprocess_block>(a.mlp_weights, reinterpret_cast<uint16_t*>(smem), threadIdx.x);
    __syncthreads();
#endif
    const uint32_t n_chunks = (a.n + preprocess_block - 1) / preprocess_block;
    for (uint32_t chunk = blockIdx.x; chunk < n_chunks; chunk += gridDim.x) {
        const uint32_t p_raw = chunk * preprocess_block + threadIdx.x;
        const bool active = p_raw < a.n;
        const uint32_t p = active ? p_raw : a.n - 1;

        Projected pr = project(a, p, active);
        uint32_t first_tiles;
        uint32_t touched = count_touched_tiles(pr, lane, first_tiles);
        const bool visible = pr.visible && touched > 0;
        if (!visible) touched = 0;

        // per-chunk visible / instance counts (deterministic compaction offsets come from their scan)
        const uint64_t visible_mask = __ballot(visible);  // (visible implies active)
        const uint32_t wave_instances = wave_sum_u32(touched);
        const uint32_t key = __float_as_uint(pr.depth);
        const uint32_t wave_kmin = wave_min_u32(visible ? key : 0xffffffffu);
        const uint32_t wave_kmax = wave_max_u32(visible ? key : 0u);
        if (lane == 0) {
            wave_counts[4 * wave] = static_cast<uint32_t>(__popcll(visible_mask));
            wave_counts[4 * wave + 1] = wave_instances;
            wave_counts[4 * wave + 2] = wave_kmin;
            wave_counts[4 * wave + 3] = wave_kmax;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t v = 0, i = 0, kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
            for (uint32_t w = 0; w < preprocess_block / 64; w++) {
                v += wave_counts[4 * w];
                i += wave_counts[4 * w + 1];
                kmin = min(kmin, wave_counts[4 * w + 2]);
                kmax = max(kmax, wave_counts[4 * w + 3]);
            }
            a.block_counts[2 * chunk] = v;
            a.block_counts[2 * chunk + 1] = i;
            a.block_key_ranges[2 * chunk] = kmin;
            a.block_key_ranges[2 * chunk + 1] = kmax;
            if (chunk == 0) a.counters[2] = 0u;  // the emission after this kernel counts its mismatches there
        }
        if (active) {
            a.n_touched[p] = touched;
            a.depth_keys[p] = key;
        }
        // whether a block barrier follows the last read of wave_counts in this chunk (else one ends the chunk)
        bool counts_released = false;

        float3 color = make_float3(0.0f, 0.0f, 0.0f);
#if EFGS_MODEL == 0
        if (visible) color = make_float3(a.precomputed[3 * p], a.precomputed[3 * p + 1], a.precomputed[3 * p + 2]);
#else
        const float3 mean = make_float3(a.means[3 * p], a.means[3 * p + 1], a.means[3 * p + 2]);
        const float3 cam = make_float3(a.cam.cam_position[0], a.cam.cam_position[1], a.cam.cam_position[2]);
        float norm_rcp;
        const float3 d = view_direction(mean, cam, norm_rcp);
        const float* rp = a.residual + static_cast<size_t>(p) * residual_params;
        float3 res = make_float3(0.0f, 0.0f, 0.0f);
#if EFGS_MODEL == 5
        // The chunk's visible primitives, compacted in thread order into the staging rows, run the MLP on as few
        // waves as their rows fill (a wave with no row skips it): with about 70 % of a scene's primitives visible,
        // three waves of the four instead of every wave that holds one visible primitive.
        if (a.cam.degree > 0) {
            uint32_t row = static_cast<uint32_t>(__popcll(visible_mask & ((1ull << lane) - 1ull))), n_rows = 0;
#pragma unroll
            for (uint32_t w = 0; w < preprocess_block / 64; w++) {
                const uint32_t c = wave_counts[4 * w];
                row += w < wave ? c : 0u;
                n_rows += c;
            }
            if (visible) {
                float x[nn::INP];
                nn::mlp_input(rp, a.base + 3 * p, d, a.cam.degree, x);
                nn::stage_input_row(stage, x, row);
            }
            __syncthreads();  // rows staged (and every read of wave_counts done)
            counts_released = true;
            if (64 * wave < n_rows) nn::mlp_forward_rows(WL, stage + 64 * wave * nn::XS, lane);
            __syncthreads();  // outputs written over the rows
            if (visible) {
                const float* ys = reinterpret_cast<const float*>(stage + (row / 64u) * 64u * nn::XS);
                const float4 y = *reinterpret_cast<const float4*>(&ys[(row % 64u) * 4u]);
                res = make_float3(residual_activation<EFGS_RES_ACT>(y.x), residual_activation<EFGS_RES_ACT>(y.y),
                                  residual_activation<EFGS_RES_ACT>(y.z));
            }
        }
#endif
#if EFGS_MODEL >= 1 && EFGS_MODEL <= 4
        if constexpr (staged_forward) {
            // the chunk's rows through LDS (the previous chunk ended at a block barrier), one pass per unit range
            const uint32_t p0 = chunk * preprocess_block;
            const uint32_t rows = min(preprocess_block, a.n - p0);
            for (uint32_t pass = 0; pass < n_passes; pass++) {
                const uint32_t u0 = pass * pass_units;
                const uint32_t nu = min(pass_units, static_cast<uint32_t>(EFGS_N_UNITS) - u0);
                if (pass > 0) __syncthreads();  // every thread has read the previous pass's rows
                stage_residual_rows<preprocess_block, row_ld>(a.residual, p0, rows, u0 * params_per_unit, nu * params_per_unit, s_rows);
                __syncthreads();
                if (visible) {
                    const float* row = s_rows + threadIdx.x * row_ld;
#if EFGS_MODEL == 1
                    res = sh_residual<EFGS_RES_ACT>(row, d, a.cam.degree);
#elif EFGS_MODEL == 2
                    res = sv_residual<EFGS_RES_ACT>(row, d, a.cam.degree);
#else
                    const uint32_t na = a.cam.degree > u0 ? min(nu, a.cam.degree - u0) : 0u;
                    const float3 r = lobe_residual<EFGS_RES_ACT, EFGS_MODEL == 4>(row, d, na);
                    res.x += r.x;
                    res.y += r.y;
                    res.z += r.z;
#endif
                }
            }
        } else if (visible) {
#if EFGS_MODEL == 1
            res = sh_residual<EFGS_RES_ACT>(rp, d, a.cam.degree);
#elif EFGS_MODEL == 2
            res = sv_residual<EFGS_RES_ACT>(rp, d, a.cam.degree);
#elif EFGS_MODEL == 3
            res = lobe_residual<EFGS_RES_ACT, false>(rp, d, a.cam.degree);
#elif EFGS_MODEL == 4
            res = lobe_residual<EFGS_RES_ACT, true>(rp, d, a.cam.degree);
#endif
        }
#endif
        if (visible) {
            const float b0 = base_activation<EFGS_BASE_ACT>(a.base[3 * p]);
            const float b1 = base_activation<EFGS_BASE_ACT>(a.base[3 * p + 1]);
            const float b2 = base_activation<EFGS_BASE_ACT>(a.base[3 * p + 2]);
            color = make_float3(color_activation<EFGS_COLOR_ACT>(b0 + res.x), color_activation<EFGS_COLOR_ACT>(b1 + res.y),
                                color_activation<EFGS_COLOR_ACT>(b2 + res.z));
            if (!a.cam.render_base) {
                color.x = fabsf(color.x - color_activation<EFGS_COLOR_ACT>(b0));
                color.y = fabsf(color.y - color_activation<EFGS_COLOR_ACT>(b1));
                color.z = fabsf(color.z - color_activation<EFGS_COLOR_ACT>(b2));
            }
        }
#endif

        if (visible) {
            PrimRecord rec;
            rec.r0 = make_float4(pr.mean2d_x, pr.mean2d_y, pr.conic_x, pr.conic_y);
            rec.r1 = make_float4(pr.conic_z, pr.opacity, color.x, color.y);
            rec.r2 = make_float4(color.z, __uint_as_float(pr.sx0 | (pr.sx1 << 16)), __uint_as_float(pr.sy0 | (pr.sy1 << 16)),
                                 __uint_as_float(first_tiles));
            a.records[p] = rec;
        }
        if (!counts_released) __syncthreads();  // (block-uniform) wave_counts read before the next chunk writes it
    }
}
