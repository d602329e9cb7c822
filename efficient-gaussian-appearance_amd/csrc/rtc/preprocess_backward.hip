// Backward preprocess, runtime-specialised with hipRTC (same preamble and headers as the forward).
//
// One thread per primitive. The blend backward leaves one gradient record per emitted instance (dL/dmean2d xy,
// dL/dconic xyz, dL/dopacity, dL/dcolor rgb: 9 floats; with three densification rows also |dL/dmean2d| xy and a
// pad: 12) at the instance's emission slot; a visible primitive's slots are contiguous, so this kernel reduces them in a fixed order
// (deterministic, no float atomics), applies the opacity chain, backpropagates the colour through the
// activations and the appearance model, and the 2D mean and conic through the EWA projection to the 3D mean,
// log-scales and quaternion. Culled primitives get zero gradients.
//
// The neural variant splits this into two kernels: the same per-primitive geometry part (no MLP state, so it
// runs at high occupancy) and an MLP kernel on a persistent grid.
//
// Reference: B/rasterization/rtc/preprocess_backward.cu:19-404 (the per-primitive part of
// B/rasterization/include/kernels_backward.cuh:215-230 is folded in here).

namespace efgs {

constexpr uint32_t preprocess_block = 256;

__device__ __forceinline__ uint32_t active_residual_params(uint32_t degree) {
    if (EFGS_MODEL == 1) return 3u * ((degree + 1) * (degree + 1) - 1);
    if (EFGS_MODEL == 5) return degree > 0 ? residual_params : 0u;
    return params_per_unit * degree;
}

struct InstanceGrads {
    float gmx, gmy, gcx, gcy, gcz, gop, gr, gg, gb, gax, gay;
};

__device__ __forceinline__ void add_record(float4& s0, float4& s1, float4& s2, float4 t0, float4 t1, float4 t2) {
    s0.x += t0.x; s0.y += t0.y; s0.z += t0.z; s0.w += t0.w;
    s1.x += t1.x; s1.y += t1.y; s1.z += t1.z; s1.w += t1.w;
    s2.x += t2.x; s2.y += t2.y; s2.z += t2.z;
}

// four floats of a record at a 4-byte aligned address (one 16-byte load: dword-aligned vector accesses to global
// memory need no more)
struct __attribute__((aligned(4))) Float4A4 {
    float x, y, z, w;
};
__device__ __forceinline__ float4 load_record4(const float* p) {
    const Float4A4 v = *reinterpret_cast<const Float4A4*>(p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// sum of a visible primitive's per-instance gradient records (starting at emission slot `offset`), in
// emission order; two records are fetched per step so their loads are in flight together. Records are
// record_floats_abs floats with three densification rows (|dL/dmean2d| after the colour), record_floats otherwise.
template <uint32_t RECORD>
__device__ inline InstanceGrads reduce_instance_grads_of(const PreprocessBackwardArgs& a, uint32_t offset, uint32_t touched) {
    const float* ig = a.inst_grads + RECORD * static_cast<size_t>(offset);
    const auto third = [&](uint32_t k) { return RECORD == record_floats ? make_float4(ig[RECORD * k + 8], 0.0f, 0.0f, 0.0f) : load_record4(ig + RECORD * k + 8); };
    float4 s0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), s1 = s0, s2 = s0;
    uint32_t k = 0;
    for (; k + 2 <= touched; k += 2) {
        const float4 t0 = load_record4(ig + RECORD * k), t1 = load_record4(ig + RECORD * k + 4), t2 = third(k);
        const float4 u0 = load_record4(ig + RECORD * (k + 1)), u1 = load_record4(ig + RECORD * (k + 1) + 4), u2 = third(k + 1);
        add_record(s0, s1, s2, t0, t1, t2);
        add_record(s0, s1, s2, u0, u1, u2);
    }
    if (k < touched) add_record(s0, s1, s2, load_record4(ig + RECORD * k), load_record4(ig + RECORD * k + 4), third(k));
    return {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w, s2.x, s2.y, s2.z};
}
__device__ inline InstanceGrads reduce_instance_grads(const PreprocessBackwardArgs& a, uint32_t offset, uint32_t touched) {
    return a.densification_rows > 2 ? reduce_instance_grads_of<record_floats_abs>(a, offset, touched)
                                    : reduce_instance_grads_of<record_floats>(a, offset, touched);
}

// a primitive's parameters, loaded before its instance records are summed so that every load is in flight at once
struct GeometryInputs {
    float3 mean, log_scale;
    float4 rotation;
    float raw_opacity;
};

__device__ __forceinline__ GeometryInputs load_geometry(const PreprocessBackwardArgs& a, uint32_t p) {
    GeometryInputs g;
    g.mean = make_float3(a.means[3 * p], a.means[3 * p + 1], a.means[3 * p + 2]);
    g.log_scale = make_float3(a.scales[3 * p], a.scales[3 * p + 1], a.scales[3 * p + 2]);
    g.rotation = make_float4(a.rotations[4 * p], a.rotations[4 * p + 1], a.rotations[4 * p + 2], a.rotations[4 * p + 3]);
    g.raw_opacity = a.cam.proper_aa ? a.opacities[p] : 0.0f;
    return g;
}

__device__ inline void zero_primitive(const PreprocessBackwardArgs& a, uint32_t p, bool residual = true) {
    a.g_means[3 * p] = 0.0f; a.g_means[3 * p + 1] = 0.0f; a.g_means[3 * p + 2] = 0.0f;
    a.g_scales[3 * p] = 0.0f; a.g_scales[3 * p + 1] = 0.0f; a.g_scales[3 * p + 2] = 0.0f;
    a.g_rotations[4 * p] = 0.0f; a.g_rotations[4 * p + 1] = 0.0f; a.g_rotations[4 * p + 2] = 0.0f; a.g_rotations[4 * p + 3] = 0.0f;
    a.g_opacities[p] = 0.0f;
#if EFGS_MODEL == 0
    a.g_precomputed[3 * p] = 0.0f; a.g_precomputed[3 * p + 1] = 0.0f; a.g_precomputed[3 * p + 2] = 0.0f;
#else
    a.g_base[3 * p] = 0.0f; a.g_base[3 * p + 1] = 0.0f; a.g_base[3 * p + 2] = 0.0f;
    if (residual)
        for (uint32_t i = 0; i < residual_params; i++) a.g_residual[static_cast<size_t>(p) * residual_params + i] = 0.0f;
#endif
}

// colour gradient through the colour activation (reference: recovered from the stored activated colour)
__device__ __forceinline__ float3 pre_activation_grad(const PrimRecord& rec, const InstanceGrads& g) {
    return make_float3(color_activation_grad<EFGS_COLOR_ACT>(rec.r1.z) * g.gr, color_activation_grad<EFGS_COLOR_ACT>(rec.r1.w) * g.gg,
                       color_activation_grad<EFGS_COLOR_ACT>(rec.r2.x) * g.gb);
}

__device__ __forceinline__ void write_base_grad(const PreprocessBackwardArgs& a, uint32_t p, float3 dpre, float3 extra) {
    if (a.cam.render_base) {
        a.g_base[3 * p] = base_activation_grad<EFGS_BASE_ACT>(a.base[3 * p]) * dpre.x + extra.x;
        a.g_base[3 * p + 1] = base_activation_grad<EFGS_BASE_ACT>(a.base[3 * p + 1]) * dpre.y + extra.y;
        a.g_base[3 * p + 2] = base_activation_grad<EFGS_BASE_ACT>(a.base[3 * p + 2]) * dpre.z + extra.z;
    } else {
        a.g_base[3 * p] = extra.x; a.g_base[3 * p + 1] = extra.y; a.g_base[3 * p + 2] = extra.z;
    }
}

// 2D mean / conic / opacity gradients through the projection to the 3D mean, log-scales and quaternion
__device__ inline void geometry_backward(const PreprocessBackwardArgs& a, uint32_t p, const PrimRecord& rec, const GeometryInputs& gi,
                                         const InstanceGrads& ig, float3 dmean_color) {
    const float3 mean = gi.mean;
    const float gmx = ig.gmx, gmy = ig.gmy;
    const float3 gconic = make_float3(ig.gcx, ig.gcy, ig.gcz);
    const float* W = a.cam.w2c;
    const float depth = W[8] * mean.x + W[9] * mean.y + W[10] * mean.z + W[11];
    const float x = (W[0] * mean.x + W[1] * mean.y + W[2] * mean.z + W[3]) / depth;
    const float y = (W[4] * mean.x + W[5] * mean.y + W[6] * mean.z + W[7]) / depth;
    const float v0 = ef_expf(2.0f * gi.log_scale.x);
    const float v1 = ef_expf(2.0f * gi.log_scale.y);
    const float v2 = ef_expf(2.0f * gi.log_scale.z);
    const float qr = gi.rotation.x, qx = gi.rotation.y, qy = gi.rotation.z, qz = gi.rotation.w;
    float qn;
    const Mat3 R = quaternion_to_rotation(qr, qx, qy, qz, qn);
    const Mat3 S = {R.m11 * v0, R.m12 * v1, R.m13 * v2, R.m21 * v0, R.m22 * v1, R.m23 * v2, R.m31 * v0, R.m32 * v1, R.m33 * v2};
    const float c11 = S.m11 * R.m11 + S.m12 * R.m12 + S.m13 * R.m13;
    const float c12 = S.m11 * R.m21 + S.m12 * R.m22 + S.m13 * R.m23;
    const float c13 = S.m11 * R.m31 + S.m12 * R.m32 + S.m13 * R.m33;
    const float c22 = S.m21 * R.m21 + S.m22 * R.m22 + S.m23 * R.m23;
    const float c23 = S.m21 * R.m31 + S.m22 * R.m32 + S.m23 * R.m33;
    const float c33 = S.m31 * R.m31 + S.m32 * R.m32 + S.m33 * R.m33;
    const float wf = static_cast<float>(a.cam.width), hf = static_cast<float>(a.cam.height);
    const float fx = a.cam.focal_x, fy = a.cam.focal_y, cx = a.cam.center_x, cy = a.cam.center_y;
    const float xc = clampf(x, a.cam.clip_left, a.cam.clip_right), yc = clampf(y, a.cam.clip_top, a.cam.clip_bottom);
    const float j11 = fx / depth, j13 = -j11 * xc, j22 = fy / depth, j23 = -j22 * yc;
    const float a1x = j11 * W[0] + j13 * W[8], a1y = j11 * W[1] + j13 * W[9], a1z = j11 * W[2] + j13 * W[10];
    const float a2x = j22 * W[4] + j23 * W[8], a2y = j22 * W[5] + j23 * W[9], a2z = j22 * W[6] + j23 * W[10];
    const float b1x = a1x * c11 + a1y * c12 + a1z * c13, b1y = a1x * c12 + a1y * c22 + a1z * c23, b1z = a1x * c13 + a1y * c23 + a1z * c33;
    const float b2x = a2x * c11 + a2y * c12 + a2z * c13, b2y = a2x * c12 + a2y * c22 + a2z * c23, b2z = a2x * c13 + a2y * c23 + a2z * c33;
    const float a_raw = b1x * a1x + b1y * a1y + b1z * a1z;
    const float B = b1x * a2x + b1y * a2y + b1z * a2z;
    const float c_raw = b2x * a2x + b2y * a2y + b2z * a2z;
    const float ks = a.cam.proper_aa ? dilation_aa : dilation;
    const float A = a_raw + ks, C = c_raw + ks;
    const float aa = A * A, bb = B * B, cc = C * C, ac = A * C, ab = A * B, bc = B * C;
    const float det = ac - bb;
    const float det_rcp_sq = 1.0f / (det * det);
    const float dcx = det_rcp_sq * (2.0f * bc * gconic.y - cc * gconic.x - bb * gconic.z);
    const float dcy = det_rcp_sq * (bc * gconic.x - (ac + bb) * gconic.y + ab * gconic.z);
    const float dcz = det_rcp_sq * (2.0f * ab * gconic.y - bb * gconic.x - aa * gconic.z);

    // opacity: stored opacity = sigmoid(raw) [* sqrt(det_raw / det) with proper antialiasing]
    if (a.cam.proper_aa) {
        const float o = ef_sigmoid(gi.raw_opacity);
        const float rad = fmaxf((a_raw * c_raw - bb) / det, 0.0f);
        a.g_opacities[p] = ig.gop * sqrtf(rad) * o * (1.0f - o);
    } else {
        const float o = rec.r1.y;
        a.g_opacities[p] = (o - o * o) * ig.gop;
    }

    const float d11 = a1x * a1x * dcx + 2.0f * a1x * a2x * dcy + a2x * a2x * dcz;
    const float d12 = a1x * a1y * dcx + (a1x * a2y + a1y * a2x) * dcy + a2x * a2y * dcz;
    const float d13 = a1x * a1z * dcx + (a1x * a2z + a1z * a2x) * dcy + a2x * a2z * dcz;
    const float d22 = a1y * a1y * dcx + 2.0f * a1y * a2y * dcy + a2y * a2y * dcz;
    const float d23 = a1y * a1z * dcx + (a1y * a2z + a1z * a2y) * dcy + a2y * a2z * dcz;
    const float d33 = a1z * a1z * dcx + 2.0f * a1z * a2z * dcy + a2z * a2z * dcz;
    const float g1x = 2.0f * (b1x * dcx + b2x * dcy), g1y = 2.0f * (b1y * dcx + b2y * dcy), g1z = 2.0f * (b1z * dcx + b2z * dcy);
    const float g2x = 2.0f * (b1x * dcy + b2x * dcz), g2y = 2.0f * (b1y * dcy + b2y * dcz), g2z = 2.0f * (b1z * dcy + b2z * dcz);
    const float dj11 = W[0] * g1x + W[1] * g1y + W[2] * g1z;
    const float dj22 = W[4] * g2x + W[5] * g2y + W[6] * g2z;
    const float dj13 = W[8] * g1x + W[9] * g1y + W[10] * g1z;
    const float dj23 = W[8] * g2x + W[9] * g2y + W[10] * g2z;

    if (a.densification_info != nullptr) {
        const uint32_t n = a.n;
        a.densification_info[p] += 1.0f;
        const float nx = 0.5f * (gmx * wf), ny = 0.5f * (gmy * hf);
        a.densification_info[n + p] += sqrtf(nx * nx + ny * ny);
        if (a.densification_rows > 2) {
            const float ax = 0.5f * (ig.gax * wf), ay = 0.5f * (ig.gay * hf);
            a.densification_info[2 * n + p] += sqrtf(ax * ax + ay * ay);
        }
    }

    float mcx = j11 * gmx, mcy = j22 * gmy, mcz = -j11 * x * gmx - j22 * y * gmy;
    const bool vx = x >= a.cam.clip_left && x <= a.cam.clip_right, vy = y >= a.cam.clip_top && y <= a.cam.clip_bottom;
    if (vx) mcx -= j11 * dj13 / depth;
    if (vy) mcy -= j22 * dj23 / depth;
    const float fxv = 1.0f + static_cast<float>(vx), fyv = 1.0f + static_cast<float>(vy);
    mcz += (j11 * (fxv * xc * dj13 - dj11) + j22 * (fyv * yc * dj23 - dj22)) / depth;
    float gx = W[0] * mcx + W[4] * mcy + W[8] * mcz;
    float gy = W[1] * mcx + W[5] * mcy + W[9] * mcz;
    float gz = W[2] * mcx + W[6] * mcy + W[10] * mcz;
    if (EFGS_DIRECTION_GRADIENT) {
        gx += dmean_color.x;
        gy += dmean_color.y;
        gz += dmean_color.z;
    }
    a.g_means[3 * p] = gx; a.g_means[3 * p + 1] = gy; a.g_means[3 * p + 2] = gz;

    const float dv0 = R.m11 * R.m11 * d11 + R.m21 * R.m21 * d22 + R.m31 * R.m31 * d33 + 2.0f * (R.m11 * R.m21 * d12 + R.m11 * R.m31 * d13 + R.m21 * R.m31 * d23);
    const float dv1 = R.m12 * R.m12 * d11 + R.m22 * R.m22 * d22 + R.m32 * R.m32 * d33 + 2.0f * (R.m12 * R.m22 * d12 + R.m12 * R.m32 * d13 + R.m22 * R.m32 * d23);
    const float dv2 = R.m13 * R.m13 * d11 + R.m23 * R.m23 * d22 + R.m33 * R.m33 * d33 + 2.0f * (R.m13 * R.m23 * d12 + R.m13 * R.m33 * d13 + R.m23 * R.m33 * d23);
    a.g_scales[3 * p] = 2.0f * v0 * dv0;
    a.g_scales[3 * p + 1] = 2.0f * v1 * dv1;
    a.g_scales[3 * p + 2] = 2.0f * v2 * dv2;
    const Mat3 dR = {
        2.0f * (S.m11 * d11 + S.m21 * d12 + S.m31 * d13), 2.0f * (S.m12 * d11 + S.m22 * d12 + S.m32 * d13), 2.0f * (S.m13 * d11 + S.m23 * d12 + S.m33 * d13),
        2.0f * (S.m11 * d12 + S.m21 * d22 + S.m31 * d23), 2.0f * (S.m12 * d12 + S.m22 * d22 + S.m32 * d23), 2.0f * (S.m13 * d12 + S.m23 * d22 + S.m33 * d23),
        2.0f * (S.m11 * d13 + S.m21 * d23 + S.m31 * d33), 2.0f * (S.m12 * d13 + S.m22 * d23 + S.m32 * d33), 2.0f * (S.m13 * d13 + S.m23 * d23 + S.m33 * d33)};
    const float4 gq = quaternion_to_rotation_backward(qr, qx, qy, qz, dR);
    a.g_rotations[4 * p] = gq.x; a.g_rotations[4 * p + 1] = gq.y; a.g_rotations[4 * p + 2] = gq.z; a.g_rotations[4 * p + 3] = gq.w;
}

// The maximum of a value over the wave, in every lane, without LDS permutes: four row rotations (DPP), then
// two lane swaps across the rows. OP: the maximum of two 32-bit patterns.
template <typename OP>
__device__ __forceinline__ uint32_t wave_max_bits(uint32_t v, OP op) {
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xf, 0xf, false)));  // row_ror:1
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xf, 0xf, false)));  // row_ror:2
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xf, 0xf, false)));  // row_ror:4
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false)));  // row_ror:8
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return op(b[0], b[1]);
}

}  // namespace efgs

#if EFGS_MODEL != 5

namespace efgs {
// Threads per block of the non-neural backward: 128 for the appearance models, whose rows are staged through LDS
// (a CU holds whole blocks, so halving a block's LDS lets more of the CU's LDS hold rows: SV with 8 sites from 2 to
// 2.5 waves per SIMD, NASG from 3 to 3.5; on the 1M c4 scene SV 192.5 -> 174.7 us, NASG 219.5 -> 212.4 us), 256 for
// precomputed colours. The host launches the kernel with the same count (api.cpp, preprocess_backward_block).
constexpr uint32_t backward_block = EFGS_MODEL >= 1 && EFGS_MODEL <= 4 ? 128u : 256u;
}  // namespace efgs

extern "C" __global__ __launch_bounds__(efgs::backward_block) void EFGS_KERNEL_NAME(efgs::PreprocessBackwardArgs a) {
    using namespace efgs;
#if EFGS_MODEL != 0
    if constexpr (BackwardRows::staged) {
        constexpr uint32_t row_ld = BackwardRows::row_ld, pass_units = BackwardRows::pass_units, n_passes = BackwardRows::n_passes;
        __shared__ float s_rows[backward_block * row_ld];
        const uint32_t p0 = blockIdx.x * backward_block, p = p0 + threadIdx.x;
        const bool active = p < a.n;
        const uint32_t touched = active ? a.n_touched[p] : 0u;
        const uint32_t offset = active ? a.prim_offset[p] : 0u;
        const bool work = touched > 0;
        PrimRecord rec{};
        GeometryInputs gi{};
        InstanceGrads ig{};
        float3 dpre = make_float3(0.0f, 0.0f, 0.0f), d = dpre, dmean_color = dpre;
        float norm_rcp = 0.0f;
        if (work) {
            rec = a.records[p];
            gi = load_geometry(a, p);
            ig = reduce_instance_grads(a, offset, touched);
            dpre = pre_activation_grad(rec, ig);
            write_base_grad(a, p, dpre, make_float3(0.0f, 0.0f, 0.0f));
            const float3 cam = make_float3(a.cam.cam_position[0], a.cam.cam_position[1], a.cam.cam_position[2]);
            d = view_direction(gi.mean, cam, norm_rcp);
        }
        const uint32_t rows = p0 < a.n ? min(backward_block, a.n - p0) : 0u;
        for (uint32_t pass = 0; pass < n_passes; pass++) {
            const uint32_t u0 = pass * pass_units;
            const uint32_t nu = min(pass_units, static_cast<uint32_t>(EFGS_N_UNITS) - u0);
            if (pass > 0) __syncthreads();  // every thread has read the previous pass's rows
            stage_residual_rows<backward_block, row_ld>(a.residual, p0, rows, u0 * params_per_unit, nu * params_per_unit, s_rows);
            __syncthreads();
#if EFGS_MODEL == 1 || EFGS_MODEL == 2
            // (one pass: every coefficient / site of the row) the gradients replace the staged row in place (each
            // parameter is read before its gradient is written) and leave with coalesced stores; the units past the
            // active degree and the rows of primitives without instances get zeros
            float* row = s_rows + threadIdx.x * row_ld;
            if (work) {
#if EFGS_MODEL == 1
                dmean_color = sh_residual_backward<EFGS_RES_ACT>(row, dpre, row, d, norm_rcp, a.cam.degree);
#else
                dmean_color = sv_residual_backward<EFGS_RES_ACT>(row, dpre, row, d, norm_rcp, a.cam.degree);
#endif
            }
            for (uint32_t i = work ? active_residual_params(a.cam.degree) : 0u; i < residual_params; i++) row[i] = 0.0f;
            __syncthreads();
            store_residual_rows<backward_block, row_ld>(s_rows, p0, rows, 0u, residual_params, a.g_residual);
#else
            // lobes: a lobe's parameters are read before its gradients are written, so the gradients replace the
            // staged row in place (zero for inactive lobes and for primitives without instances) and leave with
            // coalesced stores
            float* row = s_rows + threadIdx.x * row_ld;
            const uint32_t na = work && a.cam.degree > u0 ? min(nu, a.cam.degree - u0) : 0u;
            if (work) {
                const float3 dm = lobe_residual_backward<EFGS_RES_ACT, EFGS_MODEL == 4>(row, dpre, row, d, norm_rcp, na);
                dmean_color.x += dm.x;
                dmean_color.y += dm.y;
                dmean_color.z += dm.z;
            }
            for (uint32_t i = na * params_per_unit; i < nu * params_per_unit; i++) row[i] = 0.0f;
            __syncthreads();
            store_residual_rows<backward_block, row_ld>(s_rows, p0, rows, u0 * params_per_unit, nu * params_per_unit, a.g_residual);
#endif
        }
        if (work) {
            geometry_backward(a, p, rec, gi, ig, dmean_color);
        } else if (active) {
            zero_primitive(a, p, false);  // (its residual gradients were stored as zeros with the block's rows)
        }
        return;
    }
#endif
    const uint32_t p = blockIdx.x * backward_block + threadIdx.x;
    if (p >= a.n) return;
    const uint32_t touched = a.n_touched[p];
    const uint32_t offset = a.prim_offset[p];
    if (touched == 0) {
        zero_primitive(a, p);
        return;
    }
    const PrimRecord rec = a.records[p];
    const GeometryInputs gi = load_geometry(a, p);
    const InstanceGrads ig = reduce_instance_grads(a, offset, touched);
    float3 dmean_color = make_float3(0.0f, 0.0f, 0.0f);
#if EFGS_MODEL == 0
    a.g_precomputed[3 * p] = ig.gr; a.g_precomputed[3 * p + 1] = ig.gg; a.g_precomputed[3 * p + 2] = ig.gb;
#else
    {
        const float3 dpre = pre_activation_grad(rec, ig);
        write_base_grad(a, p, dpre, make_float3(0.0f, 0.0f, 0.0f));
        const float3 cam = make_float3(a.cam.cam_position[0], a.cam.cam_position[1], a.cam.cam_position[2]);
        float norm_rcp;
        const float3 d = view_direction(gi.mean, cam, norm_rcp);
        const float* rp = a.residual + static_cast<size_t>(p) * residual_params;
        float* gp = a.g_residual + static_cast<size_t>(p) * residual_params;
#if EFGS_MODEL == 1
        dmean_color = sh_residual_backward<EFGS_RES_ACT>(rp, dpre, gp, d, norm_rcp, a.cam.degree);
#elif EFGS_MODEL == 2
        dmean_color = sv_residual_backward<EFGS_RES_ACT>(rp, dpre, gp, d, norm_rcp, a.cam.degree);
#elif EFGS_MODEL == 3
        dmean_color = lobe_residual_backward<EFGS_RES_ACT, false>(rp, dpre, gp, d, norm_rcp, a.cam.degree);
#elif EFGS_MODEL == 4
        dmean_color = lobe_residual_backward<EFGS_RES_ACT, true>(rp, dpre, gp, d, norm_rcp, a.cam.degree);
#endif
        for (uint32_t i = active_residual_params(a.cam.degree); i < residual_params; i++) gp[i] = 0.0f;
    }
#endif
    geometry_backward(a, p, rec, gi, ig, dmean_color);
}

#else  // neural: a geometry kernel (one thread per primitive) and an MLP kernel

#define EFGS_CAT2(a, b) a##b
#define EFGS_CAT(a, b) EFGS_CAT2(a, b)

// Everything but the MLP: instance-gradient reduction, colour and base gradients, the projection chain. The
// gradient with respect to the pre-activation colour is left in color_grads for the MLP kernel, which adds
// the MLP's view-direction and base-input terms to g_means and g_base and writes the latent gradients.
extern "C" __global__ __launch_bounds__(256) void EFGS_KERNEL_NAME(efgs::PreprocessBackwardArgs a) {
    using namespace efgs;
    __shared__ uint32_t s_max;
    if (threadIdx.x == 0) s_max = 0u;
    __syncthreads();
    const uint32_t p = blockIdx.x * preprocess_block + threadIdx.x;
    float m = 0.0f;
    if (p < a.n) {
        const uint32_t touched = a.n_touched[p];
        const uint32_t offset = a.prim_offset[p];
        if (touched == 0) {
            zero_primitive(a, p);
        } else {
            const PrimRecord rec = a.records[p];
            const GeometryInputs gi = load_geometry(a, p);
            const InstanceGrads ig = reduce_instance_grads(a, offset, touched);
            const float3 dpre = pre_activation_grad(rec, ig);
            write_base_grad(a, p, dpre, make_float3(0.0f, 0.0f, 0.0f));
            if (a.cam.degree == 0)
                for (uint32_t i = 0; i < residual_params; i++) a.g_residual[static_cast<size_t>(p) * residual_params + i] = 0.0f;
            geometry_backward(a, p, rec, gi, ig, make_float3(0.0f, 0.0f, 0.0f));
            reinterpret_cast<float4*>(a.color_grads)[p] = make_float4(dpre.x, dpre.y, dpre.z, 0.0f);
            m = fmaxf(fmaxf(fabsf(dpre.x), fabsf(dpre.y)), fabsf(dpre.z));
        }
    }
    // bound for the MLP kernel's gradient scale: the residual activations' derivatives are at most 1, so
    // |dL/d(MLP output)| <= max |dpre|; non-negative float bits order like the floats (integer max)
    m = __uint_as_float(wave_max_bits(__float_as_uint(m), [](uint32_t x, uint32_t y) { return __float_as_uint(fmaxf(__uint_as_float(x), __uint_as_float(y))); }));
    if ((threadIdx.x & 63u) == 0) atomicMax(&s_max, __float_as_uint(m));
    __syncthreads();
    if (threadIdx.x == 0) a.color_grad_max[blockIdx.x] = s_max;
}

// The MLP backward (launched only when the residual is on). Persistent grid: every wave recomputes the MLP
// forward for its 64 primitives and backpropagates it with fp16 MFMA, keeps its weight gradients in fp32
// registers across chunks; the block sums its four waves in a fixed order into one partial per block.
// Two waves per SIMD: the weight-gradient accumulators and one pass's activations fit 256 VGPRs.
extern "C" __global__ __launch_bounds__(256, 2) void EFGS_CAT(EFGS_KERNEL_NAME, _mlp)(efgs::PreprocessBackwardArgs a) {
    using namespace efgs;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    extern __shared__ __align__(16) unsigned char smem[];
    const _Float16* WL = reinterpret_cast<const _Float16*>(smem);
    _Float16* stage = reinterpret_cast<_Float16*>(smem + nn::WEIGHT_BYTES + wave * nn::STAGE_BYTES);
    nn::load_weights<preprocess_block>(a.mlp_weights, reinterpret_cast<uint16_t*>(smem), threadIdx.x);
    __syncthreads();

    nn::f4 dW[nn::NL][nn::NT][nn::KT];
#pragma unroll
    for (uint32_t l = 0; l < nn::NL; l++)
#pragma unroll
        for (uint32_t rb = 0; rb < nn::NT; rb++)
#pragma unroll
            for (uint32_t cb = 0; cb < nn::KT; cb++) dW[l][rb][cb] = nn::f4_zero();

    const uint32_t degree = a.cam.degree;
    // one gradient scale for the launch: 2^(8 - e) with e the exponent of the largest |dL/d(MLP output)| bound
    // (every block reduces the geometry kernel's per-block maxima itself: a few loads per thread)
    __shared__ uint32_t s_wave_max[preprocess_block / 64];
    {
        const uint32_t n_geometry_blocks = (a.n + preprocess_block - 1) / preprocess_block;
        // 16-byte loads, four per thread in flight (one round for up to 4,096 geometry blocks; the array sits 16 n
        // bytes after the 16-byte aligned colour gradients), then the last few entries one by one
        uint32_t m = 0u;
        const uint32_t n4 = n_geometry_blocks / 4;
        const uint4* const bounds4 = reinterpret_cast<const uint4*>(a.color_grad_max);
        for (uint32_t q0 = 0; q0 < n4; q0 += 4 * preprocess_block) {
            uint4 v[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; k++) {
                const uint32_t q = q0 + k * preprocess_block + threadIdx.x;
                v[k] = q < n4 ? bounds4[q] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (uint32_t k = 0; k < 4; k++) m = max(m, max(max(v[k].x, v[k].y), max(v[k].z, v[k].w)));
        }
        for (uint32_t b = 4 * n4 + threadIdx.x; b < n_geometry_blocks; b += preprocess_block) m = max(m, a.color_grad_max[b]);
        m = wave_max_bits(m, [](uint32_t x, uint32_t y) { return max(x, y); });
        if (lane == 0) s_wave_max[wave] = m;
        __syncthreads();
    }
    uint32_t gbits = 0u;
#pragma unroll
    for (uint32_t w = 0; w < preprocess_block / 64; w++) gbits = max(gbits, s_wave_max[w]);
    const float gmax = __uint_as_float(gbits);
    // (scale 1 when the bound is zero or not finite: non-finite gradients then propagate as they are)
    const bool finite = gmax > 0.0f && gmax < 3.0e38f;
    const int e = finite ? max(ilogbf(gmax), -110) : 8;  // the clamp keeps 2^(8 - e) finite for denormal maxima
    const float s = ldexpf(1.0f, 8 - e), inv_s = ldexpf(1.0f, e - 8);
    // work list: the visible primitives in index order (every other primitive's MLP gradients are zero), so
    // the MFMA tiles are full and the gathers nearly contiguous. A chunk's inputs are loaded during the chunk before
    // it, and its primitive indices two chunks ahead, so no chunk waits on a load of its own.
    const uint32_t n_chunks = (a.n_visible + preprocess_block - 1) / preprocess_block;
    struct ChunkInputs {
        uint32_t p;
        float4 dpre;      // upstream gradient of the activated colour (zero past the list)
        float3 mean, gm, gb;  // the mean; the geometry kernel's mean and base gradients, which this chunk adds to
        float feat[nn::FEATURES > 0 ? nn::FEATURES : 1], base[3];
    };
    // (chunks past the list read entry 0: the list is not empty when a chunk is processed)
    const auto prim_of = [&](uint32_t chunk) {
        const uint32_t v_idx = chunk * preprocess_block + threadIdx.x;
        return a.visible_prims[v_idx < a.n_visible ? v_idx : 0u];
    };
    const auto load_inputs = [&](uint32_t chunk, uint32_t p, ChunkInputs& in) {
        const bool contributes = chunk * preprocess_block + threadIdx.x < a.n_visible;
        in.p = p;
        in.dpre = contributes ? reinterpret_cast<const float4*>(a.color_grads)[p] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        in.mean = make_float3(a.means[3 * p], a.means[3 * p + 1], a.means[3 * p + 2]);
        in.gm = EFGS_DIRECTION_GRADIENT ? make_float3(a.g_means[3 * p], a.g_means[3 * p + 1], a.g_means[3 * p + 2]) : make_float3(0.0f, 0.0f, 0.0f);
        in.gb = EFGS_BASE_INPUT ? make_float3(a.g_base[3 * p], a.g_base[3 * p + 1], a.g_base[3 * p + 2]) : make_float3(0.0f, 0.0f, 0.0f);
        const float* feat = a.residual + static_cast<size_t>(p) * residual_params;
#pragma unroll
        for (uint32_t i = 0; i < nn::FEATURES; i++) in.feat[i] = feat[i];
#pragma unroll
        for (uint32_t c = 0; c < 3; c++) in.base[c] = EFGS_BASE_INPUT ? a.base[3 * p + c] : 0.0f;
    };
    const float3 cam = make_float3(a.cam.cam_position[0], a.cam.cam_position[1], a.cam.cam_position[2]);
    ChunkInputs next_in;
    uint32_t p_after = 0u;
    if (blockIdx.x < n_chunks) {
        load_inputs(blockIdx.x, prim_of(blockIdx.x), next_in);
        p_after = prim_of(blockIdx.x + gridDim.x);
    }
    for (uint32_t chunk = blockIdx.x; chunk < n_chunks; chunk += gridDim.x) {
        const ChunkInputs in = next_in;  // (loaded during the previous chunk)
        const uint32_t later = chunk + gridDim.x;
        if (later < n_chunks) {
            load_inputs(later, p_after, next_in);
            p_after = prim_of(later + gridDim.x);
        }
        const uint32_t v_idx = chunk * preprocess_block + threadIdx.x;
        const bool contributes = v_idx < a.n_visible;
        if (__ballot(contributes) == 0) continue;  // wave-uniform: the tail of the list
        const uint32_t p = in.p;
        float norm_rcp;
        const float3 d = view_direction(in.mean, cam, norm_rcp);
        float x[nn::INP];
        nn::mlp_input(in.feat, in.base, d, degree, x);
        if (!contributes) {
#pragma unroll
            for (uint32_t k = 0; k < nn::INP; k++) x[k] = 0.0f;
        }
        const float g[3] = {in.dpre.x, in.dpre.y, in.dpre.z};
        float dx[nn::INP];
        nn::mlp_train(WL, stage, x, g, [](float y, float gy) { return gy * nn::residual_activation_slope<EFGS_RES_ACT>(y); }, s, inv_s, dx,
                      dW, lane);
        if (contributes) {
            float* gp = a.g_residual + static_cast<size_t>(p) * residual_params;
#pragma unroll
            for (uint32_t i = 0; i < nn::FEATURES; i++) gp[i] = nn::feature_grad(in.feat[i], dx, i);
            if (EFGS_BASE_INPUT) {
                a.g_base[3 * p] = in.gb.x + nn::feature_grad(in.base[0], dx, nn::FEATURES);
                a.g_base[3 * p + 1] = in.gb.y + nn::feature_grad(in.base[1], dx, nn::FEATURES + 1);
                a.g_base[3 * p + 2] = in.gb.z + nn::feature_grad(in.base[2], dx, nn::FEATURES + 2);
            }
            if (EFGS_DIRECTION_GRADIENT) {
                const float3 dm = direction_grad_to_mean(nn::direction_grad(d, degree, dx), d, norm_rcp);
                a.g_means[3 * p] = in.gm.x + dm.x;
                a.g_means[3 * p + 1] = in.gm.y + dm.y;
                a.g_means[3 * p + 2] = in.gm.z + dm.z;
            }
        }
    }

    // block sum of the four waves' weight gradients, in wave order, then one partial per block
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    const uint32_t r = lane & 15u, q = lane >> 4;
    for (uint32_t w = 0; w < preprocess_block / 64; w++) {
        if (wave == w) {
#pragma unroll
            for (uint32_t l = 0; l < nn::NL; l++)
#pragma unroll
                for (uint32_t rb = 0; rb < nn::lout(l) / 16; rb++)
#pragma unroll
                    for (uint32_t cb = 0; cb < nn::lin(l) / 16; cb++)
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++) {
                            const uint32_t idx = nn::loff(l) + (rb * 16 + 4 * q + i) * nn::lin(l) + cb * 16 + r;
                            red[idx] = (w == 0 ? 0.0f : red[idx]) + dW[l][rb][cb][i] * inv_s;
                        }
        }
        __syncthreads();
    }
    float* out = a.g_mlp_partials + static_cast<size_t>(blockIdx.x) * nn::PARAMS;
    for (uint32_t i = threadIdx.x; i < nn::PARAMS; i += preprocess_block) out[i] = red[i];
}

#endif
