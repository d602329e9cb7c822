// Standalone neural decode: the configured residual MLP on per-primitive features and unit view directions,
// outside the rasterizer (tokens as the neural preprocess kernels: EFGS_KERNEL_NAME, the MLP shape, the
// feature encoding and the SH degree mask). Inputs are encoded exactly as in the preprocess kernels (frequency
// encoding of the features, optional base colour input, SH degree values of the direction), so the decode
// computes the raw MLP outputs that the rasterizer adds (after the residual activation) to the base colour.
// With no SH degree and no frequency encoding the input rows are the features as they are (the identity-encoded
// network of the tiny-cuda-nn surface): directions are then neither read nor differentiated.
//
//   EFGS_KERNEL_NAME            forward: out = MLP(x), fp16 MFMA with fp32 accumulation, outputs rounded to
//                               fp16 (one wave per 64 primitives, persistent grid, weights in LDS)
//   EFGS_KERNEL_NAME_backward   recomputes the forward and backpropagates
//                               grad_out: feature, base-input and direction gradients per primitive, weight
//                               gradients as one fp32 partial per block (reduced by reduce_partials_kernel)
//
// Reference: the tiny-cuda-nn JIT MLP the reference calls per primitive (eval_model / backward_eval_model,
// B/rasterization/rtc/appearance_neural.cuh:308-407), here as a kernel of its own so that the decode can be
// measured and tested in isolation.
#define EFGS_CAT2(a, b) a##b
#define EFGS_CAT(a, b) EFGS_CAT2(a, b)

namespace efgs {
constexpr uint32_t decode_block = 256;
}  // namespace efgs

// (at least two waves per SIMD: a budget of 256 VGPRs, within which the compiler keeps MFMA results in VGPRs
// instead of accumulation registers that every result tile would have to be copied back from)
extern "C" __global__ __launch_bounds__(256, 2) void EFGS_KERNEL_NAME(efgs::NeuralDecodeArgs a) {
    using namespace efgs;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    extern __shared__ __align__(16) unsigned char smem[];
    const _Float16* WL = reinterpret_cast<const _Float16*>(smem);
    _Float16* stage = reinterpret_cast<_Float16*>(smem + nn::WEIGHT_BYTES) + wave * 64 * nn::XS;
    nn::load_weights<decode_block>(a.mlp_weights, reinterpret_cast<uint16_t*>(smem), threadIdx.x);
    __syncthreads();
    const uint32_t n_chunks = (a.n + decode_block - 1) / decode_block;
    // the lane's raw inputs (features, base colour, direction) of its primitive in the block's next chunk, loaded
    // one chunk ahead so that the loads are in flight during the current chunk's MLP
    constexpr uint32_t NB = EFGS_BASE_INPUT ? 3u : 0u;
    constexpr bool has_dirs = EFGS_SH_DEGREE_MASK != 0;  // without SH degrees the inputs are the features alone (no direction read)
    float nf[nn::FEATURES + NB + 3];
    const auto load_inputs = [&](uint32_t chunk) {
        const uint32_t p = chunk * decode_block + threadIdx.x;
        if (chunk < n_chunks && p < a.n) {
#pragma unroll
            for (uint32_t i = 0; i < nn::FEATURES; i++) nf[i] = a.features[static_cast<size_t>(p) * nn::FEATURES + i];
#pragma unroll
            for (uint32_t i = 0; i < NB; i++) nf[nn::FEATURES + i] = a.base[3 * static_cast<size_t>(p) + i];
#pragma unroll
            for (uint32_t i = 0; i < 3; i++) nf[nn::FEATURES + NB + i] = has_dirs ? a.dirs[3 * static_cast<size_t>(p) + i] : 0.0f;
        }
    };
    load_inputs(blockIdx.x);
    for (uint32_t chunk = blockIdx.x; chunk < n_chunks; chunk += gridDim.x) {
        const uint32_t p = chunk * decode_block + threadIdx.x;
        const bool active = p < a.n;
        float cf[nn::FEATURES + NB + 3];
#pragma unroll
        for (uint32_t i = 0; i < nn::FEATURES + NB + 3; i++) cf[i] = nf[i];
        load_inputs(chunk + gridDim.x);
        if (__ballot(active) == 0) continue;  // wave-uniform: the tail of the last chunk
        float x[nn::INP];
        if (active) {
            const float3 d = make_float3(cf[nn::FEATURES + NB], cf[nn::FEATURES + NB + 1], cf[nn::FEATURES + NB + 2]);
            nn::mlp_input(cf, EFGS_BASE_INPUT ? cf + nn::FEATURES : nullptr, d, a.degree, x);
        } else {
#pragma unroll
            for (uint32_t k = 0; k < nn::INP; k++) x[k] = 0.0f;
        }
        float y[3];
        nn::mlp_forward(WL, stage, x, y, lane);
        if (active) {
            a.out[3 * p] = y[0];
            a.out[3 * p + 1] = y[1];
            a.out[3 * p + 2] = y[2];
        }
    }
}

extern "C" __global__ __launch_bounds__(256, 2) void EFGS_CAT(EFGS_KERNEL_NAME, _backward)(efgs::NeuralDecodeArgs a) {
    using namespace efgs;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    extern __shared__ __align__(16) unsigned char smem[];
    const _Float16* WL = reinterpret_cast<const _Float16*>(smem);
    _Float16* stage = reinterpret_cast<_Float16*>(smem + nn::WEIGHT_BYTES + wave * nn::STAGE_BYTES);
    nn::load_weights<decode_block>(a.mlp_weights, reinterpret_cast<uint16_t*>(smem), threadIdx.x);

    nn::f4 dW[nn::NL][nn::NT][nn::KT];
#pragma unroll
    for (uint32_t l = 0; l < nn::NL; l++)
#pragma unroll
        for (uint32_t rb = 0; rb < nn::NT; rb++)
#pragma unroll
            for (uint32_t cb = 0; cb < nn::KT; cb++) dW[l][rb][cb] = nn::f4_zero();

    // one gradient scale per block: 2^(8 - e) with e the exponent of the largest |grad_out| among the
    // block's primitives (its chunks are read once here, 8 loads in flight per thread)
    const uint32_t n_chunks = (a.n + decode_block - 1) / decode_block;
    __shared__ float s_wave_max[decode_block / 64];
    {
        float m = 0.0f;
        for (uint32_t c0 = blockIdx.x; c0 < n_chunks; c0 += 8 * gridDim.x) {
            float v[8];
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) {
                const uint32_t c = c0 + k * gridDim.x;
                const uint32_t p = c * decode_block + threadIdx.x;
                v[k] = c < n_chunks && p < a.n
                           ? fmaxf(fmaxf(fabsf(a.grad_out[3 * p]), fabsf(a.grad_out[3 * p + 1])), fabsf(a.grad_out[3 * p + 2]))
                           : 0.0f;
            }
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) m = fmaxf(m, v[k]);
        }
        // the wave's maximum without LDS permutes: four row rotations (DPP), then two lane swaps across the rows
        const auto fmax_bits = [](uint32_t x, uint32_t y) { return __float_as_uint(fmaxf(__uint_as_float(x), __uint_as_float(y))); };
        uint32_t mb = __float_as_uint(m);
        mb = fmax_bits(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x121, 0xf, 0xf, false)));  // row_ror:1
        mb = fmax_bits(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x122, 0xf, 0xf, false)));  // row_ror:2
        mb = fmax_bits(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x124, 0xf, 0xf, false)));  // row_ror:4
        mb = fmax_bits(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x128, 0xf, 0xf, false)));  // row_ror:8
        const auto sa = __builtin_amdgcn_permlane32_swap(mb, mb, false, false);
        mb = fmax_bits(sa[0], sa[1]);
        const auto sb = __builtin_amdgcn_permlane16_swap(mb, mb, false, false);
        m = __uint_as_float(fmax_bits(sb[0], sb[1]));
        if (lane == 0) s_wave_max[wave] = m;
    }
    __syncthreads();  // weights staged, wave maxima written
    float gmax = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < decode_block / 64; w++) gmax = fmaxf(gmax, s_wave_max[w]);
    // (scale 1 when the bound is zero or not finite: non-finite gradients then propagate as they are)
    const bool finite = gmax > 0.0f && gmax < 3.0e38f;
    const int e = finite ? max(ilogbf(gmax), -110) : 8;  // the clamp keeps 2^(8 - e) finite for denormal maxima
    const float s = ldexpf(1.0f, 8 - e), inv_s = ldexpf(1.0f, e - 8);

    // a chunk's inputs (direction, features, base colour, upstream gradient) are loaded during the chunk before it
    constexpr bool has_dirs = EFGS_SH_DEGREE_MASK != 0;  // without SH degrees no direction is read or differentiated
    constexpr uint32_t NB = EFGS_BASE_INPUT ? 3u : 0u;
    struct ChunkInputs {
        float3 d;
        float feat[nn::FEATURES > 0 ? nn::FEATURES : 1], base[3], g[3];
    };
    const auto load_inputs = [&](uint32_t chunk, ChunkInputs& in) {
        const uint32_t p = chunk * decode_block + threadIdx.x;
        const bool active = p < a.n;
        const uint32_t pp = active ? p : 0u;
        in.d = has_dirs ? make_float3(a.dirs[3 * pp], a.dirs[3 * pp + 1], a.dirs[3 * pp + 2]) : make_float3(0.0f, 0.0f, 0.0f);
#pragma unroll
        for (uint32_t i = 0; i < nn::FEATURES; i++) in.feat[i] = a.features[static_cast<size_t>(pp) * nn::FEATURES + i];
#pragma unroll
        for (uint32_t c = 0; c < 3; c++) in.base[c] = c < NB ? a.base[3 * static_cast<size_t>(pp) + c] : 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < 3; c++) in.g[c] = active ? a.grad_out[3 * static_cast<size_t>(p) + c] : 0.0f;
    };
    ChunkInputs next_in;
    if (blockIdx.x < n_chunks) load_inputs(blockIdx.x, next_in);
    for (uint32_t chunk = blockIdx.x; chunk < n_chunks; chunk += gridDim.x) {
        const ChunkInputs in = next_in;  // (loaded during the previous chunk)
        if (chunk + gridDim.x < n_chunks) load_inputs(chunk + gridDim.x, next_in);
        const uint32_t p = chunk * decode_block + threadIdx.x;
        const bool active = p < a.n;
        if (__ballot(active) == 0) continue;  // wave-uniform: the tail of the last chunk
        const float3 d = in.d;
        float x[nn::INP];
        nn::mlp_input(in.feat, in.base, d, a.degree, x);
        if (!active) {
#pragma unroll
            for (uint32_t k = 0; k < nn::INP; k++) x[k] = 0.0f;
        }
        const float g[3] = {in.g[0], in.g[1], in.g[2]};
        float dx[nn::INP];
        nn::mlp_train(WL, stage, x, g, [](float, float gy) { return gy; }, s, inv_s, dx, dW, lane);
        if (active) {
            float* gf = a.g_features + static_cast<size_t>(p) * nn::FEATURES;
#pragma unroll
            for (uint32_t i = 0; i < nn::FEATURES; i++) gf[i] = nn::feature_grad(in.feat[i], dx, i);
            if (EFGS_BASE_INPUT && a.g_base) {
#pragma unroll
                for (uint32_t c = 0; c < 3; c++) a.g_base[3 * p + c] = nn::feature_grad(in.base[c], dx, nn::FEATURES + c);
            }
            if (has_dirs && a.g_dirs) {
                const float3 gd = nn::direction_grad(d, a.degree, dx);
                a.g_dirs[3 * p] = gd.x;
                a.g_dirs[3 * p + 1] = gd.y;
                a.g_dirs[3 * p + 2] = gd.z;
            }
        }
    }

    // block sum of the four waves' weight gradients, in wave order, then one partial per block
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    const uint32_t r = lane & 15u, q = lane >> 4;
    for (uint32_t w = 0; w < decode_block / 64; w++) {
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
    for (uint32_t i = threadIdx.x; i < nn::PARAMS; i += decode_block) out[i] = red[i];
}
