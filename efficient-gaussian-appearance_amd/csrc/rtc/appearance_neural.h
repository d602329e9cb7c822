// Neural residual (EFGS_MODEL == 5): a bias-free ReLU MLP over per-Gaussian features (optionally frequency
// encoded, optionally with the base colour as 3 extra inputs) and the SH degree values of the view
// direction, evaluated per wave of 64 primitives with fp16 MFMA (v_mfma_f32_16x16x16f16) and fp32
// accumulation; weights live in LDS in the tcnn flat layout (row-major [out x in] per layer, input padded to
// a multiple of 16, output padded to 16 rows).
//
// Layout: each layer computes H_out^T = W H_in^T with the weights as the A operand and the activations as the
// B operand, so a 16x16 accumulator tile (lane l: rows 4(l/16)..+3, column l%16) is exactly the B fragment
// of the next layer's matching k-block: no data movement between layers. Activations are rounded to fp16
// between layers (as tcnn's half-precision network), the 3 outputs are rounded to fp16.
//
// Backward: the forward is recomputed (no stored context). The upstream gradient of the wave is scaled by a
// power of two so its maximum lies in [256, 512) before the fp16 MFMA chain, and unscaled in fp32. Weight
// gradients dW = G X accumulate per wave in fp32 registers (operands transposed through LDS), then are reduced
// across the block's waves in a fixed order.
//
// Reference: B/rasterization/rtc/appearance_neural.cuh:17-407 (encoding, SH degree values and their
// gradient, tcnn eval_model / backward_eval_model at :333, :379); weight layout viewer/export_ngsplat.py:1013-1029.
#pragma once

namespace efgs {

namespace nn {

#ifndef EFGS_MLP_U_LDS
#define EFGS_MLP_U_LDS 0
#endif
constexpr uint32_t IN = EFGS_MLP_N_IN;            // unpadded input width
constexpr uint32_t INP = EFGS_MLP_N_IN_PADDED;    // padded to a multiple of 16
constexpr uint32_t NN = EFGS_MLP_N_NEURONS;
constexpr uint32_t NH = EFGS_MLP_N_HIDDEN;
constexpr uint32_t NL = NH + 1;                   // weight matrices
constexpr uint32_t OUTP = 16;
constexpr uint32_t MAXK = INP > NN ? INP : NN;
constexpr uint32_t KT = MAXK / 16;
constexpr uint32_t NT = NN / 16;
constexpr uint32_t FEATURES = EFGS_N_UNITS;
constexpr uint32_t RAW_FEATURES = FEATURES + (EFGS_BASE_INPUT ? 3u : 0u);
constexpr uint32_t ENCODED = EFGS_N_FREQUENCIES == 0 ? RAW_FEATURES : RAW_FEATURES * 2u * EFGS_N_FREQUENCIES;
constexpr uint32_t PARAMS = NN * INP + (NH - 1) * NN * NN + OUTP * NN;

__host__ __device__ constexpr uint32_t lin(uint32_t l) { return l == 0 ? INP : NN; }
__host__ __device__ constexpr uint32_t lout(uint32_t l) { return l == NH ? OUTP : NN; }
__host__ __device__ constexpr uint32_t loff(uint32_t l) { return l == 0 ? 0u : NN * INP + (l - 1) * NN * NN; }

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ f4 f4_zero() { return f4{0.0f, 0.0f, 0.0f, 0.0f}; }
__device__ __forceinline__ float round_half(float v) { return static_cast<float>(static_cast<_Float16>(v)); }
__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront"); __builtin_amdgcn_wave_barrier(); __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront"); }

// forward-mode dual number (value and d/dx, d/dy, d/dz of the direction) for the SH degree derivatives
struct D3 {
    float v, x, y, z;
};
__device__ __forceinline__ D3 operator+(D3 a, D3 b) { return {a.v + b.v, a.x + b.x, a.y + b.y, a.z + b.z}; }
__device__ __forceinline__ D3 operator-(D3 a, D3 b) { return {a.v - b.v, a.x - b.x, a.y - b.y, a.z - b.z}; }
__device__ __forceinline__ D3 operator-(D3 a) { return {-a.v, -a.x, -a.y, -a.z}; }
__device__ __forceinline__ D3 operator*(D3 a, D3 b) { return {a.v * b.v, a.x * b.v + a.v * b.x, a.y * b.v + a.v * b.y, a.z * b.v + a.v * b.z}; }
__device__ __forceinline__ D3 operator*(float s, D3 a) { return {s * a.v, s * a.x, s * a.y, s * a.z}; }
__device__ __forceinline__ D3 operator*(D3 a, float s) { return s * a; }
__device__ __forceinline__ D3 operator+(D3 a, float s) { return {a.v + s, a.x, a.y, a.z}; }
__device__ __forceinline__ D3 operator-(D3 a, float s) { return {a.v - s, a.x, a.y, a.z}; }
__device__ __forceinline__ D3 operator-(float s, D3 a) { return {s - a.v, -a.x, -a.y, -a.z}; }
__device__ __forceinline__ float sh_value(float v) { return v; }
__device__ __forceinline__ float sh_value(D3 v) { return v.v; }

constexpr float sh_c0 = 0.28209479177387814f;

// SH degree values of the direction for the degrees of EFGS_SH_DEGREE_MASK (ascending); degree 0 is never
// gated, the i-th degree >= 1 is zero unless i < active_degree. emit(index, value) receives every value.
template <typename T, typename EMIT>
__device__ inline void sh_degree_values(T x, T y, T z, uint32_t active_degree, EMIT&& emit) {
    constexpr uint32_t mask = EFGS_SH_DEGREE_MASK;
    const T xy = x * y, xz = x * z, yz = y * z, x2 = x * x, y2 = y * y, z2 = z * z;
    const T x4 = x2 * x2, y4 = y2 * y2, z4 = z2 * z2;
    const T x6 = x4 * x2, y6 = y4 * y2, z6 = z4 * z2;
    uint32_t o = 0, rank = 0;
    if (mask & 1u) { emit(o, T{} + sh_c0); o += 1; }
    if (mask & 2u) {
        const float m = rank++ < active_degree ? 1.0f : 0.0f;
        emit(o + 0, m * (-0.48860251190291987f * y)); emit(o + 1, m * (0.48860251190291987f * z)); emit(o + 2, m * (-0.48860251190291987f * x));
        o += 3;
    }
    if (mask & 4u) {
        const float m = rank++ < active_degree ? 1.0f : 0.0f;
        emit(o + 0, m * (1.0925484305920792f * xy)); emit(o + 1, m * (-1.0925484305920792f * yz));
        emit(o + 2, m * (0.94617469575755997f * z2 - 0.31539156525251999f)); emit(o + 3, m * (-1.0925484305920792f * xz));
        emit(o + 4, m * (0.54627421529603959f * x2 - 0.54627421529603959f * y2));
        o += 5;
    }
    if (mask & 8u) {
        const float m = rank++ < active_degree ? 1.0f : 0.0f;
        emit(o + 0, m * (0.59004358992664352f * y * (-3.0f * x2 + y2))); emit(o + 1, m * (2.8906114426405538f * xy * z));
        emit(o + 2, m * (0.45704579946446572f * y * (1.0f - 5.0f * z2))); emit(o + 3, m * (0.3731763325901154f * z * (5.0f * z2 - 3.0f)));
        emit(o + 4, m * (0.45704579946446572f * x * (1.0f - 5.0f * z2))); emit(o + 5, m * (1.4453057213202769f * z * (x2 - y2)));
        emit(o + 6, m * (0.59004358992664352f * x * (-x2 + 3.0f * y2)));
        o += 7;
    }
    if (mask & 16u) {
        const float m = rank++ < active_degree ? 1.0f : 0.0f;
        emit(o + 0, m * (2.5033429417967046f * xy * (x2 - y2))); emit(o + 1, m * (1.7701307697799304f * yz * (-3.0f * x2 + y2)));
        emit(o + 2, m * (0.94617469575756008f * xy * (7.0f * z2 - 1.0f))); emit(o + 3, m * (0.66904654355728921f * yz * (3.0f - 7.0f * z2)));
        emit(o + 4, m * (-3.1735664074561294f * z2 + 3.7024941420321507f * z4 + 0.31735664074561293f));
        emit(o + 5, m * (0.66904654355728921f * xz * (3.0f - 7.0f * z2))); emit(o + 6, m * (0.47308734787878004f * (x2 - y2) * (7.0f * z2 - 1.0f)));
        emit(o + 7, m * (1.7701307697799304f * xz * (-x2 + 3.0f * y2)));
        emit(o + 8, m * (-3.7550144126950569f * x2 * y2 + 0.62583573544917614f * x4 + 0.62583573544917614f * y4));
        o += 9;
    }
    if (mask & 32u) {
        const float m = rank++ < active_degree ? 1.0f : 0.0f;
        emit(o + 0, m * (0.65638205684017015f * y * (10.0f * x2 * y2 - 5.0f * x4 - y4))); emit(o + 1, m * (8.3026492595241645f * xy * z * (x2 - y2)));
        emit(o + 2, m * (-0.48923829943525038f * y * (3.0f * x2 - y2) * (9.0f * z2 - 1.0f)));
        emit(o + 3, m * (4.7935367849733241f * xy * z * (3.0f * z2 - 1.0f)));
        emit(o + 4, m * (0.45294665119569694f * y * (14.0f * z2 - 21.0f * z4 - 1.0f)));
        emit(o + 5, m * (0.1169503224534236f * z * (-70.0f * z2 + 63.0f * z4 + 15.0f)));
        emit(o + 6, m * (0.45294665119569694f * x * (14.0f * z2 - 21.0f * z4 - 1.0f)));
        emit(o + 7, m * (2.3967683924866621f * z * (x2 - y2) * (3.0f * z2 - 1.0f)));
        emit(o + 8, m * (-0.48923829943525038f * x * (x2 - 3.0f * y2) * (9.0f * z2 - 1.0f)));
        emit(o + 9, m * (2.0756623148810411f * z * (-6.0f * x2 * y2 + x4 + y4)));
        emit(o + 10, m * (0.65638205684017015f * x * (10.0f * x2 * y2 - x4 - 5.0f * y4)));
        o += 11;
    }
    if (mask & 64u) {
        const float m = rank++ < active_degree ? 1.0f : 0.0f;
        emit(o + 0, m * (1.3663682103838286f * xy * (-10.0f * x2 * y2 + 3.0f * x4 + 3.0f * y4)));
        emit(o + 1, m * (2.3666191622317521f * yz * (10.0f * x2 * y2 - 5.0f * x4 - y4)));
        emit(o + 2, m * (2.0182596029148963f * xy * (x2 - y2) * (11.0f * z2 - 1.0f)));
        emit(o + 3, m * (-0.92120525951492349f * yz * (3.0f * x2 - y2) * (11.0f * z2 - 3.0f)));
        emit(o + 4, m * (0.92120525951492349f * xy * (-18.0f * z2 + 33.0f * z4 + 1.0f)));
        emit(o + 5, m * (0.58262136251873131f * yz * (30.0f * z2 - 33.0f * z4 - 5.0f)));
        emit(o + 6, m * (6.6747662381009842f * z2 - 20.024298714302954f * z4 + 14.684485723822165f * z6 - 0.31784601133814211f));
        emit(o + 7, m * (0.58262136251873131f * xz * (30.0f * z2 - 33.0f * z4 - 5.0f)));
        emit(o + 8, m * (0.46060262975746175f * (x2 - y2) * (11.0f * z2 * (3.0f * z2 - 1.0f) - 7.0f * z2 + 1.0f)));
        emit(o + 9, m * (-0.92120525951492349f * xz * (x2 - 3.0f * y2) * (11.0f * z2 - 3.0f)));
        emit(o + 10, m * (0.50456490072872406f * (11.0f * z2 - 1.0f) * (-6.0f * x2 * y2 + x4 + y4)));
        emit(o + 11, m * (2.3666191622317521f * xz * (10.0f * x2 * y2 - x4 - 5.0f * y4)));
        emit(o + 12, m * (10.247761577878714f * x2 * y4 - 10.247761577878714f * x4 * y2 + 0.6831841051919143f * x6 - 0.6831841051919143f * y6));
        o += 13;
    }
}

// raw feature i of a primitive: learned features, then (with base input) the 3 base values
__device__ __forceinline__ float raw_feature(const float* feat, const float* base, uint32_t i) {
    return i < FEATURES ? feat[i] : base[i - FEATURES];
}

// the lane's MLP input row (INP floats, zero padded): encoded features, then the direction's SH degree values
__device__ inline void mlp_input(const float* feat, const float* base, float3 d, uint32_t degree, float* x) {
#pragma unroll
    for (uint32_t k = 0; k < INP; k++) x[k] = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < RAW_FEATURES; i++) {
        const float v = raw_feature(feat, base, i);
        if (EFGS_N_FREQUENCIES == 0) {
            x[i] = v;
        } else {
#pragma unroll
            for (uint32_t f = 0; f < EFGS_N_FREQUENCIES; f++) {
                float s, c;
                sincosf(ldexpf(v, static_cast<int>(f)), &s, &c);
                x[i * 2 * EFGS_N_FREQUENCIES + 2 * f] = s;
                x[i * 2 * EFGS_N_FREQUENCIES + 2 * f + 1] = c;
            }
        }
    }
    sh_degree_values(d.x, d.y, d.z, degree, [&](uint32_t k, float v) { x[ENCODED + k] = v; });
}

// d(loss)/d(raw feature i) from the input gradient row (frequency encoding chain)
__device__ inline float feature_grad(float v, const float* dx, uint32_t i) {
    if (EFGS_N_FREQUENCIES == 0) return dx[i];
    float g = 0.0f;
#pragma unroll
    for (uint32_t f = 0; f < EFGS_N_FREQUENCIES; f++) {
        float s, c;
        sincosf(ldexpf(v, static_cast<int>(f)), &s, &c);
        g += static_cast<float>(1u << f) * (c * dx[i * 2 * EFGS_N_FREQUENCIES + 2 * f] - s * dx[i * 2 * EFGS_N_FREQUENCIES + 2 * f + 1]);
    }
    return g;
}

// d(loss)/d(direction) through the SH degree values (forward-mode duals)
__device__ inline float3 direction_grad(float3 d, uint32_t degree, const float* dx) {
    const D3 X{d.x, 1.0f, 0.0f, 0.0f}, Y{d.y, 0.0f, 1.0f, 0.0f}, Z{d.z, 0.0f, 0.0f, 1.0f};
    float3 g = make_float3(0.0f, 0.0f, 0.0f);
    sh_degree_values(X, Y, Z, degree, [&](uint32_t k, D3 v) {
        const float w = dx[ENCODED + k];
        g.x += w * v.x;
        g.y += w * v.y;
        g.z += w * v.z;
    });
    return g;
}

// ---- dual-orientation MLP of the backward kernel --------------------------------------------------------
//
// Tile sets of a (F x 64 primitives) matrix M held by a wave (lane = r + 16 q):
//   feature-rows    T[fb][pb]: lane (r, q) holds M[16 fb + 4 q + i][16 pb + r], i = 0..3
//   primitive-rows  U[pb][fb]: lane (r, q) holds M[16 fb + r][16 pb + 4 q + i]
// v_mfma_f32_16x16x16f16 takes A as lane (r, q) -> A[r][4 q + i], B as B[4 q + i][r] and returns D as
// D[4 q + i][r]. So a product's D is a feature-rows or primitive-rows tile as it stands; a feature-rows tile
// is a B operand with K = features or an A operand holding the block's transpose (rows = primitives,
// K = features); a primitive-rows tile is a B operand with K = primitives (N = features) or an A operand
// holding the block itself with K = primitives. Computing every activation and every gradient in both
// orientations (twice the MFMAs of the forward chain, which are cheap here) feeds every product of the
// backward, including the weight gradients (contractions over primitives), with no transposes through LDS.
//
// LDS holds W_l row-major [out][in] and its transpose [in][out]; rows are padded by 4 halves so that the 16
// lanes reading 8-byte fragments of 16 consecutive rows fall on distinct banks.
constexpr uint32_t WPAD = 4;
__host__ __device__ constexpr uint32_t wrow(uint32_t l) { return lin(l) + WPAD; }
__host__ __device__ constexpr uint32_t wtrow(uint32_t l) { return lout(l) + WPAD; }
__host__ __device__ constexpr uint32_t dual_layer_halves(uint32_t l) { return lout(l) * wrow(l) + lin(l) * wtrow(l); }
__host__ __device__ constexpr uint32_t woff(uint32_t l) {
    uint32_t o = 0;
    for (uint32_t k = 0; k < l; k++) o += dual_layer_halves(k);
    return o;
}
__host__ __device__ constexpr uint32_t wtoff(uint32_t l) { return woff(l) + lout(l) * wrow(l); }
constexpr uint32_t DUAL_WEIGHT_BYTES = (woff(NL) * 2 + 15) / 16 * 16;
constexpr uint32_t XS = INP + 4;        // staging row of the input / output-gradient rows (halves)
constexpr uint32_t YS = OUTP + 4;
constexpr uint32_t FS = INP + 4;        // staging row of the input-gradient rows (floats)
constexpr uint32_t DUAL_STAGE_BYTES = 64 * FS * 4;  // per wave; also covers 64 rows of XS or YS halves
// With EFGS_MLP_U_LDS the primitive-rows input tiles of the hidden layers wait for the backward outside the
// registers: U[1] is recomputed from the staged input tiles where it is used (one MFMA per tile for a 16-wide
// input), U[2..NH] sit in a per-wave LDS store (one 8-byte slot per lane and tile, written and read by the
// same lane). The host sets it when the store fits two blocks' LDS per CU.
constexpr uint32_t U_TILES = (NN / 16) * 4;
constexpr uint32_t U_STORE_BYTES = EFGS_MLP_U_LDS ? (NH > 1 ? NH - 1 : 0u) * U_TILES * 64 * 8 : 0u;  // per wave
__device__ __forceinline__ uint32_t u_slot(uint32_t l, uint32_t pb, uint32_t fb, uint32_t lane) {
    return (((l - 2) * U_TILES + pb * (NN / 16) + fb) * 64 + lane);
}

// copies the flat tcnn-layout weights (fp16 bits, 16-byte aligned) into the padded W / W^T layout (whole
// block of N_THREADS): 8 weights per 16-byte load, up to 8 loads per thread in flight before the LDS stores.
// Every layer holds a multiple of 256 weights, so a vector never straddles two layers or two rows.
template <uint32_t N_THREADS>
__device__ inline void load_dual_weights(const uint16_t* g, uint16_t* WL, uint32_t tid) {
    constexpr uint32_t n_vec = PARAMS / 8;
    constexpr uint32_t batch = 8;
    const uint4* gv = reinterpret_cast<const uint4*>(g);
    for (uint32_t v0 = 0; v0 < n_vec; v0 += batch * N_THREADS) {
        uint4 w[batch];
#pragma unroll
        for (uint32_t k = 0; k < batch; k++) {
            const uint32_t v = v0 + k * N_THREADS + tid;
            if (v < n_vec) w[k] = gv[v];
        }
#pragma unroll
        for (uint32_t k = 0; k < batch; k++) {
            const uint32_t v = v0 + k * N_THREADS + tid;
            if (v >= n_vec) continue;
            const uint32_t h = 8 * v;
            const uint16_t e[8] = {static_cast<uint16_t>(w[k].x), static_cast<uint16_t>(w[k].x >> 16), static_cast<uint16_t>(w[k].y),
                                   static_cast<uint16_t>(w[k].y >> 16), static_cast<uint16_t>(w[k].z), static_cast<uint16_t>(w[k].z >> 16),
                                   static_cast<uint16_t>(w[k].w), static_cast<uint16_t>(w[k].w >> 16)};
#pragma unroll
            for (uint32_t l = 0; l < NL; l++) {
                if (h < loff(l) || h >= loff(l) + lout(l) * lin(l)) continue;
                const uint32_t idx = h - loff(l);
                const uint32_t row = idx / lin(l), col = idx % lin(l);
#pragma unroll
                for (uint32_t i = 0; i < 8; i++) {
                    WL[woff(l) + row * wrow(l) + col + i] = e[i];
                    WL[wtoff(l) + (col + i) * wtrow(l) + row] = e[i];
                }
            }
        }
    }
}

// ReLU of an fp32 tile, rounded to fp16 (round to nearest even, then a packed max with zero)
__device__ __forceinline__ h4 relu_h4(f4 v) {
    const h4 x = __builtin_convertvector(v, h4);
    return __builtin_elementwise_max(x, h4{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f),
                                           static_cast<_Float16>(0.0f)});
}

// v where the activation is positive (ReLU derivative), as fp16
__device__ __forceinline__ h4 masked_h4(f4 v, h4 act) {
    const _Float16 z = static_cast<_Float16>(0.0f);
    return h4{act[0] > z ? static_cast<_Float16>(v[0]) : z, act[1] > z ? static_cast<_Float16>(v[1]) : z,
              act[2] > z ? static_cast<_Float16>(v[2]) : z, act[3] > z ? static_cast<_Float16>(v[3]) : z};
}

// ReLU masks of the feature-rows activations, 4 bits per tile (tile fb * 4 + pb), kept once the forward no
// longer needs the values themselves
constexpr uint32_t MASK_WORDS = (KT * 4 * 4 + 31) / 32;
__device__ __forceinline__ uint32_t positive_bits(h4 a) {
    const _Float16 z = static_cast<_Float16>(0.0f);
    return (a[0] > z ? 1u : 0u) | (a[1] > z ? 2u : 0u) | (a[2] > z ? 4u : 0u) | (a[3] > z ? 8u : 0u);
}
__device__ __forceinline__ h4 masked_h4_bits(f4 v, uint32_t bits) {
    const _Float16 z = static_cast<_Float16>(0.0f);
    return h4{(bits & 1u) ? static_cast<_Float16>(v[0]) : z, (bits & 2u) ? static_cast<_Float16>(v[1]) : z,
              (bits & 4u) ? static_cast<_Float16>(v[2]) : z, (bits & 8u) ? static_cast<_Float16>(v[3]) : z};
}

// Per-wave MLP forward: fp16 MFMA, fp32 accumulation, activations rounded to fp16 between layers. WL: padded
// W / W^T in LDS; stage: this wave's staging area; x: the lane's input row; y: the lane's three raw outputs,
// rounded to fp16. With DUAL (the backward's recompute) it also leaves U[l], the input activations of layer l
// as primitive-rows tiles, and Tm[l] (l >= 1), the ReLU masks of the feature-rows tiles.
template <bool DUAL>
__device__ inline void mlp_forward_tiles(const _Float16* WL, _Float16* stage, const float* x, uint32_t (&Tm)[NL][MASK_WORDS], h4 (&U)[NL][4][KT],
                                         h4 (&X)[INP / 16][4], h4* ustore, float* y, uint32_t lane) {
    h4 T[NL][KT][4];
    const uint32_t r = lane & 15u, q = lane >> 4;
#pragma unroll
    for (uint32_t k = 0; k < INP; k += 4)
        *reinterpret_cast<h4*>(&stage[lane * XS + k]) =
            h4{static_cast<_Float16>(x[k]), static_cast<_Float16>(x[k + 1]), static_cast<_Float16>(x[k + 2]), static_cast<_Float16>(x[k + 3])};
    wave_sync();
#pragma unroll
    for (uint32_t ib = 0; ib < INP / 16; ib++)
#pragma unroll
        for (uint32_t pb = 0; pb < 4; pb++) {
            T[0][ib][pb] = *reinterpret_cast<const h4*>(&stage[(16 * pb + r) * XS + 16 * ib + 4 * q]);
            if (DUAL)
                U[0][pb][ib] = h4{stage[(16 * pb + 4 * q) * XS + 16 * ib + r], stage[(16 * pb + 4 * q + 1) * XS + 16 * ib + r],
                              stage[(16 * pb + 4 * q + 2) * XS + 16 * ib + r], stage[(16 * pb + 4 * q + 3) * XS + 16 * ib + r]};
        }
    wave_sync();
    f4 yt[4];
#pragma unroll
    for (uint32_t l = 0; l < NL; l++) {
#pragma unroll
        for (uint32_t ob = 0; ob < lout(l) / 16; ob++) {
            h4 wa[KT];
#pragma unroll
            for (uint32_t ib = 0; ib < lin(l) / 16; ib++) wa[ib] = *reinterpret_cast<const h4*>(&WL[woff(l) + (16 * ob + r) * wrow(l) + 16 * ib + 4 * q]);
#pragma unroll
            for (uint32_t pb = 0; pb < 4; pb++) {
                f4 t = f4_zero();
#pragma unroll
                for (uint32_t ib = 0; ib < lin(l) / 16; ib++) t = mfma(wa[ib], T[l][ib][pb], t);  // H(ob, pb) = sum W(ob, ib) M(ib, pb)
                if (l < NH) {
                    T[l + 1][ob][pb] = relu_h4(t);
                    if (!DUAL || (EFGS_MLP_U_LDS && l == 0)) continue;  // U[1] is recomputed where it is used
                    f4 u = f4_zero();
#pragma unroll
                    for (uint32_t ib = 0; ib < lin(l) / 16; ib++) u = mfma(T[l][ib][pb], wa[ib], u);  // H^T(pb, ob) = sum M^T(pb, ib) W^T(ib, ob)
                    if (EFGS_MLP_U_LDS)
                        ustore[u_slot(l + 1, pb, ob, lane)] = relu_h4(u);
                    else
                        U[l + 1][pb][ob] = relu_h4(u);
                } else if (ob == 0) {
                    yt[pb] = t;
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // one output block in flight: bounds the live accumulators
        }
    }
    // outputs 0..2 of primitive 16 pb + c sit in lane c of output tile pb
#pragma unroll
    for (uint32_t o = 0; o < 3; o++) {
        float v = 0.0f;
#pragma unroll
        for (uint32_t pb = 0; pb < 4; pb++) {
            const float t = __shfl(yt[pb][o], static_cast<int>(r));
            if (q == pb) v = t;
        }
        y[o] = round_half(v);
    }
    if (!DUAL) return;
#pragma unroll
    for (uint32_t ib = 0; ib < INP / 16; ib++)
#pragma unroll
        for (uint32_t pb = 0; pb < 4; pb++) X[ib][pb] = T[0][ib][pb];
#pragma unroll
    for (uint32_t l = 1; l < NL; l++) {
#pragma unroll
        for (uint32_t w = 0; w < MASK_WORDS; w++) Tm[l][w] = 0u;
#pragma unroll
        for (uint32_t fb = 0; fb < lin(l) / 16; fb++)
#pragma unroll
            for (uint32_t pb = 0; pb < 4; pb++) {
                const uint32_t t = fb * 4 + pb;
                Tm[l][t / 8] |= positive_bits(T[l][fb][pb]) << (4 * (t % 8));
            }
    }
}

// Backward through the MLP from the lanes' output gradients dy (zero for lanes that do not contribute), with
// Tm / U from mlp_forward_tiles<true>. The gradients run through the fp16 MFMAs scaled by s (a power of two
// that keeps them in fp16 range; the caller picks it from a bound on |dy| over the whole launch). Writes the
// lane's input gradient row dx (INP floats, unscaled) and adds the wave's weight gradients, still scaled by s,
// to dW (MFMA accumulators, lane layout of the D operand: dW[l][ob][ib][i] = s dW_l[16 ob + 4 q + i][16 ib + r]).
__device__ inline void mlp_backward_dual(const _Float16* WL, _Float16* stage, const uint32_t (&Tm)[NL][MASK_WORDS], const h4 (&U)[NL][4][KT],
                                         const h4 (&X)[INP / 16][4], const h4* ustore, const float* dy, float s, float inv_s, float* dx,
                                         f4 (&dW)[NL][NT > 1 ? NT : 1][KT], uint32_t lane) {
    // primitive-rows input tile (pb, fb) of layer l
    auto u_tile = [&](uint32_t l, uint32_t pb, uint32_t fb) -> h4 {
        if (!EFGS_MLP_U_LDS || l == 0) return U[l][pb][fb];
        if (l >= 2) return ustore[u_slot(l, pb, fb, lane)];
        f4 u = f4_zero();  // U[1](pb, fb) = ReLU(sum_ib X^T(pb, ib) W_0^T(ib, fb))
#pragma unroll
        for (uint32_t ib = 0; ib < INP / 16; ib++)
            u = mfma(X[ib][pb], *reinterpret_cast<const h4*>(&WL[woff(0) + (16 * fb + (lane & 15u)) * wrow(0) + 16 * ib + 4 * (lane >> 4)]), u);
        return relu_h4(u);
    };
    const uint32_t r = lane & 15u, q = lane >> 4;
#pragma unroll
    for (uint32_t k = 0; k < INP; k++) dx[k] = 0.0f;
    if (__ballot(dy[0] != 0.0f || dy[1] != 0.0f || dy[2] != 0.0f) == 0) return;  // wave-uniform

    // output-layer gradient (16 padded outputs x 64 primitives) in both orientations, through LDS
    const _Float16 z = static_cast<_Float16>(0.0f);
    *reinterpret_cast<h4*>(&stage[lane * YS]) = h4{static_cast<_Float16>(dy[0] * s), static_cast<_Float16>(dy[1] * s),
                                                    static_cast<_Float16>(dy[2] * s), z};
#pragma unroll
    for (uint32_t k = 4; k < OUTP; k += 4) *reinterpret_cast<h4*>(&stage[lane * YS + k]) = h4{z, z, z, z};
    wave_sync();
    h4 G[KT][4], GT[4][KT];
#pragma unroll
    for (uint32_t pb = 0; pb < 4; pb++) {
        G[0][pb] = *reinterpret_cast<const h4*>(&stage[(16 * pb + r) * YS + 4 * q]);
        GT[pb][0] = h4{stage[(16 * pb + 4 * q) * YS + r], stage[(16 * pb + 4 * q + 1) * YS + r], stage[(16 * pb + 4 * q + 2) * YS + r],
                       stage[(16 * pb + 4 * q + 3) * YS + r]};
    }
    wave_sync();

    // output layer: dW_NH(0, ib) += sum_pb dY(0, pb) M_NH(ib, pb)^T (dY as primitive-rows A operand)
#pragma unroll
    for (uint32_t ib = 0; ib < lin(NH) / 16; ib++) {
#pragma unroll
        for (uint32_t pb = 0; pb < 4; pb++) dW[NH][0][ib] = mfma(GT[pb][0], u_tile(NH, pb, ib), dW[NH][0][ib]);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int li = static_cast<int>(NH); li >= 1; li--) {
        const uint32_t l = static_cast<uint32_t>(li);
        // input gradient of layer l in both orientations, through the ReLU of its input; each primitive-rows tile
        // goes straight into layer l-1's weight gradient (dW_{l-1}(ib, jb) += sum_pb dIn(ib, pb) M_{l-1}(jb, pb)^T)
        h4 Gn[KT][4];
#pragma unroll
        for (uint32_t ib = 0; ib < lin(l) / 16; ib++) {
            h4 wt[KT];
#pragma unroll
            for (uint32_t ob = 0; ob < lout(l) / 16; ob++)
                wt[ob] = *reinterpret_cast<const h4*>(&WL[wtoff(l) + (16 * ib + r) * wtrow(l) + 16 * ob + 4 * q]);
#pragma unroll
            for (uint32_t pb = 0; pb < 4; pb++) {
                f4 t = f4_zero(), u = f4_zero();
#pragma unroll
                for (uint32_t ob = 0; ob < lout(l) / 16; ob++) {
                    t = mfma(wt[ob], G[ob][pb], t);   // dIn(ib, pb) = sum W^T(ib, ob) dOut(ob, pb)
                    u = mfma(G[ob][pb], wt[ob], u);   // dIn^T(pb, ib) = sum dOut^T(pb, ob) W(ob, ib)
                }
                const uint32_t ti = ib * 4 + pb;
                Gn[ib][pb] = masked_h4_bits(t, (Tm[l][ti / 8] >> (4 * (ti % 8))) & 15u);
                const h4 gt = masked_h4(u, u_tile(l, pb, ib));
#pragma unroll
                for (uint32_t jb = 0; jb < lin(l - 1) / 16; jb++) dW[l - 1][ib][jb] = mfma(gt, u_tile(l - 1, pb, jb), dW[l - 1][ib][jb]);
            }
            __builtin_amdgcn_sched_barrier(0);  // one input block in flight: bounds the live accumulators
        }
#pragma unroll
        for (uint32_t ib = 0; ib < lin(l) / 16; ib++)
#pragma unroll
            for (uint32_t pb = 0; pb < 4; pb++) G[ib][pb] = Gn[ib][pb];
    }
    // input gradient rows (feature-rows tiles, unscaled) to the lanes through LDS
    float* fs = reinterpret_cast<float*>(stage);
#pragma unroll
    for (uint32_t ib = 0; ib < INP / 16; ib++) {
        h4 wt[KT];
#pragma unroll
        for (uint32_t ob = 0; ob < lout(0) / 16; ob++) wt[ob] = *reinterpret_cast<const h4*>(&WL[wtoff(0) + (16 * ib + r) * wtrow(0) + 16 * ob + 4 * q]);
#pragma unroll
        for (uint32_t pb = 0; pb < 4; pb++) {
            f4 t = f4_zero();
#pragma unroll
            for (uint32_t ob = 0; ob < lout(0) / 16; ob++) t = mfma(wt[ob], G[ob][pb], t);
            *reinterpret_cast<float4*>(&fs[(16 * pb + r) * FS + 16 * ib + 4 * q]) = make_float4(t[0] * inv_s, t[1] * inv_s, t[2] * inv_s, t[3] * inv_s);
        }
    }
    wave_sync();
#pragma unroll
    for (uint32_t k = 0; k < INP; k += 4) {
        const float4 v = *reinterpret_cast<const float4*>(&fs[lane * FS + k]);
        dx[k] = v.x; dx[k + 1] = v.y; dx[k + 2] = v.z; dx[k + 3] = v.w;
    }
    wave_sync();
}

}  // namespace nn

}  // namespace efgs
