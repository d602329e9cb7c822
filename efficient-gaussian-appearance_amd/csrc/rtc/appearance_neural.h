// Neural residual (EFGS_MODEL == 5): a bias-free ReLU MLP over per-Gaussian features (optionally frequency
// encoded, optionally with the base colour as 3 extra inputs) and the SH degree values of the view
// direction, evaluated per wave of 64 primitives with fp16 MFMA (v_mfma_f32_16x16x32_f16 wherever a
// contraction spans 32 or more, v_mfma_f32_16x16x16f16 for a trailing 16) and fp32 accumulation; the weights
// sit in LDS (tcnn flat layout in HBM: row-major [out x in] per layer, input padded to a multiple of 16,
// output padded to 16 rows).
//
// Each layer computes H_out = W H_in with W as the A operand and the activations as the B operand, so an
// accumulator tile is the next layer's B fragment as it stands: no data movement between layers.
// Activations are rounded to fp16 between layers (as tcnn's half-precision network), the 3 outputs are
// rounded to fp16.
//
// Backward: the forward is recomputed (no stored context), per pair of 16-primitive column blocks, with every
// activation kept in registers until its backward. The upstream gradient is scaled by a power of two before
// the fp16 MFMA chain and unscaled in fp32. Weight gradients accumulate per wave in fp32 registers, with
// the operands' transposes taken by MFMA against the identity, then are reduced across the block's waves
// in a fixed order.
//
// Reference: B/rasterization/rtc/appearance_neural.cuh:17-407 (encoding, SH degree values and their
// gradient, tcnn eval_model / backward_eval_model at :333, :379); weight layout viewer/export_ngsplat.py:1013-1029.
#pragma once

namespace efgs {

namespace nn {

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

// derivative of the residual activation at the raw MLP output y, for the gradients: tanh' = sech^2 y =
// 4 e / (1 + e)^2 and softplus(beta 10)' = sigmoid(10 y), from e = exp(-2|y|) resp. exp(-10|y|) (no overflow),
// with the hardware exp and reciprocal (about 1 ulp each)
template <int ACT>
__device__ __forceinline__ float residual_activation_slope(float y) {
    if (ACT == 1) {
        const float e = __expf(-2.0f * fabsf(y));
        const float d = 1.0f + e;
        return 4.0f * e * __builtin_amdgcn_rcpf(d * d);
    }
    if (ACT == 2) {
        const float e = __expf(-10.0f * fabsf(y));
        const float t = __builtin_amdgcn_rcpf(1.0f + e);
        return y >= 0.0f ? t : e * t;
    }
    return 1.0f;
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

// ---- MLP tiles ----------------------------------------------------------------------------------------
//
// A wave holds a (features x 64 primitives) matrix M as 16 x 16 blocks in one of two orientations
// (lane = r + 16 q, i = 0..3):
//   F-tile (feature rows)    lane (r, q) holds M[16 fb + 4 q + i][16 pb + r]
//   P-tile (primitive rows)  lane (r, q) holds M[16 fb + r][16 pb + 4 q + i]
// v_mfma_f32_16x16x16f16 reads A as lane (r, q) -> A[r][4 q + i], B as lane (r, q) -> B[4 q + i][r] and returns
// D[4 q + i][r]. So rows of W (A, from LDS) times F-tiles (B) give F-tiles: the layer chain, forward and
// backward, contracts over features. The weight gradients contract over primitives: A is a P-tile of the
// gradient, B a P-tile of the layer input. An F-tile taken as the A operand is the block's transpose, so its
// product with the identity is the block's P-tile: one MFMA per tile, exact (products x * 1, sums of zeros).
// v_mfma_f32_16x16x32_f16 (K = 32, same issue cost) takes two K = 16 fragments concatenated on both sides:
// A's lane (r, q) and B's lane (n, q) then hold the same k's, so every contraction over 32 or more runs
// at twice the rate of the K = 16 form.
//
// LDS holds W_l row-major [out][in] and W_l^T row-major [in][out]. Within each 32-column group a row stores
// column 32 j + 16 h + 4 q + i at 32 j + 8 q + 4 h + i, so the two K = 16 fragments a lane concatenates are one
// 16-byte read (a trailing 16-column group keeps its order). Rows are padded by 8 halves.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ h8 cat(h4 a, h4 b) { return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7); }

constexpr uint32_t WPAD = 8;
__host__ __device__ constexpr uint32_t wrow(uint32_t l) { return lin(l) + WPAD; }
__host__ __device__ constexpr uint32_t wtrow(uint32_t l) { return lout(l) + WPAD; }
__host__ __device__ constexpr uint32_t layer_halves(uint32_t l) { return lout(l) * wrow(l) + lin(l) * wtrow(l); }
__host__ __device__ constexpr uint32_t woff(uint32_t l) {
    uint32_t o = 0;
    for (uint32_t k = 0; k < l; k++) o += layer_halves(k);
    return o;
}
__host__ __device__ constexpr uint32_t wtoff(uint32_t l) { return woff(l) + lout(l) * wrow(l); }
constexpr uint32_t WEIGHT_BYTES = (woff(NL) * 2 + 15) / 16 * 16;
constexpr uint32_t XS = INP + 4;        // staging row of the input rows (halves)
constexpr uint32_t FS = INP + 4;        // staging row of the input-gradient rows (floats)
constexpr uint32_t STAGE_BYTES = 64 * FS * 4;  // per wave; covers 64 rows of XS halves and 64 output rows of 16 bytes

// position of column c in a stored row of `width` columns
__host__ __device__ constexpr uint32_t kpos(uint32_t c, uint32_t width) {
    return c < width / 32u * 32u ? (c & ~31u) | (((c >> 2) & 3u) << 3) | (((c >> 4) & 1u) << 2) | (c & 3u) : c;
}

// the fp16 bits of 8 consecutive flat weights: from fp16 bits (one 16-byte load) or from fp32 master weights (two
// 16-byte loads, rounded to nearest even, as a cast of the tensor to half would)
struct WeightVec8 {
    uint4 lo, hi;
};
__device__ __forceinline__ WeightVec8 load_weight_vec(const uint16_t* g, uint32_t v) {
    return WeightVec8{reinterpret_cast<const uint4*>(g)[v], make_uint4(0u, 0u, 0u, 0u)};
}
__device__ __forceinline__ WeightVec8 load_weight_vec(const float* g, uint32_t v) {
    const uint4* gv = reinterpret_cast<const uint4*>(g);
    return WeightVec8{gv[2 * v], gv[2 * v + 1]};
}
__device__ __forceinline__ void weight_bits(const WeightVec8& w, const uint16_t*, uint16_t (&e)[8]) {
    const uint32_t x[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        e[2 * i] = static_cast<uint16_t>(x[i]);
        e[2 * i + 1] = static_cast<uint16_t>(x[i] >> 16);
    }
}
__device__ __forceinline__ void weight_bits(const WeightVec8& w, const float*, uint16_t (&e)[8]) {
    const uint32_t x[8] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w, w.hi.x, w.hi.y, w.hi.z, w.hi.w};
#pragma unroll
    for (uint32_t i = 0; i < 8; i++) e[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(__uint_as_float(x[i])));
}

// copies the flat tcnn-layout weights (fp16 bits or fp32 master weights, 16-byte aligned) into the W / W^T layout
// above (whole block of N_THREADS): 8 weights per vector, up to 8 vectors per thread in flight before the LDS
// stores. Every layer holds a multiple of 256 weights, so a vector never straddles two layers or two rows.
template <uint32_t N_THREADS, typename SRC>
__device__ inline void load_weights(const SRC* g, uint16_t* WL, uint32_t tid) {
    constexpr uint32_t n_vec = PARAMS / 8;
    constexpr uint32_t batch = 8;
    for (uint32_t v0 = 0; v0 < n_vec; v0 += batch * N_THREADS) {
        WeightVec8 w[batch];
#pragma unroll
        for (uint32_t k = 0; k < batch; k++) {
            const uint32_t v = v0 + k * N_THREADS + tid;
            if (v < n_vec) w[k] = load_weight_vec(g, v);
        }
#pragma unroll
        for (uint32_t k = 0; k < batch; k++) {
            const uint32_t v = v0 + k * N_THREADS + tid;
            if (v >= n_vec) continue;
            const uint32_t h = 8 * v;
            uint16_t e[8];
            weight_bits(w[k], g, e);
#pragma unroll
            for (uint32_t l = 0; l < NL; l++) {
                if (h < loff(l) || h >= loff(l) + lout(l) * lin(l)) continue;
                const uint32_t idx = h - loff(l);
                const uint32_t row = idx / lin(l), col = idx % lin(l);
#pragma unroll
                for (uint32_t i = 0; i < 8; i++) {
                    WL[woff(l) + row * wrow(l) + kpos(col + i, lin(l))] = e[i];
                    WL[wtoff(l) + (col + i) * wtrow(l) + kpos(row, lout(l))] = e[i];
                }
            }
        }
    }
}

// sum over the kb_count K = 16 blocks of A(row, kb) B(kb): K = 32 pairs, then a trailing K = 16 block. row:
// the lane's stored row (16-byte aligned); b: B tiles (F-tiles with K = features). Two column blocks share
// every A fragment read.
__device__ __forceinline__ void row_times(const _Float16* row, uint32_t kb_count, const h4* b0, const h4* b1, uint32_t q, f4& acc0,
                                          f4& acc1) {
#pragma unroll
    for (uint32_t j = 0; 2 * j + 1 < kb_count; j++) {
        const h8 a = *reinterpret_cast<const h8*>(row + 32 * j + 8 * q);
        acc0 = mfma32(a, cat(b0[2 * j], b0[2 * j + 1]), acc0);
        acc1 = mfma32(a, cat(b1[2 * j], b1[2 * j + 1]), acc1);
    }
    if (kb_count & 1u) {
        const h4 a = *reinterpret_cast<const h4*>(row + 16 * (kb_count - 1) + 4 * q);
        acc0 = mfma(a, b0[kb_count - 1], acc0);
        acc1 = mfma(a, b1[kb_count - 1], acc1);
    }
}
__device__ __forceinline__ f4 row_times1(const _Float16* row, uint32_t kb_count, const h4* b, uint32_t q) {
    f4 acc = f4_zero();
#pragma unroll
    for (uint32_t j = 0; 2 * j + 1 < kb_count; j++)
        acc = mfma32(*reinterpret_cast<const h8*>(row + 32 * j + 8 * q), cat(b[2 * j], b[2 * j + 1]), acc);
    if (kb_count & 1u) acc = mfma(*reinterpret_cast<const h4*>(row + 16 * (kb_count - 1) + 4 * q), b[kb_count - 1], acc);
    return acc;
}

// The lane's row index within a 16-row block, opaque to the compiler: weight-row addresses built from it stay
// inside the caller's loop as one base plus constants (folded into the LDS instructions' offsets) instead of
// being hoisted as one register per row
__device__ __forceinline__ uint32_t opaque_row(uint32_t lane) {
    uint32_t r = lane & 15u;
    asm volatile("" : "+v"(r));
    return r;
}

// ReLU of an fp32 tile, rounded to fp16 (round to nearest even, then a packed max with zero)
__device__ __forceinline__ h4 relu_h4(f4 v) {
    const h4 x = __builtin_convertvector(v, h4);
    return __builtin_elementwise_max(x, h4{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f),
                                           static_cast<_Float16>(0.0f)});
}

// fp16 of v where the ReLU output act is positive, zero elsewhere. act >= 0, so act > 0 exactly when its bits
// without the sign are nonzero: m = min(bits & 0x7fff, 1) is 1 or 0 per half and multiplies the fp16 bits
// (three packed integer instructions per pair of values). m comes from inline assembly so that the compiler
// cannot turn the product back into a compare and a select per value; the product itself stays ordinary code,
// so the compiler still sees the write that the next MFMA reads and inserts the wait states it needs.
__device__ __forceinline__ uint32_t relu_mask2(uint32_t act) {
    uint32_t m;
    asm("v_and_b32 %0, %1, %2\n\tv_pk_min_u16 %0, %0, %3" : "=&v"(m) : "s"(0x7fff7fffu), "v"(act), "s"(0x00010001u));
    return m;
}
// fp16 bits of (a, b), rounded to nearest even by one packed conversion (kept packed: without the register
// constraint the compiler converts the four values of a tile one by one and packs them with byte permutes)
typedef float f2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t half2_bits(float a, float b) {
    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
    asm("" : "+v"(r));
    return r;
}
__device__ __forceinline__ h4 relu_grad(f4 v, h4 act) {
    const u16x4 x = __builtin_bit_cast(u16x4, make_uint2(half2_bits(v[0], v[1]), half2_bits(v[2], v[3])));
    const uint2 a = __builtin_bit_cast(uint2, act);
    const u16x4 m = __builtin_bit_cast(u16x4, make_uint2(relu_mask2(a.x), relu_mask2(a.y)));
    return __builtin_bit_cast(h4, x * m);
}

// identity B operand: lane (r, q) holds I[4 q + i][r]
__device__ __forceinline__ h4 identity_tile(uint32_t lane) {
    const uint32_t r = lane & 15u, q = lane >> 4;
    const _Float16 one = static_cast<_Float16>(1.0f), z = static_cast<_Float16>(0.0f);
    return h4{4 * q == r ? one : z, 4 * q + 1 == r ? one : z, 4 * q + 2 == r ? one : z, 4 * q + 3 == r ? one : z};
}

// P-tile of the block whose F-tile is f: the F-tile taken as the A operand is the block's transpose, so its product
// with the identity is the P-tile, exact (products x * 1, sums of zeros). One MFMA issue, in a pipe the kernels
// leave mostly idle. (A store and gfx950's transposing LDS read, ds_read_b64_tr_b16, measured slower: the MLP
// backward 60.1 -> 63.4 us on the 1M-Gaussian scene; a wave's LDS reads complete in order, so the weight
// fragments the next MFMAs need wait behind the transposes' LDS traffic.)
__device__ __forceinline__ h4 transpose_tile(h4 f, h4 eye) {
    const f4 t = mfma(f, eye, f4_zero());
    return __builtin_bit_cast(h4, make_uint2(half2_bits(t[0], t[1]), half2_bits(t[2], t[3])));
}

// input row x (INP floats) to fp16 at row `row` of a staging area (rows of XS halves)
__device__ __forceinline__ void stage_input_row(_Float16* rows, const float* x, uint32_t row) {
#pragma unroll
    for (uint32_t k = 0; k < INP; k += 4)
        *reinterpret_cast<h4*>(&rows[row * XS + k]) =
            h4{static_cast<_Float16>(x[k]), static_cast<_Float16>(x[k + 1]), static_cast<_Float16>(x[k + 2]), static_cast<_Float16>(x[k + 3])};
}

// the F-tiles X[pb][ib] of the four column blocks of 64 staged input rows
__device__ __forceinline__ void load_input_tiles(const _Float16* rows, h4 (&X)[4][INP / 16], uint32_t lane) {
    const uint32_t r = lane & 15u, q = lane >> 4;
#pragma unroll
    for (uint32_t pb = 0; pb < 4; pb++)
#pragma unroll
        for (uint32_t ib = 0; ib < INP / 16; ib++) X[pb][ib] = *reinterpret_cast<const h4*>(&rows[(16 * pb + r) * XS + 16 * ib + 4 * q]);
}

// the lane's input row (INP floats) to fp16 in the staging area, then the F-tiles X[pb][ib] of the wave's four
// column blocks
__device__ inline void stage_input_tiles(_Float16* stage, const float* x, h4 (&X)[4][INP / 16], uint32_t lane) {
    stage_input_row(stage, x, lane);
    wave_sync();
    load_input_tiles(stage, X, lane);
    wave_sync();
}

// MLP forward of 64 staged input rows (rows of XS halves, written by this wave or, before a block barrier, by
// any wave of the block): fp16 MFMA, fp32 accumulation, activations rounded to fp16 between layers. WL: the
// weights in LDS. Row i's three raw outputs, rounded to fp16, then replace the rows as float4 i = (y0, y1, y2,
// 0) (the first 1 KB of the area). Column blocks of 16 primitives run one after another (the chain is per
// primitive, so a primitive's outputs do not depend on the other rows).
__device__ inline void mlp_forward_rows(const _Float16* WL, _Float16* rows, uint32_t lane) {
    const uint32_t r = lane & 15u, q = lane >> 4, ro = opaque_row(lane);
    h4 X[4][INP / 16];
    load_input_tiles(rows, X, lane);
    wave_sync();  // every row read before the outputs overwrite them
    float* ys = reinterpret_cast<float*>(rows);
#pragma unroll
    for (uint32_t pp = 0; pp < 2; pp++) {
        h4 H[2][NT], Hn[2][NT];
        f4 yt[2];
#pragma unroll
        for (uint32_t l = 0; l < NL; l++) {
            const h4* in0 = l == 0 ? X[2 * pp] : H[0];
            const h4* in1 = l == 0 ? X[2 * pp + 1] : H[1];
#pragma unroll
            for (uint32_t ob = 0; ob < lout(l) / 16; ob++) {
                f4 a0 = f4_zero(), a1 = f4_zero();
                row_times(WL + woff(l) + (16 * ob + ro) * wrow(l), lin(l) / 16, in0, in1, q, a0, a1);
                if (l < NH) {
                    Hn[0][ob] = relu_h4(a0);
                    Hn[1][ob] = relu_h4(a1);
                } else if (ob == 0) {
                    yt[0] = a0;
                    yt[1] = a1;
                }
            }
            if (l < NH) {
#pragma unroll
                for (uint32_t ob = 0; ob < NT; ob++) {
                    H[0][ob] = Hn[0][ob];
                    H[1][ob] = Hn[1][ob];
                }
            }
        }
        // outputs 0..3 of primitive 16 pb + r sit in lane r of column block pb's output tile
        if (q == 0) {
#pragma unroll
            for (uint32_t b = 0; b < 2; b++)
                *reinterpret_cast<float4*>(&ys[(16 * (2 * pp + b) + r) * 4]) =
                    make_float4(round_half(yt[b][0]), round_half(yt[b][1]), round_half(yt[b][2]), 0.0f);
        }
    }
}

// Per-wave MLP forward of the wave's own 64 primitives: stage: this wave's staging area; x: the lane's input
// row; y: the lane's three raw outputs, rounded to fp16.
__device__ inline void mlp_forward(const _Float16* WL, _Float16* stage, const float* x, float* y, uint32_t lane) {
    stage_input_row(stage, x, lane);
    wave_sync();
    mlp_forward_rows(WL, stage, lane);
    wave_sync();
    const float4 v = *reinterpret_cast<const float4*>(&reinterpret_cast<const float*>(stage)[lane * 4]);
    y[0] = v.x;
    y[1] = v.y;
    y[2] = v.z;
    wave_sync();
}

// Forward and backward of the wave's 64 primitives in two passes of 32 (a pair of column blocks): the chain is
// independent per primitive and only the weight gradients sum over primitives, in K = 32 MFMAs over the
// pair, so every activation of a pass stays in registers until its backward.
//   x: the lane's input row; g: the lane's gradient with respect to its 3 activated outputs (zero for lanes
//   that do not contribute); dy_of(y, g): gradient with respect to the raw output y (rounded to fp16) given g;
//   s / inv_s: the gradient scale, a power of two that keeps the fp16 gradients in range (the caller picks it
//   from a bound on |dL/dy| over the launch); dx: the lane's input-gradient row (unscaled); dW: weight
//   gradient accumulators, still scaled by s (D layout: dW[l][ob][ib][i] = s dW_l[16 ob + 4 q + i][16 ib + r]).
template <typename DY>
__device__ inline void mlp_train(const _Float16* WL, _Float16* stage, const float* x, const float* g, DY&& dy_of, float s,
                                 float inv_s, float* dx, f4 (&dW)[NL][NT][KT], uint32_t lane) {
    const uint32_t r = lane & 15u, q = lane >> 4, ro = opaque_row(lane);
    const h4 eye = identity_tile(lane);
    const _Float16 z = static_cast<_Float16>(0.0f);
    const h4 zero4 = h4{z, z, z, z};
    h4 X[4][INP / 16];
    stage_input_tiles(stage, x, X, lane);
    float* fs = reinterpret_cast<float*>(stage);
    // the upstream gradients of primitive 16 pb + r (column block pb's output tile holds them in lane r), read
    // before the forward so that the cross-lane reads are not waited on between the forward and the backward
    float gsrc[4][3];
#pragma unroll
    for (uint32_t pb = 0; pb < 4; pb++)
#pragma unroll
        for (uint32_t c = 0; c < 3; c++) gsrc[pb][c] = __shfl(g[c], static_cast<int>(16 * pb + r));
#pragma unroll
    for (uint32_t pp = 0; pp < 2; pp++) {
        // forward: F[l] = input activations of layer l >= 1 (F-tiles); their P-tiles are taken in the backward, next
        // to the weight-gradient MFMAs that read them (registers for one layer's P-tiles at a time)
        h4 F[NL][2][NT];
        f4 yt[2];
#pragma unroll
        for (uint32_t l = 0; l < NL; l++) {
            const h4* in0 = l == 0 ? X[2 * pp] : F[l][0];
            const h4* in1 = l == 0 ? X[2 * pp + 1] : F[l][1];
#pragma unroll
            for (uint32_t ob = 0; ob < lout(l) / 16; ob++) {
                f4 a0 = f4_zero(), a1 = f4_zero();
                row_times(WL + woff(l) + (16 * ob + ro) * wrow(l), lin(l) / 16, in0, in1, q, a0, a1);
                if (l < NH) {
                    F[l + 1][0][ob] = relu_h4(a0);
                    F[l + 1][1][ob] = relu_h4(a1);
                } else if (ob == 0) {
                    yt[0] = a0;
                    yt[1] = a1;
                }
            }
        }
        // output gradient of column block pb: lane r of the output tile holds primitive 16 pb + r's outputs;
        // rows 3..15 of the output block are padding (zero gradient)
        h4 G[2][NT], GT[2];
#pragma unroll
        for (uint32_t b = 0; b < 2; b++) {
            const float d0 = dy_of(round_half(yt[b][0]), gsrc[2 * pp + b][0]);
            const float d1 = dy_of(round_half(yt[b][1]), gsrc[2 * pp + b][1]);
            const float d2 = dy_of(round_half(yt[b][2]), gsrc[2 * pp + b][2]);
            G[b][0] = q == 0 ? h4{static_cast<_Float16>(d0 * s), static_cast<_Float16>(d1 * s), static_cast<_Float16>(d2 * s), z} : zero4;
            GT[b] = transpose_tile(G[b][0], eye);
        }
        // backward: dW_NH += dY X_NH^T over the pair, then layer by layer the input gradient (F-tiles, through
        // the ReLU of the input), its P-tiles and dW_{l-1} += dIn X_{l-1}^T over the pair. The P-tiles of a layer's
        // input are taken right before the layer's weight-gradient MFMAs (they do not depend on the gradients, so
        // they issue while the gradient chain runs).
        {
            h4 PT[2][KT];
#pragma unroll
            for (uint32_t b = 0; b < 2; b++)
#pragma unroll
                for (uint32_t ib = 0; ib < lin(NH) / 16; ib++) PT[b][ib] = transpose_tile(F[NH][b][ib], eye);
#pragma unroll
            for (uint32_t ib = 0; ib < lin(NH) / 16; ib++) dW[NH][0][ib] = mfma32(cat(GT[0], GT[1]), cat(PT[0][ib], PT[1][ib]), dW[NH][0][ib]);
        }
#pragma unroll
        for (int li = static_cast<int>(NH); li >= 1; li--) {
            const uint32_t l = static_cast<uint32_t>(li);
            h4 Gn[2][NT], PT[2][KT];
#pragma unroll
            for (uint32_t b = 0; b < 2; b++)
#pragma unroll
                for (uint32_t jb = 0; jb < lin(l - 1) / 16; jb++) PT[b][jb] = transpose_tile(l == 1 ? X[2 * pp + b][jb] : F[l - 1][b][jb], eye);
#pragma unroll
            for (uint32_t ib = 0; ib < lin(l) / 16; ib++) {
                f4 a0 = f4_zero(), a1 = f4_zero();
                row_times(WL + wtoff(l) + (16 * ib + ro) * wtrow(l), lout(l) / 16, G[0], G[1], q, a0, a1);
                Gn[0][ib] = relu_grad(a0, F[l][0][ib]);
                Gn[1][ib] = relu_grad(a1, F[l][1][ib]);
                const h8 gt = cat(transpose_tile(Gn[0][ib], eye), transpose_tile(Gn[1][ib], eye));
#pragma unroll
                for (uint32_t jb = 0; jb < lin(l - 1) / 16; jb++) dW[l - 1][ib][jb] = mfma32(gt, cat(PT[0][jb], PT[1][jb]), dW[l - 1][ib][jb]);
            }
#pragma unroll
            for (uint32_t ib = 0; ib < NT; ib++) {
                G[0][ib] = Gn[0][ib];
                G[1][ib] = Gn[1][ib];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // input gradient rows (F-tiles, unscaled) to the lanes through LDS (the input rows were read already)
#pragma unroll
        for (uint32_t ib = 0; ib < INP / 16; ib++) {
            f4 a0 = f4_zero(), a1 = f4_zero();
            row_times(WL + wtoff(0) + (16 * ib + ro) * wtrow(0), NT, G[0], G[1], q, a0, a1);
            *reinterpret_cast<float4*>(&fs[(16 * (2 * pp) + r) * FS + 16 * ib + 4 * q]) = make_float4(a0[0] * inv_s, a0[1] * inv_s, a0[2] * inv_s, a0[3] * inv_s);
            *reinterpret_cast<float4*>(&fs[(16 * (2 * pp + 1) + r) * FS + 16 * ib + 4 * q]) = make_float4(a1[0] * inv_s, a1[1] * inv_s, a1[2] * inv_s, a1[3] * inv_s);
        }
        __builtin_amdgcn_sched_barrier(0);  // one pass in flight: bounds the live activations
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
