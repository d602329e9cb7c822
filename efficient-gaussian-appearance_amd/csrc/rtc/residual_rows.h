// Per-primitive residual parameters of the preprocess kernels: their count and the LDS staging of a block's rows.
#pragma once

namespace efgs {

// floats per appearance unit (SH coefficient rgb, SV site, NASG lobe, NASGabor lobe) and per primitive
constexpr uint32_t params_per_unit = EFGS_MODEL == 1 ? 3u : EFGS_MODEL == 2 ? 7u : EFGS_MODEL == 3 ? 8u : EFGS_MODEL == 4 ? 9u : 1u;
constexpr uint32_t residual_params = EFGS_MODEL == 0 ? 0u : params_per_unit * EFGS_N_UNITS;

// Residual rows of a block staged through LDS with coalesced loads (a thread's own row is 45-72 floats apart from
// its neighbours', so direct per-thread reads spread every load instruction of a wave over 64 cache lines). Whole
// units per pass: SH (coefficients) and SV (sites: the backward's softmax needs them all) in one pass, lobes in
// passes of at most MAX_FLOATS floats; a layout that does not fit reads its rows directly. Fewer floats per pass
// mean less LDS per block and more waves per SIMD, at one barrier and one staging round more per pass (the SV
// forward in passes of two sites, its softmax carried online, measured 105 -> 131 us: it stays unstaged): the lobe
// forward runs best at 18 (2 lobes per pass; NASG 149 -> 119 us, NASGabor 233 -> 162 us on 1M Gaussians against
// 40), the lobe backward, which also writes its gradients back through the rows, at 40 (24: 221 -> 310 us).
template <uint32_t MAX_FLOATS>
struct RowStaging {
    static constexpr uint32_t max_floats = EFGS_MODEL == 1 || EFGS_MODEL == 2 ? 63u : MAX_FLOATS;
    static constexpr uint32_t units_fit = params_per_unit > 0 ? max_floats / params_per_unit : 0u;
    static constexpr uint32_t pass_units = EFGS_MODEL == 1 || EFGS_MODEL == 2 ? EFGS_N_UNITS
                                                                               : (units_fit < EFGS_N_UNITS ? units_fit : EFGS_N_UNITS);
    static constexpr bool staged = EFGS_MODEL != 0 && EFGS_N_UNITS > 0 && pass_units > 0 && pass_units * params_per_unit <= max_floats;
    static constexpr uint32_t row_ld = (pass_units * params_per_unit) | 1u;
    static constexpr uint32_t n_passes = pass_units > 0 ? (EFGS_N_UNITS + pass_units - 1) / pass_units : 0u;
};
using ForwardRows = RowStaging<18u>;
using BackwardRows = RowStaging<40u>;

// rows [p0, p0 + rows), floats [f0, f0 + floats) of each, into s[r * ROW_LD + c] by the BLOCK threads of the block;
// (r, c) advance by (BLOCK / floats, BLOCK % floats) per step, eight loads in flight
template <uint32_t BLOCK, uint32_t ROW_LD>
__device__ __forceinline__ void stage_residual_rows(const float* residual, uint32_t p0, uint32_t rows, uint32_t f0, uint32_t floats, float* s) {
    const uint32_t total = rows * floats, dr = BLOCK / floats, dc = BLOCK - dr * floats;
    uint32_t r = threadIdx.x / floats, c = threadIdx.x - r * floats;
#pragma unroll 8
    for (uint32_t i = threadIdx.x; i < total; i += BLOCK) {
        s[r * ROW_LD + c] = residual[static_cast<size_t>(p0 + r) * residual_params + f0 + c];
        c += dc;
        r += dr;
        const bool wrap = c >= floats;
        c = wrap ? c - floats : c;
        r = wrap ? r + 1 : r;
    }
}

// the reverse of stage_residual_rows: s[r * ROW_LD + c] to rows [p0, p0 + rows), floats [f0, f0 + floats) of `out`
template <uint32_t BLOCK, uint32_t ROW_LD>
__device__ __forceinline__ void store_residual_rows(const float* s, uint32_t p0, uint32_t rows, uint32_t f0, uint32_t floats, float* out) {
    const uint32_t total = rows * floats, dr = BLOCK / floats, dc = BLOCK - dr * floats;
    uint32_t r = threadIdx.x / floats, c = threadIdx.x - r * floats;
#pragma unroll 8
    for (uint32_t i = threadIdx.x; i < total; i += BLOCK) {
        out[static_cast<size_t>(p0 + r) * residual_params + f0 + c] = s[r * ROW_LD + c];
        c += dc;
        r += dr;
        const bool wrap = c >= floats;
        c = wrap ? c - floats : c;
        r = wrap ? r + 1 : r;
    }
}

}  // namespace efgs
