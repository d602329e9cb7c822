// Internal declarations shared by the C-ABI layer and the ahead-of-time kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <string>

#include "rtc/efgs_common.h"
#include "rtc/efgs_args.h"

namespace efgs {

// error state of the calling thread, read through efgs_last_error()
void set_error(const std::string& msg);

#define EFGS_HIP_CHECK(expr)                                                                              \
    do {                                                                                                  \
        hipError_t e_ = (expr);                                                                           \
        if (e_ != hipSuccess) {                                                                           \
            ::efgs::set_error(std::string(#expr " failed: ") + hipGetErrorString(e_));                  \
            return false;                                                                                 \
        }                                                                                                 \
    } while (0)

constexpr uint32_t sort_block = 256;
constexpr uint32_t sort_rounds = 8;                     // keys per thread per sort tile
constexpr uint32_t sort_tile = sort_block * sort_rounds;  // 2048 keys per block
constexpr uint32_t sort_bins = 256;                     // 8-bit digits
constexpr uint32_t scan_block = 256;
constexpr uint32_t scan_items = 8;
constexpr uint32_t scan_tile = scan_block * scan_items;   // 2048 elements per block
constexpr uint32_t preprocess_block = 256;
constexpr uint32_t instance_block = 256;

inline uint32_t div_up(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

// ---- device-wide exclusive scan of uint32 (optionally gathering in[idx[i]]) --------------------------------
size_t scan_scratch_bytes(uint32_t n);
// out[i] = sum_{k<i} v(k), v(k) = idx ? in[idx[k]] : in[k]; total (if non-null) receives the full sum
bool scan_exclusive(const uint32_t* in, const uint32_t* idx, uint32_t* out, uint32_t* total, uint32_t n, void* scratch, hipStream_t s);

// ---- stable LSD radix sort of (key, value) pairs ------------------------------------------------------------
// keys are uint32 or uint16 (key_bytes 4 or 2), values uint32; vals_in == nullptr means values = index.
// Ping-pongs between (keys_a, vals_a) and (keys_b, vals_b); returns in *result_in_b whether the sorted data
// ended in the b buffers.
size_t sort_scratch_bytes(uint32_t n);
bool radix_sort_pairs(void* keys_a, uint32_t* vals_a, void* keys_b, uint32_t* vals_b, bool identity_vals, uint32_t n,
                      int key_bytes, int end_bit, void* scratch, bool* result_in_b, hipStream_t s);

// ---- rasterizer stages -------------------------------------------------------------------------------------
bool launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, hipStream_t s);
// counters: [0] V, [1] I, [2] instance-emission mismatches, [3] / [4] min / max depth key of the visible set
constexpr uint32_t n_counters = 8;
bool launch_scan_block_counts(const uint32_t* block_counts, const uint32_t* key_ranges, uint32_t* block_offsets, uint32_t* counters,
                              uint32_t n_blocks, hipStream_t s);
// compacted depth keys are stored relative to counters[3] (order preserving; fewer radix passes); the
// primitive indices go to vals_out (sort input) and visible_out (kept in index order)
bool launch_compact_visible(const uint32_t* n_touched, const uint32_t* depth_keys, const uint32_t* block_offsets, const uint32_t* counters,
                            uint32_t* keys_out, uint32_t* vals_out, uint32_t* visible_out, uint32_t n, hipStream_t s);
bool launch_create_instances(const uint32_t* sorted_prims, const uint32_t* offsets, const uint32_t* n_touched,
                             const PrimRecord* records, void* keys, int key_bytes, uint32_t* inst_prim, uint32_t* prim_offset,
                             uint32_t* counters, uint32_t grid_w, uint32_t n_visible, hipStream_t s);
bool launch_reduce_partials(const float* partials, uint32_t n_blocks, uint32_t n_params, float* out, hipStream_t s);
bool launch_tile_ranges(const void* keys, int key_bytes, uint2* ranges, uint32_t n_instances, uint32_t n_tiles, hipStream_t s);

struct BlendForwardArgs {
    const uint2* ranges;
    const uint32_t* sorted_inst;   // emission index per sorted instance
    const uint32_t* inst_prim;     // primitive per emission index
    const PrimRecord* records;
    const float* bg;
    float* image;                  // (3, H, W)
    float* final_T;                // (tiles x 192)
    uint32_t* n_contrib;           // (tiles x 192)
    uint32_t* tile_max;            // (tiles)
    uint32_t width, height, grid_w, n_tiles;
};
bool launch_blend_forward(const BlendForwardArgs& a, hipStream_t s);

struct BlendBackwardArgs {
    const uint2* ranges;
    const uint32_t* sorted_inst;
    const uint32_t* inst_prim;
    const PrimRecord* records;
    const float* bg;
    const float* image;
    const float* grad_image;
    const float* final_T;
    const uint32_t* n_contrib;
    const uint32_t* tile_max;
    float* inst_grads;             // (I x 12), emission order
    uint32_t width, height, grid_w, n_tiles;
    uint32_t abs_grads;            // also reduce |dL/dmean2d| (third densification row)
};
bool launch_blend_backward(const BlendBackwardArgs& a, hipStream_t s);

// ---- adam ---------------------------------------------------------------------------------------------------
constexpr int adam_max_lrs = 7;
constexpr int adam_max_groups = 16;
struct AdamGroupDevice {
    const float* grad;
    float* param;
    float* m;
    float* v;
    uint64_t n;
    float step_sizes[adam_max_lrs];  // lr * 1/(1 - beta1^t)
    int n_lrs;
    float beta1, beta2, eps, bc2_sqrt_rcp;
    uint32_t first_block;
};
bool launch_adam(const AdamGroupDevice* groups, int n_groups, hipStream_t s);

}  // namespace efgs
