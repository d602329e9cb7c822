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

constexpr uint32_t preprocess_block = 256;
constexpr uint32_t instance_block = 256;

inline uint32_t div_up(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

// ---- rasterizer stages -------------------------------------------------------------------------------------
bool launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, hipStream_t s);
// counters: [0] V, [1] I, [2] instance-emission mismatches, [3] / [4] min / max depth key of the visible set,
// [5] ticket of the tile scan's last block
constexpr uint32_t n_counters = 8;
bool launch_scan_block_counts(const uint32_t* block_counts, const uint32_t* key_ranges, uint32_t* block_offsets, uint32_t* counters,
                              uint32_t n_blocks, hipStream_t s);
// visible primitives in index order and their first emission slots (exclusive scan of the tile counts in
// index order)
bool launch_compact_visible(const uint32_t* n_touched, const uint32_t* block_offsets, uint32_t* visible_out, uint32_t* prim_offset, uint32_t n,
                            hipStream_t s);
// (tile key, primitive) at every emission slot
bool launch_create_instances(const uint32_t* visible_prims, const uint32_t* prim_offset, const uint32_t* n_touched, const PrimRecord* records,
                             void* keys, int key_bytes, uint32_t* inst_prim, uint32_t* counters, uint32_t grid_w, uint32_t n_visible,
                             hipStream_t s);
// Tile binning: per-tile counts from LDS histograms over fixed segments of the emission slots (a table of
// per-segment counts, scanned per tile) when the tile count fits the LDS, else from global atomics.
constexpr size_t tile_hist_max_lds = 64 * 1024;  // default dynamic LDS limit of a launch
constexpr uint32_t tile_hist_min_segment = 16384;  // emission slots per histogram block (at least)
constexpr uint32_t tile_hist_max_blocks = 128;
struct TileBinning {
    bool use_table;
    uint32_t blocks;   // histogram blocks (rows of the table)
    uint32_t segment;  // emission slots per histogram block
};
TileBinning tile_binning_plan(uint32_t n_instances, uint32_t n_tiles);
// Tile scan state (tile arena): totals[t] instances of tile t, local_start[t] exclusive scan of the totals
// within t's 256-tile block, block_prefix[t / 256] the totals of the earlier blocks (tile t starts at
// block_prefix[t / 256] + local_start[t]), block_sums per 256-tile block, the ticket of the block that scans
// them (counters[5], zeroed by scan_block_counts), and a per-tile cursor for the global-atomic path.
struct TileScan {
    uint32_t* totals;
    uint32_t* local_start;
    uint32_t* block_sums;
    uint32_t* block_prefix;
    uint32_t* ticket;
    uint32_t* cursor;
};
// per-tile counts (LDS histograms over segments of the emission slots with per-instance ranks and the
// segment table, or global atomics) and the scan above
bool launch_tile_counts(const TileBinning& plan, const void* keys, int key_bytes, uint32_t n_instances, uint32_t* local_rank, uint32_t* table,
                        const TileScan& ts, uint32_t n_tiles, hipStream_t s);
// every instance's sort key (depth key of its primitive << 32 | emission index) into a slot of its tile's range
bool launch_tile_buckets(const TileBinning& plan, const void* keys, int key_bytes, const uint32_t* inst_prim, const uint32_t* depth_keys,
                         const uint32_t* table, const uint32_t* local_rank, const TileScan& ts, uint64_t* bucket, uint32_t n_instances,
                         uint32_t n_tiles, hipStream_t s);
// per tile: [start, end) into ranges and its keys sorted ascending -> emission indices in sorted_inst, tile id
// in sorted_keys
bool launch_tile_sort(const TileScan& ts, uint2* ranges, uint64_t* bucket, uint32_t* sorted_inst, void* sorted_keys, int key_bytes,
                      uint32_t n_tiles, hipStream_t s);
bool launch_reduce_partials(const float* partials, uint32_t n_blocks, uint32_t n_params, float* out, hipStream_t s);

struct BlendForwardArgs {
    const uint2* ranges;
    const uint32_t* sorted_inst;   // emission index per sorted instance
    const uint32_t* inst_prim;     // primitive per emission index
    const PrimRecord* records;
    const float* bg;
    float* image;                  // (3, H, W), or (H, W, 3) with hwc
    float* final_T;                // (tiles x 192); null for an inference render (no backward state)
    uint32_t* n_contrib;           // (tiles x 192)
    uint32_t* tile_max;            // (tiles)
    uint32_t width, height, grid_w, n_tiles;
    uint32_t hwc;                  // image layout (H, W, 3)
    uint32_t clamp;                // image clamped to [0, 1] (NaN to 0)
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
    float* inst_grads;             // (I x 12), emission order (pruning scores: one float per instance)
    uint32_t width, height, grid_w, n_tiles;
    uint32_t abs_grads;            // also reduce |dL/dmean2d| (third densification row)
};
bool launch_blend_backward(const BlendBackwardArgs& a, hipStream_t s);
// pruning scores of the frame in `a` (grad_image unused): per-instance scores into a.inst_grads, then
// scores[p] += their per-primitive sums
bool launch_pruning_scores(const BlendBackwardArgs& a, const uint32_t* n_touched, const uint32_t* prim_offset, float* scores, uint32_t n,
                           hipStream_t s);

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

// ---- MCMC densification ---------------------------------------------------------------------------------------
constexpr uint32_t mcmc_max_samples = 50;  // samples per relocated Gaussian (larger counts are clamped)
bool launch_add_noise(const float* raw_scales, const float* raw_rotations, const float* raw_opacities, float* means, uint32_t n, float lr,
                      uint64_t seed, uint64_t offset, hipStream_t s);
bool launch_relocation(const float* old_opacities, const float* old_scales, const int64_t* n_samples, float* new_opacities, float* new_scales,
                       uint32_t n, hipStream_t s);

}  // namespace efgs
