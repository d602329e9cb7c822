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
// [5] 1 when I exceeds the instance capacity the binning buffers were laid out for (the binning and blend kernels
// then return at once; the host re-runs them with buffers of the exact size); the host's copy also holds, in
// [counter_sequence], the sequence number of the frame whose counters it holds (written last)
constexpr uint32_t n_counters = 8;
constexpr uint32_t counter_overflow = 5;
constexpr uint32_t counter_sequence = 7;
bool launch_scan_block_counts(const uint32_t* block_counts, const uint32_t* key_ranges, uint32_t* block_offsets, uint32_t* counters,
                              uint32_t* host_counters, uint32_t instance_capacity, uint32_t seq, uint32_t n_blocks, hipStream_t s);
// visible primitives in index order and their first emission slots (exclusive scan of the tile counts in
// index order)
bool launch_compact_visible(const uint32_t* n_touched, const uint32_t* block_offsets, uint32_t* visible_out, uint32_t* prim_offset, uint32_t n,
                            hipStream_t s);
// Tile binning: per-tile counts from LDS histograms over segments of contiguous primitives (their emission slots
// are contiguous; a table of per-segment counts, scanned per tile) when the tile count fits the LDS (the fused
// emission), else from global atomics.
constexpr size_t tile_hist_max_lds = 64 * 1024;    // default dynamic LDS limit of a launch
constexpr uint32_t tile_hist_max_blocks = 256;     // segments (the rank word keeps the segment in its top 8 bits)
constexpr uint32_t rank_segment_shift = 24;        // rank word: rank within the segment's instances of the tile | segment << 24
struct TileBinning {
    bool use_table;
    uint32_t blocks;   // histogram blocks (segments, rows of the table)
    uint32_t segment;  // visible primitives per segment
};
struct CreateInstancesArgs {
    const uint32_t* visible_prims;
    const uint32_t* prim_offset;
    uint32_t* visible_prims_out;   // the fused path writes the compaction (the same arrays)
    uint32_t* prim_offset_out;
    uint32_t* n_touched;
    const PrimRecord* records;
    void* keys;                // tile key per emission slot, key_bytes wide
    uint32_t* inst_prim;
    uint32_t* counters;        // the visible count is read here ([0]); nothing is emitted when [counter_overflow] is set
    uint32_t grid_w;
    uint32_t max_visible;      // bound on the visible count (grid size of the path without a table)
    uint32_t n_visible;        // set by the kernels from counters[0]
};
// The fused path's inputs: the preprocess's per-chunk counts and depth-key ranges, the instance capacity of the
// binning buffers, and the host's mapped copy of the counters with the frame's sequence number.
struct FusedBinningArgs {
    const uint32_t* block_counts;
    const uint32_t* key_ranges;
    uint32_t* host_counters;
    uint32_t n_prims, n_chunks, chunks_per_segment, capacity, seq;
};
// whether the fused emission's LDS (tile histogram and compaction buffers) fits a launch
bool fused_binning_fits(uint32_t n_tiles);
// segments of whole preprocess chunks for the fused emission (blocks = segments)
TileBinning fused_binning_plan(uint32_t n_prims, uint32_t n_tiles, uint32_t& chunks_per_segment);
// (tile key, primitive) at every emission slot; with a table also each instance's rank | segment << 24 and the
// segments' per-tile counts (plan.blocks segments of ceil(V / plan.blocks) visible primitives). With `fused` the
// emission also does the counter scan and the compaction (segments of whole preprocess chunks).
bool launch_create_instances(const CreateInstancesArgs& a, int key_bytes, const TileBinning& plan, uint32_t* local_rank, uint32_t* table,
                             uint32_t n_tiles, const FusedBinningArgs* fused, hipStream_t s);
// Tile scan state (tile arena): totals[t] instances of tile t, local_start[t] exclusive scan of the totals within
// t's 64-tile block, block_sums per 64-tile block (tile t starts at the sum of block_sums over the blocks before
// t / 64 plus local_start[t]), and a per-tile cursor for the global-atomic path.
// Heaviest tile first: the one-block-per-tile blends run their blocks in a permutation of the tiles ordered by
// instance count, descending (longest-processing-time-first list scheduling, so that a kernel's last blocks are
// short ones). The count is bucketed into 64 classes (1 + 4 floor(log2 n) + the next two bits, reversed; an empty
// tile is the last class); the column scan counts each 64-tile block's tiles per class and gives every tile its
// rank among them (lane order), one small kernel turns the counts into each (block, class) run's first position,
// and the tile sort writes every tile at its position. Deterministic; a tile's result does not depend on it.
constexpr uint32_t order_classes = 64;
struct TileScan {
    uint32_t* totals;
    uint32_t* local_start;
    uint32_t* block_sums;
    uint32_t* cursor;
    uint32_t* order_runs;  // per 64-tile block and class: the class's tiles in the block, then their first position
    uint32_t* order_rank;  // per tile: class << 16 | rank among the block's tiles of its class
    uint32_t* order;       // the tile order (block b of a blend runs tile order[b])
    const uint32_t* counters;  // instance count ([1]) and overflow flag ([counter_overflow]) on the device
};
// per-tile counts (global atomics without a table) and the scan above
// (max_instances: bound on the instance count, the grid size of the path without a table; the kernels read the
// count itself from ts.counters)
bool launch_tile_counts(const TileBinning& plan, const void* keys, int key_bytes, uint32_t max_instances, uint32_t* table, const TileScan& ts,
                        uint32_t n_tiles, hipStream_t s);
// every instance's bucket entry (emission index, depth key of its primitive, primitive, 0; the low 8 bytes are the
// sort key depth key << 32 | emission index) into a slot of its tile's range
bool launch_tile_buckets(const TileBinning& plan, const void* keys, int key_bytes, const uint32_t* inst_prim, const uint32_t* depth_keys,
                         const uint32_t* table, const uint32_t* local_rank, const TileScan& ts, uint4* bucket, uint32_t max_instances,
                         uint32_t n_tiles, hipStream_t s);
// per tile: [start, end) into ranges and its place in the blends' tile order (the runs are sorted by the forward blend)
bool launch_tile_ranges(const TileScan& ts, uint2* ranges, uint32_t n_tiles, hipStream_t s);
bool launch_reduce_partials(const float* partials, uint32_t n_blocks, uint32_t n_params, float* out, hipStream_t s);

struct BlendForwardArgs {
    const uint2* ranges;
    uint4* bucket;                 // per tile slot: emission index, depth key, primitive, 0 (unsorted; runs of more
                                   // than 512 are sorted in chunks in place)
    uint32_t* sorted_inst;         // emission index per sorted instance (written here)
    uint32_t* sorted_prim;         // primitive per sorted instance (written here)
    void* sorted_keys;             // tile key per sorted instance (key_bytes wide; written here)
    const uint32_t* inst_prim;     // primitive per emission index
    const uint32_t* counters;      // frame counters (counters[1]: the instance count)
    uint32_t key_bytes;
    const PrimRecord* records;
    const float* bg;
    float* image;                  // (3, H, W), or (H, W, 3) with hwc
    float* final_T;                // (tiles x 192); null for an inference render (no backward state)
    uint32_t* n_contrib;           // (tiles x 192)
    uint32_t* tile_max;            // (tiles)
    const uint32_t* order;         // tile of each block, heaviest first (null: block index)
    const uint32_t* overflow;      // nothing is rendered when *overflow != 0 (null: never)
    uint32_t width, height, grid_w, n_tiles;
    uint32_t hwc;                  // image layout (H, W, 3)
    uint32_t clamp;                // image clamped to [0, 1] (NaN to 0)
};
bool launch_blend_forward(const BlendForwardArgs& a, hipStream_t s);

struct BlendBackwardArgs {
    const uint2* ranges;
    const uint32_t* sorted_inst;   // emission index per sorted instance
    const uint32_t* sorted_prim;   // primitive per sorted instance
    const PrimRecord* records;
    const float* bg;
    const float* image;
    const float* grad_image;
    const float* final_T;
    const uint32_t* n_contrib;
    const uint32_t* tile_max;
    const uint32_t* order;         // tile of each block, heaviest first (null: block index)
    float* inst_grads;             // (I x 9, or I x 12 with abs_grads), emission order (pruning scores: one float per instance)
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

// ---- .ngsplat packing ----------------------------------------------------------------------------------------------
enum NgsplatPayload { ng_neural_features = 0, ng_neural_baked = 1, ng_sh = 2, ng_sv = 3, ng_nasg = 4, ng_nasgabor = 5 };
constexpr uint32_t ng_block = 256;          // splats (and output rows) per block
constexpr uint32_t ng_tex_width = 2048;     // texture width of the format: output rows come in multiples of it
constexpr uint32_t ng_max_row = 63;         // residual parameters per splat staged in LDS
constexpr uint32_t ng_max_values = 64;      // fp16 payload values per splat (8 textures of 8)
constexpr uint32_t ng_max_baked = 16;       // neurons of a baked layer 0
constexpr uint32_t ng_max_textures = 8;
struct NgsplatArgs {
    const float* means;            // N x 3
    const float* raw_scales;       // N x 3 log scales
    const float* raw_rotations;    // N x 4 (w, x, y, z), unnormalised
    const float* raw_opacities;    // N logits
    const float* base_colors;      // N x 3
    const float* residual_params;  // N x row_stride; the first row_used floats of each row are read
    const float* bake_matrix;      // baked neural: n_values x n_encoded, row-major
    const float* bake_bias;        // baked neural: n_values, or null
    uint32_t n, row_stride, row_used;
    int payload;                   // NgsplatPayload
    int n_items;                   // SH: coefficients exported; SV: sites; NASG / NASGabor: lobes; neural: raw features
    int n_values;                  // fp16 values per splat (neural, SV, NASG, NASGabor)
    int n_encoded;                 // neural: encoded feature width
    int base_input;                // neural: the raw base colours follow the features
    int n_frequencies;             // neural: frequency encoding (0 = identity)
    int residual_act;              // SV / NASG / NASGabor: residual activation baked into the colours
    float color_shift;             // added to the base colour before quantisation
};
struct NgsplatTextures {
    uint32_t* splat_words;         // capacity x 4
    uint32_t* params;              // payload textures back to back
    int32_t* source_index;         // capacity, optional
    uint32_t capacity;             // rows per texture, a multiple of ng_tex_width
    int n_textures;
    uint32_t texel_words[ng_max_textures];
    uint64_t texture_offset[ng_max_textures];  // u32 offset of each payload texture in params
};
// device-side result of the statistics pass, copied to the host
struct NgsplatStats {
    uint32_t n_kept;
    float base_offset, base_scale;
    float level_scale[3];
};
// u32 words per payload texture (SH: per level present) for a payload description; returns the texture count
int ngsplat_texture_plan(int payload, int n_items, int n_values, uint32_t* texel_words);
// statistics, block prefix and packing; `partials` holds div_up(capacity, ng_block) * 8 u32, `stats` one NgsplatStats;
// `events` (optional, three) are recorded before the statistics kernel, before and after the pack kernel
bool launch_ngsplat_pack(const NgsplatArgs& a, const NgsplatTextures& t, uint32_t* partials, NgsplatStats* stats, hipEvent_t* events,
                         hipStream_t s);

}  // namespace efgs
