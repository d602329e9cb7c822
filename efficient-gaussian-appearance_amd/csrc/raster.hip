// Binning stages between preprocess and blend: deterministic compaction of visible primitives, instance
// emission in depth order, and per-tile instance ranges. Compiled with -ffp-contract=off: instance emission
// re-evaluates the tile test of the preprocess and must reproduce its counts exactly.
// Reference: B/rasterization/include/kernels_common.cuh:20-157, B/rasterization/src/forward.cu:82-221.
#include "internal.h"

namespace efgs {

namespace {

__global__ void fill_u32_kernel(uint32_t* p, uint32_t value, uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

// primitive-index-ordered compaction of (depth key - min depth key, primitive) for the visible primitives
__global__ __launch_bounds__(preprocess_block) void compact_visible_kernel(const uint32_t* n_touched, const uint32_t* depth_keys,
                                                                          const uint32_t* block_offsets, const uint32_t* counters,
                                                                          uint32_t* keys_out, uint32_t* vals_out, uint32_t* visible_out,
                                                                          uint32_t n) {
    __shared__ uint32_t wave_counts[preprocess_block / 64];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t p = blockIdx.x * preprocess_block + threadIdx.x;
    const bool visible = p < n && n_touched[p] > 0;
    const uint64_t mask = __ballot(visible);
    if (lane == 0) wave_counts[wave] = static_cast<uint32_t>(__popcll(mask));
    __syncthreads();
    if (!visible) return;
    uint32_t pos = block_offsets[2 * blockIdx.x];
    for (uint32_t w = 0; w < wave; w++) pos += wave_counts[w];
    pos += static_cast<uint32_t>(__popcll(mask & ((1ull << lane) - 1ull)));
    keys_out[pos] = depth_keys[p] - counters[3];
    vals_out[pos] = p;
    visible_out[pos] = p;  // kept in index order for the backward (the sort overwrites vals_out)
}

// One thread per visible primitive in depth order: emits (tile key, primitive) for every tile of its tile
// rectangle that passes the contribution test, the first 4 tiles per lane and larger footprints
// wave-cooperatively (64 tiles per step, positions from ballot prefix counts). Emission slots are
// [offset, offset + n_touched); a count that disagrees with the preprocess is clamped to that range, the
// remainder padded with an out-of-range key and counted in counters[2].
template <typename KeyT>
__global__ __launch_bounds__(instance_block) void create_instances_kernel(const uint32_t* sorted_prims, const uint32_t* offsets,
                                                                         const uint32_t* n_touched, const PrimRecord* records,
                                                                         KeyT* keys, uint32_t* inst_prim, uint32_t* prim_offset,
                                                                         uint32_t* counters, uint32_t grid_w, uint32_t n_visible) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    const uint32_t i_raw = blockIdx.x * instance_block + threadIdx.x;
    const bool active = i_raw < n_visible;
    const uint32_t i = active ? i_raw : n_visible - 1;
    const uint32_t p = sorted_prims[i];
    const uint32_t off = offsets[i];
    const uint32_t n = n_touched[p];
    if (active) prim_offset[p] = off;
    const PrimRecord rec = records[p];
    const uint32_t bx = __float_as_uint(rec.r2.y), by = __float_as_uint(rec.r2.z);
    const TileRect t = screen_to_tile_bounds(bx & 0xffffu, bx >> 16, by & 0xffffu, by >> 16);
    const uint32_t bw = t.x1 - t.x0;
    const uint32_t cnt = active ? bw * (t.y1 - t.y0) : 0u;
    const float smx = rec.r0.x - 0.5f, smy = rec.r0.y - 0.5f;
    const float cx = rec.r0.z, cy = rec.r0.w, cz = rec.r1.x;
    const float pt = power_threshold_of(rec.r1.y);
    uint32_t k = 0;
    for (uint32_t j = 0; j < cnt && j < 4; j++) {
        const uint32_t tx = t.x0 + j % bw, ty = t.y0 + j / bw;
        if (will_primitive_contribute(smx, smy, cx, cy, cz, tx, ty, pt)) {
            if (k < n) {
                keys[off + k] = static_cast<KeyT>(ty * grid_w + tx);
                inst_prim[off + k] = p;
            }
            k++;
        }
    }
    uint64_t coop = __ballot(cnt > 4);
    while (coop != 0) {
        const uint32_t src = static_cast<uint32_t>(__ffsll(static_cast<long long>(coop)) - 1);
        coop &= coop - 1;
        const uint32_t c_x0 = __shfl(t.x0, src), c_y0 = __shfl(t.y0, src), c_bw = __shfl(bw, src), c_cnt = __shfl(cnt, src);
        const uint32_t c_off = __shfl(off, src), c_n = __shfl(n, src), c_p = __shfl(p, src);
        const float c_mx = __shfl(smx, src), c_my = __shfl(smy, src);
        const float c_cx = __shfl(cx, src), c_cy = __shfl(cy, src), c_cz = __shfl(cz, src), c_pt = __shfl(pt, src);
        uint32_t c_k = __shfl(k, src);
        for (uint32_t base = 4; base < c_cnt; base += 64) {
            const uint32_t j = base + lane;
            const uint32_t tx = c_x0 + j % c_bw, ty = c_y0 + j / c_bw;
            const bool hit = j < c_cnt && will_primitive_contribute(c_mx, c_my, c_cx, c_cy, c_cz, tx, ty, c_pt);
            const uint64_t m = __ballot(hit);
            const uint32_t pos = c_k + static_cast<uint32_t>(__popcll(m & lanes_below));
            if (hit && pos < c_n) {
                keys[c_off + pos] = static_cast<KeyT>(ty * grid_w + tx);
                inst_prim[c_off + pos] = c_p;
            }
            c_k += static_cast<uint32_t>(__popcll(m));
        }
        if (lane == src) k = c_k;
    }
    if (active && k != n) {
        for (uint32_t j = (k < n ? k : n); j < n; j++) {
            keys[off + j] = static_cast<KeyT>(~static_cast<KeyT>(0));
            inst_prim[off + j] = p;
        }
        atomicAdd(&counters[2], 1u);
    }
}

// out[i] = sum over blocks b of partials[b][i]. A block covers 64 parameters with 16 groups of 64 lanes;
// group g sums blocks g, g + 16, ... in order, then the 16 group sums are added in group order (fixed
// order, reproducible).
constexpr uint32_t reduce_groups = 16;
__global__ __launch_bounds__(64 * reduce_groups) void reduce_partials_kernel(const float* partials, uint32_t n_blocks, uint32_t n_params,
                                                                          float* out) {
    __shared__ float s_part[reduce_groups][64];
    const uint32_t lane = threadIdx.x & 63u, g = threadIdx.x >> 6;
    const uint32_t i = blockIdx.x * 64u + lane;
    float acc = 0.0f;
    if (i < n_params) {
#pragma unroll 4
        for (uint32_t b = g; b < n_blocks; b += reduce_groups) acc += partials[static_cast<size_t>(b) * n_params + i];
    }
    s_part[g][lane] = acc;
    __syncthreads();
    if (g == 0 && i < n_params) {
        float t = s_part[0][lane];
        for (uint32_t k = 1; k < reduce_groups; k++) t += s_part[k][lane];
        out[i] = t;
    }
}

template <typename KeyT>
__global__ void tile_ranges_kernel(const KeyT* keys, uint2* ranges, uint32_t n_instances, uint32_t n_tiles) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_instances) return;
    const uint32_t key = static_cast<uint32_t>(keys[i]);
    const bool valid = key < n_tiles;
    const uint32_t prev = i > 0 ? static_cast<uint32_t>(keys[i - 1]) : 0xffffffffu;
    if (key != prev) {
        if (prev < n_tiles) ranges[prev].y = i;
        if (valid) ranges[key].x = i;
    }
    if (i == n_instances - 1 && valid) ranges[key].y = n_instances;
}

}  // namespace

bool launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, hipStream_t s) {
    if (n == 0) return true;
    fill_u32_kernel<<<div_up(n, 256), 256, 0, s>>>(p, value, n);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_compact_visible(const uint32_t* n_touched, const uint32_t* depth_keys, const uint32_t* block_offsets, const uint32_t* counters,
                            uint32_t* keys_out, uint32_t* vals_out, uint32_t* visible_out, uint32_t n, hipStream_t s) {
    compact_visible_kernel<<<div_up(n, preprocess_block), preprocess_block, 0, s>>>(n_touched, depth_keys, block_offsets, counters, keys_out,
                                                                                     vals_out, visible_out, n);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_create_instances(const uint32_t* sorted_prims, const uint32_t* offsets, const uint32_t* n_touched, const PrimRecord* records,
                             void* keys, int key_bytes, uint32_t* inst_prim, uint32_t* prim_offset, uint32_t* counters, uint32_t grid_w,
                             uint32_t n_visible, hipStream_t s) {
    if (n_visible == 0) return true;
    const uint32_t blocks = div_up(n_visible, instance_block);
    if (key_bytes == 2)
        create_instances_kernel<uint16_t><<<blocks, instance_block, 0, s>>>(sorted_prims, offsets, n_touched, records, static_cast<uint16_t*>(keys),
                                                                           inst_prim, prim_offset, counters, grid_w, n_visible);
    else
        create_instances_kernel<uint32_t><<<blocks, instance_block, 0, s>>>(sorted_prims, offsets, n_touched, records, static_cast<uint32_t*>(keys),
                                                                           inst_prim, prim_offset, counters, grid_w, n_visible);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_reduce_partials(const float* partials, uint32_t n_blocks, uint32_t n_params, float* out, hipStream_t s) {
    if (n_params == 0) return true;
    reduce_partials_kernel<<<div_up(n_params, 64), 64 * reduce_groups, 0, s>>>(partials, n_blocks, n_params, out);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_tile_ranges(const void* keys, int key_bytes, uint2* ranges, uint32_t n_instances, uint32_t n_tiles, hipStream_t s) {
    if (!launch_fill_u32(reinterpret_cast<uint32_t*>(ranges), 0u, 2ull * n_tiles, s)) return false;
    if (n_instances == 0) return true;
    if (key_bytes == 2)
        tile_ranges_kernel<uint16_t><<<div_up(n_instances, 256), 256, 0, s>>>(static_cast<const uint16_t*>(keys), ranges, n_instances, n_tiles);
    else
        tile_ranges_kernel<uint32_t><<<div_up(n_instances, 256), 256, 0, s>>>(static_cast<const uint32_t*>(keys), ranges, n_instances, n_tiles);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
