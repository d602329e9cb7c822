// Binning stages between preprocess and blend. The reference orders instances in two global sorts: a
// 32-bit radix sort of the visible primitives by depth, emission of (tile, primitive) instances in that
// order, then a stable radix sort by tile. This build reaches the same per-tile order, (depth, primitive
// index), without a global sort:
//   create_instances    (fused, grids whose tile histogram fits the LDS) blocks of contiguous primitives scan
//                       the preprocess's tile counts (the compaction: visible primitives in index order and
//                       their first emission slots) and emit (tile key, primitive) at the emission slots, the
//                       tile test of the preprocess for every tile past its recorded first ones; each block
//                       counts its instances per tile in an LDS histogram (ranks from the atomics' return
//                       values) and writes its row of the segment x tile table. Larger grids: compact_visible,
//                       then one thread per visible primitive, counted per tile with global atomics;
//   tile_column_scan    the segments' counts per tile -> prefixes over the segments, tile totals and starts,
//                       and each tile's size class for the blends' heaviest-first tile order;
//   tile_buckets        every instance writes its entry (emission index, depth key, primitive) at tile start +
//                       earlier segments' count + rank; one extra block turns the size-class counts into the
//                       tile order's run positions meanwhile;
//   tile_ranges         every tile's instance range and its place in the tile order.
// The forward blend then sorts each tile's entries by (depth key, emission index) before it walks them (keys are
// unique, so the order is a deterministic function of the inputs; the emission index increases with the
// primitive index, so ties in depth keep primitive-index order) and writes the emission indices and primitives
// in that order for the backward.
// Compiled with -ffp-contract=off: instance emission re-evaluates the tile test of the preprocess and must
// reproduce its counts exactly.
// Reference: B/rasterization/include/kernels_common.cuh:20-157, B/rasterization/src/forward.cu:82-221.
#include "internal.h"

namespace efgs {

namespace {

__global__ void fill_u32_kernel(uint32_t* p, uint32_t value, uint64_t n) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

// Primitive-index-ordered compaction of the visible primitives with their first emission slots (the
// preprocess stored per-block visible and instance counts; block_offsets holds their exclusive scans).
// Wave-wide scans and reductions without LDS round trips (every lane of the wave takes part). Inclusive sum:
// shifts within each 16-lane row (DPP row_shr, zero filled), then lane 15 of rows 0 and 2 into rows 1 and 3 and
// lane 31 into rows 2 and 3 (DPP row broadcasts). Reduction: four row rotations give every lane its row's
// result, two lane swaps combine the rows; the result is in every lane.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, true));  // row_shr:1
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, true));  // row_shr:2
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, true));  // row_shr:4
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, true));  // row_shr:8
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
    return v;
}
template <typename OP>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v, OP op) {
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x121, 0xf, 0xf, false)));  // row_ror:1
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x122, 0xf, 0xf, false)));  // row_ror:2
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x124, 0xf, 0xf, false)));  // row_ror:4
    v = op(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, false)));  // row_ror:8
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return op(b[0], b[1]);
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) { return wave_reduce(v, [](uint32_t x, uint32_t y) { return x + y; }); }
// a lane's value in every lane; the lane index must be wave-uniform
__device__ __forceinline__ uint32_t lane_value(uint32_t v, uint32_t src) { return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(src))); }
__device__ __forceinline__ float lane_value(float v, uint32_t src) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), static_cast<int>(src))); }

__global__ __launch_bounds__(preprocess_block) void compact_visible_kernel(const uint32_t* n_touched, const uint32_t* block_offsets,
                                                                          uint32_t* visible_out, uint32_t* prim_offset, uint32_t n) {
    __shared__ uint32_t wave_counts[preprocess_block / 64][2];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t p = blockIdx.x * preprocess_block + threadIdx.x;
    const uint32_t touched = p < n ? n_touched[p] : 0u;
    const bool visible = touched > 0;
    const uint64_t mask = __ballot(visible);
    const uint32_t inc = wave_inclusive_sum(touched);  // inclusive wave scan of the tile counts
    if (lane == 63) {
        wave_counts[wave][0] = static_cast<uint32_t>(__popcll(mask));
        wave_counts[wave][1] = inc;
    }
    __syncthreads();
    if (!visible) return;
    uint32_t pos = block_offsets[2 * blockIdx.x], off = block_offsets[2 * blockIdx.x + 1];
    for (uint32_t w = 0; w < wave; w++) {
        pos += wave_counts[w][0];
        off += wave_counts[w][1];
    }
    pos += static_cast<uint32_t>(__popcll(mask & ((1ull << lane) - 1ull)));
    visible_out[pos] = p;
    prim_offset[p] = off + inc - touched;
}

// Emission of one visible primitive per thread (visible index i, index order): (tile key, primitive) for every
// tile of its tile rectangle that passes the contribution test, the first 8 tiles per lane from the test results
// the preprocess recorded in the primitive's record, larger footprints' further tiles tested again
// wave-cooperatively (64 tiles per step, positions from ballot prefix counts); emit(slot, tile) is
// called by the lane that writes each instance. Emission slots are [prim_offset, prim_offset + n_touched); a
// count that disagrees with the preprocess is clamped to that range, the remainder padded with an out-of-range
// key (never bucketed) and counted in counters[2]. A primitive that emitted fewer tiles than counted gets
// n_touched lowered to the emitted count, so the per-primitive sums of the backward and of the pruning scores
// cover only slots that a blend kernel writes. Every lane of the wave must call this (ballots and shuffles).
// The fields of a primitive's 48-byte record that emission reads (nine of its twelve words: not the colour).
struct EmitRecord {
    float4 r0;               // mean2d x, y, conic x, y
    float cz, opacity;       // conic z, opacity
    uint32_t bx, by, first;  // packed screen bounds x, y; the first-tiles mask
};
__device__ __forceinline__ EmitRecord load_emit_record(const PrimRecord* records, uint32_t p) {
    const float* const r = reinterpret_cast<const float*>(records + p);
    const float4 r0 = *reinterpret_cast<const float4*>(r);
    const float2 r1 = *reinterpret_cast<const float2*>(r + 4);
    return EmitRecord{r0, r1.x, r1.y, __float_as_uint(r[9]), __float_as_uint(r[10]), __float_as_uint(r[11])};
}

// n: the primitive's tile count from the preprocess, rec: its record's emission fields (both loaded by the caller).
template <typename KeyT, typename Emit>
__device__ __forceinline__ void emit_primitive_rec(const CreateInstancesArgs& a, uint32_t p, uint32_t off, uint32_t n, const EmitRecord& rec, bool active,
                                                   uint32_t lane, Emit&& emit) {
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    const uint32_t bx = rec.bx, by = rec.by;
    const TileRect t = screen_to_tile_bounds(bx & 0xffffu, bx >> 16, by & 0xffffu, by >> 16);
    const uint32_t bw = t.x1 - t.x0;
    const uint32_t cnt = active ? bw * (t.y1 - t.y0) : 0u;
    const float smx = rec.r0.x - 0.5f, smy = rec.r0.y - 0.5f;
    const float cx = rec.r0.z, cy = rec.r0.w, cz = rec.cz;
    const float pt = cnt > n_sequential_tiles ? power_threshold_of(rec.opacity) : 0.0f;  // (the tile test of the later tiles)
    const uint32_t first_tiles = rec.first;  // the preprocess's test of the first n_sequential_tiles tiles
    KeyT* keys = static_cast<KeyT*>(a.keys);
    uint32_t k = 0;
    for (uint32_t j = 0; j < cnt && j < n_sequential_tiles; j++) {
        const uint32_t tx = t.x0 + j % bw, ty = t.y0 + j / bw;
        if ((first_tiles >> j) & 1u) {
            if (k < n) {
                const uint32_t tile = ty * a.grid_w + tx;
                keys[off + k] = static_cast<KeyT>(tile);
                a.inst_prim[off + k] = p;
                emit(off + k, tile);
            }
            k++;
        }
    }
    uint64_t coop = __ballot(cnt > n_sequential_tiles);
    while (coop != 0) {
        const uint32_t src = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(__ffsll(static_cast<long long>(coop)) - 1));
        coop &= coop - 1;
        const uint32_t c_x0 = lane_value(t.x0, src), c_y0 = lane_value(t.y0, src), c_bw = lane_value(bw, src), c_cnt = lane_value(cnt, src);
        const uint32_t c_off = lane_value(off, src), c_n = lane_value(n, src), c_p = lane_value(p, src);
        const float c_mx = lane_value(smx, src), c_my = lane_value(smy, src);
        const float c_cx = lane_value(cx, src), c_cy = lane_value(cy, src), c_cz = lane_value(cz, src), c_pt = lane_value(pt, src);
        uint32_t c_k = lane_value(k, src);
        for (uint32_t base = n_sequential_tiles; base < c_cnt; base += 64) {
            const uint32_t j = base + lane;
            const uint32_t tx = c_x0 + j % c_bw, ty = c_y0 + j / c_bw;
            const bool hit = j < c_cnt && will_primitive_contribute(c_mx, c_my, c_cx, c_cy, c_cz, tx, ty, c_pt);
            const uint64_t m = __ballot(hit);
            const uint32_t pos = c_k + static_cast<uint32_t>(__popcll(m & lanes_below));
            if (hit && pos < c_n) {
                const uint32_t tile = ty * a.grid_w + tx;
                keys[c_off + pos] = static_cast<KeyT>(tile);
                a.inst_prim[c_off + pos] = c_p;
                emit(c_off + pos, tile);
            }
            c_k += static_cast<uint32_t>(__popcll(m));
        }
        if (lane == src) k = c_k;
    }
    if (active && k != n) {
        for (uint32_t j = (k < n ? k : n); j < n; j++) {
            keys[off + j] = static_cast<KeyT>(~static_cast<KeyT>(0));
            a.inst_prim[off + j] = p;
        }
        if (k < n) a.n_touched[p] = k;
        atomicAdd(&a.counters[2], 1u);
    }
}

template <typename KeyT, typename Emit>
__device__ __forceinline__ void emit_primitive_at(const CreateInstancesArgs& a, uint32_t p, uint32_t off, bool active, uint32_t lane, Emit&& emit) {
    emit_primitive_rec<KeyT>(a, p, off, a.n_touched[p], load_emit_record(a.records, p), active, lane, emit);
}

// visible primitive i (index order) of the compacted list; inactive lanes repeat the last one
template <typename KeyT, typename Emit>
__device__ __forceinline__ void emit_primitive(const CreateInstancesArgs& a, uint32_t i_raw, bool active, uint32_t lane, Emit&& emit) {
    const uint32_t i = active ? i_raw : a.n_visible - 1;
    const uint32_t p = a.visible_prims[i];
    emit_primitive_at<KeyT>(a, p, a.prim_offset[p], active, lane, emit);
}

// One thread per visible primitive (the path for grids whose tile histogram does not fit the LDS).
template <typename KeyT>
__global__ __launch_bounds__(instance_block) void create_instances_kernel(CreateInstancesArgs a) {
    if (a.counters[counter_overflow] != 0) return;
    a.n_visible = a.counters[0];
    if (blockIdx.x * instance_block >= a.n_visible) return;  // (block-uniform: the grid covers a bound on V)
    const uint32_t i = blockIdx.x * instance_block + threadIdx.x;
    emit_primitive<KeyT>(a, i, i < a.n_visible, threadIdx.x & 63u, [](uint32_t, uint32_t) {});
}

// Emission with the per-tile counts, the compaction and the counter scan in one kernel (grids whose histogram
// fits the LDS). Block s takes the primitive chunks [s C, (s + 1) C) of the preprocess (C = f.chunks_per_segment
// chunks of preprocess_block primitives; its emission slots are one contiguous run, its segment). It first sums the
// preprocess's per-chunk visible and instance counts: over all chunks (the frame's totals and depth-key range:
// block 0 publishes the counters, to the host as well, followed by the frame's sequence number) and over the
// chunks before its own (its first visible index and emission slot). More instances than the buffers hold set the
// overflow flag and nothing is emitted. Then, 1024 primitives at a time (a round), a block scan of the visible
// flags and tile counts gives every visible primitive its visible index and first emission slot (visible_prims,
// prim_offset: the compaction), and the thread that holds the primitive emits it, counted per tile in an LDS
// histogram whose atomic return values rank every instance among the segment's instances of its tile (in arbitrary
// order: the per-tile sort fixes the order later); it stores rank | s << 24 per instance and writes its histogram
// row table[s][*]. The tile counts and records of the first two rounds are loaded
// before the chunk counts are summed and every later round's during the round two before it, so the rounds wait on
// no global load of their own (a thread whose primitive is not visible loads a record it does not use).
constexpr uint32_t fused_block = 1024;
template <typename KeyT>
__global__ __launch_bounds__(fused_block) void create_instances_fused_kernel(CreateInstancesArgs a, FusedBinningArgs f, uint32_t* local_rank,
                                                                           uint32_t* table, uint32_t n_tiles) {
    extern __shared__ uint32_t hist[];  // n_tiles counters
    __shared__ uint32_t s_red[fused_block / 64][8];
    __shared__ uint32_t s_scan[2][fused_block / 64][2];  // the rounds' wave totals, alternating between rounds
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t seg = blockIdx.x;
    const uint32_t c0 = seg * f.chunks_per_segment, c1 = min(f.n_chunks, c0 + f.chunks_per_segment);
    const uint32_t p_begin = c0 * preprocess_block, p_end = min(f.n_prims, c1 * preprocess_block);  // (p_end > p_begin)
    // the tile counts and records of a round (threads past the segment: count 0, the segment's last record)
    const auto load_round = [&](uint32_t it, uint32_t& touched, EmitRecord& rec) {
        const uint32_t p = p_begin + it * fused_block + tid;
        touched = p < p_end ? a.n_touched[p] : 0u;
        rec = load_emit_record(a.records, min(p, p_end - 1u));
    };
    uint32_t touched_a, touched_b;
    EmitRecord rec_a, rec_b;
    load_round(0, touched_a, rec_a);
    load_round(1, touched_b, rec_b);

    // totals, depth-key range and the segment's prefix from the per-chunk counts
    uint32_t tv = 0, ti = 0, bv = 0, bi = 0, kmin = 0xffffffffu, kmax = 0u;
    for (uint32_t c = tid; c < f.n_chunks; c += fused_block) {
        const uint2 cnt = reinterpret_cast<const uint2*>(f.block_counts)[c];
        const uint2 kr = reinterpret_cast<const uint2*>(f.key_ranges)[c];
        tv += cnt.x;
        ti += cnt.y;
        bv += c < c0 ? cnt.x : 0u;
        bi += c < c0 ? cnt.y : 0u;
        kmin = min(kmin, kr.x);
        kmax = max(kmax, kr.y);
    }
    tv = wave_sum(tv);
    ti = wave_sum(ti);
    bv = wave_sum(bv);
    bi = wave_sum(bi);
    kmin = wave_reduce(kmin, [](uint32_t x, uint32_t y) { return min(x, y); });
    kmax = wave_reduce(kmax, [](uint32_t x, uint32_t y) { return max(x, y); });
    if (lane == 0) {
        s_red[wave][0] = tv; s_red[wave][1] = ti; s_red[wave][2] = bv; s_red[wave][3] = bi; s_red[wave][4] = kmin; s_red[wave][5] = kmax;
    }
    for (uint32_t t = tid; t < n_tiles; t += fused_block) hist[t] = 0;
    __syncthreads();
    tv = ti = bv = bi = 0;
    kmin = 0xffffffffu;
    kmax = 0u;
#pragma unroll
    for (uint32_t w = 0; w < fused_block / 64; w++) {
        tv += s_red[w][0]; ti += s_red[w][1]; bv += s_red[w][2]; bi += s_red[w][3];
        kmin = min(kmin, s_red[w][4]);
        kmax = max(kmax, s_red[w][5]);
    }
    const bool overflow = ti > f.capacity;
    if (seg == 0 && tid == 0) {
        // [2] (emission mismatches) was cleared by the preprocess and is counted by the emission below
        const uint32_t c[6] = {tv, ti, 0u, tv > 0 ? kmin : 0u, tv > 0 ? kmax : 0u, overflow ? 1u : 0u};
#pragma unroll
        for (uint32_t k = 0; k < 6; k++) {
            if (k != 2) a.counters[k] = c[k];
            f.host_counters[k] = c[k];
        }
        __threadfence_system();
        __hip_atomic_store(&f.host_counters[counter_sequence], f.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        __threadfence_system();
    }
    if (overflow) return;  // (block-uniform)

    const uint32_t tag = seg << rank_segment_shift;
    uint32_t run_v = bv, run_i = bi;
    // A round's scan partials alternate between two buffers: a wave writes round r + 2's partials only after the
    // barrier of round r + 1, which every wave reaches after its reads of round r's.
    const auto round = [&](uint32_t it, uint32_t touched, const EmitRecord& rec) {
        const uint32_t p = p_begin + it * fused_block + tid;
        const uint32_t vis = touched > 0 ? 1u : 0u;
        const uint32_t iv = wave_inclusive_sum(vis), ii = wave_inclusive_sum(touched);  // inclusive wave scans
        uint32_t(*const sc)[2] = s_scan[it & 1u];
        if (lane == 63) {
            sc[wave][0] = iv;
            sc[wave][1] = ii;
        }
        __syncthreads();
        uint32_t pv = 0, pi = 0, nv = 0, ni = 0;
#pragma unroll
        for (uint32_t w = 0; w < fused_block / 64; w++) {
            const uint32_t wv = sc[w][0], wi = sc[w][1];
            pv += w < wave ? wv : 0u;
            pi += w < wave ? wi : 0u;
            nv += wv;
            ni += wi;
        }
        const uint32_t vpos = pv + iv - vis, off = run_i + pi + ii - touched;
        if (vis) {
            a.visible_prims_out[run_v + vpos] = p;
            a.prim_offset_out[p] = off;
        }
        emit_primitive_rec<KeyT>(a, p, off, touched, rec, vis != 0u, lane, [&](uint32_t slot, uint32_t tile) {
            local_rank[slot] = tag | atomicAdd(&hist[tile], 1u);
        });
        run_v += nv;
        run_i += ni;
    };
    // two register sets, each loaded a round before its use (no loaded value is copied between loop-carried
    // registers: a copy would wait for the load)
    const uint32_t n_rounds = (p_end - p_begin + fused_block - 1u) / fused_block;
    for (uint32_t it = 0; it < n_rounds; it += 2) {  // (block-uniform)
        round(it, touched_a, rec_a);
        if (it + 2 < n_rounds) load_round(it + 2, touched_a, rec_a);
        if (it + 1 >= n_rounds) break;
        round(it + 1, touched_b, rec_b);
        if (it + 3 < n_rounds) load_round(it + 3, touched_b, rec_b);
    }
    __syncthreads();
    uint32_t* row = table + static_cast<size_t>(seg) * n_tiles;
    for (uint32_t t = tid; t < n_tiles; t += fused_block) row[t] = hist[t];
}

// Per-tile offsets, 64 tiles per block, one tile per lane. With a count table (S segment rows): wave w of 16 loads
// the column entries of its sixteenth of the segments into registers; the sixteen partial sums give each wave its
// offset and the tile's total; wave 0 scans the block's 64 totals (local_start: the tile's start within the block,
// and the block total, block_sums); then every entry is rewritten as local_start + the tile's count in the earlier
// segments, so a bucket slot is block prefix + table entry + rank. Without a table the totals come from the
// global counts. The start of tile t is the sum of block_sums over the blocks before t / 64 plus local_start[t]:
// consumers add those few block sums themselves, so no block waits for another and no cross-block fence is needed.
constexpr uint32_t scan_tiles = 64;
constexpr uint32_t scan_waves = 16;
constexpr uint32_t scan_per_wave = tile_hist_max_blocks / scan_waves;
// class of a tile with n instances: 0 for the heaviest, order_classes - 1 for an empty tile
__device__ __forceinline__ uint32_t order_class(uint32_t n) {
    if (n == 0) return order_classes - 1;
    const uint32_t e = 31u - static_cast<uint32_t>(__clz(static_cast<int>(n)));
    const uint32_t m = e >= 2 ? (n >> (e - 2)) & 3u : (n << (2 - e)) & 3u;
    return order_classes - 1 - min(1u + 4u * e + m, order_classes - 1);
}

__global__ __launch_bounds__(64 * scan_waves) void tile_column_scan_kernel(uint32_t* table, uint32_t n_segments, uint32_t n_tiles,
                                                                          uint32_t* totals, uint32_t* local_start, uint32_t* block_sums,
                                                                          uint32_t* order_runs, uint32_t* order_rank, const uint32_t* counters) {
    if (counters[counter_overflow] != 0) return;
    __shared__ uint32_t s_part[scan_waves][scan_tiles];
    __shared__ uint32_t s_start[scan_tiles];
    __shared__ uint32_t s_runs[order_classes];
    static_assert(order_classes == 64 && scan_tiles == 64, "one class and one tile per lane");
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * scan_tiles + lane;
    const bool in = t < n_tiles;
    const uint32_t per = (n_segments + scan_waves - 1) / scan_waves;
    const uint32_t s0 = wave * per;
    uint32_t c[scan_per_wave];
    uint32_t sum = 0;
#pragma unroll
    for (uint32_t k = 0; k < scan_per_wave; k++) {
        c[k] = (table && in && k < per && s0 + k < n_segments) ? table[static_cast<size_t>(s0 + k) * n_tiles + t] : 0u;
        sum += c[k];
    }
    s_part[wave][lane] = sum;
    __syncthreads();
    if (wave == 0) {
        uint32_t total = 0;
#pragma unroll
        for (uint32_t w = 0; w < scan_waves; w++) total += s_part[w][lane];
        if (!table) total = in ? totals[t] : 0u;
        else if (in) totals[t] = total;
        const uint32_t inc = wave_inclusive_sum(total);
        if (in) local_start[t] = inc - total;
        s_start[lane] = inc - total;
        if (lane == 63) block_sums[blockIdx.x] = inc;
        // tile order: the block's tiles per class and each tile's rank among its class (the lanes of a class
        // are found by one ballot per class bit)
        const uint32_t cls = in ? order_class(total) : order_classes;
        uint64_t same = __ballot(in);
#pragma unroll
        for (uint32_t bit = 1; bit < order_classes; bit <<= 1) {
            const uint64_t set = __ballot((cls & bit) != 0);
            same &= (cls & bit) ? set : ~set;
        }
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(same >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(same), 0u));
        s_runs[lane] = 0u;  // order_classes == 64: one class per lane
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (in && rank == 0) s_runs[cls] = static_cast<uint32_t>(__popcll(same));
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        order_runs[static_cast<size_t>(blockIdx.x) * order_classes + lane] = s_runs[lane];
        if (in) order_rank[t] = cls << 16 | rank;
    }
    if (!table) return;
    __syncthreads();
    uint32_t prefix = s_start[lane];
    for (uint32_t w = 0; w < wave; w++) prefix += s_part[w][lane];
#pragma unroll
    for (uint32_t k = 0; k < scan_per_wave; k++) {
        if (in && k < per && s0 + k < n_segments) table[static_cast<size_t>(s0 + k) * n_tiles + t] = prefix;
        prefix += c[k];
    }
}

template <typename KeyT>
__global__ __launch_bounds__(256) void tile_count_global_kernel(const KeyT* keys, const uint32_t* counters, uint32_t* totals, uint32_t n_tiles) {
    if (counters[counter_overflow] != 0) return;
    const uint32_t e = blockIdx.x * 256u + threadIdx.x;
    if (e >= counters[1]) return;
    const uint32_t t = static_cast<uint32_t>(keys[e]);
    if (t < n_tiles) atomicAdd(&totals[t], 1u);
}

// exclusive prefix of block_sums over the scan blocks before `b`, for one wave (every lane gets it)
__device__ __forceinline__ uint32_t scan_block_prefix_wave(const uint32_t* block_sums, uint32_t b, uint32_t lane) {
    uint32_t s = 0;
    for (uint32_t k = lane; k < b; k += 64) s += block_sums[k];
    return wave_sum(s);
}

// One block: order_runs[b][c] (tiles of class c in 64-tile block b) becomes the first position of that run in
// the tile order: the tiles of the classes before c, then those of class c in the blocks before b. Lane c of every
// wave handles class c (a block's 64 counts are one coalesced row); wave w the w-th part of the blocks, whose
// rows it holds in registers (16 at a time), so each row is read once and written once.
template <uint32_t N_WAVES>
__device__ inline void order_runs_block(uint32_t* order_runs, uint32_t n_blocks, uint32_t (*s_part)[order_classes]) {
    constexpr uint32_t rows = 16;  // rows per lane in registers per pass
    const uint32_t c = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t per = (n_blocks + N_WAVES - 1) / N_WAVES;
    const uint32_t b0 = min(wave * per, n_blocks), b1 = min(b0 + per, n_blocks);
    uint32_t sum = 0;
    for (uint32_t r0 = b0; r0 < b1; r0 += rows) {
        uint32_t v[rows];
#pragma unroll
        for (uint32_t k = 0; k < rows; k++) v[k] = r0 + k < b1 ? order_runs[static_cast<size_t>(r0 + k) * order_classes + c] : 0u;
#pragma unroll
        for (uint32_t k = 0; k < rows; k++) sum += v[k];
    }
    s_part[wave][c] = sum;
    __syncthreads();
    uint32_t total = 0, before = 0;
#pragma unroll
    for (uint32_t w = 0; w < N_WAVES; w++) {
        const uint32_t x = s_part[w][c];
        total += x;
        before += w < wave ? x : 0u;
    }
    uint32_t inc = total;  // classes in lane order: prefix over the lanes
#pragma unroll
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t x = static_cast<uint32_t>(__shfl_up(static_cast<int>(inc), o));
        if (c >= o) inc += x;
    }
    uint32_t running = inc - total + before;
    for (uint32_t r0 = b0; r0 < b1; r0 += rows) {
        uint32_t v[rows];
#pragma unroll
        for (uint32_t k = 0; k < rows; k++) v[k] = r0 + k < b1 ? order_runs[static_cast<size_t>(r0 + k) * order_classes + c] : 0u;
#pragma unroll
        for (uint32_t k = 0; k < rows; k++) {
            if (r0 + k < b1) order_runs[static_cast<size_t>(r0 + k) * order_classes + c] = running;
            running += v[k];
        }
    }
}

// the tile order's run positions alone (frames without instances: no bucket pass to carry them)
__global__ __launch_bounds__(1024) void tile_order_runs_kernel(uint32_t* order_runs, uint32_t n_blocks, const uint32_t* counters) {
    if (counters[counter_overflow] != 0) return;
    __shared__ uint32_t s_part[1024 / 64][order_classes];
    order_runs_block<1024 / 64>(order_runs, n_blocks, s_part);
}

// Every emitted instance goes to a slot of its tile's range: start of the tile + the tile's count in the
// earlier segments + its rank within its segment (with a table: the scanned table entry holds the tile's start
// within its 64-tile block plus that count), or + the next slot of an atomic cursor (without one). The slot
// receives the instance's sort key, the depth key of its primitive above its emission index. Each block first
// scans the per-64-tile block sums into dynamic LDS (256 at a time with a running carry), one entry per 64-tile
// block: up to max_scan_blocks of them (1,015,808 tiles); larger grids add the block sums per instance. A thread
// takes bucket_per_thread instances (256 apart, so every load stays coalesced) and issues the loads of all of them
// before their gathers and those before the stores: the kernel waits on memory, and half the waves then keep twice
// the requests in flight each (and half the blocks repeat the block-sum scan). Two per thread measured best on the
// 1M-Gaussian 1080p step (bucket stage 21.3-22.2 us with four, 19.8 with two, 22.2 with eight).
constexpr uint32_t max_scan_blocks = static_cast<uint32_t>((tile_hist_max_lds - 2048) / 4);
constexpr uint32_t bucket_per_thread = 2;
constexpr uint32_t bucket_chunk = 256 * bucket_per_thread;  // instances per block
template <typename KeyT>
__global__ __launch_bounds__(256) void tile_buckets_kernel(const KeyT* keys, const uint32_t* inst_prim, const uint32_t* depth_keys,
                                                          const uint32_t* table, const uint32_t* local_rank, const uint32_t* block_sums,
                                                          const uint32_t* local_start, uint32_t* cursor, uint4* bucket, const uint32_t* counters,
                                                          uint32_t n_tiles, uint32_t* order_runs, uint32_t order_blocks) {
    extern __shared__ uint32_t s_prefix[];  // n_blocks entries (the launch sizes it; none above max_scan_blocks)
    __shared__ uint32_t s_waves[4];
    __shared__ uint32_t s_order[4][order_classes];
    if (counters[counter_overflow] != 0) return;
    if (blockIdx.x == 0) {  // the first block (dispatched first): the tile order's run positions, beside the buckets
        order_runs_block<4>(order_runs, order_blocks, s_order);
        return;
    }
    const uint32_t block = blockIdx.x - 1u;
    const uint32_t n_instances = counters[1];
    const uint32_t n_chunks = (n_instances + bucket_chunk - 1u) / bucket_chunk;
    if (block >= n_chunks) return;  // (block-uniform: the grid covers a bound on I)
    // XCD-aware chunk: the hardware deals workgroups to the 8 XCDs round robin (workgroup w on XCD w % 8, so bucket
    // block b on XCD (b + 1) % 8); the blocks of one XCD take one contiguous run of the chunks, so the table rows of
    // a segment (whose instances are contiguous) are fetched into one XCD's L2 instead of all eight
    const uint32_t xcd = block % 8u, per = n_chunks / 8u, extra = n_chunks % 8u;
    const uint32_t chunk = xcd * per + min(xcd, extra) + block / 8u;
    // the instances' tile keys, primitives and ranks (clamped indices past the count: every load unconditional, all
    // in flight together), then the depth keys and table entries they select, then the slots
    uint32_t e[bucket_per_thread], t[bucket_per_thread], prim[bucket_per_thread], rank[bucket_per_thread];
    const uint32_t last = n_instances - 1u;
#pragma unroll
    for (uint32_t k = 0; k < bucket_per_thread; k++) {
        e[k] = chunk * bucket_chunk + k * 256u + threadIdx.x;
        const uint32_t ec = min(e[k], last);
        t[k] = static_cast<uint32_t>(keys[ec]);
        prim[k] = inst_prim[ec];
        rank[k] = table ? local_rank[ec] : 0u;
    }
    uint32_t depth[bucket_per_thread], pos[bucket_per_thread];
#pragma unroll
    for (uint32_t k = 0; k < bucket_per_thread; k++) {
        // (an instance past the count or padded after an emission mismatch has no rank: table row 0, tile 0)
        const bool valid = e[k] < n_instances && t[k] < n_tiles;
        const uint32_t tc = valid ? t[k] : 0u, r = valid ? rank[k] : 0u;
        depth[k] = depth_keys[prim[k]];
        pos[k] = 0;
        if (table) {  // the table entry already holds the tile's start within its block
            pos[k] = table[static_cast<size_t>(r >> rank_segment_shift) * n_tiles + tc] + (r & ((1u << rank_segment_shift) - 1u));
        } else if (valid) {
            pos[k] = local_start[tc] + atomicAdd(&cursor[tc], 1u);
        }
    }
    // the block sums' prefix (after the instances' loads and gathers were issued: those do not wait for it)
    const uint32_t n_blocks = (n_tiles + scan_tiles - 1) / scan_tiles;
    if (n_blocks <= max_scan_blocks) {
        const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
        uint32_t carry = 0;  // block-uniform: the sum of the earlier passes
        for (uint32_t b0 = 0; b0 < n_blocks; b0 += 256) {
            const uint32_t i = b0 + threadIdx.x;
            const uint32_t v = i < n_blocks ? block_sums[i] : 0u;
            const uint32_t inc = wave_inclusive_sum(v);
            if (lane == 63) s_waves[wave] = inc;
            __syncthreads();
            uint32_t off = carry;
            for (uint32_t w = 0; w < wave; w++) off += s_waves[w];
            if (i < n_blocks) s_prefix[i] = off + inc - v;
            carry += s_waves[0] + s_waves[1] + s_waves[2] + s_waves[3];
            __syncthreads();  // s_waves read by every wave before the next pass writes it (and s_prefix complete)
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < bucket_per_thread; k++) {
        if (e[k] >= n_instances || t[k] >= n_tiles) continue;
        const uint32_t b = t[k] / scan_tiles;
        uint32_t base = 0;
        if (n_blocks <= max_scan_blocks) {
            base = s_prefix[b];
        } else {
            for (uint32_t j = 0; j < b; j++) base += block_sums[j];
        }
        bucket[base + pos[k]] = make_uint4(e[k], depth[k], prim[k], 0u);  // one 16-byte store: key (low 8 bytes) and primitive
    }
}

// Every tile's range and its place in the blends' tile order, one tile per lane: a wave's 64 tiles are one scan
// block, so the wave computes the prefix of the block sums once for all of them. (Each tile's run is sorted by the
// forward blend of the tile, before its walk.)
__global__ __launch_bounds__(256) void tile_ranges_kernel(const uint32_t* totals, const uint32_t* block_sums, const uint32_t* local_start,
                                                          const uint32_t* order_runs, const uint32_t* order_rank, uint32_t* order,
                                                          const uint32_t* counters, uint2* ranges, uint32_t n_tiles) {
    static_assert(scan_tiles == 64, "one scan block per wave");
    if (counters[counter_overflow] != 0) return;
    const uint32_t lane = threadIdx.x & 63u, tile = blockIdx.x * 256u + threadIdx.x;
    const uint32_t tile0 = tile - lane;
    if (tile0 >= n_tiles) return;  // the whole wave
    const uint32_t prefix = scan_block_prefix_wave(block_sums, tile0 / scan_tiles, lane);
    if (tile >= n_tiles) return;
    const uint32_t n = totals[tile];
    const uint32_t start = prefix + local_start[tile];
    ranges[tile] = n > 0 ? make_uint2(start, start + n) : make_uint2(0u, 0u);  // (0, 0) for an empty tile, as the reference
    const uint32_t cr = order_rank[tile];
    order[order_runs[static_cast<size_t>(tile / scan_tiles) * order_classes + (cr >> 16)] + (cr & 0xffffu)] = tile;
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

}  // namespace

bool launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, hipStream_t s) {
    if (n == 0) return true;
    fill_u32_kernel<<<div_up(n, 256), 256, 0, s>>>(p, value, n);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_compact_visible(const uint32_t* n_touched, const uint32_t* block_offsets, uint32_t* visible_out, uint32_t* prim_offset, uint32_t n,
                            hipStream_t s) {
    if (n == 0) return true;
    compact_visible_kernel<<<div_up(n, preprocess_block), preprocess_block, 0, s>>>(n_touched, block_offsets, visible_out, prim_offset, n);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_create_instances(const CreateInstancesArgs& a, int key_bytes, const TileBinning& plan, uint32_t* local_rank, uint32_t* table,
                             uint32_t n_tiles, const FusedBinningArgs* fused, hipStream_t s) {
    if (a.max_visible == 0) return true;
    if (fused) {
        const size_t lds = static_cast<size_t>(n_tiles) * 4;
        if (key_bytes == 2)
            create_instances_fused_kernel<uint16_t><<<plan.blocks, fused_block, lds, s>>>(a, *fused, local_rank, table, n_tiles);
        else
            create_instances_fused_kernel<uint32_t><<<plan.blocks, fused_block, lds, s>>>(a, *fused, local_rank, table, n_tiles);
    } else {
        const uint32_t blocks = div_up(a.max_visible, instance_block);
        if (key_bytes == 2)
            create_instances_kernel<uint16_t><<<blocks, instance_block, 0, s>>>(a);
        else
            create_instances_kernel<uint32_t><<<blocks, instance_block, 0, s>>>(a);
    }
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool fused_binning_fits(uint32_t n_tiles) { return n_tiles > 0 && static_cast<size_t>(n_tiles) * 4 <= tile_hist_max_lds; }

TileBinning fused_binning_plan(uint32_t n_prims, uint32_t n_tiles, uint32_t& chunks_per_segment) {
    TileBinning b;
    b.use_table = true;
    const uint32_t n_chunks = n_prims > 0 ? div_up(n_prims, preprocess_block) : 1u;
    // segments of at least one round of the fused kernel (1024 primitives), at most tile_hist_max_blocks of them
    const uint32_t want = n_prims > 0 ? div_up(n_prims, fused_block) : 1u;
    chunks_per_segment = div_up(n_chunks, want < tile_hist_max_blocks ? want : tile_hist_max_blocks);
    b.blocks = div_up(n_chunks, chunks_per_segment);
    b.segment = chunks_per_segment * preprocess_block;
    (void)n_tiles;
    return b;
}

bool launch_tile_counts(const TileBinning& plan, const void* keys, int key_bytes, uint32_t max_instances, uint32_t* table, const TileScan& ts,
                        uint32_t n_tiles, hipStream_t s) {
    if (n_tiles == 0) return true;
    const bool with_table = plan.use_table && max_instances > 0;
    if (!with_table) {
        if (!launch_fill_u32(ts.totals, 0u, n_tiles, s) || !launch_fill_u32(ts.cursor, 0u, n_tiles, s)) return false;
        if (max_instances > 0) {
            if (key_bytes == 2)
                tile_count_global_kernel<uint16_t><<<div_up(max_instances, 256), 256, 0, s>>>(static_cast<const uint16_t*>(keys), ts.counters,
                                                                                           ts.totals, n_tiles);
            else
                tile_count_global_kernel<uint32_t><<<div_up(max_instances, 256), 256, 0, s>>>(static_cast<const uint32_t*>(keys), ts.counters,
                                                                                           ts.totals, n_tiles);
        }
    }
    tile_column_scan_kernel<<<div_up(n_tiles, scan_tiles), 64 * scan_waves, 0, s>>>(with_table ? table : nullptr, with_table ? plan.blocks : 0u, n_tiles,
                                                                        ts.totals, ts.local_start, ts.block_sums, ts.order_runs, ts.order_rank,
                                                                        ts.counters);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_tile_buckets(const TileBinning& plan, const void* keys, int key_bytes, const uint32_t* inst_prim, const uint32_t* depth_keys,
                         const uint32_t* table, const uint32_t* local_rank, const TileScan& ts, uint4* bucket, uint32_t max_instances,
                         uint32_t n_tiles, hipStream_t s) {
    if (n_tiles == 0) return true;
    const uint32_t order_blocks = div_up(n_tiles, scan_tiles);
    if (max_instances == 0) {
        tile_order_runs_kernel<<<1, 1024, 0, s>>>(ts.order_runs, order_blocks, ts.counters);
        EFGS_HIP_CHECK(hipGetLastError());
        return true;
    }
    // one block that places the tile order's runs, then one block per bucket_chunk instances (a bound on I)
    const uint32_t blocks = div_up(max_instances, bucket_chunk) + 1;
    const uint32_t* tab = plan.use_table ? table : nullptr;
    const uint32_t prefix_bytes = order_blocks <= max_scan_blocks ? order_blocks * 4u : 0u;  // (order_blocks: the 64-tile blocks)
    if (key_bytes == 2)
        tile_buckets_kernel<uint16_t><<<blocks, 256, prefix_bytes, s>>>(static_cast<const uint16_t*>(keys), inst_prim, depth_keys, tab, local_rank, ts.block_sums,
                                                            ts.local_start, ts.cursor, bucket, ts.counters, n_tiles, ts.order_runs, order_blocks);
    else
        tile_buckets_kernel<uint32_t><<<blocks, 256, prefix_bytes, s>>>(static_cast<const uint32_t*>(keys), inst_prim, depth_keys, tab, local_rank, ts.block_sums,
                                                            ts.local_start, ts.cursor, bucket, ts.counters, n_tiles, ts.order_runs, order_blocks);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_tile_ranges(const TileScan& ts, uint2* ranges, uint32_t n_tiles, hipStream_t s) {
    if (n_tiles == 0) return true;
    tile_ranges_kernel<<<div_up(n_tiles, 256), 256, 0, s>>>(ts.totals, ts.block_sums, ts.local_start, ts.order_runs, ts.order_rank, ts.order,
                                                            ts.counters, ranges, n_tiles);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

bool launch_reduce_partials(const float* partials, uint32_t n_blocks, uint32_t n_params, float* out, hipStream_t s) {
    if (n_params == 0) return true;
    reduce_partials_kernel<<<div_up(n_params, 64), 64 * reduce_groups, 0, s>>>(partials, n_blocks, n_params, out);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}

}  // namespace efgs
