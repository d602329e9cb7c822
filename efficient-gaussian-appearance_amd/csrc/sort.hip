// Stable LSD radix sort of (key, value) pairs for wave64, 8-bit digits, 2048 keys per 256-thread block.
// Per pass (three launches):
//   histogram : per-block digit counts, counts[block][digit] (each block's row contiguous);
//   row scan  : one block per digit scans its row over the blocks (exclusive) and records the digit total;
//   scatter   : each wave ranks a contiguous quarter of the block's keys (8 rounds of 64, no block barrier),
//               the four waves' digit counts are combined once, the keys are placed digit-sorted in LDS,
//               then every digit run is written to its global position contiguously, so consecutive lanes
//               store consecutive addresses. Global position = (exclusive scan of the digit totals) + (row
//               scan of the digit over the previous blocks) + (rank within the block).
// A wave ranks its 64 keys per digit with 64-bit ballots (lanes sharing a digit form a peer mask; rank =
// peers below the lane) against the wave's per-digit running counts in LDS; segments and rounds are in input
// order, so equal keys keep their input order. Replaces cub::DeviceRadixSort (B/rasterization/src/forward.cu:88-96 depth keys,
// :182-190 tile keys).
#include "internal.h"

namespace efgs {

namespace {

constexpr uint32_t sort_waves = sort_block / 64;

// lanes whose 8-bit digit equals this lane's (restricted to valid lanes)
__device__ __forceinline__ uint64_t match_peers(uint32_t d, bool valid) {
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const bool bit = (d >> b) & 1u;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

// exclusive scan of one value per thread over a 256-thread block (wave scans with DPP-free shuffles)
__device__ __forceinline__ uint32_t block_exclusive_scan_256(uint32_t v, uint32_t* s_waves) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    if (lane == 63) s_waves[wave] = inc;
    __syncthreads();
    uint32_t prefix = 0;
#pragma unroll
    for (uint32_t w = 0; w < sort_waves; w++)
        if (w < wave) prefix += s_waves[w];
    __syncthreads();
    return prefix + inc - v;
}

template <typename KeyT>
__global__ __launch_bounds__(sort_block) void sort_histogram_kernel(const KeyT* keys, uint32_t* counts, uint32_t n, uint32_t shift, uint32_t n_blocks) {
    __shared__ uint32_t h[sort_bins];
    const uint32_t lane = threadIdx.x & 63u;
    h[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t start = blockIdx.x * sort_tile;
#pragma unroll
    for (uint32_t r = 0; r < sort_rounds; r++) {
        const uint32_t i = start + r * sort_block + threadIdx.x;
        const bool valid = i < n;
        const uint32_t d = valid ? (static_cast<uint32_t>(keys[i]) >> shift) & 255u : 0u;
        const uint64_t peers = match_peers(d, valid);
        if (valid && lane == static_cast<uint32_t>(__ffsll(static_cast<long long>(peers)) - 1))
            atomicAdd(&h[d], static_cast<uint32_t>(__popcll(peers)));
    }
    __syncthreads();
    counts[blockIdx.x * sort_bins + threadIdx.x] = h[threadIdx.x];
}

// block d: offsets[b][d] = sum of counts[b'][d] for b' < b, totals[d] = column sum
__global__ __launch_bounds__(sort_block) void sort_row_scan_kernel(const uint32_t* counts, uint32_t* offsets, uint32_t* totals, uint32_t n_blocks) {
    __shared__ uint32_t s_waves[sort_waves];
    const uint32_t d = blockIdx.x;
    const uint32_t per = (n_blocks + sort_block - 1) / sort_block;  // consecutive blocks per thread
    const uint32_t b0 = threadIdx.x * per;
    uint32_t sum = 0;
    for (uint32_t k = 0; k < per; k++)
        if (b0 + k < n_blocks) sum += counts[static_cast<size_t>(b0 + k) * sort_bins + d];
    uint32_t run = block_exclusive_scan_256(sum, s_waves);
    for (uint32_t k = 0; k < per; k++)
        if (b0 + k < n_blocks) {
            const size_t e = static_cast<size_t>(b0 + k) * sort_bins + d;
            const uint32_t c = counts[e];
            offsets[e] = run;
            run += c;
        }
    if (threadIdx.x == sort_block - 1) totals[d] = run;
}

template <typename KeyT>
__global__ __launch_bounds__(sort_block) void sort_scatter_kernel(const KeyT* keys_in, const uint32_t* vals_in, KeyT* keys_out, uint32_t* vals_out,
                                                                 const uint32_t* counts, const uint32_t* offsets, const uint32_t* totals, uint32_t n,
                                                                 uint32_t shift, uint32_t n_blocks) {
    constexpr uint32_t wave_keys = sort_tile / sort_waves;  // each wave ranks a contiguous segment
    constexpr uint32_t wave_rounds = wave_keys / 64;
    __shared__ KeyT s_key[sort_tile];
    __shared__ uint32_t s_val[sort_tile];
    __shared__ uint32_t local_base[sort_bins];   // first slot of each digit in the block's sorted tile
    __shared__ uint32_t global_base[sort_bins];  // global position of that slot
    __shared__ uint32_t wave_count[sort_waves][sort_bins];  // per wave: keys of each digit so far, then the wave's offset
    __shared__ uint32_t s_waves[sort_waves];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    const uint32_t start = blockIdx.x * sort_tile + wave * wave_keys;
    KeyT kr[wave_rounds];
    uint32_t vr[wave_rounds], slot[wave_rounds];
#pragma unroll
    for (uint32_t r = 0; r < wave_rounds; r++) {
        const uint32_t i = start + r * 64 + lane;
        kr[r] = 0;
        vr[r] = 0;
        if (i < n) {
            kr[r] = keys_in[i];
            vr[r] = vals_in ? vals_in[i] : i;
        }
    }
    // the block's table entries, loaded with the keys before the first barrier (one memory latency)
    const uint32_t my_count = counts[static_cast<size_t>(blockIdx.x) * sort_bins + threadIdx.x];
    const uint32_t my_total = totals[threadIdx.x];
    const uint32_t my_offset = offsets[static_cast<size_t>(blockIdx.x) * sort_bins + threadIdx.x];
#pragma unroll
    for (uint32_t w = 0; w < sort_waves; w++) wave_count[w][threadIdx.x] = 0;
    {
        const uint32_t d = threadIdx.x;
        const uint32_t lb = block_exclusive_scan_256(my_count, s_waves);  // also orders the clears
        const uint32_t digit_start = block_exclusive_scan_256(my_total, s_waves);
        local_base[d] = lb;
        global_base[d] = digit_start + my_offset;
    }
    // wave-local ranking: a wave's LDS reads and writes execute in issue order, so no barrier is needed
    // between its rounds (every lane of a digit reads the count before the digit's first lane writes it)
    uint32_t* count = wave_count[wave];
#pragma unroll
    for (uint32_t r = 0; r < wave_rounds; r++) {
        const bool valid = start + r * 64 + lane < n;
        const uint32_t d = (static_cast<uint32_t>(kr[r]) >> shift) & 255u;
        const uint64_t peers = match_peers(d, valid);
        const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lanes_below));
        const uint32_t base = count[d];
        slot[r] = base + rank;
        if (valid && rank == 0) count[d] = base + static_cast<uint32_t>(__popcll(peers));
        __builtin_amdgcn_wave_barrier();  // keeps the next round's reads after this round's writes
    }
    __syncthreads();
    {
        const uint32_t d = threadIdx.x;
        uint32_t run = 0;
#pragma unroll
        for (uint32_t w = 0; w < sort_waves; w++) {
            const uint32_t c = wave_count[w][d];
            wave_count[w][d] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < wave_rounds; r++) {
        if (start + r * 64 + lane >= n) continue;
        const uint32_t d = (static_cast<uint32_t>(kr[r]) >> shift) & 255u;
        const uint32_t k = local_base[d] + count[d] + slot[r];
        s_key[k] = kr[r];
        s_val[k] = vr[r];
    }
    __syncthreads();
    const uint32_t tile_start = blockIdx.x * sort_tile;
    const uint32_t tile_n = min(sort_tile, n - tile_start);
    for (uint32_t k = threadIdx.x; k < tile_n; k += sort_block) {
        const KeyT key = s_key[k];
        const uint32_t d = (static_cast<uint32_t>(key) >> shift) & 255u;
        const uint32_t pos = global_base[d] + (k - local_base[d]);
        if (pos < n) {
            keys_out[pos] = key;
            vals_out[pos] = s_val[k];
        }
    }
}

}  // namespace

size_t sort_scratch_bytes(uint32_t n) {
    const uint32_t blocks = div_up(n > 0 ? n : 1, sort_tile);
    const size_t table = (sizeof(uint32_t) * static_cast<size_t>(sort_bins) * blocks + 255) & ~static_cast<size_t>(255);
    return 2 * table + sizeof(uint32_t) * sort_bins;
}

template <typename KeyT>
static bool sort_impl(KeyT* ka, uint32_t* va, KeyT* kb, uint32_t* vb, bool identity_vals, uint32_t n, int end_bit, void* scratch,
                      bool* result_in_b, hipStream_t s) {
    *result_in_b = false;
    if (n == 0) return true;
    const uint32_t blocks = div_up(n, sort_tile);
    const size_t table = (sizeof(uint32_t) * static_cast<size_t>(sort_bins) * blocks + 255) & ~static_cast<size_t>(255);
    uint32_t* counts = static_cast<uint32_t*>(scratch);
    uint32_t* offsets = reinterpret_cast<uint32_t*>(static_cast<char*>(scratch) + table);
    uint32_t* totals = reinterpret_cast<uint32_t*>(static_cast<char*>(scratch) + 2 * table);
    // at least one pass, so identity values are always materialised
    const int passes = end_bit > 0 ? (end_bit + 7) / 8 : 1;
    KeyT* kin = ka;
    uint32_t* vin = va;
    KeyT* kout = kb;
    uint32_t* vout = vb;
    bool in_b = false;
    for (int pass = 0; pass < passes; pass++) {
        const uint32_t shift = 8u * static_cast<uint32_t>(pass);
        sort_histogram_kernel<KeyT><<<blocks, sort_block, 0, s>>>(kin, counts, n, shift, blocks);
        sort_row_scan_kernel<<<sort_bins, sort_block, 0, s>>>(counts, offsets, totals, blocks);
        sort_scatter_kernel<KeyT><<<blocks, sort_block, 0, s>>>(kin, (pass == 0 && identity_vals) ? nullptr : vin, kout, vout, counts, offsets,
                                                                totals, n, shift, blocks);
        EFGS_HIP_CHECK(hipGetLastError());
        std::swap(kin, kout);
        std::swap(vin, vout);
        in_b = !in_b;
    }
    *result_in_b = in_b;
    return true;
}

bool radix_sort_pairs(void* keys_a, uint32_t* vals_a, void* keys_b, uint32_t* vals_b, bool identity_vals, uint32_t n, int key_bytes,
                      int end_bit, void* scratch, bool* result_in_b, hipStream_t s) {
    if (key_bytes == 4)
        return sort_impl(static_cast<uint32_t*>(keys_a), vals_a, static_cast<uint32_t*>(keys_b), vals_b, identity_vals, n, end_bit, scratch, result_in_b, s);
    if (key_bytes == 2)
        return sort_impl(static_cast<uint16_t*>(keys_a), vals_a, static_cast<uint16_t*>(keys_b), vals_b, identity_vals, n, end_bit, scratch, result_in_b, s);
    set_error("radix_sort_pairs: unsupported key width");
    return false;
}

}  // namespace efgs
