// Stable LSD radix sort of (key, value) pairs for wave64, 8-bit digits, 1024 keys per 256-thread block.
// Per pass: per-block digit histogram -> device exclusive scan in digit-major order -> stable scatter.
// Within a block, keys are taken in index order (4 rounds of 256); a wave ranks its 64 keys per digit with
// 64-bit ballots (lanes sharing a digit form a peer mask; rank = peers below the lane), waves are ordered
// through a per-round digit prefix in LDS. Replaces cub::DeviceRadixSort
// (B/rasterization/src/forward.cu:88-96 depth keys, :182-190 tile keys).
#include "internal.h"

namespace efgs {

namespace {

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

template <typename KeyT>
__global__ __launch_bounds__(sort_block) void sort_histogram_kernel(const KeyT* keys, uint32_t* hist, uint32_t n, uint32_t shift, uint32_t n_blocks) {
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
    hist[threadIdx.x * n_blocks + blockIdx.x] = h[threadIdx.x];
}

template <typename KeyT>
__global__ __launch_bounds__(sort_block) void sort_scatter_kernel(const KeyT* keys_in, const uint32_t* vals_in, KeyT* keys_out, uint32_t* vals_out,
                                                                 const uint32_t* offsets, uint32_t n, uint32_t shift, uint32_t n_blocks) {
    __shared__ uint32_t digit_base[sort_bins];
    __shared__ uint32_t wave_hist[sort_block / 64][sort_bins];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint64_t lanes_below = (1ull << lane) - 1ull;
    digit_base[threadIdx.x] = offsets[threadIdx.x * n_blocks + blockIdx.x];
    const uint32_t start = blockIdx.x * sort_tile;
    for (uint32_t r = 0; r < sort_rounds; r++) {
#pragma unroll
        for (uint32_t w = 0; w < sort_block / 64; w++) wave_hist[w][threadIdx.x] = 0;
        __syncthreads();
        const uint32_t i = start + r * sort_block + threadIdx.x;
        const bool valid = i < n;
        KeyT key = 0;
        uint32_t val = 0;
        if (valid) {
            key = keys_in[i];
            val = vals_in ? vals_in[i] : i;
        }
        const uint32_t d = (static_cast<uint32_t>(key) >> shift) & 255u;
        const uint64_t peers = match_peers(d, valid);
        const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lanes_below));
        if (valid && rank == 0) wave_hist[wave][d] = static_cast<uint32_t>(__popcll(peers));
        __syncthreads();
        {
            uint32_t run = digit_base[threadIdx.x];
#pragma unroll
            for (uint32_t w = 0; w < sort_block / 64; w++) {
                const uint32_t c = wave_hist[w][threadIdx.x];
                wave_hist[w][threadIdx.x] = run;
                run += c;
            }
            digit_base[threadIdx.x] = run;
        }
        __syncthreads();
        if (valid) {
            const uint32_t pos = wave_hist[wave][d] + rank;
            keys_out[pos] = key;
            vals_out[pos] = val;
        }
        __syncthreads();
    }
}

}  // namespace

size_t sort_scratch_bytes(uint32_t n) {
    const uint32_t blocks = div_up(n > 0 ? n : 1, sort_tile);
    const size_t hist = sizeof(uint32_t) * static_cast<size_t>(sort_bins) * blocks;
    return 2 * ((hist + 255) & ~static_cast<size_t>(255)) + scan_scratch_bytes(sort_bins * blocks);
}

template <typename KeyT>
static bool sort_impl(KeyT* ka, uint32_t* va, KeyT* kb, uint32_t* vb, bool identity_vals, uint32_t n, int end_bit, void* scratch,
                      bool* result_in_b, hipStream_t s) {
    *result_in_b = false;
    if (n == 0) return true;
    const uint32_t blocks = div_up(n, sort_tile);
    const size_t hist_bytes = (sizeof(uint32_t) * static_cast<size_t>(sort_bins) * blocks + 255) & ~static_cast<size_t>(255);
    uint32_t* hist = static_cast<uint32_t*>(scratch);
    uint32_t* offsets = reinterpret_cast<uint32_t*>(static_cast<char*>(scratch) + hist_bytes);
    void* scan_scratch = static_cast<char*>(scratch) + 2 * hist_bytes;
    // at least one pass, so identity values are always materialised
    const int passes = end_bit > 0 ? (end_bit + 7) / 8 : 1;
    KeyT* kin = ka;
    uint32_t* vin = va;
    KeyT* kout = kb;
    uint32_t* vout = vb;
    bool in_b = false;
    for (int pass = 0; pass < passes; pass++) {
        const uint32_t shift = 8u * static_cast<uint32_t>(pass);
        sort_histogram_kernel<KeyT><<<blocks, sort_block, 0, s>>>(kin, hist, n, shift, blocks);
        if (!scan_exclusive(hist, nullptr, offsets, nullptr, sort_bins * blocks, scan_scratch, s)) return false;
        sort_scatter_kernel<KeyT><<<blocks, sort_block, 0, s>>>(kin, (pass == 0 && identity_vals) ? nullptr : vin, kout, vout, offsets, n, shift, blocks);
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
