// Scan of the preprocess's per-block (visible, instance) counts on wave64 (one block): the offsets that the
// compaction and the instance emission use, the visible and instance totals read back by the host, and the
// visible depth-key range. Replaces the reference's cub::DeviceScan calls (B/rasterization/src/forward.cu:
// 107-114) together with the per-block counts the preprocess kernels produce.
#include "internal.h"

namespace efgs {

namespace {

// inclusive scan of v over the 64 lanes of a wave (Hillis-Steele with lane shuffles)
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v, uint32_t lane) {
#pragma unroll
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(v, o);
        if (lane >= o) v += t;
    }
    return v;
}

// exclusive scan over the block's threads; returns the thread's exclusive prefix and the block total
template <uint32_t BLOCK>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t& total) {
    __shared__ uint32_t wave_totals[BLOCK / 64];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_inclusive_scan(v, lane);
    if (lane == 63) wave_totals[wave] = inc;
    __syncthreads();
    uint32_t wave_prefix = 0;
    total = 0;
#pragma unroll
    for (uint32_t w = 0; w < BLOCK / 64; w++) {
        const uint32_t t = wave_totals[w];
        if (w < wave) wave_prefix += t;
        total += t;
    }
    __syncthreads();
    return wave_prefix + inc - v;
}

// one block: offsets of the per-preprocess-block (visible, instance) counts; counters[0] = V, counters[1] = I,
// counters[3] / counters[4] = min / max depth key of the visible primitives, also written to the host's pinned
// buffer (device address host_counters), followed, after a system-scope fence, by the frame's sequence number
// in host_counters[counter_sequence]: the host polls that word instead of waiting for an event or a copy
constexpr uint32_t scan_regs = 8;  // chunks per thread held in registers (up to 8,192 chunks, 2M primitives)
__global__ __launch_bounds__(1024) void scan_block_counts_kernel(const uint32_t* counts, const uint32_t* key_ranges, uint32_t* offsets,
                                                                 uint32_t* counters, uint32_t* host_counters, uint32_t capacity, uint32_t seq,
                                                                 uint32_t n) {
    __shared__ uint32_t s_range[2 * 16];
    const uint32_t per = (n + 1023) / 1024;
    const uint32_t base = threadIdx.x * per;
    const uint2* counts2 = reinterpret_cast<const uint2*>(counts);
    const uint2* ranges2 = reinterpret_cast<const uint2*>(key_ranges);
    uint32_t sv = 0, si = 0, kmin = 0xffffffffu, kmax = 0u;
    uint2 c[scan_regs];
    const bool in_regs = per <= scan_regs;  // (block-uniform)
    if (in_regs) {
        // every load of the thread's chunks in flight at once (one memory round trip, not one per chunk)
        uint2 r[scan_regs];
#pragma unroll
        for (uint32_t k = 0; k < scan_regs; k++) {
            const bool in = k < per && base + k < n;
            c[k] = in ? counts2[base + k] : make_uint2(0u, 0u);
            r[k] = in ? ranges2[base + k] : make_uint2(0xffffffffu, 0u);
        }
#pragma unroll
        for (uint32_t k = 0; k < scan_regs; k++) {
            sv += c[k].x;
            si += c[k].y;
            kmin = min(kmin, r[k].x);
            kmax = max(kmax, r[k].y);
        }
    } else {
        for (uint32_t k = 0; k < per; k++) {
            if (base + k < n) {
                sv += counts[2 * (base + k)];
                si += counts[2 * (base + k) + 1];
                kmin = min(kmin, key_ranges[2 * (base + k)]);
                kmax = max(kmax, key_ranges[2 * (base + k) + 1]);
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        kmin = min(kmin, static_cast<uint32_t>(__shfl_xor(kmin, o)));
        kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(kmax, o)));
    }
    if ((threadIdx.x & 63u) == 0) {
        s_range[2 * (threadIdx.x >> 6)] = kmin;
        s_range[2 * (threadIdx.x >> 6) + 1] = kmax;
    }
    __syncthreads();
    uint32_t tv, ti;
    uint32_t pv = block_exclusive_scan<1024>(sv, tv);
    uint32_t pi = block_exclusive_scan<1024>(si, ti);
    uint2* offsets2 = reinterpret_cast<uint2*>(offsets);
    if (in_regs) {
#pragma unroll
        for (uint32_t k = 0; k < scan_regs; k++) {
            if (k < per && base + k < n) {
                offsets2[base + k] = make_uint2(pv, pi);
                pv += c[k].x;
                pi += c[k].y;
            }
        }
    } else {
        for (uint32_t k = 0; k < per; k++) {
            if (base + k < n) {
                offsets[2 * (base + k)] = pv;
                offsets[2 * (base + k) + 1] = pi;
                pv += counts[2 * (base + k)];
                pi += counts[2 * (base + k) + 1];
            }
        }
    }
    if (threadIdx.x == 0) {
        uint32_t lo = 0xffffffffu, hi = 0u;
        for (uint32_t w = 0; w < 16; w++) {
            lo = min(lo, s_range[2 * w]);
            hi = max(hi, s_range[2 * w + 1]);
        }
        // [2]: emission mismatches, see create_instances; [5]: the instances do not fit the binning buffers
        const uint32_t c[6] = {tv, ti, 0u, tv > 0 ? lo : 0u, tv > 0 ? hi : 0u, ti > capacity ? 1u : 0u};
#pragma unroll
        for (uint32_t k = 0; k < 6; k++) {
            counters[k] = c[k];
            host_counters[k] = c[k];
        }
        __threadfence_system();
        __hip_atomic_store(&host_counters[counter_sequence], seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        __threadfence_system();
    }
}

}  // namespace

bool launch_scan_block_counts(const uint32_t* block_counts, const uint32_t* key_ranges, uint32_t* block_offsets, uint32_t* counters,
                              uint32_t* host_counters, uint32_t capacity, uint32_t seq, uint32_t n_blocks, hipStream_t s) {
    scan_block_counts_kernel<<<1, 1024, 0, s>>>(block_counts, key_ranges, block_offsets, counters, host_counters, capacity, seq, n_blocks);
    EFGS_HIP_CHECK(hipGetLastError());
    return true;
}


}  // namespace efgs
