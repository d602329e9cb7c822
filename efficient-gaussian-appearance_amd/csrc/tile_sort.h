// The per-tile sort of bucket entries, run by the forward blend of each tile before its walk (no sort kernel: the
// blend reads its run's primitives from registers and LDS, and the sorted arrays it writes serve the backward).
// Keys are unique 64-bit values (depth key << 32 | emission index), sorted ascending by bitonic networks:
//   n <= 64, 128, 256 in registers, K = 1, 2, 4 keys per lane (element x = K lane + i): exchanges at distance
//                     j < K within a lane, j >= K with the lane at xor distance j / K (128 < n <= 192: a
//                     128-key and a 64-key network merged by rank);
//   256 < n <= 512    in the wave's LDS slab;
//   n > 512           chunks of 512 sorted in the slab and written back to the tile's range, then every key
//                     placed at (its index in its chunk) + (its rank in each other chunk).
#pragma once

#include "internal.h"

namespace efgs {

// runs of at most this many instances are sorted in registers (their primitives also go to LDS for the walk)
constexpr uint32_t forward_sort_max = 256;

// orders a wave's own LDS accesses across the steps of a network (the LDS executes a wave's instructions in
// order; the fence keeps the compiler from moving them)
__device__ __forceinline__ void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// The value of lane (lane ^ d) (d a power of two below 64, a constant after unrolling): one DPP move within a row
// for d = 1, 2 (quad permutations) and 8 (row rotation by 8), an LDS permute otherwise (the row swaps of gfx950
// overwrite both operands: two copies and a select per exchange cost more VALU than the permute).
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, uint32_t d) {
    if (d == 1) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf, true));  // quad_perm [1,0,3,2]
    if (d == 2) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf, true));  // quad_perm [2,3,0,1]
    if (d == 8) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x128, 0xf, 0xf, true));  // row_ror:8
    return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), static_cast<int>(d)));
}
__device__ __forceinline__ uint64_t xor_lane_u64(uint64_t v, uint32_t d) {
    const uint32_t lo = xor_lane(static_cast<uint32_t>(v), d);
    const uint32_t hi = xor_lane(static_cast<uint32_t>(v >> 32), d);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <uint32_t K>
__device__ __forceinline__ void wave_bitonic(uint64_t (&k)[K], uint32_t lane) {
#pragma unroll
    for (uint32_t size = 2; size <= 64 * K; size <<= 1) {
#pragma unroll
        for (uint32_t j = size >> 1; j > 0; j >>= 1) {
            if (j >= K) {
#pragma unroll
                for (uint32_t i = 0; i < K; i++) {
                    const uint32_t x = K * lane + i;
                    const uint64_t o = xor_lane_u64(k[i], j / K);
                    const bool keep_min = ((x & size) == 0) == ((x & j) == 0);
                    // the partner's key belongs here exactly when it is the smaller one where the lane keeps the
                    // minimum and the larger one elsewhere: one compare and one select (equal keys: either)
                    k[i] = (o < k[i]) == keep_min ? o : k[i];
                }
            } else {
#pragma unroll
                for (uint32_t i = 0; i < K; i++) {
                    if ((i & j) != 0) continue;
                    const uint32_t x = K * lane + i;
                    const uint64_t a = k[i], b = k[i ^ j];
                    const bool swap = (a > b) == ((x & size) == 0);
                    k[i] = swap ? b : a;
                    k[i ^ j] = swap ? a : b;
                }
            }
        }
    }
}

// A bucket entry: emission index, depth key, primitive, 0 (the first eight bytes, little-endian, are the sort key
// depth key << 32 | emission index).
__device__ __forceinline__ uint64_t key_of(uint4 b) { return (static_cast<uint64_t>(b.y) << 32) | b.x; }

// Where a tile's sorted instances go: the emission index, the instance's primitive and the tile key. The bucket
// holds each key's primitive beside it. Runs of at most 256 keys whose emission indices fit 24 bits sort the key
// (depth << 32 | e << 8 | u), u the key's index in the run: e is unique, so the order is that of (depth, e), and
// the primitive is read back from the wave's slab at u (put_packed). Other runs gather it from inst_prim (put).
template <typename KeyT>
struct SortedOut {
    uint32_t* inst;
    uint32_t* prim;
    KeyT* keys;
    const uint32_t* inst_prim;
    uint32_t tile;
    uint32_t* lds_prim;  // (optional) the primitives in sorted order in LDS as well
    __device__ __forceinline__ void put(uint32_t pos, uint64_t key) const {
        const uint32_t e = static_cast<uint32_t>(key);
        const uint32_t p = inst_prim[e];
        inst[pos] = e;
        prim[pos] = p;
        keys[pos] = static_cast<KeyT>(tile);
        if (lds_prim) lds_prim[pos] = p;
    }
    __device__ __forceinline__ void put_packed(uint32_t pos, uint64_t key, const uint32_t* s_prim) const {
        const uint32_t lo = static_cast<uint32_t>(key);
        const uint32_t p = s_prim[lo & 0xffu];
        inst[pos] = lo >> 8;
        prim[pos] = p;
        keys[pos] = static_cast<KeyT>(tile);
        if (lds_prim) lds_prim[pos] = p;
    }
};
// the sort key of run index u (< 256) when every emission index fits 24 bits
__device__ __forceinline__ uint64_t pack_run_index(uint64_t key, uint32_t u) {
    return (key & 0xffffffff00000000ull) | (static_cast<uint64_t>(static_cast<uint32_t>(key) << 8)) | u;
}

// n <= 64 K keys of the tile's run, sorted in registers (K keys per lane, element x = K lane + i), written out
template <uint32_t K, typename KeyT>
__device__ __forceinline__ void sort_run_in_registers(const uint4* run, uint32_t n, const SortedOut<KeyT>& o, uint32_t lane, bool packed,
                                                      uint32_t* s_prim) {
    uint64_t k[K];
#pragma unroll
    for (uint32_t i = 0; i < K; i++) {
        const uint32_t x = K * lane + i;
        const uint4 b = x < n ? run[x] : make_uint4(~0u, ~0u, 0u, 0u);
        k[i] = key_of(b);
        if (packed && x < n) {
            s_prim[x] = b.z;
            k[i] = pack_run_index(k[i], x);
        }
    }
    wave_lds_fence();
    wave_bitonic<K>(k, lane);
#pragma unroll
    for (uint32_t i = 0; i < K; i++) {
        const uint32_t x = K * lane + i;
        if (x < n) {
            if (packed) o.put_packed(x, k[i], s_prim);
            else o.put(x, k[i]);
        }
    }
    wave_lds_fence();  // (the slab is free again after every lane's reads)
}

// number of keys below x in the ascending run [0, n)
__device__ __forceinline__ uint32_t rank_in(const uint64_t* run, uint32_t n, uint64_t x) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (run[mid] < x) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// 128 < n <= 192: the first 128 keys (two per lane) and the other n - 128 (one per lane) are sorted by their own
// register networks and merged: a key's position is its index in its own sorted part plus the number of keys of
// the other part below it (keys are unique), found by binary search in the wave's slab. About half the work of
// the 256-key network the run would otherwise be padded to.
template <typename KeyT>
__device__ __forceinline__ void sort_run_split192(const uint4* run, uint32_t n, const SortedOut<KeyT>& o, uint32_t lane, uint64_t* s,
                                                  bool packed) {
    const uint4 ba0 = run[2 * lane], ba1 = run[2 * lane + 1];
    const uint4 bb0 = 128 + lane < n ? run[128 + lane] : make_uint4(~0u, ~0u, 0u, 0u);
    uint64_t a[2] = {key_of(ba0), key_of(ba1)}, b[1] = {key_of(bb0)};
    uint32_t* const s_prim = reinterpret_cast<uint32_t*>(s + 256);  // (the keys take s[0 .. 192))
    if (packed) {
        s_prim[2 * lane] = ba0.z;
        s_prim[2 * lane + 1] = ba1.z;
        a[0] = pack_run_index(a[0], 2 * lane);
        a[1] = pack_run_index(a[1], 2 * lane + 1);
        if (128 + lane < n) {
            s_prim[128 + lane] = bb0.z;
            b[0] = pack_run_index(b[0], 128 + lane);
        }
    }
    wave_bitonic<2>(a, lane);
    wave_bitonic<1>(b, lane);
    s[2 * lane] = a[0];
    s[2 * lane + 1] = a[1];
    s[128 + lane] = b[0];
    wave_lds_fence();
    const uint32_t nb = n - 128;
#pragma unroll
    for (uint32_t i = 0; i < 2; i++) {
        const uint32_t pos = 2 * lane + i + rank_in(s + 128, nb, a[i]);
        if (packed) o.put_packed(pos, a[i], s_prim);
        else o.put(pos, a[i]);
    }
    if (lane < nb) {
        const uint32_t pos = lane + rank_in(s, 128, b[0]);
        if (packed) o.put_packed(pos, b[0], s_prim);
        else o.put(pos, b[0]);
    }
    wave_lds_fence();  // the slab is free again only after every lane's searches
}

// A run of n <= forward_sort_max bucket entries sorted by the smallest register network that holds it (the sizes
// are wave-uniform); slab: the wave's LDS scratch, 3 KB (keys of the merge and the packed runs' primitives).
template <typename KeyT>
__device__ __forceinline__ void sort_small_run(const uint4* run, uint32_t n, const SortedOut<KeyT>& o, uint32_t lane, bool packed, uint64_t* slab) {
    uint32_t* const s_prim = reinterpret_cast<uint32_t*>(slab);
    if (n <= 64) sort_run_in_registers<1>(run, n, o, lane, packed, s_prim);
    else if (n <= 128) sort_run_in_registers<2>(run, n, o, lane, packed, s_prim);
    else if (n <= 192) sort_run_split192(run, n, o, lane, slab, packed);
    else sort_run_in_registers<4>(run, n, o, lane, packed, s_prim);
}

constexpr uint32_t wave_slab = 512;  // keys of a wave's LDS slab

// ascending bitonic sort of m (a power of two, <= wave_slab) keys in the wave's slab
__device__ inline void wave_bitonic_lds(uint64_t* s, uint32_t m, uint32_t lane) {
    for (uint32_t size = 2; size <= m; size <<= 1) {
        for (uint32_t j = size >> 1; j > 0; j >>= 1) {
            for (uint32_t x = lane; x < m; x += 64) {
                const uint32_t y = x ^ j;
                if (y > x) {
                    const uint64_t a = s[x], b = s[y];
                    if ((a > b) == ((x & size) == 0)) {
                        s[x] = b;
                        s[y] = a;
                    }
                }
            }
            wave_lds_fence();
        }
    }
}

// number of keys below x in the ascending run of bucket entries [0, n)
__device__ __forceinline__ uint32_t rank_in_bucket(const uint4* run, uint32_t n, uint64_t x) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (key_of(run[mid]) < x) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// One run of n > forward_sort_max keys (the wave's slab s: wave_slab keys); the sorted arrays in global memory only.
template <typename KeyT>
__device__ inline void sort_big_run(uint4* bucket, uint2 r, uint32_t n, uint32_t tile, uint32_t* sorted_inst, KeyT* sorted_keys,
                             const uint32_t* inst_prim, uint32_t* sorted_prim, uint32_t lane, uint64_t* s) {
    uint4* run = bucket + r.x;
    const SortedOut<KeyT> o{sorted_inst + r.x, sorted_prim + r.x, sorted_keys + r.x, inst_prim, tile, nullptr};
    if (n <= wave_slab) {
        uint32_t m = 512;
        while (m < n) m <<= 1;
        for (uint32_t x = lane; x < m; x += 64) s[x] = x < n ? key_of(run[x]) : ~0ull;
        wave_lds_fence();
        wave_bitonic_lds(s, m, lane);
        for (uint32_t x = lane; x < n; x += 64) o.put(x, s[x]);
        return;
    }
    const uint32_t n_chunks = (n + wave_slab - 1) / wave_slab;
    for (uint32_t c = 0; c < n_chunks; c++) {
        const uint32_t c0 = c * wave_slab, cn = min(wave_slab, n - c0);
        for (uint32_t x = lane; x < wave_slab; x += 64) s[x] = x < cn ? key_of(run[c0 + x]) : ~0ull;
        wave_lds_fence();
        wave_bitonic_lds(s, wave_slab, lane);
        for (uint32_t x = lane; x < cn; x += 64) run[c0 + x] = make_uint4(static_cast<uint32_t>(s[x]), static_cast<uint32_t>(s[x] >> 32), 0u, 0u);
        wave_lds_fence();
    }
    __threadfence();  // the wave reads back the chunks it wrote
    for (uint32_t idx = lane; idx < n; idx += 64) {
        const uint64_t key = key_of(run[idx]);
        const uint32_t c = idx / wave_slab;
        uint32_t pos = idx - c * wave_slab;
        for (uint32_t oc = 0; oc < n_chunks; oc++) {
            if (oc == c) continue;
            const uint32_t o0 = oc * wave_slab;
            pos += rank_in_bucket(run + o0, min(wave_slab, n - o0), key);
        }
        o.put(pos, key);
    }
}

}  // namespace efgs
