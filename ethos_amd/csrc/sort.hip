// Reordering of (token, head, k) pairs by expert id: an LSD radix sort of the expert
// ids carrying the pair index, followed by segmentation into unique experts.
// (No reference code: the reference loops over pairs in token order, model.py:306-334;
// the paper's Algorithm 1 reorders by expert, paper/ETHOS.pdf p.10.)
//
// Sort: 9-bit digits, ceil(bits / 9) passes over keys < n_experts (two for 262,144
// experts).  Each pass is
//   upsweep     per-tile digit histogram                 -> hist[digit][tile]
//   scan_tiles  per digit, exclusive scan over the tiles  -> hist[digit][tile], total[digit]
//   downsweep   stable scatter: digit base (scan of the totals, in LDS) + tile prefix +
//               rank inside the tile by wave-level multisplit
// A tile is 1024 keys = 4 waves x 4 chunks of 64 consecutive keys.  Inside a wave, the
// lanes holding the same digit are found with nine ballots ("peer mask"); the rank of a
// key is (keys of that digit in earlier waves) + (in earlier chunks of its wave) + (peers
// in lower lanes), which keeps the order of equal keys.  No global atomics; LDS counters
// are updated by one leader lane per digit.
//
// Segment: flags[i] = (i == 0 || key[i] != key[i-1]); slot = inclusive scan - 1.
// Outputs: perm (pair ids by expert), uniq (expert id per slot), seg_off (U + 1),
// pair_slot[p] (slot of pair p), sorted_slot[i] (slot of position i), n_unique.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"

namespace ethos {

constexpr int kSortChunks = 4;                  // chunks of 64 keys per wave
constexpr int kSortTile = 4 * kSortChunks * 64; // 1024 keys
constexpr int kRadixBits = 9;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kScanThreads = 1024;

__device__ __forceinline__ uint64_t peer_mask(uint32_t digit, uint64_t valid) {
    uint64_t peers = valid;
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
        const uint32_t bit = (digit >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
    }
    return peers;
}

__device__ __forceinline__ uint64_t lanemask_lt(int lane) { return (1ull << lane) - 1ull; }

__global__ __launch_bounds__(256) void sort_upsweep(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                    uint32_t* __restrict__ hist, int n_tiles) {
    __shared__ uint32_t cnt[4][kRadix];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = tid; i < 4 * kRadix; i += 256) cnt[i / kRadix][i % kRadix] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortTile + wave * (kSortChunks * 64);
#pragma unroll
    for (int c = 0; c < kSortChunks; ++c) {
        const int64_t idx = base + c * 64 + lane;
        const bool v = idx < n;
        const uint32_t key = v ? keys[idx] : 0u;
        const uint32_t dg = (key >> shift) & (kRadix - 1);
        const uint64_t peers = peer_mask(dg, __ballot(v));
        if (v && lane == 63 - __clzll((long long)peers)) cnt[wave][dg] += (uint32_t)__popcll(peers);
    }
    __syncthreads();
    for (int d = tid; d < kRadix; d += 256)
        hist[(int64_t)d * n_tiles + blockIdx.x] = cnt[0][d] + cnt[1][d] + cnt[2][d] + cnt[3][d];
}

// One wave per digit: exclusive scan of hist[digit][0 .. n_tiles) in place, the digit's
// total to total[digit].
__global__ __launch_bounds__(256) void sort_scan_tiles(uint32_t* __restrict__ hist, int n_tiles,
                                                       uint32_t* __restrict__ total) {
    const int lane = threadIdx.x & 63;
    const int d = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (d >= kRadix) return;
    uint32_t* row = hist + (int64_t)d * n_tiles;
    uint32_t carry = 0;
    for (int t0 = 0; t0 < n_tiles; t0 += 64 * 8) {
        uint32_t v[8], s = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int t = t0 + lane * 8 + j;
            v[j] = t < n_tiles ? row[t] : 0u;
            s += v[j];
        }
        uint32_t inc = s;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t u = __shfl_up(inc, off, 64);
            if (lane >= off) inc += u;
        }
        uint32_t run = carry + inc - s;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int t = t0 + lane * 8 + j;
            if (t < n_tiles) row[t] = run;
            run += v[j];
        }
        carry += __shfl(inc, 63, 64);
    }
    if (lane == 0) total[d] = carry;
}

template <bool kFirst>
__global__ __launch_bounds__(256) void sort_downsweep(const uint32_t* __restrict__ keys_in,
                                                      const uint32_t* __restrict__ vals_in,
                                                      uint32_t* __restrict__ keys_out,
                                                      uint32_t* __restrict__ vals_out, int64_t n, int shift,
                                                      const uint32_t* __restrict__ hist,
                                                      const uint32_t* __restrict__ total, int n_tiles) {
    __shared__ uint32_t cnt[4][kRadix];
    __shared__ uint32_t wsum[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int i = tid; i < 4 * kRadix; i += 256) cnt[i / kRadix][i % kRadix] = 0;
    // digit bases: exclusive scan of the digit totals (two digits per thread)
    const uint32_t ta = total[2 * tid], tb = total[2 * tid + 1];
    const uint32_t s = ta + tb;
    uint32_t inc = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t u = __shfl_up(inc, off, 64);
        if (lane >= off) inc += u;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    uint32_t wpre = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) wpre += w < wave ? wsum[w] : 0u;
    const uint32_t base_a = wpre + inc - s, base_b = base_a + ta;

    const int64_t base = (int64_t)blockIdx.x * kSortTile + wave * (kSortChunks * 64);
    uint32_t key[kSortChunks], val[kSortChunks], rank[kSortChunks];
#pragma unroll
    for (int c = 0; c < kSortChunks; ++c) {
        const int64_t idx = base + c * 64 + lane;
        const bool v = idx < n;
        key[c] = v ? keys_in[idx] : 0u;
        val[c] = v ? (kFirst ? (uint32_t)idx : vals_in[idx]) : 0u;
        const uint32_t dg = (key[c] >> shift) & (kRadix - 1);
        const uint64_t peers = peer_mask(dg, __ballot(v));
        const uint32_t below = (uint32_t)__popcll(peers & lanemask_lt(lane));
        uint32_t start = 0;
        if (v) start = cnt[wave][dg];
        __builtin_amdgcn_wave_barrier();
        rank[c] = start + below;
        if (v && lane == 63 - __clzll((long long)peers)) cnt[wave][dg] = start + (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int d = 2 * tid + j;
        uint32_t run = (j ? base_b : base_a) + hist[(int64_t)d * n_tiles + blockIdx.x];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t c = cnt[w][d];
            cnt[w][d] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kSortChunks; ++c) {
        const int64_t idx = base + c * 64 + lane;
        if (idx < n) {
            const uint32_t dg = (key[c] >> shift) & (kRadix - 1);
            const uint32_t pos = cnt[wave][dg] + rank[c];
            keys_out[pos] = key[c];
            vals_out[pos] = val[c];
        }
    }
}

// Exclusive scan of n uint32 in place by one workgroup; total -> *total (if given).
// Exclusive scan of a[0..n) in place, one workgroup.  Each thread holds 16 consecutive
// values in registers (four 16-byte loads issued together); thread sums are scanned
// across the wave with shuffles and across the 16 waves through LDS; chunks of 16384
// values are chained by a carry.  *total (if given) receives the sum of all values.
constexpr int kScanPer = 16;
constexpr int kScanChunk = kScanThreads * kScanPer;

__global__ __launch_bounds__(kScanThreads) void scan_exclusive(uint32_t* __restrict__ a, int64_t n,
                                                               int32_t* __restrict__ total) {
    __shared__ uint32_t wsum[kScanThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool vec = ((uintptr_t)a & 15) == 0;
    uint32_t carry = 0;
    for (int64_t base = 0; base < n; base += kScanChunk) {
        const int64_t lo = base + (int64_t)tid * kScanPer;
        const bool full = vec && lo + kScanPer <= n;
        uint32_t v[kScanPer];
        if (full) {
#pragma unroll
            for (int j = 0; j < kScanPer / 4; ++j) {
                const uint4 q = reinterpret_cast<const uint4*>(a + lo)[j];
                v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) v[j] = lo + j < n ? a[lo + j] : 0u;
        }
        uint32_t s = 0;
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) s += v[j];
        // inclusive wave scan of the thread sums
        uint32_t inc = s;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t t = __shfl_up(inc, off, 64);
            if (lane >= off) inc += t;
        }
        if (lane == 63) wsum[wave] = inc;
        __syncthreads();
        uint32_t wpre = 0, chunk_total = 0;
#pragma unroll
        for (int w = 0; w < kScanThreads / 64; ++w) {
            const uint32_t t = wsum[w];
            wpre += w < wave ? t : 0u;
            chunk_total += t;
        }
        __syncthreads();  // wsum is rewritten by the next chunk
        uint32_t run = carry + wpre + inc - s;
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) {
            const uint32_t t = v[j];
            v[j] = run;
            run += t;
        }
        if (full) {
#pragma unroll
            for (int j = 0; j < kScanPer / 4; ++j)
                reinterpret_cast<uint4*>(a + lo)[j] = make_uint4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
        } else {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j)
                if (lo + j < n) a[lo + j] = v[j];
        }
        carry += chunk_total;
    }
    if (tid == 0 && total) *total = (int32_t)carry;
}

// Head count per tile (items thread-contiguous: thread t owns 4 consecutive keys).
constexpr int kSegPer = kSortTile / 256;  // keys per thread in the segment kernels

__global__ __launch_bounds__(256) void seg_count(const uint32_t* __restrict__ keys, int64_t n,
                                                 uint32_t* __restrict__ tile_cnt) {
    __shared__ uint32_t red[256];
    const int tid = threadIdx.x;
    const int64_t lo = (int64_t)blockIdx.x * kSortTile + tid * kSegPer;
    uint32_t c = 0;
    for (int i = 0; i < kSegPer; ++i) {
        const int64_t idx = lo + i;
        if (idx < n && (idx == 0 || keys[idx] != keys[idx - 1])) ++c;
    }
    red[tid] = c;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) red[tid] += red[tid + off];
        __syncthreads();
    }
    if (tid == 0) tile_cnt[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(256) void seg_write(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ perm,
                                                 int64_t n, const uint32_t* __restrict__ tile_base,
                                                 int32_t* __restrict__ uniq, int32_t* __restrict__ seg_off,
                                                 int32_t* __restrict__ pair_slot, int32_t* __restrict__ sorted_slot,
                                                 int32_t* __restrict__ n_unique, int32_t max_unique) {
    __shared__ uint32_t part[256];
    const int tid = threadIdx.x;
    const int64_t lo = (int64_t)blockIdx.x * kSortTile + tid * kSegPer;
    uint32_t c = 0;
    for (int i = 0; i < kSegPer; ++i) {
        const int64_t idx = lo + i;
        if (idx < n && (idx == 0 || keys[idx] != keys[idx - 1])) ++c;
    }
    part[tid] = c;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const uint32_t v = tid >= off ? part[tid - off] : 0u;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    // slot of the item just before this thread's first head
    int32_t slot = (int32_t)(tile_base[blockIdx.x] + part[tid] - c) - 1;
    for (int i = 0; i < kSegPer; ++i) {
        const int64_t idx = lo + i;
        if (idx >= n) break;
        const uint32_t k = keys[idx];
        if (idx == 0 || k != keys[idx - 1]) {
            ++slot;
            if (slot < max_unique) {
                uniq[slot] = (int32_t)k;
                seg_off[slot] = (int32_t)idx;
            }
        }
        // Ids >= n_experts (a caller error) could make more slots than the buffers hold;
        // clamp so every later kernel stays in bounds.
        const int32_t s = slot < max_unique ? slot : max_unique - 1;
        sorted_slot[idx] = s;
        pair_slot[perm[idx]] = s;
        if (idx == n - 1) {
            const int32_t u = *n_unique < max_unique ? *n_unique : max_unique;
            *n_unique = u;
            seg_off[u] = (int32_t)n;
        }
    }
}

__global__ void seg_empty(int32_t* __restrict__ seg_off, int32_t* __restrict__ n_unique) {
    seg_off[0] = 0;
    *n_unique = 0;
}

int launch_sort_empty(int32_t* seg_off, int32_t* n_unique, hipStream_t stream) {
    hipLaunchKernelGGL(seg_empty, dim3(1), dim3(1), 0, stream, seg_off, n_unique);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Small batches (n <= kSmallMax pairs): the whole reordering in one workgroup.  Each pair
// becomes one 32-bit word, key << vb | pair index (vb bits for the index), so a stable LSD
// radix sort of the key digits orders the words by (expert id, pair id) -- the order of
// the multi-kernel path -- and carries the pair index along.  The words live in LDS (two
// buffers).  The 64-word chunks are split evenly over 16 waves in order, and every pass
// is: per-wave digit ranks by multisplit (as sort_downsweep), a scan of the per-wave digit
// counts in (digit, wave) order, a scatter between the buffers.  Segmentation works chunk
// by chunk: head flags as a ballot per chunk, a scan of the chunks' head counts, then
// every output written with coalesced stores (pair_slot scattered by pair).
// ---------------------------------------------------------------------------------
constexpr int kSmallWaves = 16;
constexpr int kSmallMax = 16384;
constexpr int kSmallChunks = kSmallMax / 64;                 // 256
constexpr int kSmallPer = kSmallChunks / kSmallWaves;        // chunks per wave at most

__global__ __launch_bounds__(kSmallWaves * 64) void sort_small_kernel(const int32_t* __restrict__ ids, int n,
                                                                      int key_bits_, int vb, int passes,
                                                                      int32_t* __restrict__ perm,
                                                                      int32_t* __restrict__ uniq,
                                                                      int32_t* __restrict__ seg_off,
                                                                      int32_t* __restrict__ pair_slot,
                                                                      int32_t* __restrict__ sorted_slot,
                                                                      int32_t* __restrict__ n_unique,
                                                                      int32_t max_unique) {
    __shared__ uint32_t buf[2][kSmallMax];
    __shared__ uint16_t cnt[kSmallWaves][kRadix];  // per-wave digit counts, then bases (< 2^14)
    __shared__ uint64_t cmask[kSmallChunks];       // head flags per chunk
    __shared__ uint32_t cbase[kSmallChunks];       // heads before each chunk
    __shared__ uint32_t wsum[kSmallWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t kmax = (1u << key_bits_) - 1u;
    const int n_chunks = (n + 63) / 64;
    const int cpw = (n_chunks + kSmallWaves - 1) / kSmallWaves;  // chunks per wave (<= kSmallPer)
    const int c0 = wave * cpw;
    {
        // all of the thread's ids in flight at once (one workgroup: latency, not bandwidth)
        constexpr int kIn = kSmallMax / (kSmallWaves * 64);
        uint32_t k[kIn];
#pragma unroll
        for (int j = 0; j < kIn; ++j) {
            const int i = tid + j * kSmallWaves * 64;
            k[j] = i < n ? (uint32_t)ids[i] : 0u;
        }
#pragma unroll
        for (int j = 0; j < kIn; ++j) {
            const int i = tid + j * kSmallWaves * 64;
            const uint32_t kk = k[j] > kmax ? kmax : k[j];  // ids outside [0, 2^key_bits) (a caller error) stay in range
            if (i < n) buf[0][i] = (kk << vb) | (uint32_t)i;
        }
    }
    int cur = 0;
    for (int p = 0; p < passes; ++p) {
        const int shift = vb + kRadixBits * p;
        for (int e = tid; e < kSmallWaves * kRadix; e += kSmallWaves * 64) cnt[e / kRadix][e % kRadix] = 0;
        __syncthreads();
        uint32_t word[kSmallPer], rank[kSmallPer];
#pragma unroll
        for (int j = 0; j < kSmallPer; ++j) {
            const int idx = (c0 + j) * 64 + lane;
            const bool v = j < cpw && idx < n;
            word[j] = v ? buf[cur][idx] : 0u;
            const uint32_t dg = (word[j] >> shift) & (kRadix - 1);
            const uint64_t peers = peer_mask(dg, __ballot(v));
            const uint32_t below = (uint32_t)__popcll(peers & lanemask_lt(lane));
            uint32_t start = 0;
            if (v) start = cnt[wave][dg];
            __builtin_amdgcn_wave_barrier();
            rank[j] = start + below;
            if (v && lane == 63 - __clzll((long long)peers)) cnt[wave][dg] = (uint16_t)(start + __popcll(peers));
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
        // digit d (threads 0 .. 511): bases of (d, wave) in digit-major, wave-minor order
        uint32_t tot = 0, inc = 0;
        if (tid < kRadix) {
#pragma unroll
            for (int w = 0; w < kSmallWaves; ++w) tot += cnt[w][tid];
            inc = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t u = __shfl_up(inc, off, 64);
                if (lane >= off) inc += u;
            }
            if (lane == 63) wsum[wave] = inc;
        }
        __syncthreads();
        if (tid < kRadix) {
            uint32_t run = inc - tot;
#pragma unroll
            for (int w = 0; w < kRadix / 64; ++w) run += w < wave ? wsum[w] : 0u;
#pragma unroll
            for (int w = 0; w < kSmallWaves; ++w) {
                const uint32_t c = cnt[w][tid];
                cnt[w][tid] = (uint16_t)run;
                run += c;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kSmallPer; ++j) {
            const int idx = (c0 + j) * 64 + lane;
            if (j < cpw && idx < n) buf[cur ^ 1][cnt[wave][(word[j] >> shift) & (kRadix - 1)] + rank[j]] = word[j];
        }
        cur ^= 1;
        __syncthreads();
    }
    // segments: head flags per chunk
    const uint32_t* w_ = buf[cur];
    for (int c = wave; c < n_chunks; c += kSmallWaves) {
        const int i = c * 64 + lane;
        const bool head = i < n && (i == 0 || (w_[i] >> vb) != (w_[i - 1] >> vb));
        const uint64_t m = __ballot(head);
        if (lane == 0) cmask[c] = m;
    }
    __syncthreads();
    // heads before each chunk: one wave scans the chunk counts (4 per lane)
    if (wave == 0) {
        uint32_t v[kSmallChunks / 64], sum = 0;
#pragma unroll
        for (int j = 0; j < kSmallChunks / 64; ++j) {
            const int c = lane * (kSmallChunks / 64) + j;
            v[j] = c < n_chunks ? (uint32_t)__popcll(cmask[c]) : 0u;
            sum += v[j];
        }
        uint32_t inc = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t u = __shfl_up(inc, off, 64);
            if (lane >= off) inc += u;
        }
        uint32_t run = inc - sum;
#pragma unroll
        for (int j = 0; j < kSmallChunks / 64; ++j) {
            const int c = lane * (kSmallChunks / 64) + j;
            if (c < kSmallChunks) cbase[c] = run;
            run += v[j];
        }
        if (lane == 63) wsum[0] = inc;  // all heads
    }
    __syncthreads();
    const int32_t u_all = (int32_t)wsum[0];
    const int32_t u_clamped = u_all < max_unique ? u_all : max_unique;
    const uint32_t imask = (1u << vb) - 1u;
    for (int c = wave; c < n_chunks; c += kSmallWaves) {
        const int i = c * 64 + lane;
        if (i < n) {
            const uint64_t m = cmask[c];
            const uint32_t wd = w_[i];
            // slot of position i: heads at positions <= i, minus one
            const int32_t slot = (int32_t)(cbase[c] + (uint32_t)__popcll(m & (lanemask_lt(lane) | (1ull << lane)))) - 1;
            if ((m >> lane) & 1ull) {
                if (slot < max_unique) {
                    uniq[slot] = (int32_t)(wd >> vb);
                    seg_off[slot] = i;
                }
            }
            const int32_t sc = slot < max_unique ? slot : max_unique - 1;
            const int32_t pi = (int32_t)(wd & imask);
            perm[i] = pi;
            sorted_slot[i] = sc;
            pair_slot[pi] = sc;
        }
    }
    if (tid == 0) {
        *n_unique = u_clamped;
        seg_off[u_clamped] = n;
    }
}

static int key_bits(int64_t n_experts) {
    int b = 0;
    while (b < 32 && ((int64_t)1 << b) < n_experts) ++b;
    return b;
}

size_t sort_workspace_bytes(int64_t n) {
    const int64_t tiles = (n + kSortTile - 1) / kSortTile;
    const size_t words = (size_t)4 * n + (size_t)kRadix * tiles + kRadix + (size_t)tiles + 64;
    return words * sizeof(uint32_t);
}

int launch_sort_segment(const int32_t* ids, int64_t n, int64_t n_experts, void* ws, int32_t* perm, int32_t* uniq,
                        int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique,
                        hipStream_t stream) {
    const int bits = key_bits(n_experts);
    const int passes = bits <= kRadixBits ? 1 : (bits + kRadixBits - 1) / kRadixBits;
    int vb = 0;
    while (vb < 31 && ((int64_t)1 << vb) < n) ++vb;
    if (n <= kSmallMax && bits + vb <= 32) {
        hipLaunchKernelGGL(sort_small_kernel, dim3(1), dim3(kSmallWaves * 64), 0, stream, ids, (int)n, bits, vb,
                           passes, perm, uniq, seg_off, pair_slot, sorted_slot, n_unique,
                           (int32_t)(n < n_experts ? n : n_experts));
        return (int)hipGetLastError();
    }
    const int n_tiles = (int)((n + kSortTile - 1) / kSortTile);
    uint32_t* w = reinterpret_cast<uint32_t*>(ws);
    uint32_t* kbuf[2] = {w, w + n};
    uint32_t* vbuf[2] = {w + 2 * n, w + 3 * n};
    uint32_t* hist = w + 4 * n;
    uint32_t* total = hist + (size_t)kRadix * n_tiles;
    uint32_t* tcnt = total + kRadix;
    hipError_t err;
    for (int p = 0; p < passes; ++p) {
        const uint32_t* kin = p == 0 ? reinterpret_cast<const uint32_t*>(ids) : kbuf[(p - 1) & 1];
        const uint32_t* vin = p == 0 ? nullptr : vbuf[(p - 1) & 1];
        uint32_t* kout = kbuf[p & 1];
        uint32_t* vout = p == passes - 1 ? reinterpret_cast<uint32_t*>(perm) : vbuf[p & 1];
        const int shift = kRadixBits * p;
        hipLaunchKernelGGL(sort_upsweep, dim3(n_tiles), dim3(256), 0, stream, kin, n, shift, hist, n_tiles);
        hipLaunchKernelGGL(sort_scan_tiles, dim3(kRadix / 4), dim3(256), 0, stream, hist, n_tiles, total);
        if (p == 0)
            hipLaunchKernelGGL(sort_downsweep<true>, dim3(n_tiles), dim3(256), 0, stream, kin, vin, kout, vout, n,
                               shift, (const uint32_t*)hist, (const uint32_t*)total, n_tiles);
        else
            hipLaunchKernelGGL(sort_downsweep<false>, dim3(n_tiles), dim3(256), 0, stream, kin, vin, kout, vout, n,
                               shift, (const uint32_t*)hist, (const uint32_t*)total, n_tiles);
        if ((err = hipGetLastError()) != hipSuccess) return (int)err;
    }
    const uint32_t* sorted = kbuf[(passes - 1) & 1];
    hipLaunchKernelGGL(seg_count, dim3(n_tiles), dim3(256), 0, stream, sorted, n, tcnt);
    hipLaunchKernelGGL(scan_exclusive, dim3(1), dim3(kScanThreads), 0, stream, tcnt, (int64_t)n_tiles, n_unique);
    hipLaunchKernelGGL(seg_write, dim3(n_tiles), dim3(256), 0, stream, sorted, (const uint32_t*)perm, n, tcnt, uniq,
                       seg_off, pair_slot, sorted_slot, n_unique, (int32_t)(n < n_experts ? n : n_experts));
    return (int)hipGetLastError();
}

}  // namespace ethos
