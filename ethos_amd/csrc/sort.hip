// Reordering of (token, head, k) pairs by expert id: an LSD radix sort of the expert
// ids carrying the pair index, with the segmentation into unique experts done in its
// last pass.
// (No reference code: the reference loops over pairs in token order, model.py:306-334;
// the paper's Algorithm 1 reorders by expert, paper/ETHOS.pdf p.10.)
//
// Sort: 9-bit digits, P = ceil(bits / 9) passes over keys < n_experts (two for 262,144
// experts), over tiles of 4096 keys (one workgroup of 16 waves each).  A pass is
//   count/stats  per-tile digit counts (last pass: also per digit the number of distinct
//                keys, and the lower bits of the first and last key)
//   scan         per digit, exclusive prefix over the tiles (last pass: also of the new
//                distinct keys, and the lower bits of the last earlier key)
//   down         stable scatter: digit base (scan of the totals) + tile prefix + rank in
//                the tile by wave-level multisplit; the tile is first ranked by digit into
//                LDS, then written with consecutive output positions on consecutive lanes
// Inside a wave, the lanes holding the same digit are found with nine ballots ("peer
// mask"); the rank of a key is (keys of that digit in earlier waves) + (in earlier chunks
// of its wave) + (peers in lower lanes), which keeps the order of equal keys.  No global
// atomics and no waiting between workgroups; LDS counters are updated by one leader lane
// per digit.
//
// Segmentation (last pass).  Equal keys are adjacent in the final order, and inside a
// tile's group of one digit the keys come in the order of their lower bits (the earlier
// passes' order), so the tile can rank its keys locally (LDS) and tell its heads (first
// key of a segment): a key differs from the one before it in the tile's group, or, for
// the group's first key, from the last key of that digit in earlier tiles (the scan's
// prefix maximum of the tiles' last lower bits; keys of one digit are non-decreasing over
// the tiles).  Slot = (new distinct keys of smaller digits and of this digit in earlier
// tiles) + (heads so far in the group) - 1.
// Outputs: perm (pair ids by expert), uniq (expert id per slot), seg_off (U + 1),
// pair_slot[p] (slot of pair p), sorted_slot[i] (slot of position i), n_unique.  The last
// pass scatters pair_slot by pair (one 4-byte store per pair to a random place).  Above
// 2^20 pairs with ids of at most 18 bits, where those stores cost more than a launch, it
// writes an expert -> slot table at the heads instead (one store per unique expert) and a
// gather over the ids in pair order writes pair_slot with coalesced stores.

#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_tp.hpp"

namespace ethos {

constexpr int kRadixBits = 9;
constexpr int kRadix = 1 << kRadixBits;

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

// ---------------------------------------------------------------------------------
// Tile passes: a tile is kTile = kSortTileKeys (4096) consecutive keys, one workgroup of
// kTW = 16 waves; wave w owns chunks w kTC .. w kTC + kTC - 1 of 64 keys (kTC = 4).
// Every kernel issues its per-digit table loads first, so that they overlap the key loads.
// ---------------------------------------------------------------------------------
constexpr int kTW = 16;
constexpr int kTThreads = kTW * 64;
constexpr int kTile = kSortTileKeys;
constexpr int kTC = kTile / (kTW * 64);
constexpr int kTPer = kTile / kTThreads;  // tile-local positions per thread in the segment phase
static_assert(kTC * kTW * 64 == kTile && kTPer == 4, "tile shape");

// The tile of this workgroup.  Workgroup b runs on XCD b % 8.  The per-digit statistics
// are rows of sort_tile_pitch(n_tiles) words, one per tile, so that each aligned group of
// 8 tiles shares 32-byte sectors; the groups are dealt to the XCDs in turn (group g to XCD
// g % 8) and a group's 8 tiles run on its XCD, so that their statistics stores merge in
// that XCD's L2 while runs of hot keys still spread over all XCDs.  The grid is padded to
// 64 workgroups per 8 groups: -1 for the padding workgroups.
__device__ __forceinline__ int tsort_tile(int n_tiles) {
    const int x = (int)(blockIdx.x & 7), j = (int)(blockIdx.x >> 3);
    const int t = ((j >> 3) * 8 + x) * 8 + (j & 7);
    return t < n_tiles ? t : -1;
}
static unsigned tsort_grid(int n_tiles) { return 64u * (unsigned)(((n_tiles + 7) / 8 + 7) / 8); }

// Exclusive scans of NV values per thread over threads 0 .. 511 (waves 0 .. 7; the other
// threads pass zeros), in one pass.  Every thread of the workgroup calls it (it holds
// barriers); tot[] receives the sums.  wsum: 8 NV words of LDS.  The waves' totals are read
// with one LDS load (one per lane) and combined with lane reads into scalar registers.
template <int NV>
__device__ __forceinline__ void scan512(const uint32_t (&v)[NV], uint32_t (&ex)[NV], uint32_t (&tot)[NV],
                                        uint32_t* wsum) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t inc[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) inc[c] = v[c];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const uint32_t u = __shfl_up(inc[c], off, 64);
            if (lane >= off) inc[c] += u;
        }
    }
    if (wave < kRadix / 64 && lane == 63) {
#pragma unroll
        for (int c = 0; c < NV; ++c) wsum[wave * NV + c] = inc[c];
    }
    __syncthreads();
    static_assert(kRadix / 64 * NV <= 64, "one wave total per lane");
    const int uwave = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t x = lane < kRadix / 64 * NV ? wsum[lane] : 0u;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        uint32_t pre = 0, t = 0;
#pragma unroll
        for (int w = 0; w < kRadix / 64; ++w) {
            const uint32_t y = __builtin_amdgcn_readlane(x, w * NV + c);
            pre += w < uwave ? y : 0u;
            t += y;
        }
        ex[c] = pre + inc[c] - v[c];
        tot[c] = t;
    }
    __syncthreads();  // wsum may be reused by the caller
}

// Exclusive scan of one value per thread over the workgroup's 1024 threads; tot gets the
// sum.  wsum: kTW words of LDS.
__device__ __forceinline__ uint32_t scan1024(uint32_t v, uint32_t* wsum, uint32_t& tot) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t u = __shfl_up(inc, off, 64);
        if (lane >= off) inc += u;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    const int uwave = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t x = lane < kTW ? wsum[lane] : 0u;
    uint32_t pre = 0, t = 0;
#pragma unroll
    for (int w = 0; w < kTW; ++w) {
        const uint32_t y = __builtin_amdgcn_readlane(x, w);
        pre += w < uwave ? y : 0u;
        t += y;
    }
    __syncthreads();
    tot = t;
    return pre + inc - v;
}

// Phase A of a tile pass: load the wave's chunks (key; value = the key's index on the first
// pass) and rank them by digit in order.  wcnt[w][d] must be zero on entry; on exit it holds
// wave w's count of digit d, and rank[j] the number of keys of the same digit before chunk
// j's key in wave w.
template <bool kFirst>
__device__ __forceinline__ void tile_load(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
                                          int64_t n, int tile, uint32_t (&key)[kTC], uint32_t (&val)[kTC]) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t base = (int64_t)tile * kTile + wave * (kTC * 64);
#pragma unroll
    for (int j = 0; j < kTC; ++j) {
        const int64_t idx = base + j * 64 + lane;
        const bool v = idx < n;
        key[j] = v ? keys[idx] : 0u;
        val[j] = v ? (kFirst ? (uint32_t)idx : vals[idx]) : 0u;
    }
}
__device__ __forceinline__ void tile_rank(int64_t n, int tile, int shift, uint32_t (*wcnt)[kRadix],
                                          const uint32_t (&key)[kTC], uint32_t (&rank)[kTC]) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t base = (int64_t)tile * kTile + wave * (kTC * 64);
#pragma unroll
    for (int j = 0; j < kTC; ++j) {
        const bool v = base + j * 64 + lane < n;
        const uint32_t dg = (key[j] >> shift) & (kRadix - 1);
        const uint64_t peers = peer_mask(dg, __ballot(v));
        const uint32_t below = (uint32_t)__popcll(peers & lanemask_lt(lane));
        uint32_t start = 0;
        if (v) start = wcnt[wave][dg];
        __builtin_amdgcn_wave_barrier();
        rank[j] = start + below;
        if (v && lane == 63 - __clzll((long long)peers)) wcnt[wave][dg] = start + (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
}

// After phase A (and a barrier): thread d < 512 turns wcnt[.][d] into the exclusive prefix
// over the waves and returns the tile's count of digit d (0 for the other threads).
__device__ __forceinline__ uint32_t tile_digit_counts(uint32_t (*wcnt)[kRadix]) {
    const int d = threadIdx.x;
    if (d >= kRadix) return 0u;
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kTW; ++w) {
        const uint32_t c = wcnt[w][d];
        wcnt[w][d] = run;
        run += c;
    }
    return run;
}

__device__ __forceinline__ void zero_wcnt(uint32_t (*wcnt)[kRadix]) {
    uint4* w = reinterpret_cast<uint4*>(&wcnt[0][0]);
    for (int e = threadIdx.x; e < kTW * kRadix / 4; e += kTThreads) w[e] = make_uint4(0u, 0u, 0u, 0u);
}

// Per-tile digit counts of one (non-last) pass: cnt[d * sort_tile_pitch(n_tiles) + tile].
__global__ __launch_bounds__(kTThreads) void tsort_count(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                         int n_tiles, uint32_t* __restrict__ cnt) {
    const int tile = tsort_tile(n_tiles);
    if (tile < 0) return;
    __shared__ uint32_t c[kRadix];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)tile * kTile + tid;
    uint32_t k[kTPer];
#pragma unroll
    for (int j = 0; j < kTPer; ++j) k[j] = base + j * kTThreads < n ? keys[base + j * kTThreads] : 0u;
    if (tid < kRadix) c[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTPer; ++j)
        if (base + j * kTThreads < n) atomicAdd(&c[(k[j] >> shift) & (kRadix - 1)], 1u);
    __syncthreads();
    if (tid < kRadix) cnt[(int64_t)tid * sort_tile_pitch(n_tiles) + tile] = c[tid];
}

// Per-tile statistics of the last pass (keys sorted by their lower bits lo = key & lomask),
// for each digit d of the tile: cnt (keys), dist (distinct keys), flo / llo (lower bits of
// the digit's first and last key in the tile's order, i.e. the smallest and largest).
// Keys of at most 18 bits (two passes): every key sets its bit in a bitmap of all keys in
// LDS; with shift = 9 a digit's keys are the 512 bits [512 d, 512 d + 512) of it, so its
// distinct keys are their population count and flo / llo the lowest and highest set bit
// (two threads per digit, 256 bits each); with shift = 0 (one pass) a digit is one key.
// The only atomics per key are the count and the (no-return) bit set.
__global__ __launch_bounds__(kTThreads) void tsort_stats_map(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                             uint32_t mkmask, int n_tiles, uint32_t* __restrict__ cnt,
                                                             uint32_t* __restrict__ dist, uint32_t* __restrict__ flo,
                                                             uint32_t* __restrict__ llo) {
    const int tile = tsort_tile(n_tiles);
    if (tile < 0) return;
    constexpr int kMapWords = (1 << (2 * kRadixBits)) / 32;
    static_assert(kTThreads == 2 * kRadix, "two threads per digit");
    __shared__ uint4 seen[kMapWords / 4];
    __shared__ uint32_t c[kRadix];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)tile * kTile + tid;
    // (positions past the batch load its last key, unused: no load waits on a branch)
    uint32_t k[kTPer];
#pragma unroll
    for (int j = 0; j < kTPer; ++j) k[j] = keys[base + j * kTThreads < n ? base + j * kTThreads : n - 1] & mkmask;
    for (int e = tid; e < kMapWords / 4; e += kTThreads) seen[e] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < kRadix) c[tid] = 0u;
    __syncthreads();
    uint32_t* sw = reinterpret_cast<uint32_t*>(seen);
#pragma unroll
    for (int j = 0; j < kTPer; ++j) {
        if (base + j * kTThreads < n) {
            atomicAdd(&c[(k[j] >> shift) & (kRadix - 1)], 1u);
            __hip_atomic_fetch_or(&sw[(k[j] >> 5) & (kMapWords - 1)], 1u << (k[j] & 31u), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    __syncthreads();
    // digit d = tid / 2; this thread's half of the digit's 512 bits: words 16 d + 8 h .. + 7
    const int d = tid >> 1, h = tid & 1;
    uint32_t pc = 0, lo_b = 0xffffffffu, hi_b = 0u;
    if (shift != 0) {
        const uint4 a = seen[4 * d + 2 * h], b = seen[4 * d + 2 * h + 1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 7; i >= 0; --i) {
            pc += __popc(w[i]);
            if (w[i]) lo_b = 256u * h + 32u * i + __builtin_ctz(w[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (w[i]) hi_b = 256u * h + 32u * i + 31u - __builtin_clz(w[i]);
    }
    const uint32_t pc_o = __shfl_xor(pc, 1, 64), lo_o = __shfl_xor(lo_b, 1, 64), hi_o = __shfl_xor(hi_b, 1, 64);
    if (h == 0) {
        const int64_t o = (int64_t)d * sort_tile_pitch(n_tiles) + tile;
        const uint32_t cc = c[d];
        cnt[o] = cc;
        if (shift != 0) {
            dist[o] = pc + pc_o;
            flo[o] = cc ? min(lo_b, lo_o) : 0u;
            llo[o] = cc ? (hi_o ? hi_o : hi_b) : 0u;
        } else {
            dist[o] = cc ? 1u : 0u;
            flo[o] = 0u;
            llo[o] = 0u;
        }
    }
}

// The same statistics for wider keys (three or more passes): the tile's keys are ranked by
// digit into LDS, where equal keys are adjacent.
__global__ __launch_bounds__(kTThreads) void tsort_stats(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                         uint32_t mkmask, int n_tiles, uint32_t* __restrict__ cnt,
                                                         uint32_t* __restrict__ dist, uint32_t* __restrict__ flo,
                                                         uint32_t* __restrict__ llo) {
    const int tile = tsort_tile(n_tiles);
    if (tile < 0) return;
    __shared__ uint32_t wcnt[kTW][kRadix];
    __shared__ uint32_t sk[kTile];
    __shared__ uint32_t lstart[kRadix], dcnt[kRadix], wsum[8];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t key[kTC], val[kTC], rank[kTC];
    tile_load<true>(keys, nullptr, n, tile, key, val);
    zero_wcnt(wcnt);
    if (tid < kRadix) dcnt[tid] = 0;
    __syncthreads();
    tile_rank(n, tile, shift, wcnt, key, rank);
    __syncthreads();
    const uint32_t tcv[1] = {tile_digit_counts(wcnt)};
    uint32_t ls[1], tile_n[1];
    scan512<1>(tcv, ls, tile_n, wsum);
    if (tid < kRadix) lstart[tid] = ls[0];
    __syncthreads();
    const int64_t base = (int64_t)tile * kTile + wave * (kTC * 64);
#pragma unroll
    for (int j = 0; j < kTC; ++j) {
        if (base + j * 64 + (tid & 63) < n) {
            const uint32_t d = (key[j] >> shift) & (kRadix - 1);
            const uint32_t lp = lstart[d] + wcnt[wave][d] + rank[j];
            if (lp < (uint32_t)kTile) sk[lp] = key[j] & mkmask;
        }
    }
    __syncthreads();
    for (int p = tid; p < (int)tile_n[0]; p += kTThreads) {
        const uint32_t k = sk[p];
        const uint32_t d = (k >> shift) & (kRadix - 1);
        if (p == (int)lstart[d] || k != sk[p - 1]) atomicAdd(&dcnt[d], 1u);
    }
    __syncthreads();
    if (tid < kRadix) {
        const int64_t o = (int64_t)tid * sort_tile_pitch(n_tiles) + tile;
        const uint32_t lomask = (1u << shift) - 1u, tc = tcv[0];
        cnt[o] = tc;
        dist[o] = dcnt[tid];
        flo[o] = tc ? sk[ls[0]] & lomask : 0u;
        llo[o] = tc ? sk[ls[0] + tc - 1] & lomask : 0u;
    }
}

// One workgroup per digit: exclusive prefix of the digit's tile counts over the tiles (in
// place), the total to tot[d].  Last pass (kLast): also the lower bits of the last key of
// the digit in earlier tiles, as llo + 1 (0: none; in place of llo), by a prefix maximum
// (the keys of one digit do not decrease over the tiles), and the exclusive prefix of the
// new distinct keys, dist - [the tile's first key equals that last key] (in place of dist),
// its total to stot[d].  Thread i takes 4 consecutive tiles per round of 1,024 (16-byte
// loads: rows start at multiples of 8 words), the waves' totals meet in LDS.
constexpr int kScanThreads = 256, kScanPer = 4, kScanRound = kScanThreads * kScanPer;

// Inclusive scan over the workgroup's threads in order of a sum and a maximum, returning
// the exclusive prefixes; *tot_c / *tot_m get the workgroup's totals.  Ends with a barrier,
// so sh can be used again at once.
__device__ __forceinline__ void scan_block_sum_max(uint32_t c, uint32_t m, uint32_t* sh, uint32_t* ex_c,
                                                   uint32_t* ex_m, uint32_t* tot_c, uint32_t* tot_m) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t ic = c, im = m;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t u = __shfl_up(ic, off, 64), w = __shfl_up(im, off, 64);
        if (lane >= off) {
            ic += u;
            im = max(im, w);
        }
    }
    if (lane == 63) {
        sh[wave] = ic;
        sh[4 + wave] = im;
    }
    __syncthreads();
    uint32_t pc = 0, pm = 0, tc = 0, tm = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
        const uint32_t a = sh[w], b = sh[4 + w];
        if (w < wave) {
            pc += a;
            pm = max(pm, b);
        }
        tc += a;
        tm = max(tm, b);
    }
    *ex_c = pc + ic - c;
    const uint32_t pmw = __shfl_up(im, 1, 64);
    *ex_m = max(pm, lane == 0 ? 0u : pmw);
    *tot_c = tc;
    *tot_m = tm;
    __syncthreads();
}

template <bool kLast>
__global__ __launch_bounds__(kScanThreads) void tsort_scan(uint32_t* __restrict__ cnt, uint32_t* __restrict__ dist,
                                                           const uint32_t* __restrict__ flo,
                                                           uint32_t* __restrict__ llo, int n_tiles,
                                                           uint32_t* __restrict__ tot, uint32_t* __restrict__ stot) {
    __shared__ uint32_t sh[8];
    const int d = blockIdx.x;
    const int64_t pitch = sort_tile_pitch(n_tiles);
    uint32_t* crow = cnt + (int64_t)d * pitch;
    uint32_t* drow = dist + (int64_t)d * pitch;
    const uint32_t* frow = flo + (int64_t)d * pitch;
    uint32_t* lrow = llo + (int64_t)d * pitch;
    uint32_t carry_c = 0, carry_s = 0, carry_l = 0;
    for (int t0 = 0; t0 < n_tiles; t0 += kScanRound) {
        const int tb = t0 + kScanPer * (int)threadIdx.x;
        // a row holds pitch >= n_tiles words, pitch % 8 == 0: the 16-byte load at tb < n_tiles
        // stays in the row; tiles from n_tiles on count as empty
        uint4 c4 = make_uint4(0u, 0u, 0u, 0u), d4 = c4, f4 = c4, l4 = c4;
        if (tb < n_tiles) {
            c4 = *reinterpret_cast<const uint4*>(crow + tb);
            if (kLast) {
                d4 = *reinterpret_cast<const uint4*>(drow + tb);
                f4 = *reinterpret_cast<const uint4*>(frow + tb);
                l4 = *reinterpret_cast<const uint4*>(lrow + tb);
            }
        }
        uint32_t c[kScanPer] = {c4.x, c4.y, c4.z, c4.w}, ds[kScanPer] = {d4.x, d4.y, d4.z, d4.w};
        const uint32_t fl[kScanPer] = {f4.x, f4.y, f4.z, f4.w}, lv[kScanPer] = {l4.x, l4.y, l4.z, l4.w};
        uint32_t sc = 0, ml = 0, le[kScanPer];
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) {
            if (tb + j >= n_tiles) c[j] = ds[j] = 0u;
            sc += c[j];
            le[j] = c[j] ? lv[j] + 1u : 0u;
            ml = max(ml, le[j]);
        }
        uint32_t ex_c, ex_l, tc, tl;
        scan_block_sum_max(sc, kLast ? ml : 0u, sh, &ex_c, &ex_l, &tc, &tl);
        uint32_t run_c = carry_c + ex_c, run_l = max(carry_l, ex_l);
        uint32_t oc[kScanPer], ol[kScanPer], nd[kScanPer], sn = 0;
#pragma unroll
        for (int j = 0; j < kScanPer; ++j) {
            oc[j] = run_c;
            run_c += c[j];
            nd[j] = ds[j] - (c[j] && run_l != 0u && fl[j] + 1u == run_l ? 1u : 0u);
            sn += nd[j];
            ol[j] = run_l;
            run_l = max(run_l, le[j]);
        }
        uint32_t os[kScanPer];
        if (kLast) {
            uint32_t ex_s, ts, unused_m, unused_t;
            scan_block_sum_max(sn, 0u, sh, &ex_s, &unused_m, &ts, &unused_t);
            uint32_t run_s = carry_s + ex_s;
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) {
                os[j] = run_s;
                run_s += nd[j];
            }
            carry_s += ts;
            carry_l = max(carry_l, tl);
        }
        carry_c += tc;
        if (tb + kScanPer <= n_tiles) {
            *reinterpret_cast<uint4*>(crow + tb) = make_uint4(oc[0], oc[1], oc[2], oc[3]);
            if (kLast) {
                *reinterpret_cast<uint4*>(drow + tb) = make_uint4(os[0], os[1], os[2], os[3]);
                *reinterpret_cast<uint4*>(lrow + tb) = make_uint4(ol[0], ol[1], ol[2], ol[3]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kScanPer; ++j) {
                if (tb + j < n_tiles) {
                    crow[tb + j] = oc[j];
                    if (kLast) {
                        drow[tb + j] = os[j];
                        lrow[tb + j] = ol[j];
                    }
                }
            }
        }
    }
    if (threadIdx.x == 0) {
        tot[d] = carry_c;
        if (kLast) stot[d] = carry_s;
    }
}

// Scatter of one non-last pass: key and value of each element to digit base + tile prefix
// + rank.
template <bool kFirst>
__global__ __launch_bounds__(kTThreads) void tsort_down(const uint32_t* __restrict__ keys_in,
                                                        const uint32_t* __restrict__ vals_in,
                                                        uint32_t* __restrict__ keys_out,
                                                        uint32_t* __restrict__ vals_out, int64_t n, int shift,
                                                        int n_tiles, const uint32_t* __restrict__ pre,
                                                        const uint32_t* __restrict__ tot) {
    __shared__ uint32_t wcnt[kTW][kRadix];
    __shared__ __align__(16) uint32_t sk[kTile];
    __shared__ __align__(16) uint32_t sv[kTile];
    __shared__ uint32_t gbase[kRadix], lstart[kRadix], wsum[2 * 8];
    const int tile = tsort_tile(n_tiles);
    if (tile < 0) return;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t my_pre = tid < kRadix ? pre[(int64_t)tid * sort_tile_pitch(n_tiles) + tile] : 0u;
    uint32_t tv[2] = {tid < kRadix ? tot[tid] : 0u, 0u};
    uint32_t key[kTC], val[kTC], rank[kTC];
    tile_load<kFirst>(keys_in, vals_in, n, tile, key, val);
    zero_wcnt(wcnt);
    __syncthreads();
    tile_rank(n, tile, shift, wcnt, key, rank);
    __syncthreads();
    tv[1] = tile_digit_counts(wcnt);
    uint32_t ex[2], sums[2];
    scan512<2>(tv, ex, sums, wsum);
    const uint32_t tile_n = sums[1];
    if (tid < kRadix) {
        gbase[tid] = ex[0] + my_pre;
        lstart[tid] = ex[1];
    }
    __syncthreads();
    // the tile ranked by digit into LDS, then written with consecutive positions of a
    // digit's group on consecutive lanes
    const int64_t base = (int64_t)tile * kTile + wave * (kTC * 64);
#pragma unroll
    for (int j = 0; j < kTC; ++j) {
        if (base + j * 64 + (tid & 63) < n) {
            const uint32_t d = (key[j] >> shift) & (kRadix - 1);
            const uint32_t lp = lstart[d] + wcnt[wave][d] + rank[j];
            if (lp < (uint32_t)kTile) {
                sk[lp] = key[j];
                sv[lp] = val[j];
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTPer; ++j) {
        const int p = tid + j * kTThreads;
        if (p >= (int)tile_n) break;
        const uint32_t k = sk[p];
        const uint32_t d = (k >> shift) & (kRadix - 1);
        const uint32_t pos = gbase[d] + (uint32_t)p - lstart[d];
        if (pos < (uint64_t)n) {  // always, for ids from one consistent pass
            keys_out[pos] = k;
            vals_out[pos] = sv[p];
        }
    }
}

// The last pass with the segmentation: the tile's keys and values ranked by digit into LDS,
// then each thread takes kTPer consecutive positions of that order: head flags, their
// prefix over the tile (one scan), slots, and every output.
template <bool kFirst>
__global__ __launch_bounds__(kTThreads) void tsort_down_last(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n, int shift,
    uint32_t mkmask, int n_tiles, const uint32_t* __restrict__ pre, const uint32_t* __restrict__ spre,
    const uint32_t* __restrict__ plast, const uint32_t* __restrict__ tot, const uint32_t* __restrict__ stot,
    int32_t* __restrict__ perm, int32_t* __restrict__ uniq, int32_t* __restrict__ seg_off,
    int32_t* __restrict__ pair_slot, int32_t* __restrict__ sorted_slot, int32_t* __restrict__ n_unique,
    int32_t max_unique, int32_t* __restrict__ slot_table) {
    // wcnt while the tile is ranked; afterwards the same LDS holds sslot, the slot + 1 of each
    // position (bit 31: a head), so that two workgroups fit a CU
    __shared__ __align__(16) uint32_t wcnt_sslot[kTW * kRadix];
    static_assert(kTile <= kTW * kRadix, "sslot aliases wcnt");
    uint32_t (*wcnt)[kRadix] = reinterpret_cast<uint32_t (*)[kRadix]>(wcnt_sslot);
    uint32_t* sslot = wcnt_sslot;
    __shared__ __align__(16) uint32_t sk[kTile];
    __shared__ __align__(16) uint32_t sv[kTile];
    __shared__ uint32_t gbase[kRadix], sbase[kRadix], lst[kRadix], lstart[kRadix], hstart[kRadix];
    __shared__ uint32_t wsum[3 * 8];
    const int tile = tsort_tile(n_tiles);
    if (tile < 0) return;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int64_t o = (int64_t)tid * sort_tile_pitch(n_tiles) + tile;
    const bool dl = tid < kRadix;
    const uint32_t my_pre = dl ? pre[o] : 0u, my_spre = dl ? spre[o] : 0u, my_plast = dl ? plast[o] : 0u;
    uint32_t tv[3] = {dl ? tot[tid] : 0u, dl ? stot[tid] : 0u, 0u};
    uint32_t key[kTC], val[kTC], rank[kTC];
    tile_load<kFirst>(keys_in, vals_in, n, tile, key, val);
    zero_wcnt(wcnt);
    __syncthreads();
    tile_rank(n, tile, shift, wcnt, key, rank);
    __syncthreads();
    tv[2] = tile_digit_counts(wcnt);
    uint32_t ex[3], sums[3];
    scan512<3>(tv, ex, sums, wsum);
    const uint32_t u_all = sums[1], tile_n = sums[2];
    if (dl) {
        gbase[tid] = ex[0] + my_pre;
        sbase[tid] = ex[1] + my_spre;
        lst[tid] = my_plast;
        lstart[tid] = ex[2];
    }
    __syncthreads();
    const int64_t base = (int64_t)tile * kTile + wave * (kTC * 64);
#pragma unroll
    for (int j = 0; j < kTC; ++j) {
        if (base + j * 64 + lane < n) {
            const uint32_t d = (key[j] >> shift) & (kRadix - 1);
            const uint32_t lp = lstart[d] + wcnt[wave][d] + rank[j];
            if (lp < (uint32_t)kTile) {
                sk[lp] = key[j];
                sv[lp] = val[j];
            }
        }
    }
    __syncthreads();
    // heads: a key differs from the one before it in its digit's group; a group's first key
    // continues the last earlier key of its digit when their lower bits agree (lst holds
    // those bits + 1, 0 for none)
    const uint32_t lomask = (1u << shift) - 1u;
    const int p0 = tid * kTPer;
    const uint4 k4 = reinterpret_cast<const uint4*>(sk)[tid];
    const uint32_t kk[kTPer] = {k4.x, k4.y, k4.z, k4.w};
    uint32_t prev = p0 > 0 ? sk[p0 - 1] : 0u;
    uint32_t dd[kTPer];
    bool st[kTPer], head[kTPer];
    uint32_t nh = 0;
#pragma unroll
    for (int i = 0; i < kTPer; ++i) {
        const int p = p0 + i;
        const bool valid = p < (int)tile_n;
        dd[i] = (kk[i] >> shift) & (kRadix - 1);
        st[i] = valid && p == (int)lstart[dd[i]];
        head[i] = valid && (st[i] ? (lst[dd[i]] == 0u || (kk[i] & lomask) + 1u != lst[dd[i]])
                                  : ((kk[i] ^ prev) & mkmask) != 0u);
        prev = kk[i];
        nh += head[i] ? 1u : 0u;
    }
    uint32_t all_heads;
    uint32_t run = scan1024(nh, wsum, all_heads);
    (void)all_heads;
#pragma unroll
    for (int i = 0; i < kTPer; ++i) {
        if (st[i]) hstart[dd[i]] = run;
        run += head[i] ? 1u : 0u;
    }
    __syncthreads();
    // each position's slot (and head flag) into LDS, then the outputs with position
    // p = tid + 1024 j per thread, so that consecutive lanes write consecutive positions of a
    // digit's group
    run -= nh;
#pragma unroll
    for (int i = 0; i < kTPer; ++i) {
        const int p = p0 + i;
        if (p >= (int)tile_n) break;
        const uint32_t d = dd[i];
        run += head[i] ? 1u : 0u;
        const int32_t slot = (int32_t)(sbase[d] + run - hstart[d]) - 1;
        sslot[p] = (uint32_t)(slot + 1) | (head[i] ? 0x80000000u : 0u);  // slot + 1 < 2^31
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTPer; ++j) {
        const int p = tid + j * kTThreads;
        if (p >= (int)tile_n) break;
        const uint32_t key = sk[p], val = sv[p], sw = sslot[p];
        const uint32_t d = (key >> shift) & (kRadix - 1);
        const int32_t slot = (int32_t)(sw & 0x7fffffffu) - 1;
        // ids outside [0, n_experts) (a caller error) could make more slots than the buffers
        // hold: clamp so that every later kernel stays in bounds
        const int32_t sc = slot < 0 ? 0 : (slot < max_unique ? slot : max_unique - 1);
        const uint32_t pos = gbase[d] + (uint32_t)p - lstart[d];
        if (pos < (uint64_t)n) {
            perm[pos] = (int32_t)val;
            sorted_slot[pos] = sc;
        }
        if (slot_table) {
            if (sw >> 31) slot_table[key & mkmask] = sc;
        } else if (val < (uint64_t)n) {
            pair_slot[val] = sc;
        }
        if ((sw >> 31) && slot >= 0 && slot < max_unique) {
            uniq[slot] = (int32_t)key;
            seg_off[slot] = (int32_t)pos;
        }
    }
    if (tile == 0 && tid == 0) {
        // unsigned comparison: the count is at most n, and the clamp keeps u in [0, max_unique]
        const int32_t u = u_all < (uint32_t)max_unique ? (int32_t)u_all : max_unique;
        *n_unique = u;
        seg_off[u] = (int32_t)n;
    }
}

// pair_slot[p] = slot_table[ids[p] & mkmask]: the slot of pair p's expert, from the table
// the last pass wrote at the heads (the same clamped slot it gives the pair's sorted
// position).  Four pairs per thread, 1024 per workgroup, coalesced.
constexpr int kPsThreads = 256, kPsPer = 4;
__global__ __launch_bounds__(kPsThreads) void tsort_pair_slot(const uint32_t* __restrict__ ids, int64_t n,
                                                              uint32_t mkmask,
                                                              const int32_t* __restrict__ slot_table,
                                                              int32_t* __restrict__ pair_slot) {
    const int64_t base = (int64_t)blockIdx.x * (kPsThreads * kPsPer) + threadIdx.x;
    // every id, then every table entry, loaded before any store (positions past the batch
    // repeat its last pair, not stored): no load waits on a branch or on another's use
    uint32_t k[kPsPer];
    int32_t v[kPsPer];
#pragma unroll
    for (int j = 0; j < kPsPer; ++j) k[j] = ids[base + j * kPsThreads < n ? base + j * kPsThreads : n - 1] & mkmask;
#pragma unroll
    for (int j = 0; j < kPsPer; ++j) v[j] = slot_table[k[j]];
#pragma unroll
    for (int j = 0; j < kPsPer; ++j)
        if (base + j * kPsThreads < n) pair_slot[base + j * kPsThreads] = v[j];
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

// LDS of the small sort: the words twice, per-wave digit counts (then bases, < 2^14), head
// flags per chunk, heads before each chunk, wave sums.
constexpr size_t kSmallBufB = 2 * (size_t)kSmallMax * 4, kSmallCntB = (size_t)kSmallWaves * kRadix * 2;
constexpr size_t kSmallLds = kSmallBufB + kSmallCntB + (size_t)kSmallChunks * 8 + (size_t)kSmallChunks * 4 +
                             (size_t)kSmallWaves * 4;

__device__ __forceinline__ void sort_small_body(unsigned char* lds, const int32_t* __restrict__ ids, int n,
                                                int key_bits_, int vb, int passes, int32_t* __restrict__ perm,
                                                int32_t* __restrict__ uniq, int32_t* __restrict__ seg_off,
                                                int32_t* __restrict__ pair_slot, int32_t* __restrict__ sorted_slot,
                                                int32_t* __restrict__ n_unique, int32_t max_unique) {
    uint32_t (*buf)[kSmallMax] = reinterpret_cast<uint32_t (*)[kSmallMax]>(lds);
    uint16_t (*cnt)[kRadix] = reinterpret_cast<uint16_t (*)[kRadix]>(lds + kSmallBufB);
    uint64_t* cmask = reinterpret_cast<uint64_t*>(lds + kSmallBufB + kSmallCntB);
    uint32_t* cbase = reinterpret_cast<uint32_t*>(lds + kSmallBufB + kSmallCntB + kSmallChunks * 8);
    uint32_t* wsum = reinterpret_cast<uint32_t*>(lds + kSmallBufB + kSmallCntB + kSmallChunks * 12);
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
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
            if (j >= cpw) break;  // wave-uniform: the wave's chunks end here
            const int idx = (c0 + j) * 64 + lane;
            const bool v = idx < n;
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
            if (j >= cpw) break;
            const int idx = (c0 + j) * 64 + lane;
            if (idx < n) buf[cur ^ 1][cnt[wave][(word[j] >> shift) & (kRadix - 1)] + rank[j]] = word[j];
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
    const uint32_t u_all = wsum[0];
    const int32_t u_clamped = u_all < (uint32_t)max_unique ? (int32_t)u_all : max_unique;
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

__global__ __launch_bounds__(kSmallWaves * 64) void sort_small_kernel(const int32_t* __restrict__ ids, int n,
                                                                      int key_bits_, int vb, int passes,
                                                                      int32_t* __restrict__ perm,
                                                                      int32_t* __restrict__ uniq,
                                                                      int32_t* __restrict__ seg_off,
                                                                      int32_t* __restrict__ pair_slot,
                                                                      int32_t* __restrict__ sorted_slot,
                                                                      int32_t* __restrict__ n_unique,
                                                                      int32_t max_unique) {
    __shared__ __align__(16) unsigned char lds[kSmallLds];
    sort_small_body(lds, ids, n, key_bits_, vb, passes, perm, uniq, seg_off, pair_slot, sorted_slot, n_unique,
                    max_unique);
}

// The small sort in workgroup 0 and the bf16 token projection xp = RN(x W_u) in the
// others (tile b - 1: column tile (b - 1) % nct, token tile (b - 1) / nct), which needs
// only x: the tiles run on CUs the single sorting workgroup leaves idle.
static_assert(kSmallLds >= (size_t)kTpLds, "the projection tile's ring fits the sort's LDS");
__global__ __launch_bounds__(kSmallWaves * 64) void sort_small_tp_kernel(
    const int32_t* __restrict__ ids, int n, int key_bits_, int vb, int passes, int32_t* __restrict__ perm,
    int32_t* __restrict__ uniq, int32_t* __restrict__ seg_off, int32_t* __restrict__ pair_slot,
    int32_t* __restrict__ sorted_slot, int32_t* __restrict__ n_unique, int32_t max_unique,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wut, int n_tok, int d, int dh, int nct,
    uint16_t* __restrict__ xp) {
    __shared__ __align__(16) unsigned char lds[kSmallLds];
    if (blockIdx.x == 0) {
        sort_small_body(lds, ids, n, key_bits_, vb, passes, perm, uniq, seg_off, pair_slot, sorted_slot, n_unique,
                        max_unique);
    } else {
        const int b = (int)blockIdx.x - 1;
        token_proj_bf16_tile(lds, x, wut, n_tok, d, dh, xp, (b % nct) * kTpCols, (b / nct) * kTpRows);
    }
}

int launch_sort_segment_tp(const int32_t* ids, int64_t n, int64_t n_experts, int32_t* perm, int32_t* uniq,
                           int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique,
                           const void* x, const void* wut, int64_t n_tok, int d, int dh, void* xp,
                           hipStream_t stream) {
    const int bits = sort_key_bits(n_experts);
    const int passes = sort_passes(n_experts);
    int vb = 0;
    while (vb < 31 && ((int64_t)1 << vb) < n) ++vb;
    const int32_t max_unique = (int32_t)(n < n_experts ? n : n_experts);
    if (!(n <= kSmallMax && bits + vb <= 32) || wut == nullptr || d % kTpK || dh % 8 || n_tok < 1 ||
        n_tok > INT32_MAX)
        return -1;  // not the single-workgroup sort, or not the MFMA projection: two launches
    const int nct = (dh + kTpCols - 1) / kTpCols;
    const int64_t tiles = (int64_t)nct * ((n_tok + kTpRows - 1) / kTpRows);
    hipLaunchKernelGGL(sort_small_tp_kernel, dim3((unsigned)(1 + tiles)), dim3(kSmallWaves * 64), 0, stream, ids,
                       (int)n, bits, vb, passes, perm, uniq, seg_off, pair_slot, sorted_slot, n_unique, max_unique,
                       (const uint16_t*)x, (const uint16_t*)wut, (int)n_tok, d, dh, nct, (uint16_t*)xp);
    return (int)hipGetLastError();
}

size_t sort_workspace_bytes(int64_t n, int64_t n_experts) {
    return sort_workspace_words(n, n_experts) * sizeof(uint32_t);
}

int launch_sort_segment(const int32_t* ids, int64_t n, int64_t n_experts, void* ws, int32_t* perm, int32_t* uniq,
                        int32_t* seg_off, int32_t* pair_slot, int32_t* sorted_slot, int32_t* n_unique,
                        hipStream_t stream) {
    const int bits = sort_key_bits(n_experts);
    const int passes = sort_passes(n_experts);
    int vb = 0;
    while (vb < 31 && ((int64_t)1 << vb) < n) ++vb;
    const int32_t max_unique = (int32_t)(n < n_experts ? n : n_experts);
    if (n <= kSmallMax && bits + vb <= 32) {
        hipLaunchKernelGGL(sort_small_kernel, dim3(1), dim3(kSmallWaves * 64), 0, stream, ids, (int)n, bits, vb,
                           passes, perm, uniq, seg_off, pair_slot, sorted_slot, n_unique, max_unique);
        return (int)hipGetLastError();
    }
    const int n_tiles = (int)((n + kTile - 1) / kTile);
    uint32_t* w = reinterpret_cast<uint32_t*>(ws);
    uint32_t* kbuf[2] = {w, w + n};
    uint32_t* vbuf[2] = {w + 2 * n, w + 3 * n};
    const size_t pitch = (size_t)sort_tile_pitch(n_tiles);
    uint32_t* cnt = w + 4 * n;
    uint32_t* dist = cnt + (size_t)kRadix * pitch;
    uint32_t* flo = dist + (size_t)kRadix * pitch;
    uint32_t* llo = flo + (size_t)kRadix * pitch;
    uint32_t* tot = llo + (size_t)kRadix * pitch;
    uint32_t* stot = tot + kRadix;
    // the expert -> slot table (large batches, ids of at most 18 bits), after the totals and
    // their padding
    int32_t* table = sort_table_words(n, n_experts) ? reinterpret_cast<int32_t*>(stot + kRadix + 64) : nullptr;
    // keys compare on the bits the passes sort (those of ids below n_experts)
    const uint32_t mkmask = kRadixBits * passes >= 32 ? 0xffffffffu : (1u << (kRadixBits * passes)) - 1u;
    const dim3 tg(tsort_grid(n_tiles)), tb(kTThreads), sg((unsigned)kRadix), sb(kScanThreads);
    for (int p = 0; p < passes; ++p) {
        const uint32_t* kin = p == 0 ? reinterpret_cast<const uint32_t*>(ids) : kbuf[(p - 1) & 1];
        const uint32_t* vin = p == 0 ? nullptr : vbuf[(p - 1) & 1];
        const int shift = kRadixBits * p;
        if (p < passes - 1) {
            hipLaunchKernelGGL(tsort_count, tg, tb, 0, stream, kin, n, shift, n_tiles, cnt);
            hipLaunchKernelGGL(tsort_scan<false>, sg, sb, 0, stream, cnt, dist, flo, llo, n_tiles, tot, stot);
            if (p == 0)
                hipLaunchKernelGGL(tsort_down<true>, tg, tb, 0, stream, kin, vin, kbuf[p & 1], vbuf[p & 1], n, shift,
                                   n_tiles, (const uint32_t*)cnt, (const uint32_t*)tot);
            else
                hipLaunchKernelGGL(tsort_down<false>, tg, tb, 0, stream, kin, vin, kbuf[p & 1], vbuf[p & 1], n, shift,
                                   n_tiles, (const uint32_t*)cnt, (const uint32_t*)tot);
        } else {
            if (passes <= 2)
                hipLaunchKernelGGL(tsort_stats_map, tg, tb, 0, stream, kin, n, shift, mkmask, n_tiles, cnt, dist, flo,
                                   llo);
            else
                hipLaunchKernelGGL(tsort_stats, tg, tb, 0, stream, kin, n, shift, mkmask, n_tiles, cnt, dist, flo,
                                   llo);
            hipLaunchKernelGGL(tsort_scan<true>, sg, sb, 0, stream, cnt, dist, flo, llo, n_tiles, tot, stot);
            if (p == 0)
                hipLaunchKernelGGL(tsort_down_last<true>, tg, tb, 0, stream, kin, vin, n, shift, mkmask, n_tiles,
                                   (const uint32_t*)cnt, (const uint32_t*)dist, (const uint32_t*)llo,
                                   (const uint32_t*)tot, (const uint32_t*)stot, perm, uniq, seg_off, pair_slot,
                                   sorted_slot, n_unique, max_unique, table);
            else
                hipLaunchKernelGGL(tsort_down_last<false>, tg, tb, 0, stream, kin, vin, n, shift, mkmask, n_tiles,
                                   (const uint32_t*)cnt, (const uint32_t*)dist, (const uint32_t*)llo,
                                   (const uint32_t*)tot, (const uint32_t*)stot, perm, uniq, seg_off, pair_slot,
                                   sorted_slot, n_unique, max_unique, table);
            if (table)
                hipLaunchKernelGGL(tsort_pair_slot, dim3((unsigned)((n + kPsThreads * kPsPer - 1) / (kPsThreads * kPsPer))),
                                   dim3(kPsThreads), 0, stream, reinterpret_cast<const uint32_t*>(ids), n, mkmask,
                                   (const int32_t*)table, pair_slot);
        }
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return (int)err;
    }
    return 0;
}

}  // namespace ethos
