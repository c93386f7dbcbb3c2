// Product-key routing: sub-key scoring, canonical top-(k_cand) per query half,
// k_cand x k_cand combination, canonical top-k, fp32 softmax gates, expert-id decode.
// (reference: model.py:217-245 per head; heads stacked as rows = token * H + head,
// model.py:250-252).
//
// Numeric contract (identical to the CPU oracle's, written independently):
//   s[j]   = RN_T(fp64 FMA chain over the half-query and sub-key j, index order)
//            (for bf16 operands: the correctly rounded dot product)
//   order  = (score descending, index ascending), -0 == +0; the index is the sub-key
//            index for the per-half lists and the expert id e = i1*K + i2 for the
//            combined list -- "ties broken to the lowest index".
//   c[a,b] = RN_T(fp32(v1[a] + v2[b]))
//   gate_i = RN_T(ex_i / sum_i ex_i), ex_i = RN_f32(exp(c_i - c_0)) with exp evaluated in
//            fp64 (the correctly rounded fp32 exponential whenever the fp64 result is not
//            within its own error of an fp32 rounding boundary), fp32 sum in list order.
//
// Certified filter, exact refinement.  Computing all K sub-key scores exactly is
// the expensive way; instead:
//   1. MFMA (fp32 accumulation) gives approximate scores s~ for a 32-row x K tile.
//      Whatever the accumulation order, |s~ - s| <= e_j = gamma * ||q|| * ||k_j||
//      with gamma = (dh2 + 16) * 2^-22 (every partial sum rounded at worst like a
//      truncating fp32 add), by Cauchy-Schwarz on sum |q_i k_ij|.
//   2. tau_s = the k_cand-th largest of the 64 per-lane maxima of s~ is at most the
//      k_cand-th largest s~, so at least k_cand keys have s >= tau_s - max_j e_j =: tau.
//      A key whose exact score rounds below RN_T(tau) rounds strictly below k_cand
//      other keys and cannot be selected; a key is dropped when even s~ plus its
//      margin lies below the interval that rounds to RN_T(tau).
//   3. The survivors (about 40 of 512) whose interval [s~ - e, s~ + e] rounds to one T
//      value have it as their exact score; the others are scored exactly (the fp64
//      chain), one per lane.  The survivors are ranked with 64-lane bitonic sort /
//      merge networks on canonical keys.
// The output therefore equals exhaustive exact scoring bit for bit.
#pragma clang fp contract(off)

#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_mfma.hpp"

namespace ethos {

constexpr int kRtWaves = 8;                            // two workgroups per CU: four waves per SIMD
constexpr int kRtRows = 32;                            // rows of the MFMA tile (and LDS row slots)
// rows per wave: 4 (32 rows per workgroup) for large batches; 1 (8 rows per workgroup,
// the MFMA tile's other rows zero) for small ones, which spreads them over 4x as many
// workgroups and cuts each wave's sequential work by 4
constexpr int kRtSmallRows = 4096;                     // batches up to this many rows take 1 row per wave
constexpr int kRtMaxKc = 32;                           // k_cand <= 32, top_k <= 32
static_assert(kRtMaxKc <= kWave, "candidate lists hold one entry per lane");
constexpr int kRtMaxK = 512;                           // sub-keys per table
constexpr int kRtSlots = kRtMaxK / kWave;              // approximate scores per lane per row
constexpr int kRtStSlots = 2;                          // staircase pairs per lane (<= 119 for top_k <= 32)
constexpr int kRtMaxDh2 = 256;

// ---------------------------------------------------------------- wave networks
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    const int lo = __shfl((int)(uint32_t)v, src, kWave);
    const int hi = __shfl((int)(uint32_t)(v >> 32), src, kWave);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// v of lane (lane ^ mask), mask a compile-time constant after inlining, with VALU lane
// exchanges only (no LDS round trip): DPP quad permutes for 1 and 2, a half-row mirror
// (lane ^ 7) or row mirror (lane ^ 15) composed with a second DPP move for 4 and 8,
// v_permlane16_swap for 16 and v_permlane32_swap for 32.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {  // every lane reads: no "old" operand
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kCtrl, 0xf, 0xf, true);
}
constexpr int kDppXor3 = 0x1b;  // quad_perm [3,2,1,0]

__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v, int mask) {
    uint32_t r = v;
    if (mask & 32) {
        const auto sw = __builtin_amdgcn_permlane32_swap(r, r, false, false);
        r = (__lane_id() & 32) ? sw[0] : sw[1];
    }
    if (mask & 16) {
        const auto sw = __builtin_amdgcn_permlane16_swap(r, r, false, false);
        r = (__lane_id() & 16) ? sw[0] : sw[1];
    }
    switch (mask & 15) {
        case 0: break;
        case 1: r = dpp_mov<kDppXor1>(r); break;
        case 2: r = dpp_mov<kDppXor2>(r); break;
        case 4: r = dpp_mov<kDppXor3>(dpp_mov<kDppRowHalfMirror>(r)); break;  // (l ^ 7) ^ 3
        case 8: r = dpp_mov<kDppRowHalfMirror>(dpp_mov<kDppRowMirror>(r)); break;  // (l ^ 15) ^ 7
        case 15: r = dpp_mov<kDppRowMirror>(r); break;
        default: r = (uint32_t)__shfl_xor((int)r, mask & 15, kWave); break;
    }
    return r;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const uint32_t lo = xor_lane_u32((uint32_t)v, mask);
    const uint32_t hi = xor_lane_u32((uint32_t)(v >> 32), mask);
    return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort of one value per lane, descending in lane order.
template <typename V>
__device__ __forceinline__ V shfl_xor_v(V v, int mask);
template <>
__device__ __forceinline__ uint64_t shfl_xor_v<uint64_t>(uint64_t v, int mask) { return shfl_xor_u64(v, mask); }
template <>
__device__ __forceinline__ uint32_t shfl_xor_v<uint32_t>(uint32_t v, int mask) {
    return xor_lane_u32(v, mask);
}

// Lanes of a bitonic stage (partner distance j, block size k) that keep the larger of
// their own and their partner's value: (lane & j) == 0 exactly when (lane & k) == 0.  A
// compile-time constant after unrolling.
__host__ __device__ constexpr uint64_t bitonic_keep_max(int j, int k) {
    uint64_t m = 0;
    for (int l = 0; l < 64; ++l)
        if (((l & j) == 0) == ((l & k) == 0)) m |= 1ull << l;
    return m;
}

// Per-lane select by a wave-uniform lane mask: lane l gets t if bit l of m is set, else f.
__device__ __forceinline__ uint32_t select_by_mask(uint32_t f, uint32_t t, uint64_t m) {
    uint32_t r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(f), "v"(t), "s"(m));
    return r;
}
__device__ __forceinline__ uint64_t select_by_mask(uint64_t f, uint64_t t, uint64_t m) {
    const uint32_t lo = select_by_mask((uint32_t)f, (uint32_t)t, m);
    const uint32_t hi = select_by_mask((uint32_t)(f >> 32), (uint32_t)(t >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

// One compare-exchange stage: every lane takes its partner's value p when p is larger
// and the lane keeps the maximum, or when p is not larger and it keeps the minimum;
// the comparison mask and the constant keep mask combine in scalar registers.
// For partner distance 16 or 32 one v_permlane{16,32}_swap of v with itself leaves every
// lane holding its own and its partner's value, in an order that differs between lanes;
// keeping the larger or smaller of the two is symmetric, so the order does not matter.
template <int kJ>
__device__ __forceinline__ void swap_pair(uint32_t v, uint32_t& a, uint32_t& b) {
    if constexpr (kJ == 16) {
        const auto sw = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = sw[0];
        b = sw[1];
    } else {
        const auto sw = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = sw[0];
        b = sw[1];
    }
}
template <int kJ>
__device__ __forceinline__ void swap_pair(uint64_t v, uint64_t& a, uint64_t& b) {
    uint32_t al, bl, ah, bh;
    swap_pair<kJ>((uint32_t)v, al, bl);
    swap_pair<kJ>((uint32_t)(v >> 32), ah, bh);
    a = ((uint64_t)ah << 32) | al;
    b = ((uint64_t)bh << 32) | bl;
}

template <typename V>
__device__ __forceinline__ V bitonic_stage(V v, int j, uint64_t keep_max) {
    if (j == 16 || j == 32) {
        V a, b;
        if (j == 16) swap_pair<16>(v, a, b);
        else swap_pair<32>(v, a, b);
        return select_by_mask(b, a, ~(ballot(a > b) ^ keep_max));
    }
    const V p = shfl_xor_v<V>(v, j);
    return select_by_mask(v, p, ~(ballot(p > v) ^ keep_max));
}

template <typename V>
__device__ __forceinline__ V wave_sort_desc(V v, int lane) {
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) v = bitonic_stage<V>(v, j, bitonic_keep_max(j, k));
    }
    return v;
}

// run and chunk are each sorted descending across the lanes; returns the 64 largest
// of their union, sorted descending.
__device__ __forceinline__ uint64_t wave_merge_desc(uint64_t run, uint64_t chunk, int lane) {
    const uint64_t rev = shfl_xor_u64(chunk, kWave - 1);  // chunk[63 - lane]
    uint64_t v = select_by_mask(rev, run, ballot(run > rev));  // bitonic top-64
#pragma unroll
    for (int j = kWave >> 1; j > 0; j >>= 1) v = bitonic_stage<uint64_t>(v, j, bitonic_keep_max(j, 2 * kWave));
    return v;
}

// 32-bit form of a canonical key whose score is a bf16 value and whose index is below
// 2^16: the upper 16 bits of ord32(score) (its lower 16 bits are all zero or all one
// for such a score), then 0xffff - index.  Same order as the 64-bit key; 0 <-> 0 (no
// key; a finite score never maps to 0).
__device__ __forceinline__ uint32_t key32_of(uint64_t k) {
    return k == 0ull ? 0u : ((uint32_t)(k >> 48) << 16) | (0xffffu - key_idx(k));
}
__device__ __forceinline__ uint64_t key64_of32(uint32_t k) {
    if (k == 0u) return 0ull;
    const uint32_t o16 = k >> 16;
    const uint32_t o32 = (o16 << 16) | ((o16 & 0x8000u) ? 0u : 0xffffu);
    return ((uint64_t)o32 << 32) | (uint64_t)(~(0xffffu - (k & 0xffffu)));
}

// A row's candidate list as held between the halves: for bf16 scores the 32-bit key form
// (half the registers), else the canonical key.
template <typename T> struct ListKey {
    using type = uint64_t;
    __device__ __forceinline__ static uint64_t pack(uint64_t k) { return k; }
    __device__ __forceinline__ static uint64_t unpack(uint64_t k) { return k; }
    // descending sort of one key per lane, in list form
    __device__ __forceinline__ static uint64_t sort(uint64_t k, int lane) { return wave_sort_desc<uint64_t>(k, lane); }
};
template <> struct ListKey<uint16_t> {
    using type = uint32_t;
    __device__ __forceinline__ static uint32_t pack(uint64_t k) { return key32_of(k); }
    __device__ __forceinline__ static uint64_t unpack(uint32_t k) { return key64_of32(k); }
    // keys of bf16 scores sort in their 32-bit form (half the lane exchanges)
    __device__ __forceinline__ static uint32_t sort(uint64_t k, int lane) {
        return wave_sort_desc<uint32_t>(key32_of(k), lane);
    }
};

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<kDppXor1>(v));
    v = max(v, dpp_u32<kDppXor2>(v));
    v = max(v, dpp_u32<kDppRowHalfMirror>(v));
    v = max(v, dpp_u32<kDppRowMirror>(v));
    const uint32_t a = max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16));
    const uint32_t b = max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48));
    return max(a, b);
}

// 16 bytes of a key row -> doubles, in order.
template <typename T> struct KeyVec;
template <> struct KeyVec<uint16_t> {
    static constexpr int kN = 8;
    __device__ __forceinline__ static void load(const uint16_t* p, double* d) {
        from_raw(*reinterpret_cast<const uint4*>(p), d);
    }
    __device__ __forceinline__ static void from_raw(const uint4 r, double* d) {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            d[2 * i] = (double)__uint_as_float(w[i] << 16);
            d[2 * i + 1] = (double)__uint_as_float(w[i] & 0xffff0000u);
        }
    }
};
template <> struct KeyVec<float> {
    static constexpr int kN = 4;
    __device__ __forceinline__ static void load(const float* p, double* d) {
        from_raw(*reinterpret_cast<const uint4*>(p), d);
    }
    __device__ __forceinline__ static void from_raw(const uint4 r, double* d) {
        d[0] = __uint_as_float(r.x);
        d[1] = __uint_as_float(r.y);
        d[2] = __uint_as_float(r.z);
        d[3] = __uint_as_float(r.w);
    }
};

// 16 bytes of a query row -> floats (bf16 and fp32 elements are exact in float).
template <typename T> struct QVecF;
template <> struct QVecF<uint16_t> {
    static constexpr int kN = 8;
    __device__ __forceinline__ static void load(const uint16_t* p, float* f) {
        const uint4 r = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};
template <> struct QVecF<float> {
    static constexpr int kN = 4;
    __device__ __forceinline__ static void load(const float* p, float* f) {
        const float4 r = *reinterpret_cast<const float4*>(p);
        f[0] = r.x;
        f[1] = r.y;
        f[2] = r.z;
        f[3] = r.w;
    }
};

struct RouteSmem {
    size_t s_off, kn_off, qs_off, xch_off, total;
    int qs_pitch;  // bytes per staged query-half row
};

// Row pitch of the score tile (floats).  Once a row's K approximate scores are in
// registers, its storage holds up to 64 8-byte candidate keys (bytes [0, 512)) and the
// row's list of candidates still to be scored exactly (bytes [512, 768)); 4 floats of
// padding spread the MFMA result stores over the banks.
constexpr int kRtPendOff = 2 * kWave;  // float offset of the pending list
__host__ __device__ inline int route_pitch(int K) {
    const int p = ((K + 31) / 32) * 32;
    return (p > 3 * kWave ? p : 3 * kWave) + 4;
}

// hp: the half-parallel form (two groups of kRtWaves waves, one per query half, kRtWaves rows):
// score rows for the workgroup's rows of both halves, both halves' staged query tiles, and the
// second half's candidate lists handed to the first group.
__host__ __device__ inline RouteSmem route_smem_layout(int K, int dh2, int elem_bytes, bool hp = false) {
    RouteSmem L;
    size_t off = 0;
    L.s_off = off;
    off += (size_t)(hp ? 2 * kRtWaves : kRtRows) * route_pitch(K) * sizeof(float);
    L.kn_off = off;
    off += (size_t)2 * ((K + 31) / 32) * 32 * sizeof(float);
    L.qs_off = off;
    // 16 bytes of padding put the query rows of one wave's lanes on different banks
    L.qs_pitch = dh2 * elem_bytes + 16;
    off += (size_t)(hp ? 2 : 1) * kRtRows * L.qs_pitch;
    L.xch_off = off;
    off += hp ? (size_t)kRtWaves * kWave * sizeof(uint64_t) : 0;
    L.total = off;
    return L;
}

// Exact score key of sub-key j: the fp64 FMA chain over the query half qh (staged in
// LDS) and key row j (global, L2-resident), index order, rounded once to T.
// The key row's 16-byte vectors are loaded kG at a time ahead of their FMAs, so that
// their L2 latencies overlap.
template <typename T, int kG>
__device__ __forceinline__ uint64_t exact_key(const T* qh, const T* __restrict__ keys, int dh2, int j) {
    constexpr int kN = KeyVec<T>::kN;
    const T* kr = keys + (int64_t)j * dh2;
    double acc = 0.0;
    int i0 = 0;
    for (; i0 + kG * kN <= dh2; i0 += kG * kN) {
        uint4 raw[kG];
#pragma unroll
        for (int g = 0; g < kG; ++g) raw[g] = *reinterpret_cast<const uint4*>(kr + i0 + g * kN);
#pragma unroll
        for (int g = 0; g < kG; ++g) {
            double qv[kN], kv[kN];
            KeyVec<T>::load(qh + i0 + g * kN, qv);
            KeyVec<T>::from_raw(raw[g], kv);
#pragma unroll
            for (int t = 0; t < kN; ++t) acc = fma(qv[t], kv[t], acc);
        }
    }
    for (int i = i0; i < dh2; i += kN) {
        double qv[KeyVec<T>::kN], kv[KeyVec<T>::kN];
        KeyVec<T>::load(qh + i, qv);
        KeyVec<T>::load(kr + i, kv);
#pragma unroll
        for (int t = 0; t < KeyVec<T>::kN; ++t) acc = fma(qv[t], kv[t], acc);
    }
    return make_key(Elem<T>::round64(acc), (uint32_t)j);
}

// kHP (small batches): 2 kRtWaves waves, one row per wave and group of kRtWaves waves per
// query half, so that the two halves' scoring, filter, exact chains and sorts run at the same
// time; the second group hands its candidate lists to the first, which combines.  The
// operations on each row are the same as in the one-group form, so the outputs are too.
template <typename T, int RPW, bool kHP = false, bool kPrep = false>
__global__ __launch_bounds__((kHP ? 2 : 1) * kRtWaves * 64, 4) void route_kernel(const T* __restrict__ q, const T* __restrict__ keys1,
                                                    const T* __restrict__ keys2, const float* __restrict__ key_norms,
                                                    int64_t rows, int dq, int K, int top_k, int kc,
                                                    T* __restrict__ out_gates, int32_t* __restrict__ out_ids,
                                                    const T* __restrict__ kfrag) {
    using M = Mfma<T>;
    extern __shared__ __align__(16) unsigned char smem[];
    const int dh2 = dq / 2;
    static_assert(!kHP || RPW == 1, "the half-parallel form takes one row per wave");
    constexpr int kThreads = (kHP ? 2 : 1) * kRtWaves * 64;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    // hw: this wave's query half (kHP; else both, in turn); wv: its index within its group
    const int hw = kHP ? wave / kRtWaves : 0, wv = kHP ? wave % kRtWaves : wave;
    const int gtid = kHP ? tid % (kRtWaves * 64) : tid;
    const int lrow = lane & 31, lk = (lane >> 5) * M::kKL;
    const RouteSmem L = route_smem_layout(K, dh2, (int)sizeof(T), kHP);
    const int pitch = route_pitch(K);
    const int kpad = ((K + 31) / 32) * 32;
    constexpr int kRowsWG = kRtWaves * RPW;  // rows of this workgroup (<= kRtRows)
    // this group's score rows and staged query tile
    float* S = reinterpret_cast<float*>(smem + L.s_off) + (kHP ? (size_t)hw * kRowsWG * pitch : 0);
    unsigned char* const qsb = smem + L.qs_off + (kHP ? (size_t)hw * kRtRows * L.qs_pitch : 0);
    float* kn = reinterpret_cast<float*>(smem + L.kn_off);
    // lst[rr][half]: the canonical top-k_cand list of this wave's row rr and query half,
    // entry i held by lane i
    // key vectors in flight per exact chain (one row per wave leaves registers for more)
    constexpr int kExG = RPW == 1 ? 8 : 4;
    using LK = ListKey<T>;
    typename LK::type lst[RPW][2];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) lst[rr][0] = lst[rr][1] = 0;

    const int64_t row0 = (int64_t)blockIdx.x * kRowsWG;
    const int nkb = kpad / 32;
    const float gamma = (float)(dh2 + 16) * 0x1p-22f * 1.01f;

    // Sub-key norms (upper bounds) for both tables: given ones all requested before any is
    // stored (positions past the tables read entry 0, unused)
    if (key_norms != nullptr) {
        constexpr int kKnIt = (2 * kRtMaxK + kThreads - 1) / kThreads;
        float kv[kKnIt];
#pragma unroll
        for (int it = 0; it < kKnIt; ++it) {
            const int e = tid + it * kThreads, half = e / kpad, j = e - half * kpad;
            kv[it] = key_norms[e < 2 * kpad && j < K ? half * K + j : 0];
        }
#pragma unroll
        for (int it = 0; it < kKnIt; ++it) {
            const int e = tid + it * kThreads, half = e / kpad, j = e - half * kpad;
            if (e < 2 * kpad) kn[e] = j < K ? kv[it] : 0.0f;
        }
    } else {
        for (int e = tid; e < 2 * kpad; e += kThreads) {
            const int half = e / kpad, j = e - half * kpad;
            float nrm = 0.0f;
            if (j < K) {
                const T* kr = (half ? keys2 : keys1) + (int64_t)j * dh2;
                double s2 = 0.0;
                for (int i = 0; i < dh2; ++i) {
                    const double v = Elem<T>::to_f64(kr[i]);
                    s2 = fma(v, v, s2);
                }
                nrm = (float)(sqrt(s2) * (1.0 + 0x1p-20));
            }
            kn[e] = nrm;
        }
    }

    const int qs_ld = L.qs_pitch / (int)sizeof(T);  // staged query row pitch (elements)
    for (int hh = 0; hh < (kHP ? 1 : 2); ++hh) {
        const int half = kHP ? hw : hh;
        const T* keys = half ? keys2 : keys1;
        // 0. stage the query halves of the tile's rows in LDS, one 16-byte vector per
        //    thread and step; rows past the batch or past this workgroup's rows are zero
        {
            constexpr int kV = 16 / (int)sizeof(T);
            const int vpr = dh2 / kV;
            for (int e = gtid; e < kRtRows * vpr; e += kRtWaves * 64) {
                const int lr = e / vpr, c = e - lr * vpr;
                const int64_t r = row0 + lr;
                uint4 v = make_uint4(0u, 0u, 0u, 0u);
                if (lr < kRowsWG && r < rows) v = *reinterpret_cast<const uint4*>(q + r * dq + half * dh2 + c * kV);
                *reinterpret_cast<uint4*>(qsb + (size_t)lr * L.qs_pitch + (size_t)c * 16) = v;
            }
        }
        __syncthreads();
        const T* qtile = reinterpret_cast<const T*>(qsb);

        // 1. approximate scores for the 32-row tile: wave w takes key blocks w, w + 8, ...
        //    The key fragments of kU reduction steps are loaded before their MFMAs, so
        //    their L2 latencies overlap.
        constexpr int kU = sizeof(T) == 2 ? (RPW == 1 ? 4 : 2) : (RPW == 1 ? 16 : 8);
        for (int kb0 = wv; kb0 < nkb; kb0 += 2 * kRtWaves) {
            f32x16_t acc[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c] = f32x16_zero();
            for (int k0 = 0; k0 < dh2; k0 += kU * M::kK) {
                typename M::frag a[kU], b[2][kU];
#pragma unroll
                for (int u = 0; u < kU; ++u) {
                    const int kk = k0 + u * M::kK;
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const int kb = kb0 + kRtWaves * c, j = kb * 32 + lrow;
                        if constexpr (kPrep)  // fragment-major copy: one contiguous 64-lane block
                            b[c][u] = kk < dh2 && kb < nkb
                                          ? M::load(kfrag + ((((int64_t)half * nkb + kb) * (dh2 / M::kK) + kk / M::kK) * kWave +
                                                             lane) * M::kKL)
                                          : M::zero();
                        else
                            b[c][u] = kk < dh2 && j < K ? M::load(keys + (int64_t)j * dh2 + kk + lk) : M::zero();
                    }
                }
#pragma unroll
                for (int u = 0; u < kU; ++u) {
                    const int kk = k0 + u * M::kK;
                    a[u] = kk < dh2 ? M::load(qtile + lrow * qs_ld + kk + lk) : M::zero();
                }
#pragma unroll
                for (int u = 0; u < kU; ++u) {
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        if (kb0 + kRtWaves * c < nkb) acc[c] = M::mma(a[u], b[c][u], acc[c]);
                }
            }
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int kb = kb0 + kRtWaves * c;
                if (kb < nkb) {
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (!kHP || mfma32_row(i, lane) < kRowsWG)  // (kHP: only the live rows have storage)
                            S[mfma32_row(i, lane) * pitch + kb * 32 + lrow] = acc[c][i];
                }
            }
        }
        __syncthreads();

        // 2. per row: candidate filter, then certification of the survivors.
        //    Filter: with the query-half norm bound qn >= ||q|| and the sub-key norm bounds
        //    kn_j >= ||k_j||, every approximate score satisfies |s~_j| <= (qn + e'_j) kn_j
        //    (e'_j = gamma qn), so the margin m_j = gamma qn kn_j + |s~_j| 2^-21 + 2^-120
        //    is at most m'_j = gamma qn kn_j + A and at most E = gamma qn kn_max + A, with
        //    A = (qn + gamma qn) kn_max 2^-21 + 2^-120 the same for the whole row.  A key
        //    whose upper bound s~_j + m_j rounds to a T value below RN_T(tau) cannot be
        //    selected; every such key has s~_j + gamma qn kn_j < cut - A, where cut is at
        //    most the lower end of the interval that rounds to RN_T(tau) (the filter keeps
        //    a superset of the keys that can be selected).
        //    Certification: a survivor whose interval [s~ - m, s~ + m] rounds to a single T
        //    value has that value as its exact score: rounding is monotone and the fp64
        //    chain lies inside the interval (its own error is below 2^-45 ||q|| ||k||, far
        //    inside the 1% slack of the margin).  The others go on the row's pending list,
        //    and step 3 scores the pending lists of all the wave's rows together.  A row
        //    with more than 64 survivors (rare) is scored exactly in full in step 4.
        // zero for every row slot, including the slots past the last row of a partial
        // tile (the loop below stops at that row, and step 3 sums all of n_pend)
        int n_cand[RPW], n_pend[RPW];
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) n_cand[rr] = n_pend[rr] = 0;
        uint32_t slow_rows = 0;
        // this lane's sub-key norm bounds (keys lane + 64 m) and their largest value over
        // the half (wave-uniform)
        float knr[kRtSlots];
        float kn_max;
        {
            uint32_t kb = 0;
#pragma unroll
            for (int m = 0; m < kRtSlots; ++m) {
                const int j = lane + m * kWave;
                knr[m] = j < K ? kn[half * kpad + j] : 0.0f;
                kb = max(kb, __float_as_uint(knr[m]));
            }
            kn_max = __uint_as_float(wave_max_u32(kb));
        }
        // sums of squares of the wave's staged query halves, all its rows at once: 64 / RPW
        // lanes per row (one DPP row of 16 lanes when a wave has four rows); every lane of
        // a row's group receives the row's sum
        float sq_row = 0.0f;
        {
            constexpr int kLPR = kWave / RPW;
            constexpr int kN = QVecF<T>::kN;
            static_assert(RPW == 1 || RPW == 4, "row groups of 64 or 16 lanes");
            const int lr = wv * RPW + lane / kLPR;
            const T* qs = reinterpret_cast<const T*>(qsb + (size_t)lr * L.qs_pitch);
            for (int i = (lane % kLPR) * kN; i < dh2; i += kLPR * kN) {
                float v[kN];
                QVecF<T>::load(qs + i, v);
#pragma unroll
                for (int t = 0; t < kN; ++t) sq_row = __builtin_fmaf(v[t], v[t], sq_row);
            }
            if constexpr (RPW == 1) {
                sq_row = wave_sum(sq_row);
            } else {
                sq_row += dpp_f32<kDppXor1>(sq_row);
                sq_row += dpp_f32<kDppXor2>(sq_row);
                sq_row += dpp_f32<kDppRowHalfMirror>(sq_row);
                sq_row += dpp_f32<kDppRowMirror>(sq_row);
            }
        }
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
            const int lr = wv * RPW + rr;
            const int64_t r = row0 + lr;
            if (r >= rows) break;
            // bound the norm of the staged query half (the 2^-12 slack covers the fp32
            // rounding of the sum of squares; v_sqrt_f32 is within 1 ulp for a normal
            // argument, and the offset keeps it normal)
            const float sq = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sq_row), rr * (kWave / RPW)));
            const float qn = __builtin_amdgcn_sqrtf(sq + 0x1p-100f) * (1.0f + 0x1p-12f);
            const float gq = gamma * qn;
            const float A = (qn + gq) * kn_max * 0x1p-21f * (1.0f + 0x1p-20f) + 0x1p-120f;
            const float E = __builtin_fmaf(gq, kn_max, A) * (1.0f + 0x1p-20f);

            // approximate scores of the row (registers) and the lane maxima
            float sv[kRtSlots];
            float lane_max = -__builtin_huge_valf();
#pragma unroll
            for (int m = 0; m < kRtSlots; ++m) {
                const int j = lane + m * kWave;
                sv[m] = j < K ? S[lr * pitch + j] : -__builtin_huge_valf();
                lane_max = fmaxf(lane_max, sv[m]);
            }
            // o: the largest value with 16 low zero bits such that at least kc lane maxima
            // are >= o (as ordered keys); it is at most the kc-th largest lane maximum
            const uint32_t lkey = lane < K ? ord32(lane_max) : 0u;
            uint32_t o = 0;
#pragma unroll
            for (int b = 31; b >= 16; --b) {
                const uint32_t cand_o = o | (1u << b);
                if ((int)__popcll(ballot(lkey >= cand_o)) >= kc) o = cand_o;
            }
            const float tau_s = __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
            const float tau = tau_s - E - fabsf(tau_s) * 0x1p-21f;
            const float cut = Elem<T>::round_down_cut(Elem<T>::round32(tau)) - A;

            // the row's scores are in registers now: its LDS row takes the survivors
            // (approximate score bits << 32 | sub-key), in slot order
            __builtin_amdgcn_wave_barrier();
            uint64_t* ck = reinterpret_cast<uint64_t*>(S + lr * pitch);
            int32_t* cand = reinterpret_cast<int32_t*>(S + lr * pitch);
            // the survivors, counted and (the first 64, in slot order) written as they are found
            int n = 0;
#pragma unroll
            for (int m = 0; m < kRtSlots; ++m) {
                const int j = lane + m * kWave;
                const bool f = j < K && __builtin_fmaf(gq, knr[m], sv[m]) >= cut;
                const uint64_t fb = ballot(f);
                const int pos = n + count_below(fb);
                if (f && pos < kWave) ck[pos] = ((uint64_t)__float_as_uint(sv[m]) << 32) | (uint32_t)j;
                n += (int)__popcll(fb);
            }
            n_cand[rr] = n;
            if (n <= kWave) {
                __builtin_amdgcn_wave_barrier();
                // certify each survivor; certified ones become final keys, the others join
                // the pending list as (sub-key << 8 | slot)
                const uint64_t e = lane < n ? ck[lane] : 0ull;
                const float sj = __uint_as_float((uint32_t)(e >> 32));
                const uint32_t j = (uint32_t)e;
                bool pend = false;
                uint32_t lo = 0;
                if (lane < n) {
                    const float marg = __builtin_fmaf(fabsf(sj), 0x1p-21f, __builtin_fmaf(gq, kn[half * kpad + j], 0x1p-120f));
                    float lo_f = sj - marg, hi_f = sj + marg;
                    Elem<T>::round32x2(lo_f, hi_f);  // RN_T of both ends (rounding is monotone)
                    lo = __float_as_uint(lo_f);
                    pend = !(lo == __float_as_uint(hi_f) && (lo & 0x7f800000u) != 0x7f800000u);
                }
                const uint64_t bal = ballot(pend);
                if (lane < n) {
                    if (pend) reinterpret_cast<uint32_t*>(S + lr * pitch + kRtPendOff)[count_below(bal)] = (j << 8) | (uint32_t)lane;
                    else ck[lane] = make_key(__uint_as_float(lo), j);
                }
                n_pend[rr] = (int)__popcll(bal);
            } else {
                // (rare) every survivor's sub-key, over the keys written above
                __builtin_amdgcn_wave_barrier();
                int pos = 0;
#pragma unroll
                for (int m = 0; m < kRtSlots; ++m) {
                    const int j = lane + m * kWave;
                    const bool f = j < K && __builtin_fmaf(gq, knr[m], sv[m]) >= cut;
                    const uint64_t fb = ballot(f);
                    if (f) cand[pos + count_below(fb)] = j;
                    pos += (int)__popcll(fb);
                }
                slow_rows |= 1u << rr;
            }
            __builtin_amdgcn_wave_barrier();
        }

        // 3. exact scores of the pending candidates of all the wave's rows, one per lane,
        //    written to their slots
        {
            int p_end[RPW];
            int nq = 0;
#pragma unroll
            for (int rr = 0; rr < RPW; ++rr) p_end[rr] = (nq += n_pend[rr]);
            for (int c0 = 0; c0 < nq; c0 += kWave) {
                const int idx = c0 + lane;
                if (idx < nq) {
                    int rr = 0, start = 0;
#pragma unroll
                    for (int t = 0; t < RPW - 1; ++t) {
                        if (idx >= p_end[t]) {
                            rr = t + 1;
                            start = p_end[t];
                        }
                    }
                    const int lr = wv * RPW + rr;
                    const uint32_t e = reinterpret_cast<const uint32_t*>(S + lr * pitch + kRtPendOff)[idx - start];
                    const T* qs = reinterpret_cast<const T*>(qsb + (size_t)lr * L.qs_pitch);
                    reinterpret_cast<uint64_t*>(S + lr * pitch)[e & 0xffu] = exact_key<T, kExG>(qs, keys, dh2, (int)(e >> 8));
                }
            }
        }
        __builtin_amdgcn_wave_barrier();

        // 4. canonical top-k_cand list of each row
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
            const int lr = wv * RPW + rr;
            const int64_t r = row0 + lr;
            if (r >= rows) break;
            const int n = n_cand[rr];
            typename LK::type run_l;
            if (!((slow_rows >> rr) & 1u)) {
                const uint64_t* ck = reinterpret_cast<const uint64_t*>(S + lr * pitch);
                run_l = LK::sort(lane < n ? ck[lane] : 0ull, lane);
            } else {
                uint64_t run = 0;
                const int32_t* cand = reinterpret_cast<const int32_t*>(S + lr * pitch);
                const T* qs = reinterpret_cast<const T*>(qsb + (size_t)lr * L.qs_pitch);
                for (int c0 = 0; c0 < n; c0 += kWave) {
                    const int idx = c0 + lane;
                    uint64_t key = idx < n ? exact_key<T, kExG>(qs, keys, dh2, cand[idx]) : 0ull;
                    key = wave_sort_desc<uint64_t>(key, lane);
                    run = c0 == 0 ? key : wave_merge_desc(run, key, lane);
                }
                run_l = LK::pack(run);
            }
            if (half == 0) lst[rr][0] = run_l;
            else lst[rr][1] = run_l;
        }
        __syncthreads();
    }
    if constexpr (kHP) {
        // the second group's lists to the first group's waves (row wv), which combine
        typename LK::type* xch = reinterpret_cast<typename LK::type*>(smem + L.xch_off);
        if (hw == 1) xch[wv * kWave + lane] = lst[0][1];
        __syncthreads();
        if (hw == 1) return;
        lst[0][1] = xch[wv * kWave + lane];
    }

    // Combine the two candidate lists of each row and take the canonical top-k.
    // Both lists are sorted (score descending), so c[a][b] = RN_T(v1[a] + v2[b]) does
    // not increase in a or b, and a pair with (a+1)(b+1) > top_k is dominated by at
    // least top_k pairs of the staircase {(a+1)(b+1) <= top_k} (at most 119 pairs).
    // Hence theta, the top_k-th largest staircase value, bounds every pair outside the
    // staircase, and an outside pair can enter the top-k only by tying theta (it may
    // win the tie on its expert id).  So: rank the staircase, then merge in the rare
    // outside pairs equal to theta.
    // Staircase pair t of this lane: entry lane + 64 t of the list of (a, b), a-major, with
    // b < nb(a) = min(top_k / (a + 1), kc).  Lane a (< kc) holds nb(a) and its exclusive
    // prefix cum(a) (a wave scan); an entry's row is the last a with nb(a) > 0 and
    // cum(a) <= its index (nb does not increase with a).
    int st_a[kRtStSlots], st_b[kRtStSlots];
    // fr_b: the first column outside the staircase in row a = lane (a <= top_k, a < kc), or
    // -1 when the row has none: the largest pair of the row outside the staircase
    int fr_b;
    {
        const int nbl = lane < kc ? min(top_k / (lane + 1), kc) : 0;
        int incl = nbl;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int v = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += v;
        }
        const int cuml = incl - nbl;
        const int total = __shfl(incl, kWave - 1, kWave);  // (lanes from kc on add 0)
        fr_b = lane < kc && lane <= top_k && nbl < kc ? nbl : -1;
        int arow[kRtStSlots];
#pragma unroll
        for (int t = 0; t < kRtStSlots; ++t) arow[t] = 0;
        for (int a = 1; a < kc; ++a) {
            const int nba = __builtin_amdgcn_readlane(nbl, a), ca = __builtin_amdgcn_readlane(cuml, a);
            if (nba == 0) break;
#pragma unroll
            for (int t = 0; t < kRtStSlots; ++t)
                if (ca <= lane + t * kWave) arow[t] = a;
        }
#pragma unroll
        for (int t = 0; t < kRtStSlots; ++t) {
            const int idx = lane + t * kWave;
            const int ca = __shfl(cuml, arow[t], kWave);
            st_a[t] = idx < total ? arow[t] : -1;
            st_b[t] = idx < total ? idx - ca : 0;
        }
    }
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
        const int lr = wv * RPW + rr;
        const int64_t r = row0 + lr;
        if (r >= rows) break;
        const uint64_t L1 = LK::unpack(lst[rr][0]), L2 = LK::unpack(lst[rr][1]);
        // (lane shuffles: call with every lane active, then select)
        auto pair_key = [&](int a, int b) {
            const uint64_t ka = shfl_u64(L1, a), kb = shfl_u64(L2, b);
            const float v = Elem<T>::round32(key_score(ka) + key_score(kb));
            return make_key(v, key_idx(ka) * (uint32_t)K + key_idx(kb));
        };
        uint64_t run = 0;
#pragma unroll
        for (int t = 0; t < kRtStSlots; ++t) {
            if (t > 0 && ballot(st_a[t] >= 0) == 0) break;
            const uint64_t pk = pair_key(st_a[t] >= 0 ? st_a[t] : 0, st_b[t]);
            uint64_t key = st_a[t] >= 0 ? pk : 0ull;
            key = wave_sort_desc<uint64_t>(key, lane);
            run = t == 0 ? key : wave_merge_desc(run, key, lane);
        }
        const float theta = key_score(readlane_u64(run, top_k - 1));
        // A tie with theta needs c[a][0] >= theta and c[0][b] >= theta: a < na, b < nb.
        const float v1_0 = key_score(readlane_u64(L1, 0)), v2_0 = key_score(readlane_u64(L2, 0));
        float ca = key_score(L1) + v2_0, cb = v1_0 + key_score(L2);
        Elem<T>::round32x2(ca, cb);
        const bool in_a = lane < kc && ca >= theta;
        const bool in_b = lane < kc && cb >= theta;
        const int na = (int)__popcll(ballot(in_a)), nb = (int)__popcll(ballot(in_b));
        // No pair outside the staircase exceeds theta, and within a row they do not
        // increase with b (rows beyond top_k are bounded by row top_k), so unless one of
        // the rows' first outside pairs equals theta there is no tie to merge in.
        const uint64_t fk = shfl_u64(L2, fr_b >= 0 ? fr_b : 0);
        const bool fr_tie = fr_b >= 0 && Elem<T>::round32(key_score(L1) + key_score(fk)) == theta;
        if (ballot(fr_tie) != 0)
        for (int p0 = 0; p0 < na * nb; p0 += kWave) {
            const int p = p0 + lane;
            const bool in = p < na * nb;
            const int a = in ? p / nb : 0, b = in ? p - (p / nb) * nb : 0;
            uint64_t key = pair_key(a, b);
            const bool tie = in && (a + 1) * (b + 1) > top_k && key_score(key) == theta;
            if (ballot(tie) == 0) continue;
            key = wave_sort_desc<uint64_t>(tie ? key : 0ull, lane);
            run = wave_merge_desc(run, key, lane);
        }
        // gates: exponentials in parallel, their sum in list order
        const float m = key_score(readlane_u64(run, 0));
        const float ex = lane < top_k ? (float)exp((double)(key_score(run) - m)) : 0.0f;
        float sum = 0.0f;
        for (int i = 0; i < top_k; ++i) sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(ex), i));
        if (lane < top_k) {
            out_ids[r * top_k + lane] = (int32_t)key_idx(run);
            out_gates[r * top_k + lane] = Elem<T>::from_f32_rne(ex / sum);
        }
    }
}

size_t route_smem_bytes(int K, int dh2, int elem_bytes) { return route_smem_layout(K, dh2, elem_bytes).total; }

// Fragment-major copy of both sub-key tables for the scoring MFMAs: block (half, key block kb
// of 32 keys, k-step s) holds, for lane l of the wave, the M::kKL elements that lane loads as
// its B fragment, keys[32 kb + l % 32][s kK + (l / 32) kKL ..] (zero past the last key), so
// that each fragment load of a wave reads one contiguous block instead of 32 key rows.
size_t route_keys_bytes(int K, int dh2, int dtype) {
    const int kpad = (K + 31) / 32 * 32;
    return (size_t)2 * kpad * dh2 * (dtype == kBF16 ? 2 : 4);
}

template <typename T>
__global__ __launch_bounds__(256) void route_keys_kernel(const T* __restrict__ k1, const T* __restrict__ k2, int K,
                                                         int dh2, T* __restrict__ out) {
    using M = Mfma<T>;
    const int nkb = (K + 31) / 32, nks = dh2 / M::kK;
    const int64_t n = (int64_t)2 * nkb * nks * kWave;
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const int l = (int)(e % kWave);
    const int64_t blk = e / kWave;
    const int s = (int)(blk % nks), kb = (int)((blk / nks) % nkb), half = (int)(blk / ((int64_t)nks * nkb));
    const T* keys = half ? k2 : k1;
    const int j = kb * 32 + l % 32, k0 = s * M::kK + (l / 32) * M::kKL;
#pragma unroll
    for (int i = 0; i < M::kKL; ++i) out[e * M::kKL + i] = j < K ? keys[(int64_t)j * dh2 + k0 + i] : T{};
}

int launch_route_prepare_keys(const void* k1, const void* k2, int K, int dq, int dtype, void* out,
                              hipStream_t stream) {
    const int dh2 = dq / 2;
    const int kk = dtype == kBF16 ? Mfma<uint16_t>::kK : Mfma<float>::kK;
    const int64_t n = (int64_t)2 * ((K + 31) / 32) * (dh2 / kk) * kWave;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (dtype == kBF16)
        hipLaunchKernelGGL(route_keys_kernel<uint16_t>, grid, dim3(256), 0, stream, (const uint16_t*)k1,
                           (const uint16_t*)k2, K, dh2, (uint16_t*)out);
    else
        hipLaunchKernelGGL(route_keys_kernel<float>, grid, dim3(256), 0, stream, (const float*)k1, (const float*)k2, K,
                           dh2, (float*)out);
    return (int)hipGetLastError();
}

bool route_supported(int K, int dh2, int dtype) {
    const int kq = dtype == kBF16 ? 16 : 4;
    return K <= kRtMaxK && dh2 <= kRtMaxDh2 && dh2 % kq == 0 && route_smem_bytes(K, dh2, dtype == kBF16 ? 2 : 4) <= 160 * 1024;
}

template <typename T, bool kPrep>
static void launch_route_t(const void* q, const void* k1, const void* k2, const float* key_norms, const void* kfrag,
                           int64_t rows, int dq, int K, int top_k, int kc, void* gates, int32_t* ids,
                           hipStream_t stream) {
    const int dh2 = dq / 2;
    const bool small = rows <= kRtSmallRows;
    const int per_wg = kRtWaves * (small ? 1 : 4);
    const dim3 grid((unsigned)((rows + per_wg - 1) / per_wg));
    if (small)  // one row per wave, the two query halves in parallel
        hipLaunchKernelGGL((route_kernel<T, 1, true, kPrep>), grid, dim3(2 * kRtWaves * 64),
                           route_smem_layout(K, dh2, (int)sizeof(T), true).total, stream, (const T*)q, (const T*)k1,
                           (const T*)k2, key_norms, rows, dq, K, top_k, kc, (T*)gates, ids, (const T*)kfrag);
    else
        hipLaunchKernelGGL((route_kernel<T, 4, false, kPrep>), grid, dim3(kRtWaves * 64),
                           route_smem_bytes(K, dh2, (int)sizeof(T)), stream, (const T*)q, (const T*)k1, (const T*)k2,
                           key_norms, rows, dq, K, top_k, kc, (T*)gates, ids, (const T*)kfrag);
}

int launch_route(const void* q, const void* k1, const void* k2, const float* key_norms, const void* kfrag,
                 int64_t rows, int dq, int K, int top_k, int kc, int dtype, void* gates, int32_t* ids,
                 hipStream_t stream) {
    if (dtype == kBF16) {
        if (kfrag)
            launch_route_t<uint16_t, true>(q, k1, k2, key_norms, kfrag, rows, dq, K, top_k, kc, gates, ids, stream);
        else
            launch_route_t<uint16_t, false>(q, k1, k2, key_norms, kfrag, rows, dq, K, top_k, kc, gates, ids, stream);
    } else {
        if (kfrag)
            launch_route_t<float, true>(q, k1, k2, key_norms, kfrag, rows, dq, K, top_k, kc, gates, ids, stream);
        else
            launch_route_t<float, false>(q, k1, k2, key_norms, kfrag, rows, dq, K, top_k, kc, gates, ids, stream);
    }
    return (int)hipGetLastError();
}

}  // namespace ethos
