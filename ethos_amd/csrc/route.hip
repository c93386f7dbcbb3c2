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
//      A key whose upper bound rounds below RN_T(tau) rounds strictly below k_cand
//      other keys and cannot be selected: it is dropped.
//   3. The survivors (about 40 of 512) are scored exactly (the fp64 chain) one per
//      lane and ranked with 64-lane bitonic sort / merge networks on canonical keys.
// The output therefore equals exhaustive exact scoring bit for bit.
#pragma clang fp contract(off)

#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_mfma.hpp"

namespace ethos {

constexpr int kRtWaves = 8;                            // two workgroups per CU: four waves per SIMD
constexpr int kRtRows = 32;                            // rows per workgroup (one MFMA row block)
constexpr int kRtRowsPerWave = kRtRows / kRtWaves;
constexpr int kRtMaxKc = 32;                           // k_cand <= 32, top_k <= 32
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

// v of lane (lane ^ mask), mask a compile-time constant after inlining: DPP quad
// permutes for 1 and 2, ds_swizzle (xor mode, within 32 lanes) up to 31, and
// v_permlane32_swap for the half-wave exchange; no LDS addressing.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {  // every lane reads: no "old" operand
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kCtrl, 0xf, 0xf, true);
}

__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v, int mask) {
    if (mask == 1) return dpp_mov<kDppXor1>(v);
    if (mask == 2) return dpp_mov<kDppXor2>(v);
    uint32_t r = v;
    if (mask & 32) {
        const auto sw = __builtin_amdgcn_permlane32_swap(r, r, false, false);
        r = (__lane_id() & 32) ? sw[0] : sw[1];
    }
    switch (mask & 31) {
        case 0: break;
        case 1: r = dpp_mov<kDppXor1>(r); break;
        case 2: r = dpp_mov<kDppXor2>(r); break;
        case 4: r = (uint32_t)__builtin_amdgcn_ds_swizzle((int)r, (4 << 10) | 0x1f); break;
        case 8: r = (uint32_t)__builtin_amdgcn_ds_swizzle((int)r, (8 << 10) | 0x1f); break;
        case 16: r = (uint32_t)__builtin_amdgcn_ds_swizzle((int)r, (16 << 10) | 0x1f); break;
        case 31: r = (uint32_t)__builtin_amdgcn_ds_swizzle((int)r, (31 << 10) | 0x1f); break;
        default: r = (uint32_t)__shfl_xor((int)r, mask & 31, kWave); break;
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

template <typename V>
__device__ __forceinline__ V wave_sort_desc(V v, int lane) {
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const V p = shfl_xor_v<V>(v, j);
            const bool desc = (lane & k) == 0;
            const bool lower = (lane & j) == 0;
            const bool keep_max = lower == desc;
            // take the partner's value when it is larger (keep_max) or not larger
            v = (p > v) == keep_max ? p : v;
        }
    }
    return v;
}

// run and chunk are each sorted descending across the lanes; returns the 64 largest
// of their union, sorted descending.
__device__ __forceinline__ uint64_t wave_merge_desc(uint64_t run, uint64_t chunk, int lane) {
    const uint64_t rev = shfl_xor_u64(chunk, kWave - 1);  // chunk[63 - lane]
    uint64_t v = run > rev ? run : rev;                    // bitonic top-64
#pragma unroll
    for (int j = kWave >> 1; j > 0; j >>= 1) {
        const uint64_t p = shfl_xor_u64(v, j);
        const bool lower = (lane & j) == 0;
        v = (p > v) == lower ? p : v;
    }
    return v;
}

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
        const uint4 r = *reinterpret_cast<const uint4*>(p);
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
        const float4 r = *reinterpret_cast<const float4*>(p);
        d[0] = r.x;
        d[1] = r.y;
        d[2] = r.z;
        d[3] = r.w;
    }
};

struct RouteSmem {
    size_t s_off, kn_off, qs_off, total;
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

__host__ __device__ inline RouteSmem route_smem_layout(int K, int dh2, int elem_bytes) {
    RouteSmem L;
    size_t off = 0;
    L.s_off = off;
    off += (size_t)kRtRows * route_pitch(K) * sizeof(float);
    L.kn_off = off;
    off += (size_t)2 * ((K + 31) / 32) * 32 * sizeof(float);
    L.qs_off = off;
    // 16 bytes of padding put the query rows of one wave's lanes on different banks
    L.qs_pitch = dh2 * elem_bytes + 16;
    off += (size_t)kRtRows * L.qs_pitch;
    L.total = off;
    return L;
}

// Exact score key of sub-key j: the fp64 FMA chain over the query half qh (staged in
// LDS) and key row j (global, L2-resident), index order, rounded once to T.
template <typename T>
__device__ __forceinline__ uint64_t exact_key(const T* qh, const T* __restrict__ keys, int dh2, int j) {
    const T* kr = keys + (int64_t)j * dh2;
    double acc = 0.0;
    for (int i = 0; i < dh2; i += KeyVec<T>::kN) {
        double qv[KeyVec<T>::kN], kv[KeyVec<T>::kN];
        KeyVec<T>::load(qh + i, qv);
        KeyVec<T>::load(kr + i, kv);
#pragma unroll
        for (int t = 0; t < KeyVec<T>::kN; ++t) acc = fma(qv[t], kv[t], acc);
    }
    return make_key(Elem<T>::round64(acc), (uint32_t)j);
}

// Certified score of a candidate slot, or this pattern (a NaN, never a certified score)
// when the slot still needs the exact chain.
constexpr uint32_t kRtPending = 0xffffffffu;

template <typename T>
__global__ __launch_bounds__(kRtWaves * 64, 4) void route_kernel(const T* __restrict__ q, const T* __restrict__ keys1,
                                                    const T* __restrict__ keys2, const float* __restrict__ key_norms,
                                                    int64_t rows, int dq, int K, int top_k, int kc,
                                                    T* __restrict__ out_gates, int32_t* __restrict__ out_ids) {
    using M = Mfma<T>;
    extern __shared__ __align__(16) unsigned char smem[];
    const int dh2 = dq / 2;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lrow = lane & 31, lk = (lane >> 5) * M::kKL;
    const RouteSmem L = route_smem_layout(K, dh2, (int)sizeof(T));
    const int pitch = route_pitch(K);
    const int kpad = ((K + 31) / 32) * 32;
    float* S = reinterpret_cast<float*>(smem + L.s_off);
    float* kn = reinterpret_cast<float*>(smem + L.kn_off);
    // lst[rr][half]: the canonical top-k_cand list of this wave's row rr and query half,
    // entry i held by lane i
    uint64_t lst[kRtRowsPerWave][2];
#pragma unroll
    for (int rr = 0; rr < kRtRowsPerWave; ++rr) lst[rr][0] = lst[rr][1] = 0;

    const int64_t row0 = (int64_t)blockIdx.x * kRtRows;
    const int nkb = kpad / 32;
    const float gamma = (float)(dh2 + 16) * 0x1p-22f * 1.01f;

    // Sub-key norms (upper bounds) for both tables.
    for (int e = tid; e < 2 * kpad; e += kRtWaves * 64) {
        const int half = e / kpad, j = e - half * kpad;
        float nrm = 0.0f;
        if (j < K) {
            if (key_norms) {
                nrm = key_norms[half * K + j];
            } else {
                const T* kr = (half ? keys2 : keys1) + (int64_t)j * dh2;
                double s2 = 0.0;
                for (int i = 0; i < dh2; ++i) {
                    const double v = Elem<T>::to_f64(kr[i]);
                    s2 = fma(v, v, s2);
                }
                nrm = (float)(sqrt(s2) * (1.0 + 0x1p-20));
            }
        }
        kn[e] = nrm;
    }

    for (int half = 0; half < 2; ++half) {
        const T* keys = half ? keys2 : keys1;
        // 1. approximate scores for the 32-row tile: wave w takes key blocks w, w + 8, ...
        for (int kb0 = wave; kb0 < nkb; kb0 += 2 * kRtWaves) {
            f32x16_t acc[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c] = f32x16_zero();
            const int64_t arow = row0 + lrow;
            for (int k0 = 0; k0 < dh2; k0 += M::kK) {
                const typename M::frag a = arow < rows ? M::load(q + arow * dq + half * dh2 + k0 + lk) : M::zero();
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int kb = kb0 + kRtWaves * c;
                    if (kb < nkb) {
                        const int j = kb * 32 + lrow;
                        const typename M::frag b = j < K ? M::load(keys + (int64_t)j * dh2 + k0 + lk) : M::zero();
                        acc[c] = M::mma(a, b, acc[c]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int kb = kb0 + kRtWaves * c;
                if (kb < nkb) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) S[mfma32_row(i, lane) * pitch + kb * 32 + lrow] = acc[c][i];
                }
            }
        }
        __syncthreads();

        // 2. per row: certified candidate filter.  A candidate whose certified interval
        //    [s~ - e, s~ + e] rounds to a single T value has that value as its exact score:
        //    rounding is monotone and the fp64 chain lies inside the interval (its own
        //    error is below 2^-45 ||q|| ||k||, far inside the 1% slack of e).  The others
        //    go on the row's pending list, and step 3 scores the pending lists of all the
        //    wave's rows together.  A row with more than 64 candidates (rare) is scored
        //    exactly in full in step 4.
        // zero for every row slot, including the slots past the last row of a partial
        // tile (the loop below stops at that row, and step 3 sums all of n_pend)
        int n_cand[kRtRowsPerWave], n_pend[kRtRowsPerWave];
#pragma unroll
        for (int rr = 0; rr < kRtRowsPerWave; ++rr) n_cand[rr] = n_pend[rr] = 0;
        uint32_t slow_rows = 0;
        const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
        for (int rr = 0; rr < kRtRowsPerWave; ++rr) {
            const int lr = wave * kRtRowsPerWave + rr;
            const int64_t r = row0 + lr;
            if (r >= rows) break;
            // stage the query half in LDS (16 bytes per lane) and bound its norm
            T* qs = reinterpret_cast<T*>(smem + L.qs_off + (size_t)lr * L.qs_pitch);
            float sq = 0.0f;
            for (int i = lane * KeyVec<T>::kN; i < dh2; i += kWave * KeyVec<T>::kN) {
                const uint4 raw = *reinterpret_cast<const uint4*>(q + r * dq + half * dh2 + i);
                *reinterpret_cast<uint4*>(qs + i) = raw;
                double v[KeyVec<T>::kN];
                KeyVec<T>::load(qs + i, v);
#pragma unroll
                for (int t = 0; t < KeyVec<T>::kN; ++t) sq = __builtin_fmaf((float)v[t], (float)v[t], sq);
            }
            const float qn = sqrtf(wave_sum(sq)) * (1.0f + 0x1p-12f);

            // up: upper bounds of the scores (filter); cs: certified scores or kRtPending
            float up[kRtSlots];   // RN_T of the upper bounds
            uint32_t cs[kRtSlots];
            float lane_max = -__builtin_huge_valf();
            uint32_t emax_bits = 0;
#pragma unroll
            for (int m = 0; m < kRtSlots; ++m) {
                const int j = lane + m * kWave;
                up[m] = -__builtin_huge_valf();
                cs[m] = kRtPending;
                if (j < K) {
                    const float sj = S[lr * pitch + j];
                    const float marg = gamma * qn * kn[half * kpad + j] + fabsf(sj) * 0x1p-21f + 0x1p-120f;
                    float lo_f = sj - marg, hi_f = sj + marg;
                    Elem<T>::round32x2(lo_f, hi_f);  // RN_T of both ends (rounding is monotone)
                    up[m] = hi_f;
                    const uint32_t lo = __float_as_uint(lo_f);
                    const uint32_t hi = __float_as_uint(hi_f);
                    if (lo == hi && (lo & 0x7f800000u) != 0x7f800000u) cs[m] = lo;
                    lane_max = fmaxf(lane_max, sj);
                    emax_bits = max(emax_bits, __float_as_uint(marg));
                }
            }
            const float emax = __uint_as_float(wave_max_u32(emax_bits));
            // o: the largest value with 16 low zero bits such that at least kc lane maxima
            // are >= o (as ordered keys); it is at most the kc-th largest lane maximum
            const uint32_t lkey = lane < K ? ord32(lane_max) : 0u;
            uint32_t o = 0;
#pragma unroll
            for (int b = 31; b >= 16; --b) {
                const uint32_t cand_o = o | (1u << b);
                if ((int)__popcll(__ballot(lkey >= cand_o)) >= kc) o = cand_o;
            }
            const float tau_s = __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
            const float tau = tau_s - emax * (1.0f + 0x1p-20f) - fabsf(tau_s) * 0x1p-21f;
            const float thr = Elem<T>::round32(tau);

            uint32_t fbits = 0;
            int n = 0;
#pragma unroll
            for (int m = 0; m < kRtSlots; ++m) {
                const bool f = lane + m * kWave < K && up[m] >= thr;
                fbits |= (uint32_t)f << m;
                n += (int)__popcll(__ballot(f));
            }
            n_cand[rr] = n;
            // the row's scores are in registers now: its LDS row holds the candidates
            __builtin_amdgcn_wave_barrier();
            if (n <= kWave) {
                uint64_t* ck = reinterpret_cast<uint64_t*>(S + lr * pitch);
                int pos = 0;
#pragma unroll
                for (int m = 0; m < kRtSlots; ++m) {
                    const bool f = (fbits >> m) & 1u;
                    const uint64_t bal = __ballot(f);
                    if (f) ck[pos + __popcll(bal & below)] = ((uint64_t)cs[m] << 32) | (uint32_t)(lane + m * kWave);
                    pos += (int)__popcll(bal);
                }
                __builtin_amdgcn_wave_barrier();
                // certified slots become final keys; the others join the pending list as
                // (sub-key << 8 | slot)
                const uint64_t e = lane < n ? ck[lane] : 0ull;
                const uint32_t sc = (uint32_t)(e >> 32), j = (uint32_t)e;
                const bool pend = lane < n && sc == kRtPending;
                const uint64_t bal = __ballot(pend);
                if (lane < n) {
                    if (pend) reinterpret_cast<uint32_t*>(S + lr * pitch + kRtPendOff)[__popcll(bal & below)] = (j << 8) | (uint32_t)lane;
                    else ck[lane] = make_key(__uint_as_float(sc), j);
                }
                n_pend[rr] = (int)__popcll(bal);
            } else {
                int32_t* cand = reinterpret_cast<int32_t*>(S + lr * pitch);
                int pos = 0;
#pragma unroll
                for (int m = 0; m < kRtSlots; ++m) {
                    const bool f = (fbits >> m) & 1u;
                    const uint64_t bal = __ballot(f);
                    if (f) cand[pos + __popcll(bal & below)] = lane + m * kWave;
                    pos += (int)__popcll(bal);
                }
                slow_rows |= 1u << rr;
            }
            __builtin_amdgcn_wave_barrier();
        }

        // 3. exact scores of the pending candidates of all the wave's rows, one per lane,
        //    written to their slots
        {
            int p_end[kRtRowsPerWave];
            int nq = 0;
#pragma unroll
            for (int rr = 0; rr < kRtRowsPerWave; ++rr) p_end[rr] = (nq += n_pend[rr]);
            for (int c0 = 0; c0 < nq; c0 += kWave) {
                const int idx = c0 + lane;
                if (idx < nq) {
                    int rr = 0, start = 0;
#pragma unroll
                    for (int t = 0; t < kRtRowsPerWave - 1; ++t) {
                        if (idx >= p_end[t]) {
                            rr = t + 1;
                            start = p_end[t];
                        }
                    }
                    const int lr = wave * kRtRowsPerWave + rr;
                    const uint32_t e = reinterpret_cast<const uint32_t*>(S + lr * pitch + kRtPendOff)[idx - start];
                    const T* qs = reinterpret_cast<const T*>(smem + L.qs_off + (size_t)lr * L.qs_pitch);
                    reinterpret_cast<uint64_t*>(S + lr * pitch)[e & 0xffu] = exact_key<T>(qs, keys, dh2, (int)(e >> 8));
                }
            }
        }
        __builtin_amdgcn_wave_barrier();

        // 4. canonical top-k_cand list of each row
#pragma unroll
        for (int rr = 0; rr < kRtRowsPerWave; ++rr) {
            const int lr = wave * kRtRowsPerWave + rr;
            const int64_t r = row0 + lr;
            if (r >= rows) break;
            const int n = n_cand[rr];
            uint64_t run = 0;
            if (!((slow_rows >> rr) & 1u)) {
                const uint64_t* ck = reinterpret_cast<const uint64_t*>(S + lr * pitch);
                run = wave_sort_desc<uint64_t>(lane < n ? ck[lane] : 0ull, lane);
            } else {
                const int32_t* cand = reinterpret_cast<const int32_t*>(S + lr * pitch);
                const T* qs = reinterpret_cast<const T*>(smem + L.qs_off + (size_t)lr * L.qs_pitch);
                for (int c0 = 0; c0 < n; c0 += kWave) {
                    const int idx = c0 + lane;
                    uint64_t key = idx < n ? exact_key<T>(qs, keys, dh2, cand[idx]) : 0ull;
                    key = wave_sort_desc<uint64_t>(key, lane);
                    run = c0 == 0 ? key : wave_merge_desc(run, key, lane);
                }
            }
            if (half == 0) lst[rr][0] = run;
            else lst[rr][1] = run;
        }
        __syncthreads();
    }

    // Combine the two candidate lists of each row and take the canonical top-k.
    // Both lists are sorted (score descending), so c[a][b] = RN_T(v1[a] + v2[b]) does
    // not increase in a or b, and a pair with (a+1)(b+1) > top_k is dominated by at
    // least top_k pairs of the staircase {(a+1)(b+1) <= top_k} (at most 119 pairs).
    // Hence theta, the top_k-th largest staircase value, bounds every pair outside the
    // staircase, and an outside pair can enter the top-k only by tying theta (it may
    // win the tie on its expert id).  So: rank the staircase, then merge in the rare
    // outside pairs equal to theta.
    int st_a[kRtStSlots], st_b[kRtStSlots];
#pragma unroll
    for (int t = 0; t < kRtStSlots; ++t) {
        int idx = lane + t * kWave, a = 0;
        st_a[t] = -1;
        st_b[t] = 0;
        for (; a < kc; ++a) {
            int nb = top_k / (a + 1);
            nb = nb < kc ? nb : kc;
            if (nb == 0) break;
            if (idx < nb) {
                st_a[t] = a;
                st_b[t] = idx;
                break;
            }
            idx -= nb;
        }
    }
#pragma unroll
    for (int rr = 0; rr < kRtRowsPerWave; ++rr) {
        const int lr = wave * kRtRowsPerWave + rr;
        const int64_t r = row0 + lr;
        if (r >= rows) break;
        const uint64_t L1 = lst[rr][0], L2 = lst[rr][1];
        // (lane shuffles: call with every lane active, then select)
        auto pair_key = [&](int a, int b) {
            const uint64_t ka = shfl_u64(L1, a), kb = shfl_u64(L2, b);
            const float v = Elem<T>::round32(key_score(ka) + key_score(kb));
            return make_key(v, key_idx(ka) * (uint32_t)K + key_idx(kb));
        };
        uint64_t run = 0;
#pragma unroll
        for (int t = 0; t < kRtStSlots; ++t) {
            if (t > 0 && __ballot(st_a[t] >= 0) == 0) break;
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
        const int na = (int)__popcll(__ballot(in_a)), nb = (int)__popcll(__ballot(in_b));
        for (int p0 = 0; p0 < na * nb; p0 += kWave) {
            const int p = p0 + lane;
            const bool in = p < na * nb;
            const int a = in ? p / nb : 0, b = in ? p - (p / nb) * nb : 0;
            uint64_t key = pair_key(a, b);
            const bool tie = in && (a + 1) * (b + 1) > top_k && key_score(key) == theta;
            if (__ballot(tie) == 0) continue;
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
            out_gates[r * top_k + lane] = Elem<T>::from_f32(ex / sum);
        }
    }
}

size_t route_smem_bytes(int K, int dh2, int elem_bytes) { return route_smem_layout(K, dh2, elem_bytes).total; }

bool route_supported(int K, int dh2, int dtype) {
    const int kq = dtype == kBF16 ? 16 : 4;
    return K <= kRtMaxK && dh2 <= kRtMaxDh2 && dh2 % kq == 0 && route_smem_bytes(K, dh2, dtype == kBF16 ? 2 : 4) <= 160 * 1024;
}

int launch_route(const void* q, const void* k1, const void* k2, const float* key_norms, int64_t rows, int dq, int K,
                 int top_k, int kc, int dtype, void* gates, int32_t* ids, hipStream_t stream) {
    const int dh2 = dq / 2;
    const size_t smem = route_smem_bytes(K, dh2, dtype == kBF16 ? 2 : 4);
    dim3 grid((unsigned)((rows + kRtRows - 1) / kRtRows));
    if (dtype == kBF16)
        hipLaunchKernelGGL(route_kernel<uint16_t>, grid, dim3(kRtWaves * 64), smem, stream, (const uint16_t*)q,
                           (const uint16_t*)k1, (const uint16_t*)k2, key_norms, rows, dq, K, top_k, kc,
                           (uint16_t*)gates, ids);
    else
        hipLaunchKernelGGL(route_kernel<float>, grid, dim3(kRtWaves * 64), smem, stream, (const float*)q, (const float*)k1,
                           (const float*)k2, key_norms, rows, dq, K, top_k, kc, (float*)gates, ids);
    return (int)hipGetLastError();
}

}  // namespace ethos
