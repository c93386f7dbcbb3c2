// Expert apply and weighted scatter-back (reference: model.py:320-341).
//
// Token projection, once per token (the reference forms it inside the pair loop,
// model.py:326, but it depends only on the token):
//   xp_t = RN_T( x_t W_u )          W_u = net.2.weight[:d]^T  ([d, dh])
// Per pair p = (t, h, j) with expert slot s:
//   a_p = RN_T( RN_T(gelu_erf( RN_T(h_s . xp_t) )) * g_p )                 (phase 1)
//   y_t = RN_T( sum_h^T RN_T( sum_j RN_T(a_p * v_s) ) / H )                (phase 2)
// where the inner sum is fp32 in j order, the head sum is taken in T one head at a
// time, and RN_T is rounding to the layer dtype -- the reference's rounding points
// (x_proj and torch.dot in T model.py:326-329, fp32 token accumulator model.py:312,334,
// per-head cast :336, dtype head sum :338, dtype divide :341).
//
// Phase 1 walks the pairs in expert order (the sorted permutation): a wave takes 64
// consecutive sorted positions, so each expert's h row is read about once and the
// token projections (n_tok x dh, a few MB) are gathered from the caches.  Phase 2 is
// token-major: one wave per token gathers the v rows of its H*k pairs and reduces
// them in registers; every output element is written by exactly one lane, so no
// atomics are needed and the result is deterministic.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_rows.hpp"
#include "ethos_mfma.hpp"
#include "ethos_tp.hpp"

namespace ethos {



// ---------------------------------------------------------------------------------
// Token projection xp = RN_T(x W_u), W_u[i][j] = w2[i * dh + j] for i < d.
// ---------------------------------------------------------------------------------
constexpr int kTpT = 64;     // tokens per tile
constexpr int kTpC = 64;     // hidden columns per tile

// bf16: W_u^T (row n = hidden column, d contiguous values) is first written to the
// workspace by a tiled transpose of net.2.weight's first d rows, so that both GEMM
// operands are staged with 16-byte loads.
__global__ __launch_bounds__(256) void transpose_wu_kernel(const uint16_t* __restrict__ w2, int d, int dh,
                                                           uint16_t* __restrict__ wut) {
    // a 64 x 64 tile: rows k0.. of w2 (columns n0..), read and written as 16-byte pieces
    __shared__ uint16_t tile[64][64 + 2];
    const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int e = tid + 256 * it, r = e >> 3, c8 = (e & 7) * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (k0 + r < d && n0 + c8 < dh) v = *reinterpret_cast<const uint4*>(w2 + (int64_t)(k0 + r) * dh + n0 + c8);
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            tile[r][c8 + 2 * q] = (uint16_t)(u[q] & 0xffffu);
            tile[r][c8 + 2 * q + 1] = (uint16_t)(u[q] >> 16);
        }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int e = tid + 256 * it, n = e >> 3, k8 = (e & 7) * 8;  // output row n, columns k8..
        uint32_t u[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            u[q] = (uint32_t)tile[k8 + 2 * q][n] | ((uint32_t)tile[k8 + 2 * q + 1][n] << 16);
        if (n0 + n < dh && k0 + k8 < d)
            *reinterpret_cast<uint4*>(wut + (int64_t)(n0 + n) * d + k0 + k8) = make_uint4(u[0], u[1], u[2], u[3]);
    }
}

// Tiles for the per-XCD L2s (workgroup b runs on XCD b % 8): row block r goes to XCD r % 8,
// its nct column tiles to consecutive slots there, so that each block of x is read from HBM by
// one XCD; the grid is 8 nct ceil(row blocks / 8), and the padding workgroups return.
__global__ __launch_bounds__(256) void token_proj_bf16_kernel(const uint16_t* __restrict__ x,
                                                              const uint16_t* __restrict__ wut, int n_tok, int d,
                                                              int dh, uint16_t* __restrict__ xp, int nct, int nrb) {
    __shared__ __align__(16) unsigned char ring[kTpLds];
    const int xcd = (int)(blockIdx.x & 7), j = (int)(blockIdx.x >> 3);
    const int rb = (j / nct) * 8 + xcd, ct = j % nct;
    if (rb >= nrb) return;
    token_proj_bf16_tile(ring, x, wut, n_tok, d, dh, xp, ct * kTpCols, rb * kTpRows);
}

// x [n_tok, K] times the [N, K] operand, output [n_tok, N], by the tile kernel above.
static void launch_tp_bf16(const uint16_t* x, const uint16_t* w, int64_t n_tok, int K, int N, uint16_t* out,
                           hipStream_t stream) {
    const int nct = (N + kTpCols - 1) / kTpCols, nrb = (int)((n_tok + kTpRows - 1) / kTpRows);
    hipLaunchKernelGGL(token_proj_bf16_kernel, dim3((unsigned)(8 * nct * ((nrb + 7) / 8))), dim3(256), 0, stream, x,
                       w, (int)n_tok, K, N, out, nct, nrb);
}

// Any shape and dtype: fp64 accumulation in index order, rounded once to T.
template <typename T>
__global__ __launch_bounds__(256) void token_proj_kernel(const T* __restrict__ x, const T* __restrict__ wu, int n_tok,
                                                         int d, int dh, T* __restrict__ xp) {
    constexpr int KC = 32;
    __shared__ double xs[KC][kTpT];
    __shared__ double ws[KC][kTpC];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int c0 = blockIdx.x * kTpC;
    const int t0 = blockIdx.y * kTpT;
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    for (int k0 = 0; k0 < d; k0 += KC) {
        const int kc = min(KC, d - k0);
        for (int e = tid; e < kTpT * KC; e += 256) {
            const int r = e / KC, kk = e % KC;
            xs[kk][r] = (kk < kc && t0 + r < n_tok) ? Elem<T>::to_f64(x[(int64_t)(t0 + r) * d + k0 + kk]) : 0.0;
        }
        for (int e = tid; e < kTpC * KC; e += 256) {
            const int kk = e / kTpC, r = e % kTpC;
            ws[kk][r] = (kk < kc && c0 + r < dh) ? Elem<T>::to_f64(wu[(int64_t)(k0 + kk) * dh + c0 + r]) : 0.0;
        }
        __syncthreads();
        for (int kk = 0; kk < kc; ++kk) {
            double a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = xs[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = ws[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = t0 + ty * 4 + i;
        if (t >= n_tok) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + tx * 4 + j;
            if (c < dh) xp[(int64_t)t * dh + c] = Elem<T>::from_f32(Elem<T>::round64(acc[i][j]));
        }
    }
}

constexpr int kActGroup = 4;  // pairs whose loads are in flight together

template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_act_kernel(const T* __restrict__ xp, const T* __restrict__ hid,
                                                        const int32_t* __restrict__ perm,
                                                        const int32_t* __restrict__ sorted_slot,
                                                        const T* __restrict__ gates, int64_t n_pairs, int hk, int dh,
                                                        float* __restrict__ act) {
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    const int64_t n_chunks = (n_pairs + 63) / 64;
    for (int64_t chunk = wave_id; chunk < n_chunks; chunk += n_waves) {
        const int64_t i0 = chunk * 64;
        const int cnt = (int)min((int64_t)64, n_pairs - i0);
        const int my_p = lane < cnt ? perm[i0 + lane] : 0;
        const int my_s = lane < cnt ? sorted_slot[i0 + lane] : 0;
        // Groups of kActGroup consecutive sorted pairs: every h and xp row of a group is
        // requested before the first dot product (repeated h rows of one expert hit in
        // the cache), then the group's wave reductions run interleaved.
        for (int j0 = 0; j0 < cnt; j0 += kActGroup) {
            Raw ur[kActGroup][CH], xr[kActGroup][CH];
            int pq[kActGroup];
#pragma unroll
            for (int q = 0; q < kActGroup; ++q) {
                const int j = j0 + q < cnt ? j0 + q : cnt - 1;  // a tail group repeats the last pair
                const int s = __builtin_amdgcn_readlane(my_s, j);
                pq[q] = __builtin_amdgcn_readlane(my_p, j);
                load_raw_buf<T, CH>(hid + (int64_t)s * dh, dh, lane, ur[q]);
                load_raw_buf<T, CH>(xp + (int64_t)(pq[q] / hk) * dh, dh, lane, xr[q]);
            }
            float part[kActGroup];
#pragma unroll
            for (int q = 0; q < kActGroup; ++q) {
                part[q] = 0.0f;
#pragma unroll
                for (int c = 0; c < CH; ++c) part[q] = dot_raw(ur[q][c], xr[q][c], part[q]);
            }
#pragma unroll
            for (int q = 0; q < kActGroup; ++q) {
                const float dot = wave_sum(part[q]);
                if (lane == q && j0 + q < cnt) {
                    const float g = Elem<T>::to_f32(gates[pq[q]]);
                    const float a = Elem<T>::round32(gelu_erf(Elem<T>::round32(dot)));
                    act[pq[q]] = Elem<T>::round32(a * g);
                }
            }
        }
    }
}

// Per-pair activations with 8 lanes per pair.  A wave takes 64 consecutive sorted pairs
// and works through them 8 at a time: lane l serves pair l / 8 of the group and holds the
// 16-byte pieces (l % 8) + 8 i, i < P, of its h row and its xp row, so each load
// instruction reads 8 whole 128-byte lines.  Per lane: P pieces of dot products in fp32,
// then a 3-step reduction over the pair's 8 lanes (act_reduce8); the 64 dot products wait
// in LDS and the epilogue (act_epilogue: rounding, GELU, gate) runs once per 64 pairs, one
// pair per lane.  P = pieces per lane: dh <= 64 P elements (bf16) or 32 P (fp32).
// With seg_off given (after the hidden-row kernel has computed the activations of the
// tiles it could), the expert-order walk takes only the pairs of tiles of kActTileRows
// unique experts with more than kActFusedCap pairs; chunks without such pairs are skipped.
constexpr int kAct8Waves = 4;
constexpr int64_t kActSmallPairs = 65536;  // batches up to this many pairs take 16-pair token-order units

// kFull: the row is exactly 8 P pieces of 16 bytes, so every lane's pieces are in range and
// the row loads need no per-lane test (a masked load is a branch of its own).
template <typename T, int P, bool kFull>
__global__ __launch_bounds__(kAct8Waves * 64) void apply_act8_kernel(const T* __restrict__ xp, const T* __restrict__ hid,
                                                                     const int32_t* __restrict__ perm,
                                                                     const int32_t* __restrict__ sorted_slot,
                                                                     const int32_t* __restrict__ pair_slot,
                                                                     const int32_t* __restrict__ n_unique,
                                                                     const int32_t* __restrict__ seg_off,
                                                                     const T* __restrict__ gates, int64_t n_pairs,
                                                                     int hk, int dh, int upairs,
                                                                     float* __restrict__ act) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    __shared__ float dots[kAct8Waves][64];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int part = lane & 7, slot = lane >> 3;
    const int64_t wave_id = (int64_t)blockIdx.x * kAct8Waves + wave;
    const int64_t n_waves = (int64_t)gridDim.x * kAct8Waves;
    if (n_unique != nullptr && pair_slot != nullptr &&
        (int64_t)*n_unique * dh * (int64_t)sizeof(T) <= kActTokenOrderMaxHBytes) {
        // Units of upairs (<= 64) consecutive pairs of one token, one wave each (small
        // batches take units smaller than a token's pairs, so that they spread over more
        // waves).  Two groups' hidden rows are requested before either is summed; the loads
        // and sums are unconditional (a group past the unit's repeats the pair's first),
        // so no branch separates a load from its use.
        const int64_t n_tok = n_pairs / hk;
        const int cpt = (hk + upairs - 1) / upairs;
        for (int64_t u = wave_id; u < n_tok * cpt; u += n_waves) {
            const int64_t t = u / cpt;
            const int j0 = (int)(u - t * cpt) * upairs;
            const int cnt = hk - j0 < upairs ? hk - j0 : upairs;
            const int64_t pbase = t * hk + j0;
            // (lanes past the unit load its last pair: no select waits on these loads)
            const int lc = lane < cnt ? lane : cnt - 1;
            const int my_s = pair_slot[pbase + lc];
            const T my_g = gates[pbase + lc];
            const T* xr = xp + t * dh;
            Raw xv[P];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int e = (part + 8 * i) * N;
                xv[i] = kFull || e < dh ? *reinterpret_cast<const Raw*>(xr + e) : Raw{};
            }
            const int ng = (cnt + 7) / 8;
            for (int g0 = 0; g0 < ng; g0 += 2) {
                Raw hv[2][P];
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    // this lane's pair of the group (a tail group repeats the last pair)
                    const int g = g0 + b < ng ? g0 + b : g0;
                    const int src = g * 8 + slot < cnt ? g * 8 + slot : cnt - 1;
                    const T* hr = hid + (int64_t)__shfl(my_s, src, 64) * dh;
#pragma unroll
                    for (int i = 0; i < P; ++i) {
                        const int e = (part + 8 * i) * N;
                        hv[b][i] = kFull || e < dh ? *reinterpret_cast<const Raw*>(hr + e) : Raw{};
                    }
                }
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    float acc = 0.0f;
#pragma unroll
                    for (int i = 0; i < P; ++i) acc = dot_raw(hv[b][i], xv[i], acc);
                    acc = act_reduce8(acc);
                    if (part == 0 && g0 + b < ng) dots[wave][(g0 + b) * 8 + slot] = acc;
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (lane < cnt) act[pbase + lane] = act_epilogue<T>(dots[wave][lane], Elem<T>::to_f32(my_g));
            __builtin_amdgcn_wave_barrier();
        }
        return;
    }
    const int64_t n_chunks = (n_pairs + 63) / 64;
    const int U = seg_off != nullptr ? *n_unique : 0;
    for (int64_t chunk = wave_id; chunk < n_chunks; chunk += n_waves) {
        const int64_t i0 = chunk * 64;
        const int cnt = (int)min((int64_t)64, n_pairs - i0);
        // (lanes past the chunk read its last position, unused: no load waits on a branch)
        const int my_s = sorted_slot[i0 + (lane < cnt ? lane : cnt - 1)];
        bool mine = lane < cnt;
        if (seg_off != nullptr) {
            // pairs of tiles within the cap were done by the hidden-row kernel
            const int t0 = my_s - my_s % kActTileRows;
            const int t1 = t0 + kActTileRows < U ? t0 + kActTileRows : U;
            mine = mine && (int64_t)seg_off[t1] - (int64_t)seg_off[t0] > kActFusedCap;
        }
        if (ballot(mine) == 0) continue;
        const int my_p = mine ? perm[i0 + lane] : 0;
        for (int g = 0; g < cnt; g += 8) {
            // this lane's pair of the group (a tail group repeats the last pair)
            const int src = g + slot < cnt ? g + slot : cnt - 1;
            const int p = __shfl(my_p, src, 64);
            const int sl = __shfl(my_s, src, 64);
            const T* hr = hid + (int64_t)sl * dh;
            const T* xr = xp + (int64_t)(p / hk) * dh;
            Raw hv[P], xv[P];
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int e = (part + 8 * i) * N;
                hv[i] = kFull || e < dh ? *reinterpret_cast<const Raw*>(hr + e) : Raw{};
                xv[i] = kFull || e < dh ? *reinterpret_cast<const Raw*>(xr + e) : Raw{};
            }
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < P; ++i) acc = dot_raw(hv[i], xv[i], acc);
            // sum over the pair's 8 lanes (lanes 8 slot .. 8 slot + 7)
            acc = act_reduce8(acc);
            if (part == 0) dots[wave][g + slot] = acc;
        }
        __builtin_amdgcn_wave_barrier();
        if (mine) act[my_p] = act_epilogue<T>(dots[wave][lane], Elem<T>::to_f32(gates[my_p]));
        __builtin_amdgcn_wave_barrier();
    }
}

constexpr int kScatterUnroll = 8;  // v rows in flight per wave

// Pairs are read a chunk of up to 64 at a time, lane j holding pair p0 + j's slot and
// activation (one vector load each instead of a scalar load per pair, whose latency the
// pair's row load would wait behind); a group of U pairs j0 .. j0 + U - 1 of the chunk is then
// taken by lane reads.  A group past the chunk's last pair repeats that pair (its row is
// loaded again and not used), so that the group's row loads issue with no branch between them;
// likewise lanes past the chunk (cnt >= 1) load its last pair, so that no branch's join waits
// for the chunk's loads.
__device__ __forceinline__ void load_pair_chunk(const int32_t* __restrict__ pair_slot, const float* __restrict__ act,
                                                int64_t p0, int cnt, int lane, int& sl, float& a) {
    const int64_t p = p0 + (lane < cnt ? lane : cnt - 1);
    sl = pair_slot[p];
    a = act[p];
}
template <int U>
__device__ __forceinline__ void pair_group(int csl, float cac, int j0, int cn, int (&sl)[U], float (&a)[U]) {
#pragma unroll
    for (int q = 0; q < U; ++q) {
        const int j = j0 + q < cn ? j0 + q : cn - 1;
        sl[q] = __builtin_amdgcn_readlane(csl, j);
        a[q] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(cac), j));
    }
}

template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_scatter_kernel(const T* __restrict__ vr_,
                                                            const int32_t* __restrict__ pair_slot,
                                                            const float* __restrict__ act, int64_t n_tok, int H,
                                                            int k, int d, T* __restrict__ out) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    const float inv_h_div = (float)H;
    for (int64_t t = wave_id; t < n_tok; t += n_waves) {
        float o[CH * N];
#pragma unroll
        for (int e = 0; e < CH * N; ++e) o[e] = 0.0f;
        // chunks of a head's pairs, each loaded one chunk ahead (the next head's first after a
        // head's last)
        const int64_t tb = t * H * k;
        int nsl;
        float nac;
        load_pair_chunk(pair_slot, act, tb, k < 64 ? k : 64, lane, nsl, nac);
        for (int h = 0; h < H; ++h) {
            float hacc[CH * N];
#pragma unroll
            for (int e = 0; e < CH * N; ++e) hacc[e] = 0.0f;
            for (int c0 = 0; c0 < k; c0 += 64) {
                const int csl = nsl, cn = k - c0 < 64 ? k - c0 : 64;
                const float cac = nac;
                const int nh = c0 + 64 < k ? h : h + 1, nc0 = c0 + 64 < k ? c0 + 64 : 0;
                if (nh < H) load_pair_chunk(pair_slot, act, tb + (int64_t)nh * k + nc0, k - nc0 < 64 ? k - nc0 : 64, lane, nsl, nac);
                for (int j0 = 0; j0 < cn; j0 += kScatterUnroll) {
                    Raw vr[kScatterUnroll][CH];
                    float a[kScatterUnroll];
                    int sl[kScatterUnroll];
                    pair_group<kScatterUnroll>(csl, cac, j0, cn, sl, a);
#pragma unroll
                    for (int q = 0; q < kScatterUnroll; ++q) load_raw_buf<T, CH>(vr_ + (int64_t)sl[q] * d, d, lane, vr[q]);
#pragma unroll
                    for (int q = 0; q < kScatterUnroll; ++q) {
                        if (j0 + q < cn) {
#pragma unroll
                            for (int c = 0; c < CH; ++c) {
                                float vf[N];
                                Vec16<T>::unpack(vr[q][c], vf);
#pragma unroll
                                for (int v = 0; v < N; v += 2) {
                                    float p0 = a[q] * vf[v], p1 = a[q] * vf[v + 1];
                                    Elem<T>::round32x2(p0, p1);  // RN_T(a v)
                                    hacc[c * N + v] += p0;
                                    hacc[c * N + v + 1] += p1;
                                }
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < CH * N; e += 2) {
                float h0 = hacc[e], h1 = hacc[e + 1];
                Elem<T>::round32x2(h0, h1);  // the head's sum cast to T
                float o0 = o[e] + h0, o1 = o[e + 1] + h1;
                Elem<T>::round32x2(o0, o1);  // the running head sum in T
                o[e] = o0;
                o[e + 1] = o1;
            }
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < d) {
                float r[N];
#pragma unroll
                for (int v = 0; v < N; ++v) r[v] = o[c * N + v] / inv_h_div;
                *reinterpret_cast<typename Vec16<T>::raw*>(out + t * d + e) = Vec16<T>::pack(r);
            }
        }
    }
}

// Hidden-space reordering (paper/ETHOS.pdf p.10, Algorithm 1): per token,
// hs_t = RN_T((1/H) sum_p RN32(a_p h_s)) over its pairs in order (heads, then k), the sum in
// float32.  One wave per token; the pairs' hidden rows are gathered kScatterUnroll at a
// time, each lane owning CH chunks of N consecutive columns.
template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_hacc_kernel(const T* __restrict__ hid,
                                                         const int32_t* __restrict__ pair_slot,
                                                         const float* __restrict__ act, int64_t n_tok, int H,
                                                         int k, int dh, T* __restrict__ hs) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    const int np = H * k;
    for (int64_t t = wave_id; t < n_tok; t += n_waves) {
        float acc[CH * N];
#pragma unroll
        for (int e = 0; e < CH * N; ++e) acc[e] = 0.0f;
        const int64_t pbase = t * np;
        // chunks of the token's pairs, each loaded one chunk ahead
        int nsl;
        float nac;
        load_pair_chunk(pair_slot, act, pbase, np < 64 ? np : 64, lane, nsl, nac);
        for (int c0 = 0; c0 < np; c0 += 64) {
            const int csl = nsl, cn = np - c0 < 64 ? np - c0 : 64;
            const float cac = nac;
            if (c0 + 64 < np) load_pair_chunk(pair_slot, act, pbase + c0 + 64, np - c0 - 64 < 64 ? np - c0 - 64 : 64, lane, nsl, nac);
            for (int j0 = 0; j0 < cn; j0 += kScatterUnroll) {
                Raw hr[kScatterUnroll][CH];
                float a[kScatterUnroll];
                int sl[kScatterUnroll];
                pair_group<kScatterUnroll>(csl, cac, j0, cn, sl, a);
#pragma unroll
                for (int q = 0; q < kScatterUnroll; ++q) load_raw_buf<T, CH>(hid + (int64_t)sl[q] * dh, dh, lane, hr[q]);
#pragma unroll
                for (int q = 0; q < kScatterUnroll; ++q) {
                    if (j0 + q < cn) {
#pragma unroll
                        for (int c = 0; c < CH; ++c) {
                            float hf[N];
                            Vec16<T>::unpack(hr[q][c], hf);
#pragma unroll
                            for (int v = 0; v < N; ++v) acc[c * N + v] += a[q] * hf[v];  // float32 products
                        }
                    }
                }
            }
        }
        const float hdiv = (float)H;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < dh) {
                float r[N];
#pragma unroll
                for (int v = 0; v < N; ++v) r[v] = acc[c * N + v] / hdiv;
                *reinterpret_cast<Raw*>(hs + t * dh + e) = Vec16<T>::pack(r);
            }
        }
    }
}

// out[j][i] = in[i][j] for in [rows, cols] (32 x 32 tiles through LDS)
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ in, int rows, int cols,
                                                        T* __restrict__ out) {
    __shared__ T tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8)
        if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = in[(int64_t)(r0 + r) * cols + c0 + tx];
    __syncthreads();
    for (int c = ty; c < 32; c += 8)
        if (c0 + c < cols && r0 + tx < rows) out[(int64_t)(c0 + c) * rows + r0 + tx] = tile[tx][c];
}

// Small batches: the scatter-back split by head, so that n_tok * H waves (not n_tok) share
// the gathers.  Each (token, head)'s RN_T(sum_k RN_T(a v)) is formed by one wave, then the
// heads are added in order in T and divided by H: the same operations in the same order as
// apply_scatter_kernel, so the output is bit-identical.  When a token's H head rows fit in
// kTokHeadLds bytes of LDS, apply_scatter_tok_kernel does both in one launch (one
// workgroup per token, its waves taking the heads); otherwise apply_scatter_head_kernel
// writes the head rows to headbuf [n_tok, H, d] and apply_head_sum_kernel sums them.
constexpr int64_t kSplitHeadMaxTok = 1024;
constexpr int kTokWaves = 8;
constexpr int kTokHeadLds = 64 * 1024;

// The head sum of one (token, head) item, pairs pbase .. pbase + k - 1, into hacc (fp32,
// this lane's CH chunks of N columns), U v rows in flight (16 per wave in the per-token kernel
// was slower: 0.142 -> 0.145 ms per 64-token forward, 0.348 -> 0.371 ms at 1,024 tokens).
template <typename T, int CH, int U = kScatterUnroll>
__device__ __forceinline__ void scatter_head_sum(const T* __restrict__ vr_, const int32_t* __restrict__ pair_slot,
                                                 const float* __restrict__ act, int64_t pbase, int k, int d,
                                                 int lane, float (&hacc)[CH * Vec16<T>::kN]) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
#pragma unroll
    for (int e = 0; e < CH * N; ++e) hacc[e] = 0.0f;
    for (int c0 = 0; c0 < k; c0 += 64) {
        const int cn = k - c0 < 64 ? k - c0 : 64;
        int csl;
        float cac;
        load_pair_chunk(pair_slot, act, pbase + c0, cn, lane, csl, cac);
        for (int j0 = 0; j0 < cn; j0 += U) {
            Raw vr[U][CH];
            float a[U];
            int sl[U];
            pair_group<U>(csl, cac, j0, cn, sl, a);
#pragma unroll
            for (int q = 0; q < U; ++q) load_raw_buf<T, CH>(vr_ + (int64_t)sl[q] * d, d, lane, vr[q]);
#pragma unroll
            for (int q = 0; q < U; ++q) {
                if (j0 + q < cn) {
#pragma unroll
                    for (int c = 0; c < CH; ++c) {
                        float vf[N];
                        Vec16<T>::unpack(vr[q][c], vf);
#pragma unroll
                        for (int v = 0; v < N; v += 2) {
                            float p0 = a[q] * vf[v], p1 = a[q] * vf[v + 1];
                            Elem<T>::round32x2(p0, p1);  // RN_T(a v)
                            hacc[c * N + v] += p0;
                            hacc[c * N + v + 1] += p1;
                        }
                    }
                }
            }
        }
    }
}

template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_scatter_head_kernel(const T* __restrict__ vr_,
                                                                 const int32_t* __restrict__ pair_slot,
                                                                 const float* __restrict__ act, int64_t n_items,
                                                                 int k, int d, T* __restrict__ headbuf) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    for (int64_t it = wave_id; it < n_items; it += n_waves) {  // item = t * H + head
        float hacc[CH * N];
        scatter_head_sum<T, CH>(vr_, pair_slot, act, it * k, k, d, lane, hacc);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < d) *reinterpret_cast<Raw*>(headbuf + it * d + e) = Vec16<T>::pack(hacc + c * N);  // RN_T
        }
    }
}

// One workgroup per token (gridDim.x = n_tok): wave w forms the head rows h = w, w +
// kTokWaves, ... into LDS (H d elements of T), then the threads add the heads in order for
// 16-byte column groups and store the token's output row.
template <typename T, int CH>
__global__ __launch_bounds__(kTokWaves * 64) void apply_scatter_tok_kernel(const T* __restrict__ vr_,
                                                                           const int32_t* __restrict__ pair_slot,
                                                                           const float* __restrict__ act, int H,
                                                                           int k, int d, T* __restrict__ out) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    extern __shared__ __align__(16) unsigned char tok_lds[];
    T* hb = reinterpret_cast<T*>(tok_lds);  // [H][d]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t t = blockIdx.x;
    for (int h = wave; h < H; h += kTokWaves) {
        float hacc[CH * N];
        scatter_head_sum<T, CH>(vr_, pair_slot, act, (t * H + h) * k, k, d, lane, hacc);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < d) *reinterpret_cast<Raw*>(hb + h * d + e) = Vec16<T>::pack(hacc + c * N);  // RN_T
        }
    }
    __syncthreads();
    const float hdiv = (float)H;
    for (int g = threadIdx.x; g * N < d; g += kTokWaves * 64) {
        float o[N];
#pragma unroll
        for (int v = 0; v < N; ++v) o[v] = 0.0f;
        for (int h = 0; h < H; ++h) {
            float hv[N];
            Vec16<T>::unpack(*reinterpret_cast<const Raw*>(hb + h * d + g * N), hv);
#pragma unroll
            for (int v = 0; v < N; v += 2) {
                float o0 = o[v] + hv[v], o1 = o[v + 1] + hv[v + 1];
                Elem<T>::round32x2(o0, o1);  // the running head sum in T
                o[v] = o0;
                o[v + 1] = o1;
            }
        }
        float r[N];
#pragma unroll
        for (int v = 0; v < N; ++v) r[v] = o[v] / hdiv;
        *reinterpret_cast<Raw*>(out + t * d + g * N) = Vec16<T>::pack(r);
    }
}

template <typename T, int CH>
__global__ __launch_bounds__(256) void apply_head_sum_kernel(const T* __restrict__ headbuf, int64_t n_tok, int H,
                                                             int d, T* __restrict__ out) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    const float hdiv = (float)H;
    for (int64_t t = wave_id; t < n_tok; t += n_waves) {
        float o[CH * N];
#pragma unroll
        for (int e = 0; e < CH * N; ++e) o[e] = 0.0f;
        for (int h = 0; h < H; ++h) {
            float hv[CH * N];
            load_row<T, CH>(headbuf + (t * H + h) * d, d, lane, hv);
#pragma unroll
            for (int e = 0; e < CH * N; e += 2) {
                float o0 = o[e] + hv[e], o1 = o[e + 1] + hv[e + 1];
                Elem<T>::round32x2(o0, o1);  // the running head sum in T
                o[e] = o0;
                o[e + 1] = o1;
            }
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < d) {
                float r[N];
#pragma unroll
                for (int v = 0; v < N; ++v) r[v] = o[c * N + v] / hdiv;
                *reinterpret_cast<Raw*>(out + t * d + e) = Vec16<T>::pack(r);
            }
        }
    }
}

template <typename T, int CH1>
static void launch_act_t(const void* xp, const void* hid, const int32_t* perm, const int32_t* sorted_slot,
                         const void* gates, int64_t n_pairs, int hk, int dh, float* act, int num_cus,
                         hipStream_t stream) {
    const int64_t cap = (int64_t)num_cus * 16;
    int64_t g1 = ((n_pairs + 63) / 64 + 3) / 4;
    g1 = g1 > cap ? cap : (g1 < 1 ? 1 : g1);
    hipLaunchKernelGGL((apply_act_kernel<T, CH1>), dim3((unsigned)g1), dim3(256), 0, stream, (const T*)xp,
                       (const T*)hid, perm, sorted_slot, (const T*)gates, n_pairs, hk, dh, act);
}

template <typename T, int CH2>
static void launch_scatter_t(const void* v, const int32_t* pair_slot, const float* act, int64_t n_tok, int H, int k,
                             int d, void* headbuf, void* out, int num_cus, hipStream_t stream) {
    const int64_t cap = (int64_t)num_cus * 16;
    const size_t tok_lds = (size_t)H * d * sizeof(T);
    if (CH2 <= 4 && headbuf != nullptr && tok_lds <= (size_t)kTokHeadLds) {  // (wider rows would spill)
        hipLaunchKernelGGL((apply_scatter_tok_kernel<T, CH2>), dim3((unsigned)n_tok), dim3(kTokWaves * 64), tok_lds,
                           stream, (const T*)v, pair_slot, act, H, k, d, (T*)out);
        return;
    }
    if (headbuf != nullptr) {
        const int64_t items = n_tok * H;
        int64_t g3 = (items + 3) / 4;
        g3 = g3 > cap ? cap : (g3 < 1 ? 1 : g3);
        hipLaunchKernelGGL((apply_scatter_head_kernel<T, CH2>), dim3((unsigned)g3), dim3(256), 0, stream,
                           (const T*)v, pair_slot, act, items, k, d, (T*)headbuf);
        int64_t g4 = (n_tok + 3) / 4;
        g4 = g4 > cap ? cap : (g4 < 1 ? 1 : g4);
        hipLaunchKernelGGL((apply_head_sum_kernel<T, CH2>), dim3((unsigned)g4), dim3(256), 0, stream,
                           (const T*)headbuf, n_tok, H, d, (T*)out);
        return;
    }
    int64_t g2 = (n_tok + 3) / 4;
    g2 = g2 > cap ? cap : (g2 < 1 ? 1 : g2);
    hipLaunchKernelGGL((apply_scatter_kernel<T, CH2>), dim3((unsigned)g2), dim3(256), 0, stream, (const T*)v,
                       pair_slot, act, n_tok, H, k, d, (T*)out);
}

template <typename T, int P>
static void launch_act8_t(const void* xp, const void* hid, const int32_t* perm, const int32_t* sorted_slot,
                          const int32_t* pair_slot, const int32_t* n_unique, const int32_t* seg_off, const void* gates,
                          int64_t n_pairs, int hk, int dh, float* act, int num_cus, hipStream_t stream) {
    // token-order units: 16 pairs for small batches (more waves than tokens), else 64
    const int upairs = n_pairs <= kActSmallPairs ? 16 : 64;
    const int64_t cap = (int64_t)num_cus * 16;
    int64_t g1 = ((n_pairs + upairs - 1) / upairs + kAct8Waves - 1) / kAct8Waves;
    g1 = g1 > cap ? cap : (g1 < 1 ? 1 : g1);
    if (dh == 8 * P * Vec16<T>::kN)
        hipLaunchKernelGGL((apply_act8_kernel<T, P, true>), dim3((unsigned)g1), dim3(kAct8Waves * 64), 0, stream,
                           (const T*)xp, (const T*)hid, perm, sorted_slot, pair_slot, n_unique, seg_off, (const T*)gates,
                           n_pairs, hk, dh, upairs, act);
    else
        hipLaunchKernelGGL((apply_act8_kernel<T, P, false>), dim3((unsigned)g1), dim3(kAct8Waves * 64), 0, stream,
                           (const T*)xp, (const T*)hid, perm, sorted_slot, pair_slot, n_unique, seg_off, (const T*)gates,
                           n_pairs, hk, dh, upairs, act);
}

// Per-pair activations a_p (phase 1): 8 lanes per pair for rows of up to 64 pieces of 16
// bytes (d_hidden <= 512 bf16 / 256 fp32), one wave per pair beyond; -1 past the limits.
// With pair_slot and the device count n_unique given, the 8-lane kernel takes token order
// when the hidden rows are few (kActTokenOrderMaxHBytes).  With seg_off given too, only
// the pairs the hidden-row kernel left (tiles over kActFusedCap pairs) are computed.
static int launch_act(const void* xp, const void* hid, const int32_t* perm, const int32_t* sorted_slot,
                      const int32_t* pair_slot, const int32_t* n_unique, const int32_t* seg_off, const void* gates,
                      int64_t n_pairs, int hk, int dh, int dtype, float* act, int num_cus, hipStream_t stream) {
    const int pieces = (dh + (dtype == kBF16 ? 8 : 4) - 1) / (dtype == kBF16 ? 8 : 4);
    const int pp = (pieces + 7) / 8;
    const int P = pp <= 1 ? 1 : pp <= 2 ? 2 : pp <= 4 ? 4 : pp <= 8 ? 8 : 0;
#define ETHOS_ACT8_CASE(TT, PP)                                                                                \
    if (P == PP) {                                                                                             \
        launch_act8_t<TT, PP>(xp, hid, perm, sorted_slot, pair_slot, n_unique, seg_off, gates, n_pairs, hk, dh, \
                              act, num_cus, stream);                                                           \
        return 0;                                                                                              \
    }
    if (dtype == kBF16) {
        ETHOS_ACT8_CASE(uint16_t, 1) ETHOS_ACT8_CASE(uint16_t, 2) ETHOS_ACT8_CASE(uint16_t, 4)
        ETHOS_ACT8_CASE(uint16_t, 8)
    } else {
        ETHOS_ACT8_CASE(float, 1) ETHOS_ACT8_CASE(float, 2) ETHOS_ACT8_CASE(float, 4) ETHOS_ACT8_CASE(float, 8)
    }
#undef ETHOS_ACT8_CASE
    if (seg_off != nullptr) return -1;  // the remainder walk exists in the 8-lane kernel only
    const int c = apply_chunks(dh, dtype);
    const int ch = c <= 1 ? 1 : c <= 2 ? 2 : c <= 4 ? 4 : c <= 8 ? 8 : 0;
#define ETHOS_ACT_CASE(TT, CC)                                                                                 \
    if (ch == CC) {                                                                                            \
        launch_act_t<TT, CC>(xp, hid, perm, sorted_slot, gates, n_pairs, hk, dh, act, num_cus, stream);         \
        return 0;                                                                                              \
    }
    if (dtype == kBF16) {
        ETHOS_ACT_CASE(uint16_t, 1) ETHOS_ACT_CASE(uint16_t, 2) ETHOS_ACT_CASE(uint16_t, 4) ETHOS_ACT_CASE(uint16_t, 8)
    } else {
        ETHOS_ACT_CASE(float, 1) ETHOS_ACT_CASE(float, 2) ETHOS_ACT_CASE(float, 4) ETHOS_ACT_CASE(float, 8)
    }
#undef ETHOS_ACT_CASE
    return -1;
}

// Weighted scatter-back (phase 2) for lane chunk counts 1, 2, 4 or 8; -1 beyond.
static int launch_scatter(const void* v, const int32_t* pair_slot, const float* act, int64_t n_tok, int H, int k,
                          int d, int dtype, void* headbuf, void* out, int num_cus, hipStream_t stream) {
    const int c = apply_chunks(d, dtype);
    const int ch = c <= 1 ? 1 : c <= 2 ? 2 : c <= 4 ? 4 : c <= 8 ? 8 : 0;
#define ETHOS_SCATTER_CASE(TT, CC)                                                                             \
    if (ch == CC) {                                                                                            \
        launch_scatter_t<TT, CC>(v, pair_slot, act, n_tok, H, k, d, headbuf, out, num_cus, stream);            \
        return 0;                                                                                              \
    }
    if (dtype == kBF16) {
        ETHOS_SCATTER_CASE(uint16_t, 1) ETHOS_SCATTER_CASE(uint16_t, 2) ETHOS_SCATTER_CASE(uint16_t, 4)
        ETHOS_SCATTER_CASE(uint16_t, 8)
    } else {
        ETHOS_SCATTER_CASE(float, 1) ETHOS_SCATTER_CASE(float, 2) ETHOS_SCATTER_CASE(float, 4)
        ETHOS_SCATTER_CASE(float, 8)
    }
#undef ETHOS_SCATTER_CASE
    return -1;
}

int apply_chunks(int d, int dtype) {
    const int per = 64 * (dtype == kBF16 ? 8 : 4);
    return (d + per - 1) / per;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// workspace: x_proj [n_tok, dh] T | act [N] fp32 | (bf16) W_u^T [dh, d]
static size_t wut_offset(int64_t n_tok, int H, int k, int dh, size_t eb) {
    return align256(align256((size_t)n_tok * dh * eb) + (size_t)n_tok * H * k * sizeof(float));
}

// d is not an argument here: the W_u^T block and the per-head rows of small batches are
// sized for d <= 4096, the ABI's limit
static size_t headbuf_offset(int64_t n_tok, int H, int k, int dh, size_t eb, int dtype) {
    return align256(wut_offset(n_tok, H, k, dh, eb) + (dtype == kBF16 ? (size_t)dh * 4096 * eb : 0));
}

size_t apply_workspace_bytes(int64_t n_tok, int H, int k, int dh, int dtype) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    return headbuf_offset(n_tok, H, k, dh, eb, dtype) +
           (n_tok <= kSplitHeadMaxTok ? (size_t)n_tok * H * 4096 * eb : 0);
}

// xp = RN_T(x W_u) into the workspace (W_u^T = the first d rows of net.2.weight, row
// length dh)
// `wut_in` (bf16, may be null): W_u^T [dh, d] prepared by the caller; otherwise it is
// transposed into the workspace here.
static void launch_token_proj(const void* x, const void* w2, const void* wut_in, int64_t n_tok, int H, int k, int d,
                              int dh, int dtype, void* ws, hipStream_t stream) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    void* xp = ws;
    const dim3 tgrid((unsigned)((dh + kTpC - 1) / kTpC), (unsigned)((n_tok + kTpT - 1) / kTpT));
    if (dtype == kBF16 && d % kTpK == 0 && dh % 8 == 0) {
        const uint16_t* wut = static_cast<const uint16_t*>(wut_in);
        if (wut == nullptr) {
            uint16_t* w = reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(ws) + wut_offset(n_tok, H, k, dh, eb));
            hipLaunchKernelGGL(transpose_wu_kernel, dim3((unsigned)((dh + 63) / 64), (unsigned)((d + 63) / 64)),
                               dim3(256), 0, stream, (const uint16_t*)w2, d, dh, w);
            wut = w;
        }
        launch_tp_bf16((const uint16_t*)x, (const uint16_t*)wut, n_tok, d, dh, (uint16_t*)xp, stream);
    } else if (dtype == kBF16)
        hipLaunchKernelGGL(token_proj_kernel<uint16_t>, tgrid, dim3(256), 0, stream, (const uint16_t*)x,
                           (const uint16_t*)w2, (int)n_tok, d, dh, (uint16_t*)xp);
    else
        hipLaunchKernelGGL(token_proj_kernel<float>, tgrid, dim3(256), 0, stream, (const float*)x, (const float*)w2,
                           (int)n_tok, d, dh, (float*)xp);
}

int launch_token_proj_out(const void* x, const void* w2, const void* wut, int64_t n_tok, int d, int dh, int dtype,
                          void* xp, hipStream_t stream) {
    // the bf16 MFMA form reads W_u^T; without it the kernel would transpose into scratch
    if (dtype == kBF16 && d % kTpK == 0 && dh % 8 == 0 && wut == nullptr) return -1;
    launch_token_proj(x, w2, wut, n_tok, 1, 1, d, dh, dtype, xp, stream);
    return (int)hipGetLastError();
}

int launch_apply(const void* x, const void* w2, const void* hid, const void* v, const int32_t* perm,
                 const int32_t* sorted_slot, const int32_t* pair_slot, const void* gates, int64_t n_tok, int H, int k,
                 int d, int dh, int dtype, void* ws, void* out, int num_cus, hipStream_t stream) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    void* xp = ws;
    float* act = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + align256((size_t)n_tok * dh * eb));
    void* headbuf = n_tok <= kSplitHeadMaxTok
                        ? static_cast<unsigned char*>(ws) + headbuf_offset(n_tok, H, k, dh, eb, dtype)
                        : nullptr;
    if (apply_chunks(dh, dtype) > 8 || apply_chunks(d, dtype) > 8) return -1;
    launch_token_proj(x, w2, nullptr, n_tok, H, k, d, dh, dtype, ws, stream);
    launch_act(xp, hid, perm, sorted_slot, nullptr, nullptr, nullptr, gates, n_tok * H * k, H * k, dh, dtype, act,
               num_cus, stream);
    launch_scatter(v, pair_slot, act, n_tok, H, k, d, dtype, headbuf, out, num_cus, stream);
    return (int)hipGetLastError();
}

// workspace for the hidden-space form: the apply workspace, then hs [n_tok, dh] T, then
// (fp32, or shapes the MFMA projection does not take) W_v^T [dh, d] T
static bool hidden_proj_mfma(int d, int dh, int dtype) { return dtype == kBF16 && dh % kTpK == 0 && d % 8 == 0; }

static size_t hs_offset(int64_t n_tok, int H, int k, int dh, int dtype) {
    return align256(apply_workspace_bytes(n_tok, H, k, dh, dtype));
}

size_t apply_hidden_workspace_bytes(int64_t n_tok, int H, int k, int d, int dh, int dtype) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    size_t b = hs_offset(n_tok, H, k, dh, dtype) + align256((size_t)n_tok * dh * eb);
    if (!hidden_proj_mfma(d, dh, dtype)) b += (size_t)d * dh * eb;
    return b;
}

template <typename T, int CH1>
static void launch_hacc_t(const void* hid, const int32_t* pair_slot, const float* act, int64_t n_tok, int H, int k,
                          int dh, void* hs, int num_cus, hipStream_t stream) {
    const int64_t cap = (int64_t)num_cus * 16;
    int64_t g2 = (n_tok + 3) / 4;
    g2 = g2 > cap ? cap : (g2 < 1 ? 1 : g2);
    hipLaunchKernelGGL((apply_hacc_kernel<T, CH1>), dim3((unsigned)g2), dim3(256), 0, stream, (const T*)hid,
                       pair_slot, act, n_tok, H, k, dh, (T*)hs);
}

// The hidden-space form after the activations: hs = RN_T((1/H) sum_p a_p h_s), then
// out = RN_T(hs W_v^T).
static int launch_hidden_tail(const void* w2, const void* hid, const int32_t* pair_slot, const float* act,
                              int64_t n_tok, int H, int k, int d, int dh, int dtype, void* ws, void* out, int num_cus,
                              hipStream_t stream);

int launch_apply_hidden(const void* x, const void* w2, const void* hid, const int32_t* perm,
                        const int32_t* sorted_slot, const int32_t* pair_slot, const void* gates, int64_t n_tok, int H,
                        int k, int d, int dh, int dtype, void* ws, void* out, int num_cus, hipStream_t stream) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    void* xp = ws;
    float* act = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + align256((size_t)n_tok * dh * eb));
    if (apply_chunks(dh, dtype) > 8) return -1;
    launch_token_proj(x, w2, nullptr, n_tok, H, k, d, dh, dtype, ws, stream);
    launch_act(xp, hid, perm, sorted_slot, nullptr, nullptr, nullptr, gates, n_tok * H * k, H * k, dh, dtype, act,
               num_cus, stream);
    return launch_hidden_tail(w2, hid, pair_slot, act, n_tok, H, k, d, dh, dtype, ws, out, num_cus, stream);
}

static int launch_hidden_tail(const void* w2, const void* hid, const int32_t* pair_slot, const float* act,
                              int64_t n_tok, int H, int k, int d, int dh, int dtype, void* ws, void* out, int num_cus,
                              hipStream_t stream) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    unsigned char* hs = static_cast<unsigned char*>(ws) + hs_offset(n_tok, H, k, dh, dtype);
    const int c1 = apply_chunks(dh, dtype);
    const int ch = c1 <= 1 ? 1 : c1 <= 2 ? 2 : c1 <= 4 ? 4 : 8;
    if (dtype == kBF16) {
        if (ch == 1) launch_hacc_t<uint16_t, 1>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
        else if (ch == 2) launch_hacc_t<uint16_t, 2>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
        else if (ch == 4) launch_hacc_t<uint16_t, 4>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
        else launch_hacc_t<uint16_t, 8>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
    } else {
        if (ch == 1) launch_hacc_t<float, 1>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
        else if (ch == 2) launch_hacc_t<float, 2>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
        else if (ch == 4) launch_hacc_t<float, 4>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
        else launch_hacc_t<float, 8>(hid, pair_slot, act, n_tok, H, k, dh, hs, num_cus, stream);
    }
    // projection back: out = RN_T(hs W_v^T), W_v^T = rows d .. 2d-1 of net.2.weight, which
    // as a [d, dh] row-major block is the output-major operand layout of the token
    // projection kernels (K = dh, N = d)
    const unsigned char* wv = static_cast<const unsigned char*>(w2) + (size_t)d * dh * eb;
    if (hidden_proj_mfma(d, dh, dtype)) {
        launch_tp_bf16((const uint16_t*)hs, (const uint16_t*)wv, n_tok, dh, d, (uint16_t*)out, stream);
        return (int)hipGetLastError();
    }
    // generic: W_v as [dh, d] row-major (the token_proj_kernel operand layout), then the
    // float64-accumulating projection
    unsigned char* wvt = hs + align256((size_t)n_tok * dh * eb);
    const dim3 tg((unsigned)((dh + 31) / 32), (unsigned)((d + 31) / 32));
    const dim3 pg((unsigned)((d + kTpC - 1) / kTpC), (unsigned)((n_tok + kTpT - 1) / kTpT));
    if (dtype == kBF16) {
        hipLaunchKernelGGL(transpose_kernel<uint16_t>, tg, dim3(256), 0, stream, (const uint16_t*)wv, d, dh,
                           (uint16_t*)wvt);
        hipLaunchKernelGGL(token_proj_kernel<uint16_t>, pg, dim3(256), 0, stream, (const uint16_t*)hs,
                           (const uint16_t*)wvt, (int)n_tok, dh, d, (uint16_t*)out);
    } else {
        hipLaunchKernelGGL(transpose_kernel<float>, tg, dim3(256), 0, stream, (const float*)wv, d, dh, (float*)wvt);
        hipLaunchKernelGGL(token_proj_kernel<float>, pg, dim3(256), 0, stream, (const float*)hs, (const float*)wvt,
                           (int)n_tok, dh, d, (float*)out);
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------
// The expert stages as one call (generation, apply, scatter-back) on the sorted pairs.
// Order 0 (the layer's rounding points): xp, h rows, activations, v rows, scatter-back;
// order 1 (hidden-space reordering): xp, h rows, activations, per-token hidden sums,
// projection back.  With the two-kernel bf16 generator the hidden-row kernel computes the
// activations of its tiles' pairs from the rows it has just staged in LDS (so h is not
// read back for them), and the activation kernel takes what it leaves; other shapes
// generate first (one kernel) and apply after.
// Workspace: the apply workspace of the order, then (order 0) v [max_unique, d].
// ---------------------------------------------------------------------------------
static size_t order_ws_bytes(int64_t n_tok, int H, int k, int d, int dh, int dtype, int order) {
    return order == 0 ? apply_workspace_bytes(n_tok, H, k, dh, dtype)
                      : apply_hidden_workspace_bytes(n_tok, H, k, d, dh, dtype);
}

size_t expert_forward_workspace_bytes(int64_t n_tok, int H, int k, int64_t max_unique, int d, int dh, int dtype,
                                      int order) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    size_t b = align256(order_ws_bytes(n_tok, H, k, d, dh, dtype, order));
    if (order == 0) b += (size_t)max_unique * d * eb;
    return b;
}

int launch_expert_forward(const void* x, const void* latents, int64_t n_experts, const void* w1, const void* w2,
                          const void* wut, const void* xp_in, const int32_t* uniq, const int32_t* seg_off,
                          const int32_t* n_unique, int64_t max_unique,
                          const int32_t* perm, const int32_t* sorted_slot, const int32_t* pair_slot,
                          const void* gates, int64_t n_tok, int H, int k, int dl, int dh, int d, int dtype, int order,
                          void* ws, void* hout, void* out, int num_cus, hipStream_t stream) {
    const size_t eb = dtype == kBF16 ? 2 : 4;
    unsigned char* v = order == 0 ? static_cast<unsigned char*>(ws) +
                                        align256(order_ws_bytes(n_tok, H, k, d, dh, dtype, order))
                                  : nullptr;
    if (apply_chunks(dh, dtype) > 8 || (order == 0 && apply_chunks(d, dtype) > 8)) return -1;
    // Stage marks (stage_mark), five per call: after the token projection, the hidden rows,
    // the activations, the v rows (order 0; nothing for order 1) and the scatter-back (or
    // the hidden-space tail).  Shapes without the two-kernel generator mark the one
    // generator launch as the hidden rows and the whole apply as the scatter-back.
    if (!generate_split_supported(n_experts, max_unique, dl, dh, d, dtype, num_cus)) {
        stage_mark(stream);
        int rc = launch_generate(latents, n_experts, uniq, n_unique, max_unique, w1, w2, dl, dh, d, dtype, hout, v,
                                 num_cus, stream);
        if (rc != 0) return rc;
        stage_mark(stream);
        stage_mark(stream);
        stage_mark(stream);
        rc = order == 0 ? launch_apply(x, w2, hout, v, perm, sorted_slot, pair_slot, gates, n_tok, H, k, d, dh, dtype,
                                       ws, out, num_cus, stream)
                        : launch_apply_hidden(x, w2, hout, perm, sorted_slot, pair_slot, gates, n_tok, H, k, d, dh,
                                              dtype, ws, out, num_cus, stream);
        stage_mark(stream);
        return rc;
    }
    // the token projection, unless the caller computed it (e.g. on another stream, while
    // the routing ran)
    void* xp = xp_in ? const_cast<void*>(xp_in) : ws;
    float* act = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) + align256((size_t)n_tok * dh * eb));
    if (!xp_in) launch_token_proj(x, w2, wut, n_tok, H, k, d, dh, dtype, ws, stream);
    stage_mark(stream);
    // the hidden rows, with the activations of every tile of at most kActFusedCap pairs
    // computed while its rows are in LDS; then the activation kernel for the rest (the
    // pairs of larger tiles, or all pairs in token order when the hidden rows are few)
    int rc = launch_hidden_act(latents, n_experts, uniq, n_unique, max_unique, w1, dl, dh, hout, xp, perm,
                               sorted_slot, seg_off, gates, H * k, act, n_tok * H * k, num_cus,
                               stream);
    if (rc != 0) return rc;
    stage_mark(stream);
    rc = launch_act(xp, hout, perm, sorted_slot, pair_slot, n_unique, seg_off, gates, n_tok * H * k, H * k, dh, dtype,
                    act, num_cus, stream);
    if (rc != 0) return rc;
    stage_mark(stream);
    if (order == 1) {
        stage_mark(stream);
        rc = launch_hidden_tail(w2, hout, pair_slot, act, n_tok, H, k, d, dh, dtype, ws, out, num_cus, stream);
        stage_mark(stream);
        return rc;
    }
    rc = launch_generate_part(latents, n_experts, uniq, n_unique, max_unique, w1, w2, dl, dh, d, hout, v, 2, num_cus,
                              stream);
    if (rc != 0) return rc;
    stage_mark(stream);
    void* headbuf = n_tok <= kSplitHeadMaxTok
                        ? static_cast<unsigned char*>(ws) + headbuf_offset(n_tok, H, k, dh, eb, dtype)
                        : nullptr;
    launch_scatter(v, pair_slot, act, n_tok, H, k, d, dtype, headbuf, out, num_cus, stream);
    stage_mark(stream);
    return (int)hipGetLastError();
}

}  // namespace ethos
