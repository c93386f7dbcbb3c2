// Backward of the expert stages: the derivative of the reference layer's per-pair
// expression (model.py:312-341, differentiated by autograd there; the reference's Triton
// layer, kernels.py:145-221, has no backward).
//
// With A = W2[:d] and B = W2[d:] (net.2.weight halves), pair p of token t(p) using unique
// expert s(p), c_p = h_s . xp_t, a_p = gelu(c_p) g_p and dY_t = dy_t / H, the per-pair part
// of the backward is, given xp = x A and dYB = dY B (both float32 [n_tok, d_hidden]):
//
//   da_p  = dYB_t . h_s                 (= dY_t . v_s with v_s = h_s B^T)
//   dg_p  = gelu(c_p) da_p
//   dc_p  = g_p gelu'(c_p) da_p
//   hacc_t = sum_p a_p h_s,   dxp_t = sum_p dc_p h_s                       (token sums)
//   dh_s  += a_p dYB_t + dc_p xp_t                                          (expert sums)
//
// Three kernels, all deterministic (every sum has a fixed order, no atomics):
//  1. expert_bwd_pairs_kernel: one wave per token walks its H k pairs (kBwdUnroll hidden
//     rows in flight), keeps xp_t, dYB_t and the token sums in registers, and stores each
//     pair's scalars (a_p, dc_p);
//  2. expert_bwd_sums_kernel: the expert sums over the sorted pairs (ethos_sort_segment's
//     permutation, each expert's pairs consecutive and in pair order), one wave per block
//     of kBwdBlock sorted positions, summing each segment's terms in sorted order: a
//     segment that lies in one block is written to dh; a segment crossing blocks leaves
//     its part in its first block (tail) and in each later block (head) as partial rows;
//  3. expert_bwd_join_kernel: each crossing segment's dh = its first block's tail part plus
//     the later blocks' head parts, in block order.
// The weight, input and latent gradients that follow are GEMMs.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_rows.hpp"

namespace ethos {

constexpr int kBwdUnroll = 8;

__device__ __forceinline__ float gelu_erf_grad(float x) {
    // Phi(x) + x phi(x)
    return 0.5f * erfcf(-x * 0.70710678118654752f) + x * expf(-0.5f * x * x) * 0.39894228040143268f;
}

constexpr int kBwdBlock = 64;  // sorted positions per block of the expert-sum pass

template <typename T, int CH>
__global__ __launch_bounds__(256) void expert_bwd_pairs_kernel(const T* __restrict__ hid, const float* __restrict__ xp,
                                                               const float* __restrict__ dyb,
                                                               const int32_t* __restrict__ pair_slot,
                                                               const T* __restrict__ gates, int64_t n_tok, int hk,
                                                               int dh, float* __restrict__ dg,
                                                               float* __restrict__ hacc, float* __restrict__ dxp,
                                                               float2* __restrict__ ac) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    for (int64_t t = wave_id; t < n_tok; t += n_waves) {
        float xr[CH * N], yr[CH * N], ha[CH * N], dx[CH * N];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
#pragma unroll
            for (int v = 0; v < N; ++v) {
                const bool in = e + v < dh;
                xr[c * N + v] = in ? xp[t * dh + e + v] : 0.0f;
                yr[c * N + v] = in ? dyb[t * dh + e + v] : 0.0f;
                ha[c * N + v] = 0.0f;
                dx[c * N + v] = 0.0f;
            }
        }
        const int64_t pbase = t * hk;
        for (int j0 = 0; j0 < hk; j0 += kBwdUnroll) {
            Raw hr[kBwdUnroll][CH];
            int sq[kBwdUnroll];
            // slots first, then every row with no branch between the loads (past the last pair
            // the last pair's row again, unused)
#pragma unroll
            for (int q = 0; q < kBwdUnroll; ++q) sq[q] = pair_slot[pbase + (j0 + q < hk ? j0 + q : hk - 1)];
#pragma unroll
            for (int q = 0; q < kBwdUnroll; ++q) load_raw_buf<T, CH>(hid + (int64_t)sq[q] * dh, dh, lane, hr[q]);
#pragma unroll
            for (int q = 0; q < kBwdUnroll; ++q) {
                if (j0 + q >= hk) continue;
                float hf[CH * N];
                float cp = 0.0f, dp = 0.0f;
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    Vec16<T>::unpack(hr[q][c], hf + c * N);
#pragma unroll
                    for (int v = 0; v < N; ++v) {
                        cp = __builtin_fmaf(hf[c * N + v], xr[c * N + v], cp);
                        dp = __builtin_fmaf(hf[c * N + v], yr[c * N + v], dp);
                    }
                }
                const float cdot = wave_sum(cp);
                const float da = wave_sum(dp);
                const int64_t p = pbase + j0 + q;
                const float g = Elem<T>::to_f32(gates[p]);
                const float act = gelu_erf(cdot);
                const float a = act * g;
                const float dc = g * gelu_erf_grad(cdot) * da;
                if (lane == 0) {
                    dg[p] = act * da;
                    ac[p] = make_float2(a, dc);
                }
#pragma unroll
                for (int c = 0; c < CH; ++c) {
#pragma unroll
                    for (int v = 0; v < N; ++v) {
                        ha[c * N + v] = __builtin_fmaf(a, hf[c * N + v], ha[c * N + v]);
                        dx[c * N + v] = __builtin_fmaf(dc, hf[c * N + v], dx[c * N + v]);
                    }
                }
            }
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e = c * 64 * N + lane * N;
            if (e < dh) {
#pragma unroll
                for (int v = 0; v < N; ++v) {
                    hacc[t * dh + e + v] = ha[c * N + v];
                    dxp[t * dh + e + v] = dx[c * N + v];
                }
            }
        }
    }
}

// Expert sums, one wave per block of kBwdBlock sorted positions: lane l holds columns
// 64 j + l (j < NB) of the running sum of the segment being walked, the positions are
// taken one at a time in sorted order (their pair, token and scalars loaded a lane each
// and broadcast), and a segment's sum is stored when the walk leaves it: to dh when the
// segment lies in the block, else as the block's head part (the segment that began
// before the block) or tail part (the segment that begins in the block and continues
// past it).
template <int NB>
__global__ __launch_bounds__(256) void expert_bwd_sums_kernel(const float* __restrict__ xp,
                                                              const float* __restrict__ dyb,
                                                              const int32_t* __restrict__ perm,
                                                              const int32_t* __restrict__ sorted_slot,
                                                              const int32_t* __restrict__ seg_off,
                                                              const float2* __restrict__ ac, int64_t n_pairs, int hk,
                                                              int dh, float* __restrict__ dhs,
                                                              float* __restrict__ head, float* __restrict__ tail) {
    const int lane = threadIdx.x & 63;
    const int64_t n_blocks = (n_pairs + kBwdBlock - 1) / kBwdBlock;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    for (int64_t blk = wave_id; blk < n_blocks; blk += n_waves) {
        const int64_t b0 = blk * kBwdBlock;
        const int cnt = (int)min((int64_t)kBwdBlock, n_pairs - b0);
        // this lane's position: pair, token, scalars, slot and segment bounds
        int my_t = 0, my_s = 0;
        float my_a = 0.0f, my_dc = 0.0f;
        int64_t my_beg = 0, my_end = 0;
        if (lane < cnt) {
            const int p = perm[b0 + lane];
            my_t = p / hk;
            const float2 v = ac[p];
            my_a = v.x;
            my_dc = v.y;
            my_s = sorted_slot[b0 + lane];
            my_beg = seg_off[my_s];
            my_end = seg_off[my_s + 1];
        }
        float acc[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = 0.0f;
        for (int i = 0; i < cnt; ++i) {
            const int t = __shfl(my_t, i, 64);
            const float a = __shfl(my_a, i, 64), dc = __shfl(my_dc, i, 64);
            const float* yr = dyb + (int64_t)t * dh;
            const float* xr = xp + (int64_t)t * dh;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int e = 64 * j + lane;
                if (e < dh) acc[j] = __builtin_fmaf(dc, xr[e], __builtin_fmaf(a, yr[e], acc[j]));
            }
            const int s = __shfl(my_s, i, 64);
            const bool last = i + 1 == cnt || __shfl(my_s, i + 1, 64) != s;
            if (last) {
                const int64_t beg = (int64_t)__shfl((int)my_beg, i, 64), end = (int64_t)__shfl((int)my_end, i, 64);
                float* dst = beg < b0 ? head + blk * dh : end > b0 + kBwdBlock ? tail + blk * dh : dhs + (int64_t)s * dh;
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int e = 64 * j + lane;
                    if (e < dh) dst[e] = acc[j];
                    acc[j] = 0.0f;
                }
            }
        }
    }
}

// dh of each segment that crosses blocks: found from its first block (the segment of the
// block's last position, when it began in the block and continues past it), summed over
// that block's tail part and the head parts of the blocks it continues into, in order.
template <int NB>
__global__ __launch_bounds__(256) void expert_bwd_join_kernel(const int32_t* __restrict__ sorted_slot,
                                                              const int32_t* __restrict__ seg_off, int64_t n_pairs,
                                                              int dh, const float* __restrict__ head,
                                                              const float* __restrict__ tail,
                                                              float* __restrict__ dhs) {
    const int lane = threadIdx.x & 63;
    const int64_t n_blocks = (n_pairs + kBwdBlock - 1) / kBwdBlock;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    for (int64_t blk = wave_id; blk < n_blocks; blk += n_waves) {
        const int64_t b0 = blk * kBwdBlock, last = b0 + kBwdBlock - 1;
        if (last >= n_pairs) continue;  // the final block has no segment continuing past it
        const int s = sorted_slot[last];
        const int64_t beg = seg_off[s], end = seg_off[s + 1];
        if (beg < b0 || end <= last + 1) continue;  // not a segment that begins here and crosses
        float acc[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int e = 64 * j + lane;
            acc[j] = e < dh ? tail[blk * dh + e] : 0.0f;
        }
        const int64_t b_end = (end - 1) / kBwdBlock;  // the segment's last block
        for (int64_t b = blk + 1; b <= b_end; ++b) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int e = 64 * j + lane;
                if (e < dh) acc[j] += head[b * dh + e];
            }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int e = 64 * j + lane;
            if (e < dh) dhs[(int64_t)s * dh + e] = acc[j];
        }
    }
}

size_t expert_backward_workspace_bytes(int64_t n_pairs, int dh) {
    const int64_t n_blocks = (n_pairs + kBwdBlock - 1) / kBwdBlock;
    return (size_t)n_pairs * sizeof(float2) + 2 * (size_t)n_blocks * dh * sizeof(float) + 256;
}

template <typename T, int CH>
static void launch_bwd_t(const void* hid, const float* xp, const float* dyb, const int32_t* pair_slot,
                         const void* gates, int64_t n_tok, int hk, int dh, float* dg, float* hacc, float* dxp,
                         float2* ac, int num_cus, hipStream_t stream) {
    int64_t g = (n_tok + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 16;
    g = g > cap ? cap : (g < 1 ? 1 : g);
    hipLaunchKernelGGL((expert_bwd_pairs_kernel<T, CH>), dim3((unsigned)g), dim3(256), 0, stream, (const T*)hid, xp,
                       dyb, pair_slot, (const T*)gates, n_tok, hk, dh, dg, hacc, dxp, ac);
}

template <int NB>
static void launch_sums_t(const float* xp, const float* dyb, const int32_t* perm, const int32_t* sorted_slot,
                          const int32_t* seg_off, const float2* ac, int64_t n_pairs, int hk, int dh, float* dhs,
                          float* head, float* tail, int num_cus, hipStream_t stream) {
    const int64_t n_blocks = (n_pairs + kBwdBlock - 1) / kBwdBlock;
    int64_t g = (n_blocks + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 16;
    g = g > cap ? cap : (g < 1 ? 1 : g);
    hipLaunchKernelGGL((expert_bwd_sums_kernel<NB>), dim3((unsigned)g), dim3(256), 0, stream, xp, dyb, perm,
                       sorted_slot, seg_off, ac, n_pairs, hk, dh, dhs, head, tail);
    hipLaunchKernelGGL((expert_bwd_join_kernel<NB>), dim3((unsigned)g), dim3(256), 0, stream, sorted_slot, seg_off,
                       n_pairs, dh, (const float*)head, (const float*)tail, dhs);
}

int launch_expert_backward(const void* hid, const float* xp, const float* dyb, const int32_t* pair_slot,
                           const int32_t* perm, const int32_t* sorted_slot, const int32_t* seg_off, const void* gates,
                           int64_t n_tok, int H, int k, int dh, int dtype, void* ws, float* dg, float* hacc,
                           float* dxp, float* dhs, int num_cus, hipStream_t stream) {
    const int c = apply_chunks(dh, dtype);
    const int64_t n_pairs = n_tok * H * k, n_blocks = (n_pairs + kBwdBlock - 1) / kBwdBlock;
    float2* ac = static_cast<float2*>(ws);
    float* head = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) +
                                           (((size_t)n_pairs * sizeof(float2) + 255) & ~(size_t)255));
    float* tail = head + (size_t)n_blocks * dh;
    bool done = false;
#define ETHOS_BWD_CASE(TT, C)                                                                                    \
    if (!done && c <= C) {                                                                                       \
        launch_bwd_t<TT, C>(hid, xp, dyb, pair_slot, gates, n_tok, H * k, dh, dg, hacc, dxp, ac, num_cus, stream); \
        done = true;                                                                                             \
    }
    if (dtype == kBF16) {
        ETHOS_BWD_CASE(uint16_t, 1)
        ETHOS_BWD_CASE(uint16_t, 2)
        ETHOS_BWD_CASE(uint16_t, 4)
        ETHOS_BWD_CASE(uint16_t, 8)
    } else {
        ETHOS_BWD_CASE(float, 1)
        ETHOS_BWD_CASE(float, 2)
        ETHOS_BWD_CASE(float, 4)
        ETHOS_BWD_CASE(float, 8)
    }
#undef ETHOS_BWD_CASE
    if (!done) return -1;
    const int nb = (dh + 63) / 64;
#define ETHOS_SUMS_CASE(NBC)                                                                                      \
    if (nb <= NBC) {                                                                                              \
        launch_sums_t<NBC>(xp, dyb, perm, sorted_slot, seg_off, ac, n_pairs, H * k, dh, dhs, head, tail, num_cus, \
                           stream);                                                                               \
        return (int)hipGetLastError();                                                                            \
    }
    ETHOS_SUMS_CASE(1) ETHOS_SUMS_CASE(2) ETHOS_SUMS_CASE(4) ETHOS_SUMS_CASE(8) ETHOS_SUMS_CASE(16)
    ETHOS_SUMS_CASE(32) ETHOS_SUMS_CASE(64)
#undef ETHOS_SUMS_CASE
    return -1;
}

}  // namespace ethos
