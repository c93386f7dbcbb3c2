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
// One wave per token walks its H k pairs (kBwdUnroll hidden rows in flight), keeps xp_t,
// dYB_t and the token sums in registers and adds each pair's expert term into dh with
// vector float atomics (the expert sums are therefore order-nondeterministic in float32,
// as a scatter-add is).  The weight, input and latent gradients that follow are GEMMs.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_rows.hpp"

namespace ethos {

constexpr int kBwdUnroll = 8;

__device__ __forceinline__ float gelu_erf_grad(float x) {
    // Phi(x) + x phi(x)
    return 0.5f * erfcf(-x * 0.70710678118654752f) + x * expf(-0.5f * x * x) * 0.39894228040143268f;
}

template <typename T, int CH>
__global__ __launch_bounds__(256) void expert_bwd_pairs_kernel(const T* __restrict__ hid, const float* __restrict__ xp,
                                                               const float* __restrict__ dyb,
                                                               const int32_t* __restrict__ pair_slot,
                                                               const T* __restrict__ gates, int64_t n_tok, int hk,
                                                               int dh, float* __restrict__ dg,
                                                               float* __restrict__ hacc, float* __restrict__ dxp,
                                                               float* __restrict__ dhs) {
    constexpr int N = Vec16<T>::kN;
    typedef typename Vec16<T>::raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t wave_id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t n_waves = (int64_t)gridDim.x * 4;
    constexpr int NB = CH * N;  // elements per lane (lane-major layout for the expert sums)
    for (int64_t t = wave_id; t < n_tok; t += n_waves) {
        float xr[CH * N], yr[CH * N], ha[CH * N], dx[CH * N];
        // xp_t and dyb_t again with element e = 64 j + lane, so that each expert-sum atomic
        // instruction covers 64 consecutive floats (two cache lines)
        float xb[NB], yb[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int e = 64 * j + lane;
            xb[j] = e < dh ? xp[t * dh + e] : 0.0f;
            yb[j] = e < dh ? dyb[t * dh + e] : 0.0f;
        }
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
#pragma unroll
            for (int q = 0; q < kBwdUnroll; ++q) {
                sq[q] = 0;
                if (j0 + q < hk) {
                    sq[q] = pair_slot[pbase + j0 + q];
                    load_raw<T, CH>(hid + (int64_t)sq[q] * dh, dh, lane, hr[q]);
                }
            }
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
                if (lane == 0) dg[p] = act * da;
#pragma unroll
                for (int c = 0; c < CH; ++c) {
#pragma unroll
                    for (int v = 0; v < N; ++v) {
                        ha[c * N + v] = __builtin_fmaf(a, hf[c * N + v], ha[c * N + v]);
                        dx[c * N + v] = __builtin_fmaf(dc, hf[c * N + v], dx[c * N + v]);
                    }
                }
                float* drow = dhs + (int64_t)sq[q] * dh;
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    if (64 * j + lane < dh) unsafeAtomicAdd(drow + 64 * j + lane, a * yb[j] + dc * xb[j]);
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

template <typename T, int CH>
static void launch_bwd_t(const void* hid, const float* xp, const float* dyb, const int32_t* pair_slot,
                         const void* gates, int64_t n_tok, int hk, int dh, float* dg, float* hacc, float* dxp,
                         float* dhs, int num_cus, hipStream_t stream) {
    int64_t g = (n_tok + 3) / 4;
    const int64_t cap = (int64_t)num_cus * 16;
    g = g > cap ? cap : (g < 1 ? 1 : g);
    hipLaunchKernelGGL((expert_bwd_pairs_kernel<T, CH>), dim3((unsigned)g), dim3(256), 0, stream, (const T*)hid, xp,
                       dyb, pair_slot, (const T*)gates, n_tok, hk, dh, dg, hacc, dxp, dhs);
}

int launch_expert_backward(const void* hid, const float* xp, const float* dyb, const int32_t* pair_slot,
                           const void* gates, int64_t n_tok, int H, int k, int dh, int dtype, float* dg, float* hacc,
                           float* dxp, float* dhs, int num_cus, hipStream_t stream) {
    const int c = apply_chunks(dh, dtype);
#define ETHOS_BWD_CASE(TT, C)                                                                                    \
    if (c <= C) {                                                                                                \
        launch_bwd_t<TT, C>(hid, xp, dyb, pair_slot, gates, n_tok, H * k, dh, dg, hacc, dxp, dhs, num_cus, stream); \
        return (int)hipGetLastError();                                                                           \
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
    return -1;
}

}  // namespace ethos
