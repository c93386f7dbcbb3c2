// Expert generation over the unique-expert set: [u_e ; v_e] = W2 gelu(W1 z_e)
// (reference: ExpertGenerationNetwork, model.py:168-179; the weights are read
// directly at model.py:297-300 and applied per pair at model.py:320-332 -- here
// each unique expert is generated once).
//
//   z   = latents[uniq[u]]                      gathered rows  [U, dl]
//   pre = RN_T(z W1^T)      (fp32 MFMA accumulation)          [U, dh]
//   hid = RN_T(gelu_erf(pre))                                  [U, dh]   (LDS only)
//   uv  = RN_T(hid W2^T)                                       [U, 2 d]  u = first d, v = last d
//
// One workgroup (4 waves) owns a tile of experts; the latent tile and the hidden
// tile live in LDS.  Wave w computes 32-column blocks w*4.., w*4+16.. of each GEMM
// with 32x32 MFMA tiles (bf16: v_mfma_f32_32x32x16_bf16, fp32: v_mfma_f32_32x32x2f32).
// The number of unique experts U is read on the device: the grid is sized for the
// maximum and tiles past U are skipped, so no host synchronisation is needed.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_mfma.hpp"

namespace ethos {

template <typename T> struct GenTile;
template <> struct GenTile<uint16_t> { static constexpr int kRows = 64; };  // experts per tile
template <> struct GenTile<float> { static constexpr int kRows = 32; };

constexpr int kGenPad = 8;  // LDS row padding (elements)

template <typename T>
__global__ __launch_bounds__(256) void generate_kernel(const T* __restrict__ latents, int64_t n_experts,
                                                       const int32_t* __restrict__ uniq,
                                                       const int32_t* __restrict__ n_unique, const T* __restrict__ w1,
                                                       const T* __restrict__ w2, int dl, int dh, int d2,
                                                       T* __restrict__ uv) {
    using M = Mfma<T>;
    constexpr int R = GenTile<T>::kRows;
    constexpr int RB = R / 32;
    extern __shared__ __align__(16) unsigned char smem[];
    const int zp = dl + kGenPad, hp = dh + kGenPad;
    T* zs = reinterpret_cast<T*>(smem);
    T* hs = zs + R * zp;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lrow = lane & 31, lk = (lane >> 5) * M::kKL;
    const int U = *n_unique;
    const int n_tiles = (U + R - 1) / R;
    const int nb1 = dh / 32, nb2 = d2 / 32;

    for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int u0 = tile * R;
        __syncthreads();
        for (int e = tid; e < R * dl; e += 256) {
            const int r = e / dl, k = e - r * dl;
            const int u = u0 + r;
            T v = T(0);
            if (u < U) {
                const int64_t id = uniq[u];
                if (id >= 0 && id < n_experts) v = latents[id * dl + k];
            }
            zs[r * zp + k] = v;
        }
        __syncthreads();

        // GEMM1 + GELU -> hidden tile in LDS
        for (int g = wave * 4; g < nb1; g += 16) {
            f32x16_t acc[RB][4];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.0f;
            for (int k0 = 0; k0 < dl; k0 += M::kK) {
                typename M::frag a[RB];
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) a[rb] = M::load(zs + (rb * 32 + lrow) * zp + k0 + lk);
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    if (g + cb < nb1) {
                        const typename M::frag b = M::load(w1 + (int64_t)((g + cb) * 32 + lrow) * dl + k0 + lk);
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb) acc[rb][cb] = M::mma(a[rb], b, acc[rb][cb]);
                    }
                }
            }
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                if (g + cb >= nb1) continue;
                const int col = (g + cb) * 32 + lrow;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int row = rb * 32 + mfma32_row(i, lane);
                        const float pre = Elem<T>::round32(acc[rb][cb][i]);
                        hs[row * hp + col] = Elem<T>::from_f32(gelu_erf(pre));
                    }
            }
        }
        __syncthreads();

        // GEMM2 -> [u ; v] rows
        for (int g = wave * 4; g < nb2; g += 16) {
            f32x16_t acc[RB][4];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.0f;
            for (int k0 = 0; k0 < dh; k0 += M::kK) {
                typename M::frag a[RB];
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) a[rb] = M::load(hs + (rb * 32 + lrow) * hp + k0 + lk);
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    if (g + cb < nb2) {
                        const typename M::frag b = M::load(w2 + (int64_t)((g + cb) * 32 + lrow) * dh + k0 + lk);
#pragma unroll
                        for (int rb = 0; rb < RB; ++rb) acc[rb][cb] = M::mma(a[rb], b, acc[rb][cb]);
                    }
                }
            }
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                if (g + cb >= nb2) continue;
                const int col = (g + cb) * 32 + lrow;
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int u = u0 + rb * 32 + mfma32_row(i, lane);
                        if (u < U) uv[(int64_t)u * d2 + col] = Elem<T>::from_f32(acc[rb][cb][i]);
                    }
            }
        }
    }
}

template <typename T>
static size_t gen_smem(int dl, int dh) {
    return (size_t)GenTile<T>::kRows * ((dl + kGenPad) + (dh + kGenPad)) * sizeof(T);
}

size_t generate_smem_bytes(int dl, int dh, int dtype) {
    return dtype == kBF16 ? gen_smem<uint16_t>(dl, dh) : gen_smem<float>(dl, dh);
}

int launch_generate(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                    int64_t max_unique, const void* w1, const void* w2, int dl, int dh, int d2, int dtype, void* uv,
                    int num_cus, hipStream_t stream) {
    const int R = dtype == kBF16 ? GenTile<uint16_t>::kRows : GenTile<float>::kRows;
    int64_t tiles = (max_unique + R - 1) / R;
    int64_t cap = (int64_t)num_cus * 2;
    const unsigned grid = (unsigned)(tiles < cap ? (tiles > 0 ? tiles : 1) : cap);
    const size_t smem = generate_smem_bytes(dl, dh, dtype);
    if (dtype == kBF16)
        hipLaunchKernelGGL(generate_kernel<uint16_t>, dim3(grid), dim3(256), smem, stream, (const uint16_t*)latents,
                           n_experts, uniq, n_unique, (const uint16_t*)w1, (const uint16_t*)w2, dl, dh, d2,
                           (uint16_t*)uv);
    else
        hipLaunchKernelGGL(generate_kernel<float>, dim3(grid), dim3(256), smem, stream, (const float*)latents,
                           n_experts, uniq, n_unique, (const float*)w1, (const float*)w2, dl, dh, d2, (float*)uv);
    return (int)hipGetLastError();
}

}  // namespace ethos
