// Expert generation over the unique-expert set (reference: ExpertGenerationNetwork,
// model.py:168-179; the weights are read directly at model.py:297-300 and applied per
// pair at model.py:320-332 -- here each unique expert is generated once).
//
//   z   = latents[uniq[u]]                      gathered rows  [U, dl]
//   pre = RN_T(z W1^T)      (fp32 MFMA accumulation)          [U, dh]
//   h   = RN_T(gelu_erf(pre))                                  [U, dh]   h_i of model.py:323
//   v   = RN_T(h W_v^T)                                        [U, d]    h_i @ W_v of model.py:332
//
// W_v^T is rows d .. 2d-1 of net.2.weight ([2d, dh]); the first d rows (W_u^T) are not
// used here: the reference contracts them with the token (x_proj = x W_u, model.py:326),
// which the apply stage does once per token.
//
// One workgroup (4 waves) owns a tile of experts; the latent tile and the hidden
// tile live in LDS.  Wave w computes 32-column blocks w*4.., w*4+16.. of each GEMM
// with 32x32 MFMA tiles (bf16: v_mfma_f32_32x32x16_bf16, fp32: v_mfma_f32_32x32x2f32).
// The number of unique experts U is read on the device: the grid is sized for the
// maximum and tiles past U are skipped, so no host synchronisation is needed.
#include "ethos_common.hpp"
#include "ethos_launch.hpp"
#include "ethos_mfma.hpp"
#include "ethos_rows.hpp"
#include "ethos_act.hpp"

namespace ethos {

template <typename T> struct GenTile;
template <> struct GenTile<uint16_t> { static constexpr int kRows = 64; };  // experts per tile
template <> struct GenTile<float> { static constexpr int kRows = 32; };

constexpr int kGenPad = 8;  // LDS row padding (elements)

template <typename T>
__global__ __launch_bounds__(256) void generate_kernel(const T* __restrict__ latents, int64_t n_experts,
                                                       const int32_t* __restrict__ uniq,
                                                       const int32_t* __restrict__ n_unique, int64_t max_unique,
                                                       const T* __restrict__ w1, const T* __restrict__ w2, int dl,
                                                       int dh, int d2, T* __restrict__ hout, T* __restrict__ uv) {
    using M = Mfma<T>;
    constexpr int R = GenTile<T>::kRows;
    constexpr int RB = R / 32;
    extern __shared__ __align__(16) unsigned char smem[];
    const int zp = dl + kGenPad, hp = dh + kGenPad;
    T* zs = reinterpret_cast<T*>(smem);
    T* hs = zs + R * zp;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lrow = lane & 31, lk = (lane >> 5) * M::kKL;
    // uniq, h and v hold max_unique rows
    const int U = (int)((int64_t)*n_unique < max_unique ? (int64_t)*n_unique : max_unique);
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
                        const T hv = Elem<T>::from_f32(gelu_erf(pre));
                        hs[row * hp + col] = hv;
                        if (u0 + row < U) hout[(int64_t)(u0 + row) * dh + col] = hv;
                    }
            }
        }
        __syncthreads();

        // GEMM2 -> v rows
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

// ---------------------------------------------------------------------------------
// bf16 generator for the common shapes (d_latent 128, d_hidden 256 or 512), two kernels:
// hidden_ws_bf16_kernel writes h (GEMM1 + GELU, VALU heavy) and an expand kernel reads it
// back for v = h W_v^T (MFMA bound): expand_ws_bf16_kernel (W_v-stationary) when d_model
// splits into 256-column groups, else expand_bf16_kernel (one wave per SIMD holding 64
// experts' hidden rows).
// ---------------------------------------------------------------------------------
constexpr int kG2Waves = 4;
constexpr int kG2MB = 2;                          // expert blocks of 32 per wave
constexpr int kG2Cols = 64;                       // output columns per staged W2 chunk
constexpr int kG2Rows = kG2Waves * kG2MB * 32;    // experts per tile

__device__ __forceinline__ bf16x8_t pack_bf16x8(const float* v) {
    uint4 r;
    r.x = pack_bf16x2(v[0], v[1]);
    r.y = pack_bf16x2(v[2], v[3]);
    r.z = pack_bf16x2(v[4], v[5]);
    r.w = pack_bf16x2(v[6], v[7]);
    return __builtin_bit_cast(bf16x8_t, r);
}

// The GELU table (gelu_bf16_lut.inc): the correctly rounded erf-form GELU of the bf16
// inputs that are not a closed form.
__device__ const uint16_t kGeluLut[kGeluLutSize] = {
#include "gelu_bf16_lut.inc"
};

// ---------------------------------------------------------------------------------
// Hidden rows, bf16, W1-stationary (the form of expand_ws_bf16_kernel applied to GEMM1):
// h = RN(gelu(RN(z W1^T))).  Each wave owns 64 hidden units for the whole launch, its W1
// rows in AGPRs (64 registers, loaded once); the latent rows of 64 unique experts at a
// time are gathered global -> LDS by buffer_load ... lds one tile ahead (double buffered;
// row r's 16-byte piece p at slot p ^ (r % 16), so fragment reads are conflict-free) and
// each fragment read feeds two MFMAs.  The unique ids of all of a workgroup's tiles are
// copied to LDS once at the start, so the loop issues no id loads.  GELU comes from the
// table in LDS; the rows leave through a per-wave staging area as whole 128-byte lines.
// The products are A = W1 rows, B = latent rows, k-steps in order, fp32 accumulation.
// ---------------------------------------------------------------------------------
constexpr int kHsRows = 64;       // experts per tile
constexpr int kHsMaxTiles = 32;   // tiles per workgroup whose ids fit the LDS id table
static_assert(kHsRows == kActTileRows, "activation tiles are the hidden-row tiles");

template <int DL, int DH, bool kAct>
__global__ __launch_bounds__(DH) void hidden_ws_bf16_kernel(const uint16_t* __restrict__ latents, int64_t n_experts,
                                                            const int32_t* __restrict__ uniq,
                                                            const int32_t* __restrict__ n_unique, int64_t max_unique,
                                                            const uint16_t* __restrict__ w1,
                                                            uint16_t* __restrict__ hout, HiddenActArgs A) {
    constexpr int kWaves = DH / 64;
    constexpr int KS1 = DL / 16;                 // k-steps
    constexpr int PPR = DL / 8;                  // 16-byte pieces per latent row
    constexpr int kCopies = kHsRows * PPR / 64;  // copy instructions per tile
    constexpr int kCW = kCopies / kWaves;        // per wave
    constexpr int kNSt = 8;                      // h-row stores per wave and tile
    constexpr int LA = 2;                        // fragment reads run LA k-steps ahead
    static_assert(PPR == 16 && kCopies % kWaves == 0 && KS1 >= kNSt && KS1 > LA, "latent tile shape");
    __shared__ __align__(16) f32x2_t gmc[kGeluMcSize];
    __shared__ uint4 zs[2][kHsRows * PPR];
    __shared__ u32x4_t stg[kWaves][kHsRows * 8];
    __shared__ int32_t ids_s[kHsMaxTiles][kHsRows];
    __shared__ float dsm[kAct ? kWaves : 1][64];  // per-wave dot products of the activations

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int U = (int)((int64_t)*n_unique < max_unique ? (int64_t)*n_unique : max_unique);
    const int n_tiles = (U + kHsRows - 1) / kHsRows;
    const int G = gridDim.x;
    const int hid0 = wave * 64;
    // activations here unless the token order applies (few hidden-row bytes)
    const bool act_on = kAct && (int64_t)U * DH * (int64_t)sizeof(uint16_t) > kActTokenOrderMaxHBytes;

    // the GELU table and this workgroup's tile ids (-1 past U or for ids outside the table);
    // every value is requested before any is used (positions past the end read a valid
    // element, unused), so the loads share one round trip
    {
        constexpr int kGIt = (kGeluMcSize + DH - 1) / DH, kIIt = kHsMaxTiles * kHsRows / DH;
        static_assert(kHsMaxTiles * kHsRows % DH == 0, "id table loop");
        uint16_t gv[kGIt];
        int iv[kIIt];
#pragma unroll
        for (int it = 0; it < kGIt; ++it) {
            const int e = tid + it * DH;
            gv[it] = kGeluLut[gelu_mc_lut_index(e < kGeluMcSize ? e : 0)];
        }
#pragma unroll
        for (int it = 0; it < kIIt; ++it) {
            const int e = tid + it * DH, i = e / kHsRows, r = e % kHsRows;
            const int64_t u = ((int64_t)blockIdx.x + (int64_t)i * G) * kHsRows + r;
            iv[it] = U > 0 ? uniq[u < U ? u : 0] : -1;  // (no unique expert: nothing to read)
        }
#pragma unroll
        for (int it = 0; it < kGIt; ++it) {
            const int e = tid + it * DH;
            if (e < kGeluMcSize) gmc[e] = gelu_mc_entry_from(e, gv[it]);
        }
#pragma unroll
        for (int it = 0; it < kIIt; ++it) {
            const int e = tid + it * DH, i = e / kHsRows, r = e % kHsRows;
            const int64_t u = ((int64_t)blockIdx.x + (int64_t)i * G) * kHsRows + r;
            const int v = iv[it];
            ids_s[i][r] = u < U && v >= 0 && v < n_experts ? v : -1;
        }
    }
    const uint32_t mc_bytes = lds_addr(gmc);
    // the wave's W1 rows: A fragment (cb, s) = W1[hid0 + 32 cb + l32][16 s + 8 h ..]
    bf16x8_t wf[2][KS1];
    {
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(w1), (short)0, DH * DL * (int)sizeof(uint16_t), 0x00020000);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int s = 0; s < KS1; ++s)
                wf[cb][s] = __builtin_bit_cast(
                    bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                  wr, ((hid0 + 32 * cb + l32) * DL + 16 * s + 8 * h) * (int)sizeof(uint16_t), 0, 0));
    }
    // latent rows: the whole table as one descriptor (the launch checks its size); absent
    // rows take an offset past it and read as zero
    const i32x4_t zr = buffer_rsrc(latents, (uint32_t)(n_experts * DL * (int64_t)sizeof(uint16_t)));
    constexpr int kZOOB = 0x7ffffff0;
    // copy instruction j = it * kWaves + wave of a tile moves rows 4 j .. 4 j + 3: lane i
    // takes row 4 j + i / 16, LDS slot i % 16, global piece (i % 16) ^ (row % 16)
    auto copy = [&](int i_tile, int buf) {
#pragma unroll
        for (int it = 0; it < kCW; ++it) {
            const int j = it * kWaves + wave;
            const int r = 4 * j + (lane >> 4), sl = lane & 15;
            const int id = ids_s[i_tile][r];
            const int voff = id >= 0 ? (id * DL + 8 * (sl ^ (r & 15))) * (int)sizeof(uint16_t) : kZOOB;
            lds_dma16_nt(zr, voff, 0, lds_addr(&zs[buf][64 * j]));  // each latent row is read once
        }
    };
    // B fragment (mb, s): row 32 mb + l32, piece 2 s + h, at slot (2 s + h) ^ (l32 % 16)
    const int zb_off = l32 * PPR;
    const int st_voff = ((lane >> 3) * DH + hid0 + 8 * (lane & 7)) * (int)sizeof(uint16_t);
    constexpr int kOOB = 0x40000000;
    u32x4_t* my = stg[wave];
    u32x2_t* my2 = reinterpret_cast<u32x2_t*>(my);
    constexpr int kWaitVm8 = 0x0f78;  // s_waitcnt vmcnt(8)
    constexpr int kWaitVm0 = 0x0f70;  // s_waitcnt vmcnt(0)

    __syncthreads();  // table and ids in place
    if ((int)blockIdx.x < n_tiles) copy(0, 0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // W1 rows and the first tile

    __amdgpu_buffer_rsrc_t hr_prev = __builtin_amdgcn_make_buffer_rsrc(hout, (short)0, 0, 0x00020000);
    bool have_prev = false;
    // seg_off bounds of tile t: loaded one tile ahead (tile t is clamped to the last tile)
    auto seg_bounds = [&](int64_t t, int32_t& b0, int32_t& b1) {
        const int64_t tc = t < n_tiles ? t : n_tiles - 1;
        const int64_t r0 = tc * kHsRows;
        b0 = A.seg_off[r0];
        b1 = A.seg_off[r0 + (U - (int)r0 < kHsRows ? U - (int)r0 : kHsRows)];
    };
    int32_t nb0 = 0, nb1 = 0;
    if constexpr (kAct) {
        if (act_on && (int)blockIdx.x < n_tiles) seg_bounds(blockIdx.x, nb0, nb1);
    }
    int i = 0;
    for (int64_t t = blockIdx.x; t < n_tiles; t += G, ++i) {
        __builtin_amdgcn_s_waitcnt(kWaitVm8);  // this tile's rows have landed
        __syncthreads();
        const int64_t row0 = t * kHsRows;
        const int live = U - (int)row0 < kHsRows ? U - (int)row0 : kHsRows;
        ActMeta meta{};
        if constexpr (kAct) {
            if (act_on) {
                const int32_t b0 = __builtin_amdgcn_readfirstlane(nb0), b1 = __builtin_amdgcn_readfirstlane(nb1);
                seg_bounds(t + G, nb0, nb1);
                meta = act_meta<kWaves>(A, row0, b0, b1, wave, lane);
            }
        }
        u32x4_t outv[kNSt];
#pragma unroll
        for (int k = 0; k < kNSt; ++k) {
            const int r = 8 * k + (lane >> 3);
            outv[k] = my[r * 8 + ((lane & 7) ^ (r & 7))];
        }
        const int st_base = have_prev ? st_voff : kOOB;
        if (t + G < n_tiles) copy(i + 1, (i + 1) & 1);
        const uint4* cur = zs[i & 1];
        auto bfrag = [&](int s, int mb) {
            return __builtin_bit_cast(bf16x8_t, cur[zb_off + mb * 32 * PPR + ((2 * s + h) ^ (l32 & 15))]);
        };
        bf16x8_t bfr[LA + 1][2];
        f32x16_t acc[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) acc[mb][cb] = f32x16_zero();
#pragma unroll
        for (int s = 0; s < LA; ++s)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) bfr[s][mb] = bfrag(s, mb);
#pragma unroll
        for (int s = 0; s < KS1; ++s) {
            if (s + LA < KS1) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) bfr[(s + LA) % (LA + 1)][mb] = bfrag(s + LA, mb);
            }
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) asm volatile("" : "+a"(wf[cb][s]));
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    acc[mb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[cb][s], bfr[s % (LA + 1)][mb],
                                                                         acc[mb][cb], 0, 0, 0);
            // the previous tile's rows, one store per k-step (after this tile's copies)
            if (s < kNSt)
                __builtin_amdgcn_raw_buffer_store_b128(outv[s], hr_prev, st_base + s * 8 * DH * 2, 0, 0);
        }
        // acc[mb][cb][i]: hidden unit hid0 + 32 cb + 8 (i/4) + 4h + i%4 of expert 32 mb + l32,
        // i.e. 8-byte half h of 16-byte piece 4 cb + i/4 of staged row 32 mb + l32
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int r = mb * 32 + l32;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4) {
                    const int q = 4 * cb + a4;
                    my2[r * 16 + (q ^ (r & 7)) * 2 + h] = u32x2_t{
                        gelu_bf16x2_mc(pack_bf16x2(acc[mb][cb][4 * a4], acc[mb][cb][4 * a4 + 1]), mc_bytes),
                        gelu_bf16x2_mc(pack_bf16x2(acc[mb][cb][4 * a4 + 2], acc[mb][cb][4 * a4 + 3]), mc_bytes)};
                }
        }
        hr_prev = __builtin_amdgcn_make_buffer_rsrc(hout + row0 * DH, (short)0, live * DH * (int)sizeof(uint16_t),
                                                    0x00020000);
        have_prev = true;
        if constexpr (kAct) {
            if (act_on) {
                // every wave's rows of this tile are staged; the next tile's staging writes
                // wait for the barrier at the top of the next iteration
                __syncthreads();
                // piece part + 8 i of staged row sl is 16-byte group `part` of wave area i
                auto piece = [&](int sl, int part, int i) {
                    return __builtin_bit_cast(uint4, stg[i][sl * 8 + (part ^ (sl & 7))]);
                };
                tile_activations<DH, kWaves, kHsRows>(A, piece, dsm[wave], row0, meta, wave, lane);
            }
        }
    }
    if (have_prev) {
#pragma unroll
        for (int k = 0; k < kNSt; ++k) {
            const int r = 8 * k + (lane >> 3);
            __builtin_amdgcn_raw_buffer_store_b128(my[r * 8 + ((lane & 7) ^ (r & 7))], hr_prev,
                                                   st_voff + k * 8 * DH * 2, 0, 0);
        }
    }
}

// ---------------------------------------------------------------------------------
// v rows, bf16: v = RN(h W_v^T) over tiles of 256 experts, one workgroup of 4 waves per
// CU, 64 experts (two blocks of 32) per wave.  The wave's hidden rows (64 x DH bf16,
// 256 registers per lane) are loaded into AGPRs, which the MFMAs read directly; every
// W2 fragment read from LDS feeds two MFMAs (one per expert block).  The product is
// computed transposed, v^T = W_v . h^T, over chunks of 64 output columns: the chunk's
// 64 rows of W_v are copied global -> LDS (double buffered) and each lane owns, per
// expert block, one expert and eight groups of four consecutive output columns of the
// chunk.  Results go through a per-wave LDS staging area and are stored one chunk
// later as whole 128-byte lines.
// ---------------------------------------------------------------------------------
template <int DH>
__global__ __launch_bounds__(kG2Waves * 64) __attribute__((amdgpu_waves_per_eu(1, 1))) void expand_bf16_kernel(
    const int32_t* __restrict__ n_unique, int64_t max_unique, const uint16_t* __restrict__ hin,
    const uint16_t* __restrict__ w2, int d2, uint16_t* __restrict__ uv) {
    constexpr int KS2 = DH / 16;                  // k-steps
    constexpr int GPR = DH / 8;                   // 16-byte groups per W2 row
    constexpr int kCopies = GPR * kG2Cols / 64;   // 64-lane copy instructions per chunk
    static_assert(GPR % 8 == 0 && kCopies % kG2Waves == 0 && KS2 % 4 == 0, "chunk staging shape");
    // W2 chunks, double buffered, swizzled (see w2_voff)
    __shared__ uint4 bs[2][GPR * kG2Cols];
    // Output staging, per wave: 64 experts x 64 columns of bf16; expert r's 128-byte
    // row holds its 16-byte group q at slot q ^ (r % 8).
    __shared__ u32x4_t stg[kG2Waves][kG2MB * 32 * 8];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int U = (int)((int64_t)*n_unique < max_unique ? (int64_t)*n_unique : max_unique);
    const int n_tiles = (U + kG2Rows - 1) / kG2Rows;
    const int n_chunks = d2 / kG2Cols;
    // W2 as a buffer resource (raw, byte-addressed; loads beyond its size return 0)
    const i32x4_t w2r = buffer_rsrc(w2, (uint32_t)d2 * DH * (uint32_t)sizeof(uint16_t));
    // Copy instruction i = wave + 4 it of a chunk moves eight whole 128-byte lines: rows
    // 8 (i % 8) + j / 8 = 8 wave + 32 (it % 2) + j / 8 of the chunk, line i / 8 = it / 2.
    // Lane j lands at bs[buf][64 i + j] and carries 16-byte group
    // x = (j % 8) ^ (j / 8) ^ (i % 2) of its line, so that the B-fragment reads (one
    // group, 16 consecutive rows) hit 16 distinct bank groups.
    const int w2_voff = ((8 * wave + (lane >> 3)) * DH + 8 * ((lane & 7) ^ (lane >> 3) ^ (wave & 1))) * 2;
    // W2 row (output column) r = 32 cb + l32 of a chunk, group g = 2 s + h, sits at
    // 64 (8 (g / 8) + r / 8) + 8 (r % 8) + ((g % 8) ^ (r % 8) ^ (r / 8 % 2)); only s % 4
    // changes the last term, so four lane bases cover every k-step.
    int bq_off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        bq_off[q] = (l32 >> 3) * 64 + (l32 & 7) * 8 + ((2 * q + h) ^ (l32 & 7) ^ ((l32 >> 3) & 1));

    // Work units: tiles that fill whole rounds of the grid are done whole; the
    // remaining rem tiles are split by column range into parts so that the last round
    // spreads over the grid (each part loads the tile's hidden rows).
    const int G = gridDim.x;
    const int n_full = n_tiles - n_tiles % G;
    const int rem = n_tiles - n_full;
    int parts = rem > 0 ? G / rem : 1;
    parts = parts < 1 ? 1 : (parts > n_chunks ? n_chunks : parts);
    const int cpp = (n_chunks + parts - 1) / parts;  // chunks per part
    const int n_units = n_full + rem * parts;
    constexpr int kOOB = 0x40000000;  // a byte offset past any tile's rows (and kOOB + 56 d2 * 2 < 2^31)

    for (int w = blockIdx.x; w < n_units; w += G) {
        int tile = w, c_begin = 0, c_end = n_chunks;
        if (w >= n_full) {
            tile = n_full + (w - n_full) / parts;
            c_begin = ((w - n_full) % parts) * cpp;
            c_end = c_begin + cpp < n_chunks ? c_begin + cpp : n_chunks;
            if (c_begin >= c_end) continue;
        }
        // copy instruction it of chunk c into buffer buf
        auto copy = [&](int c, int buf, int it) {
            const int soff = ((c * kG2Cols + 32 * (it & 1)) * DH + 64 * (it >> 1)) * 2;
            lds_dma16(w2r, w2_voff, soff, lds_addr(&bs[buf][(wave + it * kG2Waves) * 64]));
        };
#pragma unroll
        for (int it = 0; it < kCopies / kG2Waves; ++it) copy(c_begin, c_begin & 1, it);

        // the wave's hidden rows, k-slot s of expert block mb = h[u][16 s + 8 h ..] with
        // u = 64 wave + 32 mb + l32 (rows at or past U read as zero)
        const int64_t row0 = (int64_t)tile * kG2Rows;
        const int64_t live = U - row0;
        const int h_rows = live < kG2Rows ? (int)(live > 0 ? live : 0) : kG2Rows;
        const __amdgpu_buffer_rsrc_t hrd = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(hin) + row0 * DH, (short)0, h_rows * DH * (int)sizeof(uint16_t), 0x00020000);
        bf16x8_t hf[kG2MB][KS2];
#pragma unroll
        for (int mb = 0; mb < kG2MB; ++mb)
#pragma unroll
            for (int s = 0; s < KS2; ++s)
                hf[mb][s] = __builtin_bit_cast(
                    bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                  hrd, ((wave * kG2MB * 32 + mb * 32 + l32) * DH + 16 * s + 8 * h) * 2, 0, 0));
        const int64_t rows_left = max_unique - row0;
        const int tile_rows = rows_left < kG2Rows ? (int)(rows_left > 0 ? rows_left : 0) : kG2Rows;

        // GEMM2^T.  Each chunk's results go to the wave's staging rows; they are read
        // back at the start of the next chunk and stored between its MFMAs as whole
        // 128-byte lines with non-temporal stores (the v stream must not evict W2 from
        // L2).  The stores go through a buffer resource covering this tile's rows below
        // max_unique, so rows past the allocation are dropped by the hardware and no
        // store needs a branch; rows in [U, max_unique) receive the rows of absent
        // experts.
        //
        // Within a chunk the copies of the next chunk (k-steps 0 .. kCS-1) are issued
        // before its eight stores, so the next chunk only waits for vmcnt(8): its copies
        // have landed, the stores stay in flight across the boundary.  The first chunk
        // waits the same way: the 64 hidden-row loads follow its copies (and the MFMAs
        // wait for each of those loads themselves).
        const __amdgpu_buffer_rsrc_t uvr = __builtin_amdgcn_make_buffer_rsrc(
            uv + row0 * d2, (short)0, tile_rows * d2 * (int)sizeof(uint16_t), 0x00020000);
        // lane's store k covers row 8 k + lane / 8 of the wave, 16-byte group lane % 8
        const int st_voff = ((wave * kG2MB * 32 + (lane >> 3)) * d2 + 8 * (lane & 7)) * 2;
        u32x4_t* my = stg[wave];
        u32x2_t* my2 = reinterpret_cast<u32x2_t*>(my);
        // B fragments run LA k-steps ahead of the MFMAs in a ring of LA + 1 slots.
        constexpr int LA = 4;
        constexpr int kCopiesW = kCopies / kG2Waves;  // copies per wave, 4 per k-step
        constexpr int kCS = kCopiesW / 4;             // k-steps that issue copies
        constexpr int kNSt = kG2MB * 4;               // v-row stores per chunk
        static_assert(kCopiesW % 4 == 0 && kCS + kNSt <= KS2 && kG2MB * KS2 >= kNSt, "interleave shape");
        // s_waitcnt vmcnt(8) (gfx9 immediate: vmcnt [3:0] and [15:14], expcnt [6:4],
        // lgkmcnt [11:8]; expcnt 7 and lgkmcnt 15 do not wait)
        constexpr int kWaitVm8 = 0x0f78;
        static_assert(kNSt == 8, "kWaitVm8 assumes eight stores after the copies");
        int pend_c = -1;
        for (int c = c_begin; c < c_end; ++c) {
            __builtin_amdgcn_s_waitcnt(kWaitVm8);
            __syncthreads();
            // the previous chunk's staged rows
            u32x4_t outv[kNSt];
#pragma unroll
            for (int k = 0; k < kNSt; ++k) {
                const int r = 8 * k + (lane >> 3);
                outv[k] = my[r * 8 + ((lane & 7) ^ (r & 7))];
            }
            const int st_base = pend_c >= 0 ? st_voff + kG2Cols * 2 * pend_c : kOOB;
            const uint4* cur = bs[c & 1];
            auto bfrag = [&](int s, int cb) {
                return __builtin_bit_cast(bf16x8_t, cur[bq_off[s & 3] + (s >> 2) * 512 + cb * 256]);
            };
            bf16x8_t bfr[LA + 1][2];
            f32x16_t acc[kG2MB][2];
#pragma unroll
            for (int mb = 0; mb < kG2MB; ++mb)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) acc[mb][cb] = f32x16_zero();
#pragma unroll
            for (int s = 0; s < LA; ++s)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) bfr[s][cb] = bfrag(s, cb);
#pragma unroll
            for (int s = 0; s < KS2; ++s) {
                if (s + LA < KS2) {
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) bfr[(s + LA) % (LA + 1)][cb] = bfrag(s + LA, cb);
                }
                // the k-slots stay in AGPRs: the MFMAs take them from there directly
#pragma unroll
                for (int mb = 0; mb < kG2MB; ++mb) asm volatile("" : "+a"(hf[mb][s]));
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int mb = 0; mb < kG2MB; ++mb)
                        acc[mb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[s % (LA + 1)][cb], hf[mb][s],
                                                                             acc[mb][cb], 0, 0, 0);
                // copies of the next chunk, four per k-step (never past the unit's last
                // chunk: the buffer range check does not cover the scalar chunk offset)
                if (s < kCS && c + 1 < c_end) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) copy(c + 1, (c + 1) & 1, 4 * s + j);
                }
                // the previous chunk's rows, one store per k-step
                if (s >= kCS && s < kCS + kNSt)
                    __builtin_amdgcn_raw_buffer_store_b128(outv[s - kCS], uvr, st_base + (s - kCS) * 8 * d2 * 2, 0,
                                                           2);
            }
            // Pin that interleave in the schedule: the staged-row reads and the first LA
            // fragment reads, then per k-step its four MFMAs, the two fragment reads of
            // k-step s + LA and the store (the copies keep their place in program order).
            __builtin_amdgcn_sched_group_barrier(0x100, kNSt + 2 * LA, 0);
#pragma unroll
            for (int s = 0; s < KS2; ++s) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2 * kG2MB, 0);
                if (s + LA < KS2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                if (s >= kCS && s < kCS + kNSt) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
            }
            // acc[mb][cb][i]: column c*64 + 32 cb + 8 (i/4) + 4h + i%4 of expert
            // u_wave + 32 mb + l32, i.e. 8-byte half h of 16-byte group 4 cb + i/4 of the
            // staged row 32 mb + l32
#pragma unroll
            for (int mb = 0; mb < kG2MB; ++mb) {
                const int r = mb * 32 + l32;
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int a4 = 0; a4 < 4; ++a4) {
                        const int q = 4 * cb + a4;
                        my2[r * 16 + (q ^ (r & 7)) * 2 + h] =
                            u32x2_t{pack_bf16x2(acc[mb][cb][4 * a4], acc[mb][cb][4 * a4 + 1]),
                                    pack_bf16x2(acc[mb][cb][4 * a4 + 2], acc[mb][cb][4 * a4 + 3])};
                    }
            }
            pend_c = c;
        }
        // the last chunk's rows (the staging writes above are this wave's own LDS
        // operations, which complete in order)
#pragma unroll
        for (int k = 0; k < kNSt; ++k) {
            const int r = 8 * k + (lane >> 3);
            __builtin_amdgcn_raw_buffer_store_b128(my[r * 8 + ((lane & 7) ^ (r & 7))], uvr,
                                                   st_voff + kG2Cols * 2 * pend_c + k * 8 * d2 * 2, 0, 2);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------
// v rows, bf16, W_v-stationary: v = RN(h W_v^T) where each workgroup owns 256 output
// columns (64 per wave) for the whole launch, their W_v rows held in AGPRs (loaded
// once), and the hidden rows stream through LDS in tiles of 64 experts.  A tile's rows
// (64 x DH bf16, contiguous in h) are copied global -> LDS by buffer_load ... lds one
// tile ahead, double buffered; each B-fragment read from LDS feeds two MFMAs (one per
// 32-column block).  The d / 256 workgroups that share a tile (one per column group)
// form a group placed on one XCD, so one of them brings the tile in from HBM and the
// others find it in that XCD's L2.  Operands and k-steps are those of
// expand_bf16_kernel (A = W_v rows, B = hidden rows, k-steps in order), so v is
// bit-identical to it; the difference is that no tile waits for its hidden rows.
//
// Most of each tile's epilogue is carried out during the next tile's MFMAs: right after
// its k-steps a tile's sums are rounded to bf16 pairs in registers (32 registers, no LDS
// work), the next tile's MFMAs start at once, and the 32 remaining operations of the
// epilogue (16 staging writes, then 8 read-backs of whole 128-byte rows each followed by
// its store) are spread evenly over that tile's k-steps.
// ---------------------------------------------------------------------------------
constexpr int kWsCols = 256;  // output columns per workgroup, 64 per wave
constexpr int kWsRows = 64;   // experts per tile

template <int DH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void expand_ws_bf16_kernel(
    const int32_t* __restrict__ n_unique, int64_t max_unique, const uint16_t* __restrict__ hin,
    const uint16_t* __restrict__ w2, int d2, int n_cg, uint16_t* __restrict__ uv) {
    constexpr int KS2 = DH / 16;                         // k-steps
    constexpr int GPR = DH / 8;                          // 16-byte groups per hidden row
    constexpr int kCopiesW = kWsRows * GPR / 64 / 4;     // copy instructions per wave and tile
    constexpr int LA = 4;                                // fragment reads run LA k-steps ahead
    constexpr int kCS = kCopiesW / 4;                    // k-steps that issue copies (4 each)
    constexpr int kNSt = 8;                              // v-row stores per wave and tile
    constexpr int kEpi = 16 + 2 * kNSt;                  // epilogue operations per tile
    static_assert(GPR >= 16 && (GPR & (GPR - 1)) == 0 && kCopiesW % 4 == 0 && kEpi % KS2 == 0 && kCS <= KS2,
                  "tile staging shape");
    constexpr int kOps = kEpi / KS2;                     // epilogue operations per k-step
    // Hidden tiles: row r's 16-byte group g sits at slot g ^ (r % 16) of the row, so a
    // fragment read (one group, 16 consecutive rows per 256 bytes of banks) is
    // conflict-free.
    __shared__ uint4 hs[2][kWsRows * GPR];
    // Output staging, per wave: 64 experts x 64 columns of bf16; expert r's 128-byte
    // row holds its 16-byte group q at slot q ^ (r % 8).
    __shared__ u32x4_t stg[4][kWsRows * 8];

    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    // the h and v outputs hold max_unique rows
    const int U = (int)((int64_t)*n_unique < max_unique ? (int64_t)*n_unique : max_unique);
    const int n_tiles = (U + kWsRows - 1) / kWsRows;
    // Workgroup b runs on XCD b % 8.  Slots b / 8 of one XCD are taken n_cg at a time:
    // the members of one group, column groups 0 .. n_cg - 1.  (The launch makes the
    // grid a multiple of 8 n_cg.)
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int per_xcd = ((int)gridDim.x >> 3) / n_cg;
    const int cg = slot % n_cg, grp = xcd * per_xcd + slot / n_cg;
    const int n_groups = 8 * per_xcd;
    const int col0 = cg * kWsCols + wave * 64;  // the wave's first output column

    // the wave's W_v rows: A fragment (cb, s) = W_v[col0 + 32 cb + l32][16 s + 8 h ..]
    bf16x8_t wf[2][KS2];
    {
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(w2), (short)0, d2 * DH * (int)sizeof(uint16_t), 0x00020000);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int s = 0; s < KS2; ++s)
                wf[cb][s] = __builtin_bit_cast(
                    bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                  wr, ((col0 + 32 * cb + l32) * DH + 16 * s + 8 * h) * (int)sizeof(uint16_t), 0, 0));
    }
    // Copy instruction j = 4 it + wave of a tile moves LDS slots 64 j .. 64 j + 63 (lane
    // i: slot f = 64 j + i, row f / GPR, slot f % GPR of that row, which holds global
    // group (f % GPR) ^ (row % 16)).  Rows at or past U read as zero (the descriptor
    // covers rows below U only).
    auto copy = [&](int64_t tile, int buf, int it) {
        const int64_t row0 = tile * kWsRows;
        const int64_t live = U - row0;
        const int rows = live < kWsRows ? (int)live : kWsRows;
        const i32x4_t rs = buffer_rsrc(hin + row0 * DH, (uint32_t)rows * DH * (uint32_t)sizeof(uint16_t));
        const int j = 4 * it + wave;
        const int f = 64 * j + lane;
        const int r = f / GPR, gs = f % GPR;
        lds_dma16(rs, (r * DH + 8 * (gs ^ (r & 15))) * (int)sizeof(uint16_t), 0, lds_addr(&hs[buf][64 * j]));
    };
    // B fragment (mb, s) of the current tile: row 32 mb + l32, group 2 s + h, at slot
    // (2 s + h) ^ (l32 % 16) = ((2 (s % 8) + h) ^ (l32 % 16)) + 16 (s / 8)
    int bq_off[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) bq_off[q] = l32 * GPR + ((2 * q + h) ^ (l32 & 15));
    // lane's store k covers staged row 8 k + lane / 8, 16-byte group lane % 8
    const int st_voff = ((lane >> 3) * d2 + col0 + 8 * (lane & 7)) * (int)sizeof(uint16_t);
    constexpr int kOOB = 0x40000000;  // a byte offset past any tile's rows (and kOOB + 56 d2 * 2 < 2^31)
    u32x4_t* my = stg[wave];
    u32x2_t* my2 = reinterpret_cast<u32x2_t*>(my);
    // s_waitcnt vmcnt(8) (gfx9 immediate: vmcnt [3:0] and [15:14], expcnt [6:4],
    // lgkmcnt [11:8]; expcnt 7 and lgkmcnt 15 do not wait)
    constexpr int kWaitVm8 = 0x0f78;
    constexpr int kWaitVm0 = 0x0f70;
    // the store descriptor of a tile's rows (rows below max_unique)
    auto tile_rsrc = [&](int64_t t) {
        const int64_t row0 = t * kWsRows;
        const int64_t rows_left = max_unique - row0;
        const int tile_rows = rows_left < kWsRows ? (int)rows_left : kWsRows;
        return __builtin_amdgcn_make_buffer_rsrc(uv + row0 * d2, (short)0, tile_rows * d2 * (int)sizeof(uint16_t),
                                                 0x00020000);
    };
    // A tile's sums as bf16 pairs: pk[e] (e = 8 mb + 4 cb + a4) holds columns
    // col0 + 32 cb + 8 a4 + 4 h .. + 3 of expert 32 mb + l32, i.e. 8-byte half h of 16-byte
    // group 4 cb + a4 of staged row 32 mb + l32.
    u32x2_t pk[16];
    u32x4_t ov[kNSt];
    // epilogue operation e of the tile held in pk: e < 16 stages pk[e]; then, for k = 0 .. 7,
    // e = 16 + 2 k reads back staged row group k (rows 8 k .. 8 k + 7) and e + 1 stores it
    auto epi = [&](int e, __amdgpu_buffer_rsrc_t rsrc, int st_base) {
        if (e < 16) {
            const int mb = e / 8, q = e % 8;
            const int r = mb * 32 + l32;
            my2[r * 16 + (q ^ (r & 7)) * 2 + h] = pk[e];
        } else if ((e - 16) % 2 == 0) {
            const int k = (e - 16) / 2, r = 8 * k + (lane >> 3);
            ov[k] = my[r * 8 + ((lane & 7) ^ (r & 7))];
        } else {
            const int k = (e - 16) / 2;
            __builtin_amdgcn_raw_buffer_store_b128(ov[k], rsrc, st_base + k * 8 * d2 * 2, 0, 2);
        }
    };

    if (grp < n_tiles) {
#pragma unroll
        for (int it = 0; it < kCopiesW; ++it) copy(grp, 0, it);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the W_v rows and the first tile

#pragma unroll
    for (int e = 0; e < 16; ++e) pk[e] = u32x2_t{0u, 0u};
    // The previous tile's epilogue goes out during this tile's k-steps.  The first tile has
    // no previous one: its epilogue stores go to an offset past the descriptor (no memory is
    // written), so that every tile issues its eight stores after its copies and the
    // vmcnt(8) at the top of the next tile covers the copies.
    __amdgpu_buffer_rsrc_t prev_rsrc = tile_rsrc(0);
    bool have_prev = false;
    int i = 0;
    for (int64_t t = grp; t < n_tiles; t += n_groups, ++i) {
        __builtin_amdgcn_s_waitcnt(kWaitVm8);  // this tile's copies have landed
        __syncthreads();
        const int64_t t_next = t + n_groups;
        const int st_base = have_prev ? st_voff : kOOB;
        const uint4* cur = hs[i & 1];
        auto bfrag = [&](int s, int mb) {
            return __builtin_bit_cast(bf16x8_t, cur[bq_off[s & 7] + 16 * (s >> 3) + mb * 32 * GPR]);
        };
        bf16x8_t bfr[LA + 1][2];
        f32x16_t acc[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) acc[mb][cb] = f32x16_zero();
#pragma unroll
        for (int s = 0; s < LA; ++s)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) bfr[s][mb] = bfrag(s, mb);
#pragma unroll
        for (int s = 0; s < KS2; ++s) {
            if (s + LA < KS2) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) bfr[(s + LA) % (LA + 1)][mb] = bfrag(s + LA, mb);
            }
            // the W_v fragments stay in AGPRs: the MFMAs take them from there directly
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) asm volatile("" : "+a"(wf[cb][s]));
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    acc[mb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[cb][s], bfr[s % (LA + 1)][mb],
                                                                         acc[mb][cb], 0, 0, 0);
            if (s < kCS && t_next < n_tiles) {
#pragma unroll
                for (int j = 0; j < 4; ++j) copy(t_next, (i + 1) & 1, 4 * s + j);
            }
#pragma unroll
            for (int o = 0; o < kOps; ++o) epi(s * kOps + o, prev_rsrc, st_base);
        }
        // per k-step: its MFMAs, then the fragment reads LA k-steps ahead, then its
        // epilogue operations (staging write, read-back or store)
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * LA, 0);
#pragma unroll
        for (int s = 0; s < KS2; ++s) {
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            if (s + LA < KS2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int o = 0; o < kOps; ++o) {
                const int e = s * kOps + o;
                if (e < 16)
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                else if ((e - 16) % 2 == 0)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                else
                    __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
            }
        }
        // this tile's sums, rounded (acc[mb][cb][i]: column col0 + 32 cb + 8 (i/4) + 4h + i%4
        // of expert 32 mb + l32)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4)
                    pk[8 * mb + 4 * cb + a4] = u32x2_t{pack_bf16x2(acc[mb][cb][4 * a4], acc[mb][cb][4 * a4 + 1]),
                                                       pack_bf16x2(acc[mb][cb][4 * a4 + 2], acc[mb][cb][4 * a4 + 3])};
        prev_rsrc = tile_rsrc(t);
        have_prev = true;
    }
    // the last tile's epilogue
    if (have_prev) {
#pragma unroll
        for (int e = 0; e < kEpi; ++e) epi(e, prev_rsrc, st_voff);
    }
}

// The two-kernel bf16 generator takes d_latent DL, d_hidden DH, d_model % 64 == 0, at most
// 32 hidden-row tiles per workgroup and a latent table within one buffer descriptor.
template <int DL, int DH>
static bool generate_bf16_ok(int64_t n_experts, int64_t max_unique, int dl, int dh, int d2, int num_cus) {
    if (dl != DL || dh != DH || d2 % kG2Cols) return false;
    const int64_t htiles = (max_unique + kHsRows - 1) / kHsRows;
    const int64_t hgrid = htiles < num_cus ? (htiles > 0 ? htiles : 1) : num_cus;
    return (htiles + hgrid - 1) / hgrid <= kHsMaxTiles && n_experts * DL * 2 < 0x7ff00000ll;
}

// parts: 1 = the hidden rows (W1-stationary kernel), 2 = the v rows from them (an expand
// kernel), 3 = both.  False (nothing launched) when the shape is not one these kernels take.
template <int DL, int DH>
static bool launch_generate_bf16(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                                 int64_t max_unique, const void* w1, const void* w2, int dl, int dh, int d2, void* hout,
                                 void* uv, int parts, int num_cus, hipStream_t stream) {
    if (!generate_bf16_ok<DL, DH>(n_experts, max_unique, dl, dh, d2, num_cus)) return false;
    if (parts & 1) {
        const int64_t htiles = (max_unique + kHsRows - 1) / kHsRows;
        const int64_t hgrid = htiles < num_cus ? (htiles > 0 ? htiles : 1) : num_cus;
        hipLaunchKernelGGL((hidden_ws_bf16_kernel<DL, DH, false>), dim3((unsigned)hgrid), dim3(DH), 0, stream,
                           (const uint16_t*)latents, n_experts, uniq, n_unique, max_unique, (const uint16_t*)w1,
                           (uint16_t*)hout, HiddenActArgs{});
    }
    if (uv == nullptr || !(parts & 2)) return true;  // hidden rows only
    // W_v-stationary when d2 splits into 256-column groups that fill the XCDs evenly
    const int n_cg = d2 / kWsCols;
    const int per_xcd = d2 % kWsCols == 0 && n_cg > 0 ? (num_cus / 8) / n_cg : 0;
    if (per_xcd > 0 && (int64_t)d2 * DH * 2 < (1ll << 31)) {
        const unsigned g2 = (unsigned)(8 * per_xcd * n_cg);
        hipLaunchKernelGGL((expand_ws_bf16_kernel<DH>), dim3(g2), dim3(256), 0, stream, n_unique, max_unique,
                           (const uint16_t*)hout, (const uint16_t*)w2, d2, n_cg, (uint16_t*)uv);
        return true;
    }
    const int64_t tiles = (max_unique + kG2Rows - 1) / kG2Rows;
    const int64_t cap = num_cus;  // one workgroup per CU
    const unsigned grid = (unsigned)(tiles < cap ? (tiles > 0 ? tiles : 1) : cap);
    hipLaunchKernelGGL((expand_bf16_kernel<DH>), dim3(grid), dim3(kG2Waves * 64), 0, stream, n_unique, max_unique,
                       (const uint16_t*)hout, (const uint16_t*)w2, d2, (uint16_t*)uv);
    return true;
}

template <typename T>
static size_t gen_smem(int dl, int dh) {
    return (size_t)GenTile<T>::kRows * ((dl + kGenPad) + (dh + kGenPad)) * sizeof(T);
}

size_t generate_smem_bytes(int dl, int dh, int dtype) {
    return dtype == kBF16 ? gen_smem<uint16_t>(dl, dh) : gen_smem<float>(dl, dh);
}

int launch_generate(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                    int64_t max_unique, const void* w1, const void* w2, int dl, int dh, int d, int dtype, void* hout,
                    void* vout, int num_cus, hipStream_t stream) {
    // W_v^T: rows d .. 2d-1 of net.2.weight; vout == nullptr asks for the hidden rows only
    const size_t eb = dtype == kBF16 ? 2 : 4;
    const void* wv = vout ? static_cast<const unsigned char*>(w2) + (size_t)d * dh * eb : nullptr;
    const int d2 = vout ? d : 0;
    if (dtype == kBF16) {
        if (launch_generate_bf16<128, 512>(latents, n_experts, uniq, n_unique, max_unique, w1, wv, dl, dh, d, hout,
                                              vout, 3, num_cus, stream) ||
            launch_generate_bf16<128, 256>(latents, n_experts, uniq, n_unique, max_unique, w1, wv, dl, dh, d, hout,
                                              vout, 3, num_cus, stream))
            return (int)hipGetLastError();
    }
    const int R = dtype == kBF16 ? GenTile<uint16_t>::kRows : GenTile<float>::kRows;
    int64_t tiles = (max_unique + R - 1) / R;
    int64_t cap = (int64_t)num_cus * 2;
    const unsigned grid = (unsigned)(tiles < cap ? (tiles > 0 ? tiles : 1) : cap);
    const size_t smem = generate_smem_bytes(dl, dh, dtype);
    if (dtype == kBF16)
        hipLaunchKernelGGL(generate_kernel<uint16_t>, dim3(grid), dim3(256), smem, stream, (const uint16_t*)latents,
                           n_experts, uniq, n_unique, max_unique, (const uint16_t*)w1, (const uint16_t*)wv, dl, dh, d2,
                           (uint16_t*)hout, (uint16_t*)vout);
    else
        hipLaunchKernelGGL(generate_kernel<float>, dim3(grid), dim3(256), smem, stream, (const float*)latents,
                           n_experts, uniq, n_unique, max_unique, (const float*)w1, (const float*)wv, dl, dh, d2,
                           (float*)hout,
                           (float*)vout);
    return (int)hipGetLastError();
}

bool generate_split_supported(int64_t n_experts, int64_t max_unique, int dl, int dh, int d, int dtype, int num_cus) {
    return dtype == kBF16 && (generate_bf16_ok<128, 512>(n_experts, max_unique, dl, dh, d, num_cus) ||
                              generate_bf16_ok<128, 256>(n_experts, max_unique, dl, dh, d, num_cus));
}

int launch_generate_part(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                         int64_t max_unique, const void* w1, const void* w2, int dl, int dh, int d, void* hout,
                         void* vout, int part, int num_cus, hipStream_t stream) {
    const void* wv = static_cast<const unsigned char*>(w2) + (size_t)d * dh * 2;
    if (launch_generate_bf16<128, 512>(latents, n_experts, uniq, n_unique, max_unique, w1, wv, dl, dh, d, hout, vout,
                                       part, num_cus, stream) ||
        launch_generate_bf16<128, 256>(latents, n_experts, uniq, n_unique, max_unique, w1, wv, dl, dh, d, hout, vout,
                                       part, num_cus, stream))
        return (int)hipGetLastError();
    return -1;
}

// The hidden rows with the activations of their pairs (tiles of at most kActFusedCap
// pairs; see tile_activations) in one kernel; the activation kernel with seg_off then
// takes the pairs of larger tiles.  -1 (nothing launched) for shapes without the two-kernel
// bf16 generator.
template <int DL, int DH>
static bool launch_hidden_act_t(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                                int64_t max_unique, const void* w1, int dl, int dh, void* hout,
                                const HiddenActArgs& A, int num_cus, hipStream_t stream) {
    if (dl != DL || dh != DH) return false;
    const int64_t htiles = (max_unique + kHsRows - 1) / kHsRows;
    const int64_t hgrid = htiles < num_cus ? (htiles > 0 ? htiles : 1) : num_cus;
    if ((htiles + hgrid - 1) / hgrid > kHsMaxTiles || n_experts * DL * 2 >= 0x7ff00000ll) return false;
    hipLaunchKernelGGL((hidden_ws_bf16_kernel<DL, DH, true>), dim3((unsigned)hgrid), dim3(DH), 0, stream,
                       (const uint16_t*)latents, n_experts, uniq, n_unique, max_unique, (const uint16_t*)w1,
                       (uint16_t*)hout, A);
    return true;
}

int launch_hidden_act(const void* latents, int64_t n_experts, const int32_t* uniq, const int32_t* n_unique,
                      int64_t max_unique, const void* w1, int dl, int dh, void* hout, const void* xp,
                      const int32_t* perm, const int32_t* sorted_slot, const int32_t* seg_off, const void* gates, int hk,
                      float* act, int64_t n_pairs, int num_cus, hipStream_t stream) {
    if (n_pairs <= 0) return -1;
    const HiddenActArgs A{(const uint16_t*)xp, perm, sorted_slot, seg_off, (const uint16_t*)gates, hk, act, n_pairs};
    if (launch_hidden_act_t<128, 512>(latents, n_experts, uniq, n_unique, max_unique, w1, dl, dh, hout, A, num_cus,
                                      stream) ||
        launch_hidden_act_t<128, 256>(latents, n_experts, uniq, n_unique, max_unique, w1, dl, dh, hout, A, num_cus,
                                      stream))
        return (int)hipGetLastError();
    return -1;
}

}  // namespace ethos
