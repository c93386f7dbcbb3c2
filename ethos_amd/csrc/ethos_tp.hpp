// The bf16 token projection xp = RN(x W_u) as a workgroup tile, shared by the projection
// kernel (apply.hip) and the fused small sort (sort.hip).
#pragma once

#include "ethos_common.hpp"
#include "ethos_mfma.hpp"

namespace ethos {

// xp = RN(x W_u) with 32x32x16 MFMAs, fp32 accumulation in k order, rounded once.
// Workgroup tile: 64 tokens x 128 hidden columns; wave (wr, wc) computes tokens 32 wr ..
// and columns 64 wc .. (two 32-column blocks: each B fragment feeds two MFMAs).  Computed
// transposed (xp^T = W_u^T x^T: A = rows of W_u^T, B = rows of x) so that each lane ends
// with four consecutive hidden columns of one token (8-byte stores).  K is copied global
// -> LDS in chunks of 64 by buffer_load ... lds into a ring of three chunk buffers (two
// chunks in flight while one is multiplied; one barrier per chunk); a row's eight 16-byte
// pieces sit at slot piece ^ ((row / 2) % 8), so a fragment read (16 rows, one piece) hits
// every bank once.  Rows past the batch or past d_hidden read as zero (buffer bounds).
constexpr int kTpK = 64;       // reduction chunk (the MFMA path needs d % kTpK == 0)
constexpr int kTpRows = 64;    // tokens per workgroup tile (MFMA path)
constexpr int kTpCols = 128;   // hidden columns per workgroup tile (MFMA path)
constexpr int kTpKC = kTpK;    // K chunk (elements) per ring buffer
constexpr int kTpStages = 3;
constexpr int kTpWBytes = kTpCols * kTpKC * 2;             // 16 KB of W_u^T rows per chunk
constexpr int kTpStage = kTpWBytes + kTpRows * kTpKC * 2;  // + 8 KB of x rows
constexpr int kTpCopies = kTpStage / 1024 / 4;             // 1 KB copies per wave per chunk
__device__ __forceinline__ int tp_slot(int row, int piece) { return piece ^ ((row >> 1) & 7); }

constexpr int kTpLds = kTpStages * kTpStage;               // LDS of one tile's ring

// One workgroup tile (hidden columns c0 .., tokens t0 ..) with `ring` (kTpLds bytes of LDS,
// 16-byte aligned).  Waves 0-3 compute; every wave of the workgroup calls it (it holds the
// barriers), and waves from 4 on only take part in them, so that a larger workgroup can run
// a tile beside other work (the fused sort and token projection).
__device__ __forceinline__ void token_proj_bf16_tile(unsigned char* ring, const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ wut, int n_tok, int d, int dh,
                                                     uint16_t* __restrict__ xp, int c0, int t0) {
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const bool active = wave < 4;
    const int h = lane >> 5, l32 = lane & 31;
    const int wr = (wave & 3) >> 1, wc = wave & 1;
    const int wrows = max(0, min(kTpCols, dh - c0)), xrows = max(0, min(kTpRows, n_tok - t0));
    i32x4_t wrs = buffer_rsrc(wut + (int64_t)c0 * d, (uint32_t)(wrows * d * 2));
    i32x4_t xrs = buffer_rsrc(x + (int64_t)t0 * d, (uint32_t)(xrows * d * 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        wrs[j] = __builtin_amdgcn_readfirstlane(wrs[j]);
        xrs[j] = __builtin_amdgcn_readfirstlane(xrs[j]);
    }
    // copy block b (1 KB: rows 8 b .. 8 b + 7 of the chunk buffer, W_u^T rows first, then x
    // rows) is wave b % 4's; lane l fills row l / 8, slot l % 8 with the piece the swizzle
    // puts there
    static_assert(kTpCols / 8 % 4 == 0, "copies 0 .. kTpCols / 32 - 1 of each wave are W_u^T blocks");
    auto issue = [&](int k0, int stage) {
        unsigned char* base = ring + stage * kTpStage;
#pragma unroll
        for (int j = 0; j < kTpCopies; ++j) {
            constexpr int kWBlocks = kTpCols / 8;
            const int blk = wave + 4 * j;
            const bool isw = j < kWBlocks / 4;  // compile-time after unrolling
            const int row = (isw ? blk : blk - kWBlocks) * 8 + (lane >> 3);
            const int voff = (row * d + tp_slot(row, lane & 7) * 8) * 2;
            if (isw)
                lds_dma16(wrs, voff, k0 * 2, lds_addr(base + blk * 1024));
            else
                lds_dma16(xrs, voff, k0 * 2, lds_addr(base + blk * 1024));
        }
    };
    const int nch = d / kTpKC;
    if (active) {
        issue(0, 0);
        if (nch > 1) issue(kTpKC, 1);
    }
    f32x16_t acc[2] = {f32x16_zero(), f32x16_zero()};
    const int brow = wr * 32 + l32;
    for (int kc = 0; kc < nch; ++kc) {
        // this wave's copies of chunk kc have landed once at most those of chunk kc + 1 are
        // pending (s_waitcnt vmcnt(kTpCopies) / vmcnt(0), gfx9 encoding)
        if (kc + 1 < nch)
            __builtin_amdgcn_s_waitcnt(0x0f70 | kTpCopies);
        else
            __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();  // every wave's copies of chunk kc landed; chunk kc - 1 fully read
        if (!active) continue;
        if (kc + 2 < nch) issue((kc + 2) * kTpKC, (kc + 2) % kTpStages);
        const unsigned char* base = ring + (kc % kTpStages) * kTpStage;
#pragma unroll
        for (int s = 0; s < kTpKC / 16; ++s) {
            const int piece = 2 * s + h;
            const bf16x8_t b =
                *reinterpret_cast<const bf16x8_t*>(base + kTpWBytes + brow * 128 + tp_slot(brow, piece) * 16);
#pragma unroll
            for (int ab = 0; ab < 2; ++ab) {
                const int ar = wc * 64 + ab * 32 + l32;
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(base + ar * 128 + tp_slot(ar, piece) * 16);
                acc[ab] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[ab], 0, 0, 0);
            }
        }
    }
    // acc[ab][i]: hidden column c0 + 64 wc + 32 ab + mfma32_row(i, lane) of token t0 + 32 wr + l32
    const int t = t0 + brow;
    if (active && t < n_tok) {
#pragma unroll
        for (int ab = 0; ab < 2; ++ab)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = c0 + wc * 64 + ab * 32 + 8 * g + 4 * h;
                if (c < dh)
                    *reinterpret_cast<uint2*>(xp + (int64_t)t * dh + c) =
                        make_uint2(pack_bf16x2(acc[ab][4 * g], acc[ab][4 * g + 1]),
                                   pack_bf16x2(acc[ab][4 * g + 2], acc[ab][4 * g + 3]));
            }
    }
}

}  // namespace ethos
