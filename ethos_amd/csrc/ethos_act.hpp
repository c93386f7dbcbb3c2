// Activations of a tile's pairs computed inside a generator kernel while the tile's hidden
// rows are staged in LDS: a_p = RN(RN(gelu(RN(h_s . xp_t))) g_p), the apply's phase 1
// (model.py:326-329), with the arithmetic of apply_act8_kernel (dot_raw in piece order,
// act_reduce8, act_epilogue), so the activations are bit-identical to it whichever kernel
// computes a pair.
#pragma once
#include "ethos_common.hpp"
#include "ethos_rows.hpp"

namespace ethos {

// What a generator kernel needs to compute the activations of its tiles' pairs.
struct HiddenActArgs {
    const uint16_t* xp;          // [n_tok, DH] token projections x W_u
    const int32_t* perm;         // sorted position -> pair
    const int32_t* sorted_slot;  // sorted position -> unique slot
    const int32_t* seg_off;      // [U + 1] first sorted position of each unique slot
    const uint16_t* gates;       // [n_pairs]
    int hk;                      // pairs per token (heads x top_k)
    float* act;                  // [n_pairs] activations (fp32 holding bf16 values)
    int64_t n_pairs;             // entries of perm, sorted_slot, gates and act
};

// A tile's activations: its sorted positions and this lane's pair of the first round.
// The tile's seg_off bounds are loaded one tile ahead and its pair and row at the top of
// the tile's iteration, with no branch between a load and its use, so that all of them
// have landed by the time the tile's rows are staged.
struct ActMeta {
    int64_t s0, s1;  // the tile's pairs: sorted positions s0 .. s1 - 1
    int p, s;        // this lane's pair of the first round and its row in the tile
    bool valid;
};

template <int kWaves>
__device__ __forceinline__ int64_t act_position(int64_t r0, int wave, int lane) {
    return r0 + 8 * (wave + kWaves * (lane >> 3)) + (lane & 7);
}

// sorted position j clamped to the pair arrays, so that its loads need no branch
__device__ __forceinline__ int64_t act_index(const HiddenActArgs& A, int64_t j) {
    return j < 0 ? 0 : (j < A.n_pairs ? j : A.n_pairs - 1);
}

template <int kWaves>
__device__ __forceinline__ ActMeta act_meta(const HiddenActArgs& A, int64_t row0, int64_t s0, int64_t s1, int wave,
                                            int lane) {
    ActMeta m;
    m.s0 = s0;
    m.s1 = s1;
    const int64_t j = act_position<kWaves>(s0, wave, lane), jc = act_index(A, j);
    m.valid = j < s1 && s1 - s0 <= kActFusedCap;
    m.p = A.perm[jc];
    m.s = A.sorted_slot[jc] - (int)row0;
    return m;
}

// The activations of one tile's pairs (sorted positions s0 .. s1 - 1) from the tile's
// staged hidden rows, when they number at most kActFusedCap (larger tiles are left to the
// activation kernel).  Rounds of 64 pairs per wave: lane l of wave w holds the metadata of
// sorted position r0 + 8 (w + waves (l / 8)) + l % 8 (act_position), so the wave's groups
// of 8 consecutive pairs interleave with the other waves' and a tile's pairs spread over
// all waves.  Per group, lane (q, part) serves the group's pair q with the pieces
// part + 8 i of the pair's xp row (global) and hidden row (staged; piece(row, part, i)
// reads it), summed as apply_act8_kernel sums them.  The xp rows of kBatch groups are
// requested before any is summed, so a tile of a few hundred pairs costs one or two round
// trips to memory.
template <int DH, int kWaves, int kTileRows, typename Piece, int kBatch = 3>
__device__ __forceinline__ void tile_activations(const HiddenActArgs& A, Piece piece, float* dsm, int64_t row0,
                                                 const ActMeta& m, int wave, int lane) {
    constexpr int P = DH / 64;
    if (m.s1 - m.s0 > kActFusedCap) return;
    const int part = lane & 7, q = lane >> 3;
    for (int64_t r0 = m.s0; r0 < m.s1; r0 += 64 * kWaves) {
        int my_p = m.p, my_s = m.s;
        bool valid = m.valid;
        if (r0 != m.s0) {
            const int64_t j = act_position<kWaves>(r0, wave, lane), jc = act_index(A, j);
            valid = j < m.s1;
            my_p = A.perm[jc];
            my_s = A.sorted_slot[jc] - (int)row0;
        }
        my_s = my_s < 0 ? 0 : (my_s < kTileRows ? my_s : kTileRows - 1);  // stays inside the tile on any input
        // the gate is requested with the xp rows and used by the epilogue
        const uint16_t g_raw = A.gates[my_p];
        const int my_t = my_p / A.hk;  // the pair's token
        // this wave's groups of the round: group gi starts at r0 + 8 (wave + waves gi)
        const int64_t left = m.s1 - r0 - 8 * wave;
        const int ng =
            __builtin_amdgcn_readfirstlane(left <= 0 ? 0 : (int)min((int64_t)8, (left + 8 * kWaves - 1) / (8 * kWaves)));
        for (int g0 = 0; g0 < ng; g0 += kBatch) {
            // Every group of the batch has its xp row requested before any is summed.  The
            // loads and sums are unconditional (a group past ng repeats group g0, whose
            // result is not kept), so no branch separates a load from its use.
            uint4 xv[kBatch][P];
            int sl[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int src = (g0 + b < ng ? g0 + b : g0) * 8 + q;
                const int tb = __shfl(my_t, src, 64);
                sl[b] = __shfl(my_s, src, 64);
                const uint16_t* xr = A.xp + (int64_t)tb * DH;
#pragma unroll
                for (int i = 0; i < P; ++i) xv[b][i] = *reinterpret_cast<const uint4*>(xr + (part + 8 * i) * 8);
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < P; ++i) acc = dot_raw(piece(sl[b], part, i), xv[b][i], acc);
                acc = act_reduce8(acc);
                if (part == 0 && g0 + b < ng) dsm[(g0 + b) * 8 + q] = acc;
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (valid) A.act[my_p] = act_epilogue<uint16_t>(dsm[lane], bf16_bits_to_f32(g_raw));
        __builtin_amdgcn_wave_barrier();
    }
}

}  // namespace ethos
