// token_gemm_kernel.h -- the per-token INT8 layer in one pass: a block
// quantises a 64-row tile of fp32 activations into INT8 codes held in LDS
// (the per-token scale absmax / 127 and the reference's correctly rounded
// codes, int8_gemm.cpp:231-240 with scale_A per row), then runs the whole N
// range from them with v_mfma_i32_16x16x64_i8, dequantise + bias +
// activation in the epilogue.  The activations are read once and the codes
// never reach HBM: the layer costs one fp32 read and one fp32 write, where
// the split form (quantise launch, codes to HBM, tiled GEMM) adds a launch
// and 2 MK bytes of code traffic and re-reads the codes per column block.
//
// k_token_gemm (K = 128, 256, 512): 4 waves, 2 blocks per CU, each block
// quantising a tile and then running its product, persistent over tiles.
//
// Tile quantise: a wave quantises 16 rows, 4 at a time with 16 lanes per
// row (the reductions are DPP row steps), codes into LDS rows of K + 16
// bytes (the pad spreads the 16 rows of an operand read over the banks).
// Tile product: the N range is walked in chunks of 256 columns; wave w takes
// the 64 columns 64 w .. 64 w + 63 of the chunk for all 64 rows: 4 x 4 tiles
// of 16 x 16 accumulators.  Weights come from L2 (16 contiguous bytes of one
// weight row per lane and K step), codes from LDS.  As in the other kernels
// the weight tile is the MFMA's A operand, so a lane's four results are four
// adjacent output columns of one row, and lane group g takes k = 16 g ..
// 16 g + 15 of each 64-wide step in both operands (the product is a
// permutation of the K-sum, exact in int32).  The epilogue passes each
// 16-row strip of a wave's 16 x 64 outputs through a per-wave LDS strip, and
// the strip leaves as row-contiguous 256-byte segments.
// Column constants: lane L of a wave owns column nw0 + L of its 64 columns.
// It loads that column's weight scale, bias, zero point and given sum_W
// before the K loop (one coalesced load each, whose latency the K loop
// covers), forms the INT8 epilogue constants from the weight bytes summed
// during the K loop (as in the row-tile kernels) and files everything in the
// wave's LDS tables, which the epilogue reads as float4 / IntEpi per lane.
// Loading them per output lane after the K loop instead puts a chain of
// dependent global loads -- each also waiting for the previous chunk's
// stores -- between every product and its stores.
#pragma once

#include "common.h"
#include "rows_kernel.h"

namespace nfq {

// Output stores carry the nt (non-temporal) policy: the streamed output then
// leaves the L2 to the weights the K loops re-read (measured at C4, six
// blocks of qkv + proj on 32768 tokens: 25.35 -> 22.3 us per layer; sc1
// 24.2 us).
constexpr int kTokenStoreCpol = 2;

template <int KB>
struct TokenGemmShape {
    static constexpr int K = 64 * KB;
    static constexpr int ROW = K + 16;            // LDS code row stride (bytes)
    static constexpr int CODES = 64 * ROW;        // code tile bytes
    static constexpr int STRIP_W = 68;            // per-wave output strip row stride (floats)
    static constexpr int STRIP = 16 * STRIP_W * 4;
    static constexpr int ETAB = 64 * static_cast<int>(sizeof(IntEpi)) + 2 * 64 * 4;  // per-wave column consts
    static constexpr int ROWQ = 64 * 4 + 64 * 4;  // row scales, row code sums
    static constexpr int LDS = CODES + 4 * STRIP + 4 * ETAB + ROWQ;
};

// Activations of 4 rows (row m of this lane's group g; rows past M read row
// M - 1 and are not used): float4 r + 16 j of the row, j < J.
template <int J>
__device__ __forceinline__ void token_load4(const RowsArgs& a, int64_t m, int r, v4f (&x)[J]) {
    const int64_t M = a.M;
    const v4f* x4 = reinterpret_cast<const v4f*>(a.A + (m < M ? m : M - 1) * static_cast<int64_t>(64 * J));
#pragma unroll
    for (int j = 0; j < J; ++j) x[j] = __builtin_nontemporal_load(x4 + r + 16 * j);
}

// Codes of local row lr (= 4 q + g of the wave's rows) from x into the tile:
// the row's absmax over its 16 lanes, s = absmax / 127 (1 for a zero row),
// the codes, their byte sum; row scale and sum to lds_s / lds_sa (and the
// scale to scale_out for rows < M).
template <int J>
__device__ __forceinline__ void token_quantise_row(const RowsArgs& a, const v4f (&x)[J], int64_t m0, int lr,
                                                   int r, uint8_t* codes, int row_bytes, float* lds_s,
                                                   int32_t* lds_sa) {
    const bool live = m0 + lr < a.M;
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j)
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(x[j][0]), fabsf(x[j][1]))), fmaxf(fabsf(x[j][2]), fabsf(x[j][3])));
    mx = fmaxf(mx, dpp_mov<0xB1>(mx));   // quad_perm [1,0,3,2]
    mx = fmaxf(mx, dpp_mov<0x4E>(mx));   // quad_perm [2,3,0,1]
    mx = fmaxf(mx, dpp_mov<0x141>(mx));  // row_half_mirror
    mx = fmaxf(mx, dpp_mov<0x140>(mx));  // row_mirror
    const float s = (mx == 0.0f) ? 1.0f : mx / 127.0f;
    const float inv = 1.0f / s;
    int32_t sa = 0;
    uint32_t* crow = reinterpret_cast<uint32_t*>(codes + lr * row_bytes);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        uint32_t v = pack4(quant_i8_token(x[j][0], s, inv), quant_i8_token(x[j][1], s, inv),
                           quant_i8_token(x[j][2], s, inv), quant_i8_token(x[j][3], s, inv));
        v = live ? v : 0u;
        crow[r + 16 * j] = v;
        sa = sum_bytes_i8(v, sa);
    }
    sa += dpp_movi<0xB1>(sa);
    sa += dpp_movi<0x4E>(sa);
    sa += dpp_movi<0x141>(sa);
    sa += dpp_movi<0x140>(sa);
    if (r == 0) {
        lds_s[lr] = s;
        lds_sa[lr] = sa;
        if (a.scale_out && live) a.scale_out[m0 + lr] = s;
    }
}

__device__ __forceinline__ void token_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The product of the 64-row code tile at m0 with every column, by product
// wave `wid` (0..3): columns 64 wid .. 64 wid + 63 of each 256-column chunk.
// SUMS = false when every integer-epilogue term is zero whatever the weights
// (zp_A = 0, no weight zero points, no caller sum_W or the batched formula):
// the weight byte sums and the epilogue constants are then skipped.
template <int KB, int ACT, bool SUMS = true>
__device__ __forceinline__ void token_tile_gemm(const RowsArgs& a, const uint8_t* codes, const float* lds_s,
                                                const int32_t* lds_sa, float* strip, uint8_t* ctab, int64_t m0,
                                                int wid, int lane) {
    using S = TokenGemmShape<KB>;
    constexpr int K = S::K;
    const int r = lane & 15, g = lane >> 4;
    const int64_t M = a.M;
    const int N = a.N;
    IntEpi* etab = reinterpret_cast<IntEpi*>(ctab);                     // 64 columns' INT8 constants
    float* swtab = reinterpret_cast<float*>(ctab + 64 * sizeof(IntEpi));  // 64 weight scales
    float* btab = swtab + 64;                                             // 64 biases

    // Row scales / code sums of the lane's rows 16 rt + r.
    float srow[4];
    int32_t sarow[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        srow[rt] = lds_s[16 * rt + r];
        sarow[rt] = lds_sa[16 * rt + r];
    }

    for (int nc = 0; nc < N; nc += 256) {
        const int nw0 = nc + 64 * wid;              // the wave's first column
        if (nw0 >= N) continue;                     // wave-uniform
        // This lane's column: constants loaded branch-free (an absent
        // array reads the scales and the value is replaced by 0).
        const int cl = nw0 + lane;
        const float my_sw = a.sW[cl];
        const float my_b0 = (a.bias ? a.bias : a.sW)[cl];
        const int32_t my_zp0 = (a.zpW ? a.zpW : reinterpret_cast<const int32_t*>(a.sW))[cl];
        const int32_t my_sg0 = (a.sumW ? a.sumW : reinterpret_cast<const int32_t*>(a.sW))[cl];
        v4i acc[4][4];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = v4i{0, 0, 0, 0};
        int32_t wsum[4] = {0, 0, 0, 0};
        // Two K steps per trip: unrolled further, the weight loads hoisted
        // ahead of the products push the kernel past 256 registers.
#pragma unroll 2
        for (int kb = 0; kb < KB; ++kb) {
            v4i wv[4], xv[4];
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const uint8_t* wp = a.W + static_cast<int64_t>(nw0 + 16 * ct + r) * K + 64 * kb + 16 * g;
                wv[ct] = *reinterpret_cast<const v4i*>(wp);
                if constexpr (SUMS) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) wsum[ct] = sum_bytes_i8(static_cast<uint32_t>(wv[ct][e]), wsum[ct]);
                }
            }
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
                xv[rt] = *reinterpret_cast<const v4i*>(codes + (16 * rt + r) * S::ROW + 64 * kb + 16 * g);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int ct = 0; ct < 4; ++ct)
                    acc[rt][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[ct], xv[rt], acc[rt][ct], 0, 0, 0);
        }
        // Weight byte sums of column 16 ct + r reduced over the lane groups;
        // lane (r, g) = column 16 g + r takes tile ct = g.
        bool trivial = true;
        if constexpr (SUMS) {
            int32_t wfull = 0;
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const int32_t f = row_sum4(wsum[ct]);
                wfull = (g == ct) ? f : wfull;
            }
            const int32_t my_zp = a.zpW ? my_zp0 : 0;
            const IntEpi mine = int_epi_consts(a.formula, a.K, a.zp_A, my_zp, a.sumW ? my_sg0 : 0,
                                               a.sumW != nullptr, wfull, wfull);
            // Wave-uniform: all 64 columns' constants zero, the result is (float)D.
            trivial = !__any((mine.c0 != 0) | (mine.c1 != 0) | (mine.c2 != 0));
            if (!trivial) etab[lane] = mine;
        }
        swtab[lane] = my_sw;
        btab[lane] = a.bias ? my_b0 : 0.0f;
        token_wave_sync();
        // Epilogue, one 16-row strip at a time through the wave's LDS strip.
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const int c0 = 16 * ct + 4 * g;          // the lane's first column in the wave
                float t[4];
                if (trivial) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) t[v] = static_cast<float>(acc[rt][ct][v]);
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v) t[v] = int_epi_value(etab[c0 + v], acc[rt][ct][v], sarow[rt]);
                }
                const v4f sw4 = *reinterpret_cast<const v4f*>(swtab + c0);
                const v4f b4 = *reinterpret_cast<const v4f*>(btab + c0);
                v4f y;
#pragma unroll
                for (int v = 0; v < 4; ++v) y[v] = activate<ACT>(dequant_bias(sw4[v], srow[rt], t[v], b4[v]));
                *reinterpret_cast<v4f*>(strip + r * S::STRIP_W + 16 * ct + 4 * g) = y;
            }
            token_wave_sync();
            // The strip's rows m0 + 16 rt .. + 15 as a buffer range clipped
            // at M: rows past it are dropped by the hardware.
            const int64_t r0 = m0 + 16 * rt;
            const int64_t left = M - r0 < 0 ? 0 : (M - r0 > 16 ? 16 : M - r0);
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(static_cast<float*>(a.C) + r0 * N, 0,
                                                              static_cast<int>(left * N * 4), 0x00020000);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int sr = 4 * q + (lane >> 4);     // strip row
                const v4f v = *reinterpret_cast<const v4f*>(strip + sr * S::STRIP_W + 4 * (lane & 15));
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), rs,
                                                       (sr * N + nw0 + 4 * (lane & 15)) * 4, 0, kTokenStoreCpol);
            }
            token_wave_sync();
        }
    }
}

template <int KB, int ACT>
__global__ __launch_bounds__(256, 2) void k_token_gemm(RowsArgs a) {
    using S = TokenGemmShape<KB>;
    constexpr int J = S::K / 64;                 // float4 per lane per row in the quantise
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::LDS];
    uint8_t* codes = lds;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* strip = reinterpret_cast<float*>(lds + S::CODES) + wid * (16 * S::STRIP_W);
    uint8_t* ctab = lds + S::CODES + 4 * S::STRIP + wid * S::ETAB;
    float* lds_s = reinterpret_cast<float*>(lds + S::CODES + 4 * S::STRIP + 4 * S::ETAB);
    int32_t* lds_sa = reinterpret_cast<int32_t*>(lds_s + 64);

    const int lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int64_t ntiles = (a.M + 63) / 64;
    const bool zero_terms = a.zp_A == 0 && !a.zpW && (!a.sumW || a.formula == F_BATCHED);

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * 64;
        // Quantise 16 rows per wave (rows 16 wid + 4 q + g, q < 4).
        {
            v4f x[4][J];
#pragma unroll
            for (int q = 0; q < 4; ++q) token_load4<J>(a, m0 + 16 * wid + 4 * q + g, r, x[q]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                token_quantise_row<J>(a, x[q], m0, 16 * wid + 4 * q + g, r, codes, S::ROW, lds_s, lds_sa);
        }
        __syncthreads();
        if (zero_terms) token_tile_gemm<KB, ACT, false>(a, codes, lds_s, lds_sa, strip, ctab, m0, wid, lane);
        else token_tile_gemm<KB, ACT, true>(a, codes, lds_s, lds_sa, strip, ctab, m0, wid, lane);
        __syncthreads();   // the next tile's quantise overwrites the codes
    }
}

}  // namespace nfq
