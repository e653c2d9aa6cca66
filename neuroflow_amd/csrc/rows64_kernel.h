// rows64_kernel.h -- the fused per-token layer for K = 64, N = 64 (the
// FNO1d / FNO2d local-linear shape and the standalone 64x64 GEMM): per-token
// INT8 or FP8 quantise -> MFMA -> dequantise + bias + activation, with every
// HBM access a full-row, 1 KB-contiguous wave instruction.
//
// A wave owns 16 rows at a time (a 4 KB input tile and a 4 KB output tile).
// Two register layouts are used:
//   linear  lane l holds row 4j + (l >> 4), columns 4(l & 15) .. +3 for
//           j = 0..3: instruction j reads / writes rows 4j .. 4j+3 whole.
//   MFMA    lane l holds row r = l & 15 and k-group g = l >> 4 (operands),
//           or row r, columns 16nt + 4g .. +3 (results).
// The row absmax is a 16-lane DPP reduction in the linear layout; each row's
// scale is then computed once, in the lane that holds the row in the MFMA
// layout, and sent back with ds_bpermute.  The 1 KB of codes (2 KB of bf16
// for FP8) and the 4 KB output tile change layout through per-wave LDS.
// k-group g of the operands is k = 16g .. 16g + 15 for both the weight and
// the activation operand, so each MFMA is a permutation of the K-sum.
#pragma once

#include "common.h"
#include "rows_kernel.h"

namespace nfq {

// DPP row move (16-lane rows).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Max over the 16 lanes of a DPP row (NaN operands are ignored by fmaxf).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
    return v;
}

__device__ __forceinline__ float bperm_f(int src_lane, float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_bpermute(src_lane << 2, __builtin_bit_cast(int, v)));
}

// Exact per-token INT8 codes of four elements of a row whose absmax is amax
// (the rare slow path; out of line so the hot loop does not carry it).
__device__ __attribute__((noinline)) uint32_t pack4_token_exact_amax(v4f v, float amax) {
    const float s = (amax == 0.0f) ? 1.0f : amax / 127.0f;
    const float inv = 1.0f / s;
    return pack4(quant_i8_token(v[0], s, inv), quant_i8_token(v[1], s, inv),
                 quant_i8_token(v[2], s, inv), quant_i8_token(v[3], s, inv));
}

// Per-wave LDS: codes (row stride padded against bank conflicts) and the
// output tile (row stride 68 floats).
template <bool FP8>
struct alignas(16) Rows64Lds {
    static constexpr int CODE_DW = FP8 ? 32 : 16;        // dwords of one row's operand data
    static constexpr int CODE_STRIDE = CODE_DW + 4;      // padded
    static constexpr int OUT_STRIDE = 68;                // floats
    uint32_t codes[16 * CODE_STRIDE];
    float out[16 * OUT_STRIDE];
};

template <bool FP8, int ACT>
__global__ __launch_bounds__(256, 3) void k_rows64(RowsArgs a) {
    constexpr bool INT_EPI = !FP8;
    using L = Rows64Lds<FP8>;
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int r = lane & 15;       // MFMA layout
    const int g = lane >> 4;
    const int lr = lane >> 4;      // linear layout: row within a 4-row group
    const int lc = lane & 15;      //                4-float column chunk
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + wid;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
    const int64_t ntiles = (a.M + 15) >> 4;
    const int64_t M = a.M;

    __shared__ L lds[4];
    __shared__ IntEpi lds_e[INT_EPI ? 64 : 1];
    __shared__ v4f lds_sw[16];
    __shared__ v4f lds_b[16];
    L& my = lds[wid];

    // Linear-layout load of one tile (rows past M re-read row M-1 and are
    // never stored).
    auto load_lin = [&](int64_t tile, v4f (&x)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int64_t row = tile * 16 + 4 * j + lr;
            row = row < M ? row : M - 1;
            x[j] = *reinterpret_cast<const v4f*>(a.A + row * 64 + 4 * lc);
        }
    };

    int64_t tile = wave;
    v4f nxt[4];
    if (tile < ntiles) load_lin(tile, nxt);

    // Weights: lane (r, g) holds W[16nt + r][16g .. 16g + 15] for nt = 0..3.
    constexpr int DW = FP8 ? 8 : 4;
    uint32_t wop[4][DW];
    bool triv[4];
    if (threadIdx.x < 64) {
        const int n = threadIdx.x;
        reinterpret_cast<float*>(lds_sw)[n] = a.sW[n];
        reinterpret_cast<float*>(lds_b)[n] = a.bias ? a.bias[n] : 0.0f;
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(a.W + (16 * nt + r) * 64 + 16 * g);
        uint32_t b[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = src[q];
        int32_t ps = 0;
        if constexpr (FP8) {
            bytes_to_bf16_op(b, wop[nt]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wop[nt][q] = b[q];
                ps = sum_bytes_i8(b[q], ps);
            }
        }
        IntEpi mine;
        ColConsts cc;
        col_setup<FP8, OUT_EPI>(a, 16 * nt, r, g, ps, ps, cc, mine, false);
        triv[nt] = cc.trivial;
        if constexpr (INT_EPI) {
            if (wid == 0 && g == 0) lds_e[16 * nt + r] = mine;
        }
    }
    __syncthreads();

    for (; tile < ntiles; tile += nwaves) {
        v4f x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = nxt[j];
        if (tile + nwaves < ntiles) load_lin(tile + nwaves, nxt);

        // Row absmax in the linear layout: amax[j] = absmax of row 4j + lr.
        float amax[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            amax[j] = row16_max(fmaxf(fmaxf(fabsf(x[j][0]), fabsf(x[j][1])),
                                      fmaxf(fabsf(x[j][2]), fabsf(x[j][3]))));

        // Row r's absmax to the MFMA-layout lanes (row r = 4j + q lives in
        // lanes 16q.. of amax[j]); scale and reciprocal once per row.
        float am_r = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = bperm_f((r & 3) * 16, amax[j]);
            am_r = ((r >> 2) == j) ? v : am_r;
        }
        const float qmax = FP8 ? 448.0f : 127.0f;
        const float s_r = (am_r == 0.0f) ? 1.0f : am_r / qmax;
        const float inv_r = FP8 ? ((s_r == 0.0f) ? 1.0f : 1.0f / s_r) : 1.0f / s_r;
        const int64_t row_r = tile * 16 + r;
        if (a.scale_out && g == 0 && row_r < M) a.scale_out[row_r] = s_r;

        // Back to the linear layout: inverse scale of row 4j + lr.
        float inv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) inv[j] = bperm_f(4 * j + lr, inv_r);

        // Quantise in the linear layout and stage the operand in LDS.
        if constexpr (FP8) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = bf16_bits(fp8_value(x[j][0], inv[j])) |
                                    (bf16_bits(fp8_value(x[j][1], inv[j])) << 16);
                const uint32_t hi = bf16_bits(fp8_value(x[j][2], inv[j])) |
                                    (bf16_bits(fp8_value(x[j][3], inv[j])) << 16);
                uint32_t* dst = my.codes + (4 * j + lr) * L::CODE_STRIDE + 2 * lc;
                dst[0] = lo;
                dst[1] = hi;
            }
        } else {
            uint32_t q[4];
            bool slow = false;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int32_t q0, q1, q2, q3;
                const bool ok = quant_i8_fast(x[j][0], inv[j], q0) & quant_i8_fast(x[j][1], inv[j], q1) &
                                quant_i8_fast(x[j][2], inv[j], q2) & quant_i8_fast(x[j][3], inv[j], q3);
                slow |= !ok;
                q[j] = pack4(q0, q1, q2, q3);
            }
            if (slow) {
#pragma unroll
                for (int j = 0; j < 4; ++j) q[j] = pack4_token_exact_amax(x[j], amax[j]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) my.codes[(4 * j + lr) * L::CODE_STRIDE + lc] = q[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // Operand in the MFMA layout: row r, k = 16g .. 16g + 15.
        uint32_t xo[DW];
        {
            const v4i* src = reinterpret_cast<const v4i*>(my.codes + r * L::CODE_STRIDE + (FP8 ? 8 : 4) * g);
            const v4i p0 = src[0];
#pragma unroll
            for (int q = 0; q < 4; ++q) xo[q] = static_cast<uint32_t>(p0[q]);
            if constexpr (FP8) {
                const v4i p1 = src[1];
#pragma unroll
                for (int q = 0; q < 4; ++q) xo[4 + q] = static_cast<uint32_t>(p1[q]);
            }
        }
        int32_t SA = 0;
        if constexpr (INT_EPI) {
#pragma unroll
            for (int q = 0; q < 4; ++q) SA = sum_bytes_i8(xo[q], SA);
            SA = row_sum4(SA);
        }

#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            v4i acc_i = {0, 0, 0, 0};
            v4f acc_f = {0.f, 0.f, 0.f, 0.f};
            mfma_block<FP8>(wop[nt], xo, acc_i, acc_f);
            v4f t;
            if constexpr (FP8) {
                t = acc_f;
            } else if (triv[nt]) {
#pragma unroll
                for (int v = 0; v < 4; ++v) t[v] = static_cast<float>(acc_i[v]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) t[v] = int_epi_value(lds_e[16 * nt + 4 * g + v], acc_i[v], SA);
            }
            const v4f sw = lds_sw[4 * nt + g];
            const v4f bb = lds_b[4 * nt + g];
            v4f y;
#pragma unroll
            for (int v = 0; v < 4; ++v) y[v] = activate<ACT>(dequant_bias(sw[v], s_r, t[v], bb[v]));
            *reinterpret_cast<v4f*>(my.out + r * L::OUT_STRIDE + 16 * nt + 4 * g) = y;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // Linear-layout stores: rows 4j .. 4j + 3 whole per instruction.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t row = tile * 16 + 4 * j + lr;
            const v4f y = *reinterpret_cast<const v4f*>(my.out + (4 * j + lr) * L::OUT_STRIDE + 4 * lc);
            if (row < M) *reinterpret_cast<v4f*>(static_cast<float*>(a.C) + row * 64 + 4 * lc) = y;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
}

}  // namespace nfq
