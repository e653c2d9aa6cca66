// rows_kernel.h -- the row-tile MFMA kernel: per-token (or fixed-scale)
// activation quantise -> INT8 / FP8 product -> dequantise + bias +
// activation, in one pass over HBM.
//
// Work split: each wave owns 16 consecutive rows at a time (a "row tile") and
// loops over row tiles with a grid stride.  Lane l handles row r = l & 15 and
// k-group g = l >> 4.  For every 64-wide block kb of K the lane loads four
// float4 of its row at k = kb*64 + j*16 + g*4 (j = 0..3), so the 64 lanes of
// one load instruction read 16 rows x 64 contiguous bytes, and the four
// instructions cover the 16 rows' 256-byte block completely.
//
// INT8: v_mfma_i32_16x16x64_i8 computes D = A(16x64) * B(64x16).  The weight
// tile is passed as A (row i = output column n0 + i) and the activation codes
// as B (column j = row j of the tile), so D[i][j] = C[row j][column n0+i].
// Both operands take their k index from the same (lane group g, dword j,
// byte e) position, so the product is a permutation of the K-sum: exact in
// int32.  D's layout gives lane l the four consecutive columns
// n0 + 4g .. n0 + 4g + 3 of row r, so the epilogue writes one float4 per
// column tile and the row's scale is already in the lane that computed it.
//
// FP8: the activations are rounded to E4M3 values exactly as the reference
// codec does, and the E4M3 values (exactly representable in bfloat16) go
// through v_mfma_f32_16x16x32_bf16 with fp32 accumulation, two instructions
// per 64-wide block.  The fp8 MFMA forms (v_mfma_f32_16x16x32_fp8_fp8 and the
// scaled 16x16x128 f8f6f4) were measured on MI355X to lose about 2^-14 of
// sum|a_k w_k| inside the instruction, outside the 1e-5 tolerance; the bf16
// form stays at 2^-22.
#pragma once

#include "common.h"

namespace nfq {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

enum InMode { IN_F32_TOKEN = 0, IN_F32_FIXED = 1, IN_CODES = 2 };
enum OutMode { OUT_EPI = 0, OUT_RAW = 1 };

struct RowsArgs {
    const float* A;         // IN_F32_*: (M, K) fp32
    const uint8_t* Aq;      // IN_CODES: (M, K) codes
    const float* scale_in;  // IN_CODES: (M) per-row scales (OUT_EPI)
    int64_t M;
    int K;
    int N;
    const uint8_t* W;       // (N, K) int8 or e4m3 codes
    const float* sW;        // (N)
    const int32_t* zpW;     // (N) or null (= zeros); INT8 only
    const float* bias;      // (N) or null
    const int32_t* sumW;    // (N) or null; INT8 only
    float scale_A;          // IN_F32_FIXED
    int32_t zp_A;           // IN_F32_FIXED (and the formula's zpA)
    int formula;            // Formula
    int kb_dot;             // number of 64-wide K blocks that enter the dot
    void* C;                // (M, N) fp32 (OUT_EPI, FP8 OUT_RAW) or int32 (INT8 OUT_RAW)
    float* scale_out;       // (M) or null: per-row scales (IN_F32_TOKEN)
};

// Operand dwords per lane per 64-wide K block: 16 int8 codes, or 16 bf16.
template <bool FP8>
struct Op {
    static constexpr int DW = FP8 ? 8 : 4;
};

// Raw code dwords of the weight tile for column tile n0 and K block kb.
__device__ __forceinline__ void load_w_bytes(const uint8_t* __restrict__ W, int K, int N, int n0,
                                             int kb, int r, int g, uint32_t (&w)[4]) {
    const int n = n0 + r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = kb * 64 + j * 16 + g * 4;
        w[j] = (n < N && k < K)
                   ? *reinterpret_cast<const uint32_t*>(W + static_cast<int64_t>(n) * K + k)
                   : 0u;
    }
}

// Byte dword j -> bf16 dwords 2j (bytes 0, 1) and 2j+1 (bytes 2, 3).
__device__ __forceinline__ void bytes_to_bf16_op(const uint32_t (&b)[4], uint32_t (&o)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        o[2 * j] = e4m3_to_bf16(b[j] & 0xFFu) | (e4m3_to_bf16((b[j] >> 8) & 0xFFu) << 16);
        o[2 * j + 1] = e4m3_to_bf16((b[j] >> 16) & 0xFFu) | (e4m3_to_bf16(b[j] >> 24) << 16);
    }
}

// Weight operand (in MFMA form) and the partial byte sums used by the INT8
// epilogue constants.
template <bool FP8>
__device__ __forceinline__ void load_w_op(const uint8_t* __restrict__ W, int K, int N, int n0,
                                          int kb, int r, int g, uint32_t (&w)[Op<FP8>::DW],
                                          int32_t& psum) {
    uint32_t b[4];
    load_w_bytes(W, K, N, n0, kb, r, g, b);
    if constexpr (FP8) {
        bytes_to_bf16_op(b, w);
        psum = 0;
    } else {
        psum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            w[j] = b[j];
            psum = sum_bytes_i8(b[j], psum);
        }
    }
}

// One 64-wide K block of the product for one column tile.
template <bool FP8>
__device__ __forceinline__ void mfma_block(const uint32_t (&w)[Op<FP8>::DW],
                                           const uint32_t (&x)[Op<FP8>::DW], v4i& acc_i,
                                           v4f& acc_f) {
    if constexpr (FP8) {
        const v4i w0 = {static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]),
                        static_cast<int>(w[3])};
        const v4i w1 = {static_cast<int>(w[4]), static_cast<int>(w[5]), static_cast<int>(w[6]),
                        static_cast<int>(w[7])};
        const v4i x0 = {static_cast<int>(x[0]), static_cast<int>(x[1]), static_cast<int>(x[2]),
                        static_cast<int>(x[3])};
        const v4i x1 = {static_cast<int>(x[4]), static_cast<int>(x[5]), static_cast<int>(x[6]),
                        static_cast<int>(x[7])};
        acc_f = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w0),
                                                        __builtin_bit_cast(v8bf, x0), acc_f, 0, 0, 0);
        acc_f = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w1),
                                                        __builtin_bit_cast(v8bf, x1), acc_f, 0, 0, 0);
    } else {
        const v4i wv = {static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]),
                        static_cast<int>(w[3])};
        const v4i xv = {static_cast<int>(x[0]), static_cast<int>(x[1]), static_cast<int>(x[2]),
                        static_cast<int>(x[3])};
        acc_i = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv, xv, acc_i, 0, 0, 0);
    }
}

// Per-lane epilogue constants of one column tile: the lane's four columns
// n = n0 + 4g + v.  `trivial` (wave-uniform) is set when every INT8 formula
// constant of the tile is zero, i.e. the result is (float)D.
struct ColConsts {
    float sw[4];
    float b[4];
    IntEpi e[4];
    bool trivial;
};

// Sum of the int8 bytes of a weight operand, reduced over the 4 lanes of a
// row (lane groups g), then gathered so that lane (r, g) holds the value of
// column n0 + 4g + v in out[v].
__device__ __forceinline__ void gather_col_sums(int32_t part, int g, int32_t (&out)[4]) {
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
#pragma unroll
    for (int v = 0; v < 4; ++v) out[v] = __shfl(part, 4 * g + v);
}

template <bool FP8, int OUT>
__device__ __forceinline__ void col_consts(const RowsArgs& a, int n0, int g, int32_t part_full,
                                           int32_t part_dot, ColConsts& cc) {
    int32_t sfull[4], sdot[4];
    if constexpr (!FP8 && OUT == OUT_EPI) {
        gather_col_sums(part_full, g, sfull);
        gather_col_sums(part_dot, g, sdot);
    }
    bool nonzero = false;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int n = n0 + 4 * g + v;
        const bool ok = n < a.N;
        cc.sw[v] = ok ? a.sW[n] : 0.0f;
        cc.b[v] = (ok && a.bias) ? a.bias[n] : 0.0f;
        if constexpr (!FP8 && OUT == OUT_EPI) {
            const int32_t zpw = (ok && a.zpW) ? a.zpW[n] : 0;
            const int32_t swg = (ok && a.sumW) ? a.sumW[n] : 0;
            cc.e[v] = int_epi_consts(a.formula, a.K, a.zp_A, zpw, swg, a.sumW != nullptr,
                                     sfull[v], sdot[v]);
            nonzero |= (cc.e[v].c0 != 0) | (cc.e[v].c1 != 0) | (cc.e[v].c2 != 0);
        } else {
            cc.e[v] = IntEpi{0, 0, 0};
        }
    }
    cc.trivial = !__any(nonzero);
}

template <bool FP8, int ACT, int OUT>
__device__ __forceinline__ void store_tile(const RowsArgs& a, int64_t row, int n0, int g,
                                           const v4i& acc_i, const v4f& acc_f,
                                           const ColConsts& cc, float srow, int32_t SA) {
    if (row >= a.M) return;
    const int nb = n0 + 4 * g;
    if constexpr (OUT == OUT_RAW) {
        if constexpr (FP8) {
            float* dst = static_cast<float*>(a.C) + row * a.N + nb;
            if (nb + 3 < a.N) {
                __builtin_nontemporal_store(acc_f, reinterpret_cast<v4f*>(dst));
            } else {
                for (int v = 0; v < 4; ++v)
                    if (nb + v < a.N) dst[v] = acc_f[v];
            }
        } else {
            int32_t* dst = static_cast<int32_t*>(a.C) + row * a.N + nb;
            if (nb + 3 < a.N) {
                __builtin_nontemporal_store(acc_i, reinterpret_cast<v4i*>(dst));
            } else {
                for (int v = 0; v < 4; ++v)
                    if (nb + v < a.N) dst[v] = acc_i[v];
            }
        }
    } else {
        v4f t;
        if constexpr (FP8) {
            t = acc_f;
        } else if (cc.trivial) {
#pragma unroll
            for (int v = 0; v < 4; ++v) t[v] = static_cast<float>(acc_i[v]);
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) t[v] = int_epi_value(cc.e[v], acc_i[v], SA);
        }
        v4f y;
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = activate<ACT>(dequant_bias(cc.sw[v], srow, t[v], cc.b[v]));
        float* dst = static_cast<float*>(a.C) + row * a.N + nb;
        if (nb + 3 < a.N) {
            __builtin_nontemporal_store(y, reinterpret_cast<v4f*>(dst));
        } else {
            for (int v = 0; v < 4; ++v)
                if (nb + v < a.N) dst[v] = y[v];
        }
    }
}

// KB: number of 64-wide K blocks held per lane (K <= 64 * KB).
// HOIST: N <= 64, so the weight operands and column constants of the single
// 64-column chunk stay in registers for the whole kernel.
template <int KB, bool FP8, int IN, int OUT, int ACT, bool HOIST>
__global__ __launch_bounds__(256) void k_rows(RowsArgs a) {
    constexpr int DW = Op<FP8>::DW;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
    const int64_t ntiles = (a.M + 15) >> 4;
    const int K = a.K;
    const int N = a.N;
    const int kb_dot = a.kb_dot;

    // Hoisted weights: operands for the 4 column tiles of columns 0..63.
    uint32_t wh[HOIST ? 4 : 1][HOIST ? KB : 1][DW];
    ColConsts cch[HOIST ? 4 : 1];
    if constexpr (HOIST) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            int32_t pf = 0, pd = 0;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                int32_t ps;
                load_w_op<FP8>(a.W, K, N, nt * 16, kb, r, g, wh[nt][kb], ps);
                pf += ps;
                if (kb < kb_dot) pd += ps;
            }
            col_consts<FP8, OUT>(a, nt * 16, g, pf, pd, cch[nt]);
        }
    }

    for (int64_t tile = wave; tile < ntiles; tile += nwaves) {
        const int64_t row = tile * 16 + r;
        const bool row_ok = row < a.M;
        uint32_t xc[KB][DW];
        float srow = 1.0f;

        if constexpr (IN == IN_CODES) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                uint32_t b[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = kb * 64 + j * 16 + g * 4;
                    b[j] = (row_ok && k < K)
                               ? *reinterpret_cast<const uint32_t*>(a.Aq + row * K + k)
                               : 0u;
                }
                if constexpr (FP8) {
                    bytes_to_bf16_op(b, xc[kb]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) xc[kb][j] = b[j];
                }
            }
            if constexpr (OUT == OUT_EPI) srow = row_ok ? a.scale_in[row] : 1.0f;
        } else {
            float4 x[KB][4];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = kb * 64 + j * 16 + g * 4;
                    x[kb][j] = (row_ok && k < K)
                                   ? *reinterpret_cast<const float4*>(a.A + row * K + k)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            float inv;
            if constexpr (IN == IN_F32_TOKEN) {
                float mx = 0.0f;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        mx = fmaxf(mx, fabsf(x[kb][j].x));
                        mx = fmaxf(mx, fabsf(x[kb][j].y));
                        mx = fmaxf(mx, fabsf(x[kb][j].z));
                        mx = fmaxf(mx, fabsf(x[kb][j].w));
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const float qmax = FP8 ? 448.0f : 127.0f;
                srow = (mx == 0.0f) ? 1.0f : mx / qmax;
                if (a.scale_out && row_ok && g == 0) a.scale_out[row] = srow;
                if constexpr (FP8) {
                    inv = (srow == 0.0f) ? 1.0f : 1.0f / srow;
                } else {
                    inv = 1.0f / srow;
                }
            } else {
                srow = a.scale_A;
                inv = FP8 ? ((srow == 0.0f) ? 1.0f : 1.0f / srow) : 0.0f;
            }
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 v = x[kb][j];
                    if constexpr (FP8) {
                        xc[kb][2 * j] = bf16_bits(fp8_value(v.x, inv)) |
                                        (bf16_bits(fp8_value(v.y, inv)) << 16);
                        xc[kb][2 * j + 1] = bf16_bits(fp8_value(v.z, inv)) |
                                            (bf16_bits(fp8_value(v.w, inv)) << 16);
                    } else if constexpr (IN == IN_F32_TOKEN) {
                        xc[kb][j] = pack4(quant_i8_token(v.x, srow, inv),
                                          quant_i8_token(v.y, srow, inv),
                                          quant_i8_token(v.z, srow, inv),
                                          quant_i8_token(v.w, srow, inv));
                    } else {
                        xc[kb][j] = pack4(quant_i8_exact(v.x, srow, a.zp_A),
                                          quant_i8_exact(v.y, srow, a.zp_A),
                                          quant_i8_exact(v.z, srow, a.zp_A),
                                          quant_i8_exact(v.w, srow, a.zp_A));
                        // Padding beyond K must stay 0 even when zp_A != 0.
                        const int k = kb * 64 + j * 16 + g * 4;
                        if (!(row_ok && k < K)) xc[kb][j] = 0u;
                    }
                }
        }

        int32_t SA = 0;
        if constexpr (!FP8 && OUT == OUT_EPI) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) SA = sum_bytes_i8(xc[kb][j], SA);
            SA += __shfl_xor(SA, 16);
            SA += __shfl_xor(SA, 32);
        }

        if constexpr (HOIST) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                v4i acc_i = {0, 0, 0, 0};
                v4f acc_f = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
                    if (kb < kb_dot) mfma_block<FP8>(wh[nt][kb], xc[kb], acc_i, acc_f);
                store_tile<FP8, ACT, OUT>(a, row, nt * 16, g, acc_i, acc_f, cch[nt], srow, SA);
            }
        } else {
            for (int n0 = 0; n0 < N; n0 += 64) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const int nc = n0 + nt * 16;
                    if (nc >= N) break;
                    v4i acc_i = {0, 0, 0, 0};
                    v4f acc_f = {0.f, 0.f, 0.f, 0.f};
                    int32_t pf = 0, pd = 0;
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) {
                        uint32_t w[DW];
                        int32_t ps;
                        load_w_op<FP8>(a.W, K, N, nc, kb, r, g, w, ps);
                        pf += ps;
                        if (kb < kb_dot) {
                            pd += ps;
                            mfma_block<FP8>(w, xc[kb], acc_i, acc_f);
                        }
                    }
                    ColConsts cc;
                    col_consts<FP8, OUT>(a, nc, g, pf, pd, cc);
                    store_tile<FP8, ACT, OUT>(a, row, nc, g, acc_i, acc_f, cc, srow, SA);
                }
            }
        }
    }
}

}  // namespace nfq
