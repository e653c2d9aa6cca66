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

// Cache policy of the streaming activation reads and output writes
// (1 = non-temporal).
#ifndef NFQ_NT_LOAD
#define NFQ_NT_LOAD 0
#endif
#ifndef NFQ_NT_STORE
#define NFQ_NT_STORE 0
#endif

namespace nfq {

template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
#if NFQ_NT_LOAD
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

template <typename T>
__device__ __forceinline__ void stream_store(T v, T* p) {
#if NFQ_NT_STORE
    __builtin_nontemporal_store(v, p);
#else
    *p = v;
#endif
}

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
    const float* residual;  // (M, N) or null: added before the activation (FNO layer)
    const int32_t* sum_in;     // IN_CODES: (M) row code sums, or null (the tiled GEMM only)
    const int32_t* colsum_in;  // (N) byte sums of W's rows over K, or null (the tiled GEMM only)
    // x2 fake-quant of the FNO layer (nflow_x2_quant; k_rows64 and the FNO post-pass)
    int xq_kind;               // 0 none, 1 per-tensor, 2 per-position
    float xq_scale;
    float xq_zpf;              // the zero point as float
    const float* xq_scales;    // per-position: index j * xq_points + m % xq_points
    const int32_t* xq_zps;
    int xq_points;
};

// Operand dwords per lane per 64-wide K block: 16 int8 codes, or 16 bf16.
template <bool FP8>
struct Op {
    static constexpr int DW = FP8 ? 8 : 4;
};

// Raw code dwords of the weight tile for column tile n0 and K block kb.
// Branch-free: the column is clamped into range and the value replaced by 0
// outside it; with KFULL (K a multiple of 64) every k is in range.
template <bool KFULL>
__device__ __forceinline__ void load_w_bytes(const uint8_t* __restrict__ W, int K, int N, int n0,
                                             int kb, int r, int g, uint32_t (&w)[4]) {
    const int n = n0 + r;
    const uint8_t* rowp = W + static_cast<int64_t>(n < N ? n : N - 1) * K;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = kb * 64 + j * 16 + g * 4;
        uint32_t v;
        if constexpr (KFULL) {
            v = *reinterpret_cast<const uint32_t*>(rowp + k);
        } else {
            v = *reinterpret_cast<const uint32_t*>(rowp + (k < K ? k : K - 4));
            v = k < K ? v : 0u;
        }
        w[j] = n < N ? v : 0u;
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
template <bool FP8, bool KFULL>
__device__ __forceinline__ void load_w_op(const uint8_t* __restrict__ W, int K, int N, int n0,
                                          int kb, int r, int g, uint32_t (&w)[Op<FP8>::DW],
                                          int32_t& psum) {
    uint32_t b[4];
    load_w_bytes<KFULL>(W, K, N, n0, kb, r, g, b);
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
// constant of the tile is zero, i.e. the result is (float)D; the constants
// themselves (needed only otherwise) are kept per lane in `e`, or -- for the
// hoisted tiles -- in LDS.
struct ColConsts {
    v4f sw;
    v4f b;
    bool trivial;
};

// Reduce a lane's partial byte sum over the 4 lanes of a row (lane groups g):
// every lane (r, g) then holds the sum of column n0 + r.
__device__ __forceinline__ int32_t row_sum4(int32_t part) {
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
    return part;
}

// Column setup for the 16-column tile n0.  Lane (r, g) computes the INT8
// epilogue constants of column n0 + r from the reduced weight sums (no
// gathers needed for the triviality test), and loads scale / bias of its own
// output columns n0 + 4g + v.  The constants of column n0 + r are returned in
// `mine`; callers that need them per output column gather or stage them.
template <bool FP8, int OUT>
__device__ __forceinline__ void col_setup(const RowsArgs& a, int n0, int r, int g,
                                          int32_t part_full, int32_t part_dot, ColConsts& cc,
                                          IntEpi& mine, bool load_sw_b) {
    bool nonzero = false;
    mine = IntEpi{0, 0, 0};
    if constexpr (!FP8 && OUT == OUT_EPI) {
        const int32_t sfull = row_sum4(part_full);
        const int32_t sdot = row_sum4(part_dot);
        const int c = n0 + r;
        if (c < a.N) {
            const int32_t zpw = a.zpW ? a.zpW[c] : 0;
            const int32_t swg = a.sumW ? a.sumW[c] : 0;
            mine = int_epi_consts(a.formula, a.K, a.zp_A, zpw, swg, a.sumW != nullptr, sfull, sdot);
            nonzero = (mine.c0 != 0) | (mine.c1 != 0) | (mine.c2 != 0);
        }
    }
    if (OUT == OUT_EPI && load_sw_b) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = n0 + 4 * g + v;
            const bool ok = n < a.N;
            cc.sw[v] = ok ? a.sW[n] : 0.0f;
            cc.b[v] = (ok && a.bias) ? a.bias[n] : 0.0f;
        }
    }
    cc.trivial = !__any(nonzero);
}

// Gather the constants of the lane's output columns n0 + 4g + v from the
// lanes that computed them (lane 4g + v holds column n0 + 4g + v).
__device__ __forceinline__ void gather_consts(const IntEpi& mine, int g, IntEpi (&e)[4]) {
    const int32_t c2lo = static_cast<int32_t>(static_cast<uint64_t>(mine.c2));
    const int32_t c2hi = static_cast<int32_t>(static_cast<uint64_t>(mine.c2) >> 32);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int src = 4 * g + v;
        e[v].c0 = __shfl(mine.c0, src);
        e[v].c1 = __shfl(mine.c1, src);
        const uint32_t lo = static_cast<uint32_t>(__shfl(c2lo, src));
        const uint32_t hi = static_cast<uint32_t>(__shfl(c2hi, src));
        e[v].c2 = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
    }
}

template <bool FP8, int ACT, int OUT>
__device__ __forceinline__ void store_tile(const RowsArgs& a, int64_t row, int n0, int g,
                                           const v4i& acc_i, const v4f& acc_f, v4f sw, v4f bias,
                                           bool trivial, const IntEpi* e, float srow,
                                           int32_t SA) {
    // N % 4 == 0 (a dispatch precondition), so a column group is either
    // entirely inside or entirely outside [0, N).
    if (row >= a.M) return;
    const int nb = n0 + 4 * g;
    if constexpr (OUT == OUT_RAW) {
        if constexpr (FP8) {
            if (nb < a.N)
                stream_store(acc_f, reinterpret_cast<v4f*>(static_cast<float*>(a.C) + row * a.N + nb));
        } else {
            if (nb < a.N)
                stream_store(acc_i, reinterpret_cast<v4i*>(static_cast<int32_t*>(a.C) + row * a.N + nb));
        }
    } else {
        v4f t;
        if constexpr (FP8) {
            t = acc_f;
        } else if (trivial) {
#pragma unroll
            for (int v = 0; v < 4; ++v) t[v] = static_cast<float>(acc_i[v]);
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) t[v] = int_epi_value(e[v], acc_i[v], SA);
        }
        v4f y;
#pragma unroll
        for (int v = 0; v < 4; ++v) y[v] = activate<ACT>(dequant_bias(sw[v], srow, t[v], bias[v]));
        if (nb < a.N)
            stream_store(y, reinterpret_cast<v4f*>(static_cast<float*>(a.C) + row * a.N + nb));
    }
}

// Exact per-token codes of four elements (the rare slow path of the
// reciprocal quantiser); kept out of line so that the unrolled hot loop does
// not carry its registers.
__device__ __attribute__((noinline)) uint32_t pack4_token_exact(v4f v, float s, float inv) {
    return pack4(quant_i8_token(v[0], s, inv), quant_i8_token(v[1], s, inv),
                 quant_i8_token(v[2], s, inv), quant_i8_token(v[3], s, inv));
}

// Activation operand of one row tile, loaded (fp32 input: raw floats; code
// input: raw code dwords) ahead of its use so the next tile's HBM reads are
// in flight while the current tile is computed.
template <int KB, int IN>
struct TileIn {
    v4f x[IN == IN_CODES ? 1 : KB][4];
    uint32_t c[IN == IN_CODES ? KB : 1][4];
};

template <int KB, int IN, bool KFULL>
__device__ __forceinline__ void load_tile(const RowsArgs& a, int64_t tile, int r, int g,
                                          TileIn<KB, IN>& t) {
    // Rows past M (only in the last tile) re-read row M-1; they are never
    // stored.  Without KFULL, k past K reads a clamped address and becomes 0.
    const int K = a.K;
    const int64_t row = tile * 16 + r;
    const int64_t rowc = row < a.M ? row : a.M - 1;
    if constexpr (IN == IN_CODES) {
        const uint8_t* base = a.Aq + rowc * K;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = kb * 64 + j * 16 + g * 4;
                if constexpr (KFULL) {
                    t.c[kb][j] = *reinterpret_cast<const uint32_t*>(base + k);
                } else {
                    const uint32_t v = *reinterpret_cast<const uint32_t*>(base + (k < K ? k : K - 4));
                    t.c[kb][j] = k < K ? v : 0u;
                }
            }
    } else {
        const float* base = a.A + rowc * K;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = kb * 64 + j * 16 + g * 4;
                if constexpr (KFULL) {
                    t.x[kb][j] = stream_load(reinterpret_cast<const v4f*>(base + k));
                } else {
                    const v4f v = stream_load(
                        reinterpret_cast<const v4f*>(base + (k < K ? k : K - 4)));
                    t.x[kb][j] = k < K ? v : v4f{0.f, 0.f, 0.f, 0.f};
                }
            }
    }
}

// Waves per SIMD the register budget is sized for (512 / waves VGPRs).
#ifndef NFQ_ROWS_WAVES_KB1
#define NFQ_ROWS_WAVES_KB1 3
#endif
constexpr int rows_min_waves(int KB, bool FP8) {
    return KB == 1 ? NFQ_ROWS_WAVES_KB1 : (KB == 2 && !FP8 ? 3 : 2);
}

// Whether the weight operands of one 64-column chunk fit in registers.
#ifndef NFQ_ROWS_HOIST_DW
#define NFQ_ROWS_HOIST_DW 8
#endif
constexpr bool rows_hoist_fits(int KB, bool FP8) { return KB * (FP8 ? 8 : 4) <= NFQ_ROWS_HOIST_DW; }

// KB: number of 64-wide K blocks held per lane (K <= 64 * KB).
// HOIST: N <= 64, so the weight operands and column constants of the single
// 64-column chunk stay resident (registers; INT8 formula constants in LDS)
// for the whole kernel.
template <int KB, bool FP8, int IN, int OUT, int ACT, bool HOIST, bool KFULL>
__global__ __launch_bounds__(256, rows_min_waves(KB, FP8)) void k_rows(RowsArgs a) {
    constexpr int DW = Op<FP8>::DW;
    constexpr bool INT_EPI = !FP8 && OUT == OUT_EPI;
    const int lane = threadIdx.x & 63;
    const int wid = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + wid;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
    const int64_t ntiles = (a.M + 15) >> 4;
    const int K = a.K;
    const int N = a.N;
    const int kb_dot = a.kb_dot;

    // The first tile's HBM reads go out before the weight setup.
    int64_t tile = wave;
    TileIn<KB, IN> nxt;
    if (tile < ntiles) load_tile<KB, IN, KFULL>(a, tile, r, g, nxt);

    // Hoisted weights: operands for the 4 column tiles of columns 0..63.
    uint32_t wh[HOIST ? 4 : 1][HOIST ? KB : 1][DW];
    bool triv[HOIST ? 4 : 1];
    __shared__ IntEpi lds_e[HOIST && INT_EPI ? 64 : 1];
    __shared__ v4f lds_sw[HOIST ? 16 : 1];
    __shared__ v4f lds_b[HOIST ? 16 : 1];
    if constexpr (HOIST) {
        // Scale and bias exist only for the dequantising epilogue (the raw
        // product entry points pass no scale_W).
        if (OUT == OUT_EPI && threadIdx.x < 64) {
            const int n = threadIdx.x;
            reinterpret_cast<float*>(lds_sw)[n] = n < N ? a.sW[n] : 0.0f;
            reinterpret_cast<float*>(lds_b)[n] = (n < N && a.bias) ? a.bias[n] : 0.0f;
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            int32_t pf = 0, pd = 0;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                int32_t ps;
                load_w_op<FP8, KFULL>(a.W, K, N, nt * 16, kb, r, g, wh[nt][kb], ps);
                pf += ps;
                if (kb < kb_dot) pd += ps;
            }
            IntEpi mine;
            ColConsts cc;
            col_setup<FP8, OUT>(a, nt * 16, r, g, pf, pd, cc, mine, false);
            triv[nt] = cc.trivial;
            if constexpr (INT_EPI) {
                if (wid == 0 && g == 0) lds_e[nt * 16 + r] = mine;
            }
        }
        __syncthreads();
    }

    for (; tile < ntiles; tile += nwaves) {
        const int64_t row = tile * 16 + r;
        const bool row_ok = row < a.M;
        TileIn<KB, IN> cur = nxt;
        if (tile + nwaves < ntiles) load_tile<KB, IN, KFULL>(a, tile + nwaves, r, g, nxt);

        uint32_t xc[KB][DW];
        float srow = 1.0f;

        if constexpr (IN == IN_CODES) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                if constexpr (FP8) {
                    bytes_to_bf16_op(cur.c[kb], xc[kb]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) xc[kb][j] = cur.c[kb][j];
                }
            }
            if constexpr (OUT == OUT_EPI) srow = row_ok ? a.scale_in[row] : 1.0f;
        } else {
            float inv;
            if constexpr (IN == IN_F32_TOKEN) {
                float mx = 0.0f;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        mx = fmaxf(mx, fabsf(cur.x[kb][j][0]));
                        mx = fmaxf(mx, fabsf(cur.x[kb][j][1]));
                        mx = fmaxf(mx, fabsf(cur.x[kb][j][2]));
                        mx = fmaxf(mx, fabsf(cur.x[kb][j][3]));
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
            if constexpr (FP8) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const v4f v = cur.x[kb][j];
                        xc[kb][2 * j] = pack_bf16x2(fp8_value(v[0], inv), fp8_value(v[1], inv));
                        xc[kb][2 * j + 1] = pack_bf16x2(fp8_value(v[2], inv), fp8_value(v[3], inv));
                    }
            } else if constexpr (IN == IN_F32_TOKEN) {
                // Reciprocal fast path for all elements, then one branch per
                // lane that redoes the lane's codes exactly if any element
                // was too close to a rounding tie.
                bool slow = false;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const v4f v = cur.x[kb][j];
                        int32_t q0, q1, q2, q3;
                        const bool ok = quant_i8_fast(v[0], inv, q0) & quant_i8_fast(v[1], inv, q1) &
                                        quant_i8_fast(v[2], inv, q2) & quant_i8_fast(v[3], inv, q3);
                        slow |= !ok;
                        xc[kb][j] = pack4(q0, q1, q2, q3);
                    }
                if (slow) {
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                        for (int j = 0; j < 4; ++j) xc[kb][j] = pack4_token_exact(cur.x[kb][j], srow, inv);
                }
            } else {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const v4f v = cur.x[kb][j];
                        xc[kb][j] = pack4(quant_i8_exact(v[0], srow, a.zp_A),
                                          quant_i8_exact(v[1], srow, a.zp_A),
                                          quant_i8_exact(v[2], srow, a.zp_A),
                                          quant_i8_exact(v[3], srow, a.zp_A));
                        // Padding beyond K must stay 0 even when zp_A != 0.
                        const int k = kb * 64 + j * 16 + g * 4;
                        if (!(row_ok && k < K)) xc[kb][j] = 0u;
                    }
            }
        }

        int32_t SA = 0;
        if constexpr (INT_EPI) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) SA = sum_bytes_i8(xc[kb][j], SA);
            SA = row_sum4(SA);
        }

        if constexpr (HOIST) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                v4i acc_i = {0, 0, 0, 0};
                v4f acc_f = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
                    if (kb < kb_dot) mfma_block<FP8>(wh[nt][kb], xc[kb], acc_i, acc_f);
                IntEpi e[4];
                if constexpr (INT_EPI) {
                    if (!triv[nt]) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) e[v] = lds_e[nt * 16 + 4 * g + v];
                    }
                }
                store_tile<FP8, ACT, OUT>(a, row, nt * 16, g, acc_i, acc_f, lds_sw[nt * 4 + g],
                                          lds_b[nt * 4 + g], triv[nt], e, srow, SA);
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
                        load_w_op<FP8, KFULL>(a.W, K, N, nc, kb, r, g, w, ps);
                        pf += ps;
                        if (kb < kb_dot) {
                            pd += ps;
                            mfma_block<FP8>(w, xc[kb], acc_i, acc_f);
                        }
                    }
                    ColConsts cc;
                    IntEpi mine, e[4];
                    col_setup<FP8, OUT>(a, nc, r, g, pf, pd, cc, mine, true);
                    if constexpr (INT_EPI) {
                        if (!cc.trivial) gather_consts(mine, g, e);
                    }
                    store_tile<FP8, ACT, OUT>(a, row, nc, g, acc_i, acc_f, cc.sw, cc.b, cc.trivial, e,
                                              srow, SA);
                }
            }
        }
    }
}

}  // namespace nfq
