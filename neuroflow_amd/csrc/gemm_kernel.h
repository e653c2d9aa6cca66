// gemm_kernel.h -- tiled MFMA GEMMs on INT8 codes with the fused epilogue,
// for the wide shapes (K a multiple of 64, K >= 128): C[m][n] =
// epilogue(sum_k A_q[m][k] * W_q[n][k]).
//
// A block of 4 waves (2 x 2) computes a BM x BN tile, BM = 32 TM, BN = 32 TN;
// wave (wm, wn) owns rows 16 TM wm .. and columns 16 TN wn .. as TM x TN
// MFMA tiles of v_mfma_i32_16x16x64_i8 (W as the A operand, so lane (r, g)
// of a tile holds row r, columns 4g .. 4g + 3).  K advances 64 per step.
// Rows of both LDS tiles are 64 bytes with the 16-byte group g of row `row`
// stored at slot g ^ ((row >> 1) & 3): measured on gfx950, this reads
// 16-row x 16-byte operand fragments at the rate of a contiguous
// ds_read_b128 (a 64- or 80-byte stride without it is 2-4 way bank
// conflicted).
//
// Two K loops share the epilogue:
//  - k_gemm_pipe (the per-token hot path): the tiles go from global memory
//    straight into a ring of three LDS stages (buffer_load ... lds, no
//    registers, no LDS store instructions), issued two steps ahead of the
//    MFMAs, with one barrier per step.  It forms no byte sums: the row sums
//    come from the quantise pass and the weight-row sums from a pre-pass,
//    when the formula needs them (summing in the loop costs 30-45%).
//  - k_gemm (every other case): each thread loads 16-byte chunks into
//    registers one step ahead, adds their byte sums to its row / column
//    partial sums (the zero-point terms), and stores them into the stage
//    not being read, two stages.
#pragma once

#include <type_traits>

#include "common.h"
#include "rows_kernel.h"

namespace nfq {

constexpr int GEMM_LDS_ROW = 64;  // bytes per K row in LDS

// Byte offset of 16-byte group g of row `row` within a stage tile.
__device__ __forceinline__ int gemm_lds_off(int row, int g) {
    return row * GEMM_LDS_ROW + 16 * (g ^ ((row >> 1) & 3));
}

template <int TM, int TN>
struct GemmShape {
    static constexpr int BM = 32 * TM;
    static constexpr int BN = 32 * TN;
    static constexpr int A_CHUNKS = BM * 4 / 256;  // 16-byte chunks per thread per K step
    static constexpr int W_CHUNKS = BN * 4 / 256;
    static constexpr int STAGE = (BM + BN) * GEMM_LDS_ROW;
};

// Buffer resource over rows [row0, row0 + rows) of a row-major array with
// `row_bytes` bytes per row and `total_rows` rows (reads past the end are 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int64_t row0,
                                                            int64_t total_rows, int rows,
                                                            int64_t row_bytes) {
    int64_t left = total_rows - row0;
    left = left < 0 ? 0 : (left > rows ? rows : left);
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(base)) + row0 * row_bytes, 0,
        static_cast<int>(left * row_bytes), 0x00020000);
}

// Waves per SIMD the tile shape is built for: the 256 x 256 tile holds its
// accumulators in all 256 AGPRs (one wave per SIMD); smaller tiles fit two.
constexpr int gemm_min_waves(int TM, int TN) { return TM * TN >= 64 ? 1 : 2; }

// Tile of block `bid` among `nblk`: blocks are dealt round-robin to `groups`
// XCDs (block b runs on XCD b % groups, each with its own L2), so XCD x is
// given the contiguous tile range [x q + min(x, rem), ...) of its
// q + (x < rem) blocks (q = nblk / groups, rem = nblk % groups).  The N tiles
// of one row tile then run together behind one L2 and share its A rows.
__device__ __forceinline__ int gemm_tile_of_block(int bid, int nblk, int groups) {
    const int x = bid % groups, s = bid / groups;
    const int q = nblk / groups, rem = nblk % groups;
    return x * q + (x < rem ? x : rem) + s;
}

// Per-column epilogue tables of the block's BN columns (n0 ..): integer
// constants of the zero-point terms, scale_W and bias.  col_sum(c) is the
// byte sum of W row n0 + c over the whole K (used only by the formulas that
// need it).  Returns true when every column's integer constants are zero.
// Contains a block barrier.
template <int BN, int OUT, typename ColSum>
__device__ __forceinline__ bool gemm_epi_tables(const RowsArgs& a, int n0, ColSum col_sum,
                                                IntEpi* lds_e, float* lds_scw, float* lds_b) {
    bool nonzero = false;
    if constexpr (OUT == OUT_EPI) {
        for (int c = threadIdx.x; c < BN; c += 256) {
            const int n = n0 + c;
            IntEpi e{0, 0, 0};
            float sw = 0.0f, b = 0.0f;
            if (n < a.N) {
                const int32_t zpw = a.zpW ? a.zpW[n] : 0;
                const int32_t swg = a.sumW ? a.sumW[n] : 0;
                const int32_t s = col_sum(c);
                // K is a multiple of 64, so the dot covers every k and Wd = Sfull.
                e = int_epi_consts(a.formula, a.K, a.zp_A, zpw, swg, a.sumW != nullptr, s, s);
                sw = a.sW[n];
                b = a.bias ? a.bias[n] : 0.0f;
            }
            nonzero |= (e.c0 != 0) | (e.c1 != 0) | (e.c2 != 0);
            lds_e[c] = e;
            lds_scw[c] = sw;
            lds_b[c] = b;
        }
    }
    return __syncthreads_count(nonzero) == 0;
}

// Epilogue of a wave's TM x TN accumulator tiles, one 16-row strip (tile row
// i) at a time.  Lane (r, g) of tile (i, j) holds row 16 TM wm + 16 i + r,
// columns 16 TN wn + 16 j + 4 g .. + 3; the wave writes its strip (16 rows x
// 16 TN columns) into its own LDS area `strip` (16 (16 TN + 4) words), then
// reads it back row-contiguously, so each store instruction writes
// 64 / (4 TN) rows of 64 TN contiguous bytes.  srow[i] / sa[i]: the row
// scale and row code sum of lane row i.
template <int TM, int TN, int OUT, int ACT>
__device__ __forceinline__ void gemm_store(const RowsArgs& a, const v4i (&acc)[TM][TN], int64_t m0,
                                           int n0, int wm, int wn, uint32_t* strip,
                                           const float (&srow)[TM], const int32_t (&sa)[TM],
                                           bool trivial, const IntEpi* lds_e, const float* lds_scw,
                                           const float* lds_b) {
    constexpr int SW = 16 * TN + 4;                 // strip row stride (32-bit words)
    constexpr int CHUNKS = 4 * TN;                  // 16-byte chunks per strip row
    constexpr int ROWS_PER_INST = 64 / CHUNKS;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int64_t M = a.M;
    const int N = a.N;
    const int ncol0 = n0 + 16 * TN * wn;            // first column of the wave's tile
    const int rd_row = lane / CHUNKS, rd_chunk = lane % CHUNKS;
    const bool col_ok = ncol0 + 4 * rd_chunk < N;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int lcol = 16 * TN * wn + 16 * j + 4 * g;
            v4u bits;
            if constexpr (OUT == OUT_RAW) {
                bits = __builtin_bit_cast(v4u, acc[i][j]);
            } else {
                const v4f swv = *reinterpret_cast<const v4f*>(lds_scw + lcol);
                const v4f bv = *reinterpret_cast<const v4f*>(lds_b + lcol);
                v4f y;
                if (trivial) {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        y[v] = activate<ACT>(dequant_bias(swv[v], srow[i], static_cast<float>(acc[i][j][v]), bv[v]));
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float t = int_epi_value(lds_e[lcol + v], acc[i][j][v], sa[i]);
                        y[v] = activate<ACT>(dequant_bias(swv[v], srow[i], t, bv[v]));
                    }
                }
                bits = __builtin_bit_cast(v4u, y);
            }
            *reinterpret_cast<v4u*>(strip + r * SW + 16 * j + 4 * g) = bits;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int q = 0; q < 16 / ROWS_PER_INST; ++q) {
            const int srow_i = q * ROWS_PER_INST + rd_row;
            const v4u v = *reinterpret_cast<const v4u*>(strip + srow_i * SW + 4 * rd_chunk);
            const int64_t m = m0 + 16 * TM * wm + 16 * i + srow_i;
            if (m < M && col_ok)
                *reinterpret_cast<v4u*>(static_cast<uint32_t*>(a.C) + m * N + ncol0 + 4 * rd_chunk) = v;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

template <int TN>
constexpr int gemm_strip_bytes() { return 16 * (16 * TN + 4) * 4; }

typedef int v16i __attribute__((ext_vector_type(16)));

// Epilogue of a wave's (TM / 2) x (TN / 2) accumulator tiles of
// v_mfma_i32_32x32x32_i8 with W as the A operand: value v of lane l in tile
// (i, j) is row 32 i + l % 32, column 32 j + 8 (v / 4) + 4 (l / 32) + v % 4
// of the wave's 16 TM x 16 TN tile, so each group of four values is four
// adjacent columns of one row.  The tile rows go out 16 at a time: the
// lanes holding them (l % 32 in [16 p, 16 p + 16)) write the strip, the
// wave reads it back row-contiguously (64 TN bytes per row).
template <int TM, int TN, int OUT, int ACT>
__device__ __forceinline__ void gemm_store32(const RowsArgs& a, const v16i (&acc)[TM / 2][TN / 2], int64_t m0,
                                             int n0, int wm, int wn, uint32_t* strip,
                                             const float (&srow)[TM / 2], const int32_t (&sa)[TM / 2],
                                             bool trivial, const IntEpi* lds_e, const float* lds_scw,
                                             const float* lds_b) {
    constexpr int I = TM / 2, J = TN / 2;
    constexpr int SW = 16 * TN + 4;                 // strip row stride (32-bit words)
    constexpr int CHUNKS = 4 * TN;                  // 16-byte chunks per strip row
    constexpr int ROWS_PER_INST = 64 / CHUNKS;
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
    const int64_t M = a.M;
    const int N = a.N;
    const int ncol0 = n0 + 16 * TN * wn;
    const int rd_row = lane / CHUNKS, rd_chunk = lane % CHUNKS;
    const bool col_ok = ncol0 + 4 * rd_chunk < N;
#pragma unroll
    for (int i = 0; i < I; ++i) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            if ((r >> 4) == p) {
#pragma unroll
                for (int j = 0; j < J; ++j) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int wcol = 32 * j + 8 * q + 4 * h;      // column within the wave tile
                        const int lcol = 16 * TN * wn + wcol;         // within the block tile
                        v4u bits;
                        if constexpr (OUT == OUT_RAW) {
                            bits = v4u{static_cast<unsigned>(acc[i][j][4 * q]), static_cast<unsigned>(acc[i][j][4 * q + 1]),
                                       static_cast<unsigned>(acc[i][j][4 * q + 2]), static_cast<unsigned>(acc[i][j][4 * q + 3])};
                        } else {
                            const v4f swv = *reinterpret_cast<const v4f*>(lds_scw + lcol);
                            const v4f bv = *reinterpret_cast<const v4f*>(lds_b + lcol);
                            v4f y;
                            if (trivial) {
#pragma unroll
                                for (int v = 0; v < 4; ++v)
                                    y[v] = activate<ACT>(dequant_bias(swv[v], srow[i], static_cast<float>(acc[i][j][4 * q + v]), bv[v]));
                            } else {
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    const float t = int_epi_value(lds_e[lcol + v], acc[i][j][4 * q + v], sa[i]);
                                    y[v] = activate<ACT>(dequant_bias(swv[v], srow[i], t, bv[v]));
                                }
                            }
                            bits = __builtin_bit_cast(v4u, y);
                        }
                        *reinterpret_cast<v4u*>(strip + (r & 15) * SW + wcol) = bits;
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int u = 0; u < 16 / ROWS_PER_INST; ++u) {
                const int srow_i = u * ROWS_PER_INST + rd_row;
                const v4u v = *reinterpret_cast<const v4u*>(strip + srow_i * SW + 4 * rd_chunk);
                const int64_t m = m0 + 16 * TM * wm + 32 * i + 16 * p + srow_i;
                if (m < M && col_ok)
                    *reinterpret_cast<v4u*>(static_cast<uint32_t*>(a.C) + m * N + ncol0 + 4 * rd_chunk) = v;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

// ---------------------------------------------------------------------------
// k_gemm: register-staged K loop with in-loop byte sums (any zero points).
// ---------------------------------------------------------------------------
template <int TM, int TN, int OUT, int ACT>
__global__ __launch_bounds__(256, gemm_min_waves(TM, TN)) void k_gemm(RowsArgs a, int xcd_groups) {
    using S = GemmShape<TM, TN>;
    constexpr int BM = S::BM, BN = S::BN;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // Epilogue tables after the two stages.
    int32_t* lds_sa = reinterpret_cast<int32_t*>(lds + 2 * S::STAGE);      // BM row code sums
    int32_t* lds_sw = lds_sa + BM;                                          // BN weight sums
    IntEpi* lds_e = reinterpret_cast<IntEpi*>(lds_sw + BN);                 // BN constants
    float* lds_scw = reinterpret_cast<float*>(lds_e + BN);                  // BN scale_W
    float* lds_b = lds_scw + BN;                                            // BN bias

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const int r = lane & 15, g = lane >> 4;
    const int K = a.K;
    const int64_t M = a.M;
    const int N = a.N;
    // Tile order: consecutive tiles share an A row tile (N tiles inner).
    const int n_tiles = (N + BN - 1) / BN;
    const int tile = gemm_tile_of_block(blockIdx.x, gridDim.x, xcd_groups);
    const int64_t m0 = static_cast<int64_t>(tile / n_tiles) * BM;
    const int n0 = static_cast<int>(tile % n_tiles) * BN;

    const auto rs_a = rows_rsrc(a.Aq, m0, M, BM, K);
    const auto rs_w = rows_rsrc(a.W, n0, N, BN, K);

    // Chunk c of this thread: tile row (tid >> 2) + 64 c, 16-byte column tid & 3.
    const int crow = tid >> 2, ccol = tid & 3;
    v4u ra[S::A_CHUNKS], rw[S::W_CHUNKS];
    int32_t psa[S::A_CHUNKS], psw[S::W_CHUNKS];
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) psa[c] = 0;
#pragma unroll
    for (int c = 0; c < S::W_CHUNKS; ++c) psw[c] = 0;

    auto gload = [&](int k0) {
#pragma unroll
        for (int c = 0; c < S::A_CHUNKS; ++c)
            ra[c] = __builtin_amdgcn_raw_buffer_load_b128(rs_a, (crow + 64 * c) * K + k0 + 16 * ccol, 0, 0);
#pragma unroll
        for (int c = 0; c < S::W_CHUNKS; ++c)
            rw[c] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, (crow + 64 * c) * K + k0 + 16 * ccol, 0, 0);
    };
    auto sstore = [&](uint8_t* st) {
#pragma unroll
        for (int c = 0; c < S::A_CHUNKS; ++c) {
            *reinterpret_cast<v4u*>(st + gemm_lds_off(crow + 64 * c, ccol)) = ra[c];
#pragma unroll
            for (int q = 0; q < 4; ++q) psa[c] = sum_bytes_i8(ra[c][q], psa[c]);
        }
#pragma unroll
        for (int c = 0; c < S::W_CHUNKS; ++c) {
            *reinterpret_cast<v4u*>(st + BM * GEMM_LDS_ROW + gemm_lds_off(crow + 64 * c, ccol)) = rw[c];
#pragma unroll
            for (int q = 0; q < 4; ++q) psw[c] = sum_bytes_i8(rw[c][q], psw[c]);
        }
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int ksteps = K / 64;
    gload(0);
    sstore(lds);
    __syncthreads();
    for (int ks = 0; ks < ksteps; ++ks) {
        const uint8_t* cur = lds + (ks & 1) * S::STAGE;
        const bool more = ks + 1 < ksteps;
        if (more) gload((ks + 1) * 64);
        v4i xf[TM], wf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            xf[i] = *reinterpret_cast<const v4i*>(cur + gemm_lds_off(16 * TM * wm + 16 * i + r, g));
#pragma unroll
        for (int j = 0; j < TN; ++j)
            wf[j] = *reinterpret_cast<const v4i*>(cur + BM * GEMM_LDS_ROW + gemm_lds_off(16 * TN * wn + 16 * j + r, g));
        // All fragment reads before the first MFMA: one LDS round trip per
        // K step instead of one per row tile.
        __builtin_amdgcn_sched_group_barrier(0x0100, TM + TN, 0);  // DS reads
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[j], xf[i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x0008, TM * TN, 0);  // MFMA
        if (more) sstore(lds + ((ks + 1) & 1) * S::STAGE);
        __syncthreads();
    }

    // Row / column byte sums: reduce the 4 threads (ccol) of each tile row.
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) {
        int32_t v = psa[c];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        if (ccol == 0) lds_sa[crow + 64 * c] = v;
    }
#pragma unroll
    for (int c = 0; c < S::W_CHUNKS; ++c) {
        int32_t v = psw[c];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        if (ccol == 0) lds_sw[crow + 64 * c] = v;
    }
    __syncthreads();
    const bool trivial = gemm_epi_tables<BN, OUT>(
        a, n0, [&](int c) { return lds_sw[c]; }, lds_e, lds_scw, lds_b);

    static_assert(4 * gemm_strip_bytes<TN>() <= 2 * GemmShape<TM, TN>::STAGE, "strip areas fit the stages");
    uint32_t* strip = reinterpret_cast<uint32_t*>(lds + wid * gemm_strip_bytes<TN>());
    float srow[TM];
    int32_t sa[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int lrow = 16 * TM * wm + 16 * i + r;
        const int64_t m = m0 + lrow;
        srow[i] = 1.0f;
        sa[i] = 0;
        if constexpr (OUT == OUT_EPI) {
            srow[i] = m < M ? (a.scale_in ? a.scale_in[m] : a.scale_A) : 0.0f;
            sa[i] = lds_sa[lrow];
        }
    }
    gemm_store<TM, TN, OUT, ACT>(a, acc, m0, n0, wm, wn, strip, srow, sa, trivial, lds_e, lds_scw, lds_b);
}

template <int TM, int TN>
constexpr size_t gemm_lds_bytes() {
    using S = GemmShape<TM, TN>;
    return 2 * S::STAGE + (S::BM + S::BN) * sizeof(int32_t) + S::BN * (sizeof(IntEpi) + 2 * sizeof(float));
}

// ---------------------------------------------------------------------------
// k_gemm_pipe: LDS-DMA K loop, three stages, no byte sums in the loop.
// ---------------------------------------------------------------------------

// 16 bytes per lane from the buffer at byte voff into LDS at lds + 16 lane
// (buffer_load_dwordx4 ... lds; lds is wave-uniform).
__device__ __forceinline__ void gemm_dma16(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff,
                                             0, 0, 0);
}

// Wait until this wave's LDS reads are done and at most one step of its DMA
// loads (NL instructions) is outstanding, then the block barrier.  The
// barrier is an asm statement with a memory clobber, so no memory access
// moves across it and the compiler adds no wait of its own (its LDS-DMA
// tracking still orders each stage's fragment reads after that stage's
// loads).
template <int NL>
__device__ __forceinline__ void gemm_stage_sync() {
    // s_waitcnt: vmcnt in bits 3:0, expcnt 6:4 (7 = no wait), lgkmcnt 11:8.
    static_assert(NL <= 15, "vmcnt fits the low field");
    __builtin_amdgcn_s_waitcnt(0x070 | NL);
    asm volatile("s_barrier" ::: "memory");
}

// Row code sums come from a.sum_in and weight-row byte sums from
// a.colsum_in (null: zero; valid when zpW is null, resp. when the formula
// does not use them).  zp_A must be 0.
//
// MF selects the MFMA: 16 (v_mfma_i32_16x16x64_i8, TM x TN tiles of 16 x 16
// per wave) or 32 (v_mfma_i32_32x32x32_i8, (TM / 2) x (TN / 2) tiles of
// 32 x 32: half the operand reads per product and a higher issue rate).
template <int TM, int TN, int OUT, int ACT, int MF = 16>
__global__ __launch_bounds__(256, 2) void k_gemm_pipe(RowsArgs a, int xcd_groups) {
    static_assert(MF == 16 || (MF == 32 && TM % 2 == 0 && TN % 2 == 0), "32 x 32 tiles need even TM, TN");
    using S = GemmShape<TM, TN>;
    constexpr int BM = S::BM, BN = S::BN;
    constexpr int NL = (BM + BN) / 64;   // 1 KB DMA instructions per wave per K step
    static_assert((BM + BN) % 64 == 0 && BM % 16 == 0, "16-row regions split evenly over 4 waves");
    // Three stages as separate arrays: the compiler then tracks each
    // stage's DMA loads apart, and a fragment read waits for its own stage.
    __shared__ __attribute__((aligned(16))) uint8_t st0[S::STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t st1[S::STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t st2[S::STAGE];
    __shared__ __attribute__((aligned(16))) IntEpi lds_e[BN];
    __shared__ __attribute__((aligned(16))) float lds_scw[BN];
    __shared__ __attribute__((aligned(16))) float lds_b[BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const int r = lane & 15, g = lane >> 4;
    const int K = a.K;
    const int64_t M = a.M;
    const int N = a.N;
    const int n_tiles = (N + BN - 1) / BN;
    const int tile = gemm_tile_of_block(blockIdx.x, gridDim.x, xcd_groups);
    const int64_t m0 = static_cast<int64_t>(tile / n_tiles) * BM;
    const int n0 = static_cast<int>(tile % n_tiles) * BN;

    const auto rs_a = rows_rsrc(a.Aq, m0, M, BM, K);
    const auto rs_w = rows_rsrc(a.W, n0, N, BN, K);

    // Step k's tile into stage st: region q (16 LDS rows, 1 KB) is loaded by
    // wave q % 4; its lane l fills slot l of the region, i.e. row 16 q + l / 4,
    // slot l % 4, which holds 16-byte group (l % 4) ^ ((row >> 1) & 3).
    // A step at or past K / 64 gets an offset beyond the buffer range: it
    // writes zeros into a stage nobody reads and fetches nothing, so every
    // step issues the same loads and the loop has no branches.
    const int nk = K / 64;
    const int drow = lane >> 2, dslot = lane & 3;
    auto dma_step = [&](uint8_t* st, int step) {
        // 2^30 added past the last step, as arithmetic (a select on a
        // uniform condition may become a branch).
        const int oob = ((nk - 1 - step) >> 31) & 0x40000000;
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const int q = wid + 4 * c;
            const int row = 16 * q + drow;
            const int grp = dslot ^ ((row >> 1) & 3);
            const int trow = q < BM / 16 ? row : row - BM;
            gemm_dma16(q < BM / 16 ? rs_a : rs_w, st + 1024 * q, (trow * K + 64 * step + 16 * grp) | oob);
        }
    };

    constexpr int AI = MF == 32 ? TM / 2 : TM, AJ = MF == 32 ? TN / 2 : TN;
    using Acc = std::conditional_t<MF == 32, v16i, v4i>;
    Acc acc[AI][AJ];
#pragma unroll
    for (int i = 0; i < AI; ++i)
#pragma unroll
        for (int j = 0; j < AJ; ++j) acc[i][j] = Acc{};
    auto mma_step = [&](const uint8_t* cur) {
        if constexpr (MF == 32) {
            // Lane l reads row l % 32 of each 32-row fragment, 16-byte group
            // 2 s + l / 32 for K half s: the same k order for both operands.
            const int r32 = lane & 31, h32 = lane >> 5;
            v4i xf[2][AI], wf[2][AJ];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    xf[s][i] = *reinterpret_cast<const v4i*>(cur + gemm_lds_off(16 * TM * wm + 32 * i + r32, 2 * s + h32));
#pragma unroll
                for (int j = 0; j < AJ; ++j)
                    wf[s][j] = *reinterpret_cast<const v4i*>(cur + BM * GEMM_LDS_ROW +
                                                             gemm_lds_off(16 * TN * wn + 32 * j + r32, 2 * s + h32));
            }
            __builtin_amdgcn_sched_group_barrier(0x0100, 2 * (AI + AJ), 0);  // DS reads
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < AI; ++i)
#pragma unroll
                    for (int j = 0; j < AJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[s][j], xf[s][i], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x0008, 2 * AI * AJ, 0);  // MFMA
            return;
        } else {
        v4i xf[TM], wf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            xf[i] = *reinterpret_cast<const v4i*>(cur + gemm_lds_off(16 * TM * wm + 16 * i + r, g));
#pragma unroll
        for (int j = 0; j < TN; ++j)
            wf[j] = *reinterpret_cast<const v4i*>(cur + BM * GEMM_LDS_ROW + gemm_lds_off(16 * TN * wn + 16 * j + r, g));
        __builtin_amdgcn_sched_group_barrier(0x0100, TM + TN, 0);  // DS reads
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[j], xf[i], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x0008, TM * TN, 0);  // MFMA
        }
    };

    // Steps 0 and 1 are loaded before the loop.  Step k (stage k % 3): wait
    // for stage k's loads (only step k + 1's may still be in flight), barrier
    // (every wave has also finished reading stage k - 1), load step k + 2
    // into stage (k + 2) % 3 = (k - 1) % 3, then the MFMAs.  Conditional
    // loads would cost a full wait: the compiler's per-stage tracking does
    // not survive a branch around a DMA.
    auto iter = [&](uint8_t* cur, uint8_t* nxt2, int k) {
        gemm_stage_sync<NL>();
        dma_step(nxt2, k + 2);
        mma_step(cur);
    };
    dma_step(st0, 0);
    dma_step(st1, 1);
    int k = 0;
    for (; k + 3 <= nk; k += 3) {
        iter(st0, st2, k);
        iter(st1, st0, k + 1);
        iter(st2, st1, k + 2);
    }
    if (k < nk) iter(st0, st2, k);
    if (k + 1 < nk) iter(st1, st0, k + 1);
    // No DMA may land after this point (the stages become strip areas).
    __builtin_amdgcn_s_waitcnt(0x070);

    const bool trivial = gemm_epi_tables<BN, OUT>(
        a, n0, [&](int c) { return a.colsum_in ? a.colsum_in[n0 + c] : 0; }, lds_e, lds_scw, lds_b);

    // Strip areas: waves 0, 1 in stage 0, waves 2, 3 in stage 1 (free after
    // the last step; gemm_epi_tables ends with a barrier).
    static_assert(2 * gemm_strip_bytes<TN>() <= S::STAGE, "two strips fit a stage");
    uint32_t* strip = reinterpret_cast<uint32_t*>((wid < 2 ? st0 : st1) + (wid & 1) * gemm_strip_bytes<TN>());
    // Row of lane l in accumulator row tile i: 16 i + l % 16 (16 x 16) or
    // 32 i + l % 32 (32 x 32).
    float srow[AI];
    int32_t sa[AI];
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        const int64_t m = m0 + 16 * TM * wm + (MF == 32 ? 32 * i + (lane & 31) : 16 * i + r);
        srow[i] = 1.0f;
        sa[i] = 0;
        if constexpr (OUT == OUT_EPI) {
            srow[i] = m < M ? (a.scale_in ? a.scale_in[m] : a.scale_A) : 0.0f;
            sa[i] = (a.sum_in && m < M) ? a.sum_in[m] : 0;
        }
    }
    if constexpr (MF == 32)
        gemm_store32<TM, TN, OUT, ACT>(a, acc, m0, n0, wm, wn, strip, srow, sa, trivial, lds_e, lds_scw, lds_b);
    else
        gemm_store<TM, TN, OUT, ACT>(a, acc, m0, n0, wm, wn, strip, srow, sa, trivial, lds_e, lds_scw, lds_b);
}

}  // namespace nfq
