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

// Absmax over the 16 lanes of a DPP row of four-float chunks, NaN operands
// ignored and starting from 0 (the reference's `if (a > m) m = a` loop):
// fmaxf, so every step canonicalises.  The exact path uses it.
__device__ __forceinline__ float row16_absmax_exact(v4f x) {
    float v = fmaxf(fmaxf(fmaxf(0.0f, fabsf(x[0])), fmaxf(fabsf(x[1]), fabsf(x[2]))), fabsf(x[3]));
    v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
    return v;
}

// The same reduction as six VALU instructions: VOP3 max3 with |.| modifiers
// from 0, then max with a DPP-moved operand (the compiler would add a
// canonicalising max per DPP move).  IEEE-mode max returns the other operand
// for a quiet NaN, so the result equals row16_absmax_exact unless the row
// holds a signalling NaN, in which case it is NaN and the caller takes the
// exact path.  s_nop 1 covers the VALU-write -> DPP-read hazard.
__device__ __forceinline__ float row16_absmax_fast(v4f x) {
    float m;
    asm("v_max3_f32 %0, |%1|, |%2|, 0\n\t"
        "v_max3_f32 %0, %0, |%3|, |%4|\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf"
        : "=&v"(m)
        : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
    return m;
}

// Cache-policy operand of the buffer intrinsics: the nt (non-temporal) bit,
// and sc1 (write through the CU's L2).
constexpr int kCpolNt = 2;
constexpr int kCpolSc1 = 16;

__device__ __forceinline__ float bperm_f(int src_lane, float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_bpermute(src_lane << 2, __builtin_bit_cast(int, v)));
}

// Per-wave LDS: the operand codes (row stride padded against bank
// conflicts) and the output tile (row stride 68 floats) share one buffer --
// the codes are in registers before the first output value is written.
template <bool FP8>
union alignas(16) Rows64Lds {
    static constexpr int CODE_DW = FP8 ? 32 : 16;        // dwords of one row's operand data
    static constexpr int CODE_STRIDE = CODE_DW + 4;      // padded
    static constexpr int OUT_STRIDE = 68;                // floats
    uint32_t codes[16 * CODE_STRIDE];
    float out[16 * OUT_STRIDE];
};

// FP8 weights as the bf16 MFMA operand, shared by the block: row n holds
// W[n][0..63] (32 dwords) with a stride of 36 dwords, so the 8 lanes of a
// ds_read_b128 phase (rows r .. r + 7) fall in distinct banks.
constexpr int W_BF16_STRIDE = 36;

// Buffer resource over the 16-row tile starting at row0 of a row-major array
// of M rows of row_bytes bytes.  The hardware range check returns zeros for
// loads past row M - 1 and drops stores there, so partial and past-the-end
// tiles need no branches.  row0 must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t row0,
                                                            int64_t M, int row_bytes) {
    int64_t left = M - row0;
    left = left < 0 ? 0 : (left > 16 ? 16 : left);
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(static_cast<const char*>(base)) + row0 * row_bytes, 0,
        static_cast<int>(left) * row_bytes, 0x00020000);
}

// Fixed-scale INT8 code (QuantiseActivation with scale_A, zp_A) by the
// reciprocal, and whether it is certainly the reference's.  inv = fl(1 / s)
// correctly rounded and, for s in [2^-120, 2^120] (the caller's condition),
// normal; t = fl(a * inv) and q = fl(a / s) then each lie within
// 2^-24 |a / s| (t: 2 * 2^-24) of a / s, so |t - q| <= 3 * 2^-24 |a / s|
// < 2^-22 |t| (a subnormal product is below 2^-126 and gives r = q = 0).
// |t - r| with r = rint(t) is exact (t and r within a factor 2, or r = 0).
// If |t - r| < 0.5 - 2^-20 |t| (so |t| < 2^19), then |q - r| < 0.5:
// round-half-away(q) == r, and the code is clamp(r + zp) with the
// reference's wrapping add.  NaN / Inf elements give a NaN distance and are
// rejected.
__device__ __forceinline__ int32_t quant_i8_fixed_near(float a, float inv, int32_t zp, bool& bad) {
    const float t = a * inv;
    const float r = rintf(t);
    const float lim = __builtin_fmaf(fabsf(t), -0x1p-20f, 0.5f);
    bad = !(fabsf(t - r) < lim);
    const int32_t ri = bad ? 0 : static_cast<int32_t>(r);
    return clamp_i8(static_cast<int32_t>(static_cast<uint32_t>(ri) + static_cast<uint32_t>(zp)));
}

// The exact code of element e of x (kept out of line: the rare patch path).
__device__ __attribute__((noinline)) uint32_t patch_fixed_code(uint32_t word, float v, int e, float s, int32_t zp) {
    const uint32_t c = static_cast<uint32_t>(quant_i8_exact(v, s, zp)) & 0xFFu;
    return (word & ~(0xFFu << (8 * e))) | (c << (8 * e));
}

// A row takes the exact path when its fast absmax is NaN (a signalling NaN
// in the row) or, for INT8, when amax / 127 would be subnormal (t may then
// leave the int8 range).
template <bool FP8>
__device__ __forceinline__ bool amax_needs_exact(float amax) {
    if constexpr (FP8) return amax != amax;
    return !(amax == 0.0f || (amax >= 0x1p-119f && amax <= 0x1.fffffep+127f));
}

// Exact per-token INT8 codes of four elements with scale s (the reference's
// correctly rounded quotient and half-away rounding).
__device__ __attribute__((noinline)) uint32_t pack4_token_scale(v4f v, float s) {
    const float inv = 1.0f / s;
    return pack4(quant_i8_token(v[0], s, inv), quant_i8_token(v[1], s, inv),
                 quant_i8_token(v[2], s, inv), quant_i8_token(v[3], s, inv));
}

// RES: the FNO layer form act(x1 + x2) with x1 = a.residual (fno.cpp:650-654).
// XQ: the x2 fake-quant before it (fno.cpp:572-648): 1 per-tensor
// (a.xq_scale, a.xq_zpf), 2 per-position (index column * a.xq_points +
// row % a.xq_points into a.xq_scales / a.xq_zps).
// FIXED (INT8 only): one per-tensor scale a.scale_A and zero point a.zp_A
// for every row (QuantiseActivation, int8_gemm.cpp:507-520, as
// LinearForwardBatched and LinearForward run it) instead of the per-row
// absmax; the epilogue's integer formula is a.formula's.
// WPB: waves per block.  4: blocks of 4 waves, wave w takes tiles w,
// w + nwaves, ... (a static, balanced deal).  16: one block per CU whose 16
// waves share the block's tiles through an LDS counter: a wave takes the
// next tile when it starts one, so waves whose loads are served late take
// fewer tiles (with the static deal the slowest waves of a 256 Ki-row layer
// finished 7 us after the median wave).
template <bool FP8, int ACT, int PF = 1, bool RES = false, int XQ = 0, bool FIXED = false, int WPB = 4>
__global__ __launch_bounds__(64 * WPB, WPB == 4 ? 3 : 1) void k_rows64(RowsArgs a) {
    static_assert(!(FIXED && FP8), "the fixed-scale mode is INT8");
    static_assert(WPB == 4 || (WPB == 16 && PF == 1), "block shapes");
    constexpr bool QUEUE = WPB == 16;
    // Output stores: the small layers of the static deal write through the
    // L2 (sc1), so the dirty lines do not wait for the write-back at the end
    // of the launch (measured at 32 Ki rows: 7.4 -> 6.35 us per layer); the
    // large layers of the queue keep the default policy, under which a
    // chained next layer finds more of its input in the last-level cache
    // (sc1 at 256 Ki rows: 22.7 -> 23.0 us; nt: 27.1 us).
    constexpr int STORE_CPOL = QUEUE ? 0 : kCpolSc1;
    constexpr bool INT_EPI = !FP8;
    using L = Rows64Lds<FP8>;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;       // MFMA layout
    const int g = lane >> 4;
    const int lr = lane >> 4;      // linear layout: row within a 4-row group
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * WPB + wid;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * WPB;
    const int64_t ntiles = (a.M + 15) >> 4;
    // QUEUE: this block's tiles are blockIdx.x + G k (G blocks), as in the
    // static deal; the first WPB (k = wid) dealt one per wave, the rest taken
    // through q_next.
    const int64_t qG = gridDim.x;
    const int64_t M = a.M;
    const int lin_off = lane * 16;  // byte offset of the lane in a 4-row group
    constexpr int DW = FP8 ? 8 : 4;  // operand dwords per lane

    __shared__ L lds[WPB];
    __shared__ int q_next;
    __shared__ IntEpi lds_e[INT_EPI ? 64 : 1];
    __shared__ uint32_t lds_w[FP8 ? 64 * W_BF16_STRIDE : 1];
    __shared__ v4f lds_sw[16];
    __shared__ v4f lds_b[16];
    // W_SHARED (the queued INT8 layers): wave 0 loads the weights and forms
    // the column constants; every wave reads them from LDS after the setup
    // barrier, so the launch burst carries one 4 KB weight load per block
    // instead of one per wave (measured at 256 Ki rows, alternating runs on
    // one device: 22.33-22.39 -> 22.23-22.29 us per layer on one, 23.3-23.4
    // -> 22.5-22.7 us on another; with four waves, at 32 Ki rows, 6.3 -> 6.8
    // us, so the static deal keeps the per-wave loads).
    constexpr bool W_SHARED = QUEUE && !FP8;
    __shared__ uint32_t lds_wi8[W_SHARED ? 16 * 64 : 1];
    __shared__ int lds_triv;
    L& my = lds[wid];

    // Linear-layout load of one tile: instruction j reads rows 4j .. 4j + 3.
    // The activations are read once: non-temporal loads (cache policy nt)
    // keep them from displacing lines that are reused; measured +10% at
    // 1 Mi rows, +6-9% at 256 Ki rows over the default policy.
    auto load_lin = [&](int64_t t, v4f (&x)[4]) {
        const auto rs = tile_rsrc(a.A, t * 16, M, 256);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            x[j] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, lin_off + 1024 * j, 0, kCpolNt));
    };

    int64_t tile = QUEUE ? static_cast<int64_t>(blockIdx.x) + qG * wid : wave;
    v4f pre[PF][4];

    // Setup loads first -- the weights, the per-column constants and the
    // block's scale / bias table -- then the first tile's loads.  Loads
    // complete in issue order, so the waits for the setup data then do not
    // include the tile's HBM latency under the launch's initial burst (every
    // wave requests its first tile at once); with the tile loads first, each
    // setup wait also waited for the tile, and no tile of a 256 Ki-row layer
    // completed in its first 6 us (measured).
    // INT8 weights stay in registers: lane (r, g) holds W[16nt + r][16g ..
    // 16g + 15] for nt = 0..3.  FP8 weights go to LDS as bf16 (thread t
    // converts W[t / 4][16 (t % 4) .. + 15]).
    uint32_t wi8[4][4];
    int32_t zpw_c[4] = {0, 0, 0, 0}, sumw_c[4] = {0, 0, 0, 0};   // column 16 nt + r
    uint32_t w8[4];
    if constexpr (FP8) {
        if (threadIdx.x < 256) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(a.W + (threadIdx.x >> 2) * 64 + 16 * (threadIdx.x & 3));
#pragma unroll
            for (int q = 0; q < 4; ++q) w8[q] = src[q];
        }
    } else if (!W_SHARED || wid == 0) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(a.W + (16 * nt + r) * 64 + 16 * g);
#pragma unroll
            for (int q = 0; q < 4; ++q) wi8[nt][q] = src[q];
            zpw_c[nt] = a.zpW ? a.zpW[16 * nt + r] : 0;
            sumw_c[nt] = a.sumW ? a.sumW[16 * nt + r] : 0;
        }
    }
    float sw_n = 0.0f, b_n = 0.0f;
    if (threadIdx.x < 64) {
        sw_n = a.sW[threadIdx.x];
        b_n = a.bias ? a.bias[threadIdx.x] : 0.0f;
    }
    asm volatile("" ::: "memory");   // the tile loads stay behind the setup loads
#pragma unroll
    for (int p = 0; p < PF; ++p) load_lin(tile + p * nwaves, pre[p]);

    if (threadIdx.x < 64) {
        reinterpret_cast<float*>(lds_sw)[threadIdx.x] = sw_n;
        reinterpret_cast<float*>(lds_b)[threadIdx.x] = b_n;
    }
    bool triv[4] = {true, true, true, true};
    if constexpr (FP8) {
        if (threadIdx.x < 256) {
            const int n = threadIdx.x >> 2, c = threadIdx.x & 3;
            uint32_t o[8];
            bytes_to_bf16_op(w8, o);
            v4u* dst = reinterpret_cast<v4u*>(lds_w + n * W_BF16_STRIDE + 8 * c);
            dst[0] = v4u{o[0], o[1], o[2], o[3]};
            dst[1] = v4u{o[4], o[5], o[6], o[7]};
        }
    } else if (!W_SHARED || wid == 0) {
        // The epilogue constants of column 16 nt + r (row_sum4 reduces the
        // four k-groups' byte sums; K = 64, so the dot covers every k).
        // With zp_A = 0, no weight zero points and no caller sum_W (or the
        // batched formula, which uses sum_W only times zp_A) every constant
        // is zero whatever the weights: int_epi_consts' c0 is then
        // 128 S - 128 S, c1 = -2 zp_W and c2 = K zp_W zp_A.  The launch then
        // skips the byte sums (a branch on kernel arguments, uniform).
        const bool zero_terms = a.zp_A == 0 && !a.zpW && (!a.sumW || a.formula == F_BATCHED);
#pragma unroll
        for (int nt = 0; nt < 4 && !zero_terms; ++nt) {
            int32_t ps = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) ps = sum_bytes_i8(wi8[nt][q], ps);
            const int32_t sfull = row_sum4(ps);
            const IntEpi mine = int_epi_consts(a.formula, a.K, a.zp_A, zpw_c[nt], sumw_c[nt], a.sumW != nullptr,
                                               sfull, sfull);
            triv[nt] = !__any((mine.c0 != 0) | (mine.c1 != 0) | (mine.c2 != 0));
            if (wid == 0 && g == 0) lds_e[16 * nt + r] = mine;
        }
        if constexpr (W_SHARED) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                for (int q = 0; q < 4; ++q) lds_wi8[(4 * nt + q) * 64 + lane] = wi8[nt][q];
            if (lane == 0) lds_triv = (triv[0] ? 1 : 0) | (triv[1] ? 2 : 0) | (triv[2] ? 4 : 0) | (triv[3] ? 8 : 0);
        }
    }
    // FIXED: the correctly rounded reciprocal of the scale, and whether the
    // scale is outside the range where the reciprocal codes are certain (then
    // every element takes the exact quotient).
    const float fixed_inv = FIXED ? 1.0f / a.scale_A : 0.0f;
    const bool fixed_exact = FIXED && !(a.scale_A >= 0x1p-120f && a.scale_A <= 0x1p120f);
    if (QUEUE && threadIdx.x == 0) q_next = WPB;
    __syncthreads();
    if constexpr (W_SHARED) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int q = 0; q < 4; ++q) wi8[nt][q] = lds_wi8[(4 * nt + q) * 64 + lane];
        const int tb = lds_triv;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) triv[nt] = ((tb >> nt) & 1) != 0;
    }
    const bool all_triv = triv[0] & triv[1] & triv[2] & triv[3];

    while (tile < ntiles) {
        v4f x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = pre[0][j];
#pragma unroll
        for (int p = 0; p + 1 < PF; ++p)
#pragma unroll
            for (int j = 0; j < 4; ++j) pre[p][j] = pre[p + 1][j];
        // The next tile (a tile at or past the end loads zeros: its rows are
        // outside the buffer range).
        int64_t next;
        if constexpr (QUEUE) {
            int k = 0;
            if (lane == 0) k = atomicAdd(&q_next, 1);
            next = static_cast<int64_t>(blockIdx.x) + qG * __builtin_amdgcn_readfirstlane(k);
        } else {
            next = tile + nwaves;
        }
        load_lin(next + (PF - 1) * nwaves, pre[PF - 1]);
        // Residual tile in the MFMA result layout: lane (r, g), column tile
        // nt -> row r, columns 16 nt + 4 g .. + 3.
        // Position of row r for the per-position x2 fake-quant.
        int xq_pos = 0;
        if constexpr (XQ == 2) xq_pos = static_cast<int>((tile * 16 + r) % a.xq_points);
        v4f res[4];
        if constexpr (RES) {
            const auto rr = tile_rsrc(a.residual, tile * 16, M, 256);
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                res[nt] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rr, (r * 64 + 16 * nt + 4 * g) * 4, 0, kCpolNt));
        }

        const int lc = lane & 15;
        uint32_t q[FP8 ? 8 : 4];
        uint64_t slow = 0;
        float s_r;
        if constexpr (FIXED) {
            // One scale for all rows; the rare elements the reciprocal cannot
            // settle are patched with the exact quotient one by one.
            s_r = a.scale_A;
            uint32_t badm = 0;   // bit 4j + e: element e of x[j]
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int32_t c[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bool bad;
                    c[e] = quant_i8_fixed_near(x[j][e], fixed_inv, a.zp_A, bad);
                    badm |= (bad || fixed_exact) ? (1u << (4 * j + e)) : 0u;
                }
                q[j] = pack4(c[0], c[1], c[2], c[3]);
            }
            if (__builtin_amdgcn_ballot_w64(badm != 0)) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (badm & (1u << (4 * j + e))) q[j] = patch_fixed_code(q[j], x[j][e], e, s_r, a.zp_A);
            }
        } else {
        // Row absmax in the linear layout: amax[j] = absmax of row 4j + lr.
        float amax[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) amax[j] = row16_absmax_fast(x[j]);

        // Row r's absmax to the MFMA-layout lanes (row r = 4j + q lives in
        // lanes 16q.. of amax[j]); scale and reciprocal once per row.
        float am_r = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = bperm_f((r & 3) * 16, amax[j]);
            am_r = ((r >> 2) == j) ? v : am_r;
        }
        slow = __builtin_amdgcn_ballot_w64(amax_needs_exact<FP8>(am_r));
        const float qmax = FP8 ? 448.0f : 127.0f;
        s_r = (am_r == 0.0f) ? 1.0f : am_r / qmax;
        // FP8 scales down by the correctly rounded 1 / s, as the reference.
        float inv_r = FP8 ? ((s_r == 0.0f) ? 1.0f : 1.0f / s_r) : __builtin_amdgcn_rcpf(s_r);

        // Back to the linear layout: inverse scale of row 4j + lr.
        float inv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) inv[j] = bperm_f(4 * j + lr, inv_r);

        // Quantise in the linear layout.
        if constexpr (FP8) {
            // Fast path: no NaN among x * inv (a NaN sets the mask; the
            // reference's NaN byte makes the whole output row NaN).
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float xs = x[j][e] * inv[j];
                    slow |= __builtin_amdgcn_ballot_w64(__builtin_isnan(xs));
                    v[e] = fp8_value_of(xs);
                }
                q[2 * j] = pack_bf16x2(v[0], v[1]);
                q[2 * j + 1] = pack_bf16x2(v[2], v[3]);
            }
            if (slow) {
                // A NaN element or a signalling NaN in the absmax: the
                // canonical reduction, its scales and NaN-propagating values.
#pragma unroll
                for (int j = 0; j < 4; ++j) amax[j] = row16_absmax_exact(x[j]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float v = bperm_f((r & 3) * 16, amax[j]);
                    am_r = ((r >> 2) == j) ? v : am_r;
                }
                s_r = (am_r == 0.0f) ? 1.0f : am_r / qmax;
                inv_r = (s_r == 0.0f) ? 1.0f : 1.0f / s_r;
#pragma unroll
                for (int j = 0; j < 4; ++j) inv[j] = bperm_f(4 * j + lr, inv_r);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    q[2 * j] = pack_bf16x2(fp8_value(x[j][0], inv[j]), fp8_value(x[j][1], inv[j]));
                    q[2 * j + 1] = pack_bf16x2(fp8_value(x[j][2], inv[j]), fp8_value(x[j][3], inv[j]));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int32_t q0 = quant_i8_near(x[j][0], inv[j], slow);
                const int32_t q1 = quant_i8_near(x[j][1], inv[j], slow);
                const int32_t q2 = quant_i8_near(x[j][2], inv[j], slow);
                const int32_t q3 = quant_i8_near(x[j][3], inv[j], slow);
                q[j] = pack4(q0, q1, q2, q3);
            }
            if (slow) {
                // Exact path for the whole tile (wave-uniform branch): the
                // canonical absmax, correctly rounded scales, exact codes.
#pragma unroll
                for (int j = 0; j < 4; ++j) amax[j] = row16_absmax_exact(x[j]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float v = bperm_f((r & 3) * 16, amax[j]);
                    am_r = ((r >> 2) == j) ? v : am_r;
                }
                s_r = (am_r == 0.0f) ? 1.0f : am_r / qmax;
#pragma unroll
                for (int j = 0; j < 4; ++j) q[j] = pack4_token_scale(x[j], bperm_f(4 * j + lr, s_r));
            }
        }
        }  // per-row scales
        if (!FIXED && a.scale_out) {
            // Every lane of row r stores the same value; rows >= M are dropped.
            const auto rs = tile_rsrc(a.scale_out, tile * 16, M, 4);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s_r), rs, r * 4, 0, 0);
        }

        // Stage the operand in LDS.
        if constexpr (FP8) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t* dst = my.codes + (4 * j + lr) * L::CODE_STRIDE + 2 * lc;
                dst[0] = q[2 * j];
                dst[1] = q[2 * j + 1];
            }
        } else {
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
            if (!all_triv) {
#pragma unroll
                for (int q = 0; q < 4; ++q) SA = sum_bytes_i8(xo[q], SA);
                SA = row_sum4(SA);
            }
        }

#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            v4i acc_i = {0, 0, 0, 0};
            v4f acc_f = {0.f, 0.f, 0.f, 0.f};
            uint32_t w[DW];
            if constexpr (FP8) {
                const v4u* src = reinterpret_cast<const v4u*>(lds_w + (16 * nt + r) * W_BF16_STRIDE + 8 * g);
                const v4u w0 = src[0], w1 = src[1];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    w[q] = w0[q];
                    w[4 + q] = w1[q];
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) w[q] = wi8[nt][q];
            }
            mfma_block<FP8>(w, xo, acc_i, acc_f);
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
            for (int v = 0; v < 4; ++v) {
                float x2 = dequant_bias(sw[v], s_r, t[v], bb[v]);
                if constexpr (XQ == 1) {
                    x2 = x2_fake_quant(x2, a.xq_scale, a.xq_zpf);
                } else if constexpr (XQ == 2) {
                    const int64_t idx = static_cast<int64_t>(16 * nt + 4 * g + v) * a.xq_points + xq_pos;
                    x2 = x2_fake_quant(x2, a.xq_scales[idx], static_cast<float>(a.xq_zps[idx]));
                }
                if constexpr (RES) y[v] = activate<ACT>(res[nt][v] + x2);
                else y[v] = activate<ACT>(x2);
            }
            *reinterpret_cast<v4f*>(my.out + r * L::OUT_STRIDE + 16 * nt + 4 * g) = y;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // Linear-layout stores: rows 4j .. 4j + 3 whole per instruction.
        v4f y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            y[j] = *reinterpret_cast<const v4f*>(my.out + (4 * j + lr) * L::OUT_STRIDE + 4 * lc);
        const auto rs = tile_rsrc(a.C, tile * 16, M, 256);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, y[j]), rs, lin_off + 1024 * j, 0, STORE_CPOL);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        tile = next;
    }
}

}  // namespace nfq
