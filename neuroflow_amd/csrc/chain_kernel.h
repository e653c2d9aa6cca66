// chain_kernel.h -- the 1024-wide per-token INT8 layer with 8-bit output:
// codes (M, K) + row scales in, the next layer's per-token codes (M, N) +
// row scales out.  For every row m
//     y[m][n]  = act((scale_W[n] * s_in[m]) * float(sum_k A_q[m][k] W_q[n][k]) + bias[n])
//     s_out[m] = max_n |y[m][n]| / 127 (1 for an all-zero row)
//     C_q[m][n] = round_half_away(y[m][n] / s_out[m])
// which is, bit for bit, the fp32 layer output followed by the per-token
// quantise of the next layer (the absmax is order-independent and every
// code is the exact quotient's rounding).  The fp32 activations never reach
// HBM: a 65536 x 1024 layer moves 64 MiB of codes each way instead of
// 256 MiB of fp32 out and, for the next layer's quantise, 256 MiB in and
// 64 MiB of codes out.
//
// The K loop is k_gemm_wide's (wide_kernel.h): a persistent block of eight
// waves per CU walks 128 x BN tiles (BN = 256, or 128 for small M), K in
// 128-byte steps through a ring of LDS stages filled by buffer_load ... lds,
// one barrier per step, two accumulator sets so that the epilogue of tile
// t drains during the K loop of tile t + 1.  Differences:
//  - The weights are the MFMA's A operand and the activation codes its B
//    operand, so lane l of a 32 x 32 tile holds ONE output row (l % 32) and
//    16 columns, four adjacent ones per group of values: a row's absmax is a
//    register reduction plus one exchange between the two lane halves, and
//    four adjacent codes pack into one dword.
//  - A row's absmax needs all N columns, which N / BN blocks compute.  The
//    blocks of one row tile run in the same round of the tile deal (on the
//    same XCD); each publishes its rows' maxima to global memory as 64-bit
//    words (epoch << 32 | bits of the max), written through to memory (sc1),
//    and reads the others' two steps later.  The epoch of the launch tells a
//    fresh word from a stale one, so nothing needs clearing between
//    launches; a stale word (a block of the row tile running late, or a
//    line cached before it was written) is re-read from memory past the L2,
//    bounded: after spin_limit ticks of the 100 MHz clock the wave sets
//    *fault and goes on, so the kernel always ends.
//  - The drain of a tile is eight units of 16 values per lane, one per K
//    step after the step's MFMAs (the whole drain in four of the eight
//    steps measured 136 us against 107 us without it at 65536 x 1024 x
//    1024).  Units split into four groups, whether placed between the
//    MFMA parts or after them, gave wrong codes in some tiles, always in
//    one block of lanes (l % 16 >= 12) and values (0-3, 8-11) of one unit,
//    with nothing in the code to explain it; the drain keeps whole units.
//    A(i, j) forms
//    y (dequantise + bias + activation, kept in the accumulator registers as
//    float bits) of row block i (32 rows per wave), column block j, and the
//    rows' running maxima; B(i, j) quantises it.  Tile t's drain, by step of
//    tile t + 1 (step 7 of tile t for the first unit):
//        t.7 A(0,0) | .0 A(0,1), row block 0's wave maxima into LDS
//        .1 publish block 0, A(1,0) | .2 A(1,1), block 1's maxima into LDS
//        .3 fetch block 0's words, publish block 1 | .4 row scales of
//        block 0, B(0,0) | .5 fetch block 1, B(0,1) | .6 row scales of
//        block 1, B(1,0) | .7 B(1,1)
//    (128-column tiles have no column block 1: their A(i,1) / B(i,1) are
//    empty).  The fetch is an LDS DMA of the row block's words; the scales
//    are read from LDS one step later.
//  - Stage loads: A rows from the tile's row 0 with the row in the VGPR
//    offset against the tile's valid rows (zeros past them); W rows from
//    the matrix's start (W tiles are whole).  Stores put the lane's row in
//    the VGPR offset, so the hardware range check drops rows past M.
//  - Every wave issues the same memory instructions in every step (null
//    ranges where it has nothing to move), so each wait's vmcnt is a
//    compile-time count, as in k_gemm_wide.  The step's stage loads all go
//    out at its start, before any store of the drain.
#pragma once

#include "wide_kernel.h"

namespace nfq {

typedef unsigned v2u_c __attribute__((ext_vector_type(2)));

struct ChainArgs {
    const uint8_t* Aq;         // (M, K) int8 codes
    const float* scale_in;     // (M) row scales of Aq
    int64_t M;
    int K;                     // 1024
    int N;                     // multiple of BN, at most 1024
    const uint8_t* W;          // (N, K) int8
    const float* sW;           // (N)
    const float* bias;         // (N) or null
    uint8_t* Cq;               // (M, N) int8 codes out
    float* scale_out;          // (M) row scales of Cq
    uint64_t* part;            // (M rounded up to 128) x (1024 / BN) published row maxima
    uint32_t* fault;           // set to 1 when a wait for the other blocks of a row tile timed out
    uint32_t epoch;            // nonzero, different from every earlier launch on `part`
    int64_t spin_limit;        // wall-clock ticks (100 MHz) a wave waits before giving up
};

// Cache policy of the published words: written through to memory (sc1),
// where the CUs of every XCD see them.  The words are fetched from the L2
// (the blocks of a row tile share an XCD); a stale one is re-read past it.
constexpr int kChainXcdCpol = 16;
// Code stores: the L2 merges the 8-byte pieces of a row's 128-byte line that
// the two column waves of a line write.
constexpr int kChainCodeCpol = 0;

// Per-tile LDS tables (1 KB each, one DMA load each; `spare` takes the
// loads of waves with no table or no published words to fetch).
struct ChainTables {
    float sw[256];
    float bias[256];
    float sa[256];
    uint32_t spare[256];
};

// Per-token INT8 code of a = y / s by the reciprocal inv = 1 / s
// (correctly rounded), for |a| <= max |row| = 127 s: t = a * inv lies within
// 2^-22 |t| <= 2^-15 of the correctly rounded quotient q (|t| < 128), so if
// |t - rint(t)| < 0.5 - 2^-14 then |q - rint(t)| < 0.5 and
// round_half_away(q) = rint(t), no clamp needed.  Otherwise (near-ties,
// about one value in 8000, and NaN) `slow` gets the lane's bit and the
// caller takes the exact path.
__device__ __forceinline__ int32_t quant_i8_chain(float a, float inv, uint64_t& slow) {
    const float t = a * inv;
    const float r = rintf(t);
    slow |= __builtin_amdgcn_ballot_w64(!(fabsf(t - r) < 0.5f - 0x1p-14f));
    return static_cast<int32_t>(r);
}

// The lane's index, recomputed where it is used, so that lane-dependent
// offsets are not hoisted out of the tile loop (where each would hold a
// register for the whole loop).  The v_mbcnt pair is ordinary compiled code,
// so the compiler accounts for its wait states; only its zero seed is an
// SGPR written by a one-instruction asm, which the compiler cannot see
// through or hoist.  No VGPR is written inside asm anywhere in this kernel.
__device__ __forceinline__ int chain_lane() {
    uint32_t z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, z)));
}

// The drain's schedule (steps of the next tile) and the memory instructions
// of step k issued before its stage loads (right after the barrier) and
// after them (the codes of a B unit).
template <int TJ>
struct ChainSteps {
    static constexpr int NSLOT = 1024 / WideCfg<TJ>::BN;                 // published words per row
    static constexpr int PART_KB = 32 * NSLOT * 8 / 1024;   // 1 KB DMA loads per 32 rows (one wave row of a row block)
    static constexpr int PUB0 = 1, FETCH0 = 3, PUB1 = 3, USE0 = 4, FETCH1 = 5, USE1 = 6;
    static constexpr int pre(int k) {
        return (k == PUB0) + (k == FETCH0) + (k == PUB1) + (k == USE0) + (k == FETCH1) + (k == USE1);
    }
    // B units: (0,0) at step 4, (0,1) at 5, (1,0) at 6, (1,1) at 7; one store each.
    static constexpr int post(int k) { return (k == 4 || k == 6 || ((k == 5 || k == 7) && TJ == 2)) ? 1 : 0; }
};

// vmcnt at step k's wait: memory instructions issued after the stage loads
// of step k (issued in step k - LEAD of this or the previous tile), and at
// the steps that read fetched words, after that fetch.
template <int TJ>
constexpr int chain_wait(int k, int nk, int nl, int ntab, int lead) {
    using S = ChainSteps<TJ>;
    const int s = (k - lead + nk) % nk;
    int cnt = (s == 0 ? ntab : 0) + S::post(s);
    for (int d = lead - 1; d >= 1; --d) {
        const int j = (k - d + nk) % nk;
        cnt += S::pre(j) + nl + (j == 0 ? ntab : 0) + S::post(j);
    }
    // Step FETCH0's first instruction is the fetch (then the publish).
    if (k == S::USE0) cnt = cnt < 1 + nl + S::post(S::FETCH0) ? cnt : 1 + nl + S::post(S::FETCH0);
    if (k == S::USE1) cnt = cnt < nl + S::post(S::FETCH1) ? cnt : nl + S::post(S::FETCH1);
    return cnt;
}

template <int ACT, int NK, int TJ>
__global__ __launch_bounds__(kWideThreads, 1) void k_chain_wide(ChainArgs a, int ntiles) {
    using Cf = WideCfg<TJ>;
    using S = ChainSteps<TJ>;
    constexpr int BM = Cf::BM, BN = Cf::BN, NL = Cf::NL, ROW = Cf::ROW, TI = Cf::TI;
    constexpr int W = Cf::WAVES;
    constexpr int NSLOT = S::NSLOT;
    static_assert(NK == 8 && TI == 2, "schedule of the drain: eight K steps, two row blocks per wave");
    static_assert(Cf::THREADS == kWideThreads, "block size");
    static_assert(2 * S::PART_KB <= W, "one published-word load per wave at most");
    using Acc = v16i_w_t[TI][TJ];
    constexpr int NTAB = 1;                       // sw, bias, row scales: one load each, waves 0..2
    static_assert(chain_wait<TJ>(0, NK, NL, NTAB, Cf::LEAD) < 64 && chain_wait<TJ>(1, NK, NL, NTAB, Cf::LEAD) < 64 &&
                      chain_wait<TJ>(7, NK, NL, NTAB, Cf::LEAD) < 64,
                  "vmcnt field");
    static_assert(Cf::LEAD < NK && Cf::NS == Cf::LEAD + 1, "stage ring");
    __shared__ __attribute__((aligned(16))) uint8_t stages[Cf::NS][Cf::STAGE];
    __shared__ __attribute__((aligned(16))) ChainTables tb[2];
    __shared__ __attribute__((aligned(16))) float pmax[Cf::WN][BM];          // wave row maxima
    __shared__ __attribute__((aligned(16))) uint64_t pub[BM * NSLOT];       // the row tile's published words

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid / Cf::WN, wn = wid % Cf::WN;
    constexpr int K = 1024;                       // chain_ok
    const int64_t M = a.M;
    const int N = a.N;
    const int n_tiles_n = N / BN;
    const uint32_t st_base = wide_lds_addr(&stages[0][0]);
    const int lr = lane & 31, lg = lane >> 5;

    // ---- stage loads (as k_gemm_wide) ---------------------------------------
    // Load c of a wave: rows 8 q .. 8 q + 7 of the step's rows, q = wid + W c
    // (A rows for c < 2, as BM / 8 = 2 W, then W rows), lane row lane / 8,
    // 16-byte group (lane % 8) ^ ((row / 2) % 8).  An A load addresses from the
    // tile's row 0, the row in the VGPR offset, against the range of the
    // tile's valid rows (lanes past it read zeros).  W tiles are whole (N is
    // a multiple of BN), so a W load addresses from the matrix's start: the
    // wave's rows in the VGPR offset, the tile's and the load's in the
    // scalar one.
    static_assert(BM / 8 == 2 * W, "two A loads per wave");
    // Lane l fills slot l % 8 of stage row 8 (wid + 8 c) + l / 8, which holds
    // group (l % 8) ^ ((row >> 1) & 7) = (l % 8) ^ ((4 (wid & 1) + l / 16) & 7)
    // (wide_lds_off's layout), the same for every load c of the wave.
    const int ldma = (8 * wid + (lane >> 3)) * K + 16 * ((lane & 7) ^ ((4 * (wid & 1) + (lane >> 4)) & 7));
    auto dma_step = [&](uint32_t st, const WideTile& t, int step) {
        const int64_t rows_a = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const v4u ds_a = wide_desc(a.Aq + t.m0 * K, rows_a * K);
        const v4u ds_w = wide_desc(a.W, static_cast<int64_t>(N) * K);
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const uint32_t dst = st + 1024 * (wid + W * c);
            if (c < 2) wide_dma(ds_a, dst, ldma + 8 * W * c * K, ROW * step);
            else wide_dma(ds_w, dst, ldma, ROW * step + (t.n0 + 8 * W * (c - 2)) * K);
        }
    };
    // Tables of tile t into tb[par]: wave 0 scale_W, 1 bias, 2 the row
    // scales, the others zero bytes into the spare table.
    auto dma_tables = [&](int par, const WideTile& t) {
        ChainTables& T = tb[par];
        const int64_t cols = t.valid ? (N - t.n0 < BN ? N - t.n0 : BN) : 0;
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const void* src = wid == 0 ? static_cast<const void*>(a.sW + t.n0)
                        : wid == 1 ? static_cast<const void*>(a.bias ? a.bias + t.n0 : nullptr)
                        : wid == 2 ? static_cast<const void*>(a.scale_in + t.m0)
                        : nullptr;
        const int64_t len = wid == 2 ? 4 * rows : 4 * cols;
        const void* dst = wid == 0 ? static_cast<const void*>(T.sw)
                        : wid == 1 ? static_cast<const void*>(T.bias)
                        : wid == 2 ? static_cast<const void*>(T.sa) : static_cast<const void*>(T.spare);
        wide_dma(wide_desc(src, len), wide_lds_addr(dst), 16 * lane, 0);
    };

    // ---- MFMA: weights as A (rows = output columns), codes as B ------------
    Acc accA, accB;
    auto frag_read = [&](uint32_t st, int hh, v4i (&xf)[TI], v4i (&wf)[TJ]) {
        const int g = 2 * hh + lg;
#pragma unroll
        for (int i = 0; i < TI; ++i)
            xf[i] = *reinterpret_cast<lds_v4i_ptr>(st + wide_lds_off(32 * TI * wm + 32 * i + lr, g));
#pragma unroll
        for (int j = 0; j < TJ; ++j)
            wf[j] = *reinterpret_cast<lds_v4i_ptr>(st + BM * ROW + wide_lds_off(32 * TJ * wn + 32 * j + lr, g));
    };

    // ---- the drain ---------------------------------------------------------
    // Value v of lane l in tile (i, j): row 64 wm + 32 i + l % 32 of the block
    // tile, column 32 TJ wn + 32 j + 8 (v / 4) + 4 (l / 32) + v % 4.
    float rmax[TI];                    // running maxima of the lane's row in row block i
    float s_out[TI], inv_out[TI];      // its output row scale and the scale's reciprocal
    // Unit A(i, j): its 16 values.
    auto a_unit = [&](Acc& acc, int i, int j, int par, bool live = true) {
        if (!live) return;
        const ChainTables& T = tb[par];
        const float sa = T.sa[64 * wm + 32 * i + lr];
        float mx = j == 0 ? 0.0f : rmax[i];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int col = 32 * TJ * wn + 32 * j + 8 * g + 4 * lg;
            const v4f sw = *reinterpret_cast<const v4f*>(T.sw + col);
            const v4f bb = *reinterpret_cast<const v4f*>(T.bias + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float y = activate<ACT>(dequant_bias(sw[e], sa, static_cast<float>(acc[i][j][4 * g + e]), bb[e]));
                mx = fmaxf(mx, fabsf(y));
                acc[i][j][4 * g + e] = __builtin_bit_cast(int32_t, y);
            }
        }
        rmax[i] = mx;
    };
    // The wave's maxima of row block i (both lane halves) into LDS.  The
    // partner's value (lane l ^ 32) comes from two v_permlane32_swap with
    // zero: swap(v, 0) gives lanes 0..31 the value of lanes 32..63 in its
    // second result (zero in lanes 32..63), swap(0, v) gives lanes 32..63
    // the value of lanes 0..31 in its first (zero in lanes 0..31).
    auto put_wave_max = [&](int i) {
        const uint32_t v = __builtin_bit_cast(uint32_t, rmax[i]);
        const auto lo_gets = __builtin_amdgcn_permlane32_swap(v, 0u, false, false);
        const auto hi_gets = __builtin_amdgcn_permlane32_swap(0u, v, false, false);
        // Elements through scalars (bit_cast of an ext-vector element reads
        // element 0).
        const uint32_t from_hi = lo_gets[1], from_lo = hi_gets[0];
        pmax[wn][64 * wm + 32 * i + (chain_lane() & 31)] = fmaxf(rmax[i], __builtin_bit_cast(float, from_hi | from_lo));
    };
    // Publish the block's maxima of row block i (the waves of column 0,
    // lanes 0..31; the others store into a zero-byte range or past it).  The
    // row block's offset is in the scalar offset: `part` holds whole row
    // tiles, so a lane past the tile's valid rows still stores inside it,
    // and words of rows past M are never read.
    auto publish = [&](const WideTile& t, int i) {
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const int r0 = 64 * wm + 32 * i;
        float mx = pmax[0][r0 + lr];
#pragma unroll
        for (int w2 = 1; w2 < Cf::WN; ++w2) mx = fmaxf(mx, pmax[w2][r0 + lr]);
        const v2u_c word = {__builtin_bit_cast(uint32_t, mx), a.epoch};
        const auto rs = wide_rsrc(wn == 0 ? static_cast<void*>(a.part + t.m0 * NSLOT) : nullptr, rows * NSLOT * 8);
        const int ln = chain_lane();
        __builtin_amdgcn_raw_buffer_store_b64(word, rs, ln >= 32 ? 0x40000000 : ln * NSLOT * 8, (r0 * NSLOT + t.n0 / BN) * 8,
                                              kChainXcdCpol);
    };
    // DMA of row block i's published words into `pub`: per wm, 32 rows of
    // NSLOT words in PART_KB loads of 1 KB (waves 0 .. 2 PART_KB - 1; the
    // others zero bytes into the spare table).
    auto fetch = [&](const WideTile& t, int i, int par) {
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const bool mine = wid < 2 * S::PART_KB;
        const int fwm = wid / S::PART_KB, half = wid % S::PART_KB;
        const int row0 = 64 * fwm + 32 * i;
        const v4u d = wide_desc(mine ? static_cast<const void*>(a.part + (t.m0 + row0) * NSLOT + 128 * half) : nullptr,
                                (rows - row0) * NSLOT * 8 - 1024 * half);
        const uint32_t dst = mine ? wide_lds_addr(pub) + row0 * NSLOT * 8 + 1024 * half : wide_lds_addr(tb[par].spare);
        wide_dma(d, dst, 16 * lane, 0);
    };
    // Whether a row's words are this launch's (or the row is past M: its
    // words are never written).
    auto row_words_fresh = [&](const uint64_t* wds, bool past) {
        bool ok = true;
#pragma unroll
        for (int s2 = 0; s2 < NSLOT; ++s2)
            if (s2 < n_tiles_n) ok &= static_cast<uint32_t>(wds[s2] >> 32) == a.epoch;
        return ok || past;
    };
    // Scale and reciprocal of the lane's row in row block i from the
    // published words: from `pub` (or, with from_global, global memory),
    // re-reading global memory while any word is stale; then the row scales
    // (column tile 0's waves of column 0, lanes 0..31) into scale_out.
    auto row_scale = [&](const WideTile& t, int i, bool from_global) {
        const int row = 64 * wm + 32 * i + lr;
        // Past the tile's valid rows, compared in 32 bits (no 64-bit lane row).
        const int valid_rows = t.valid ? static_cast<int>(M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const bool past = row >= valid_rows;
        uint64_t wds[NSLOT];
#pragma unroll
        for (int s2 = 0; s2 < NSLOT; ++s2) wds[s2] = from_global ? 0 : pub[row * NSLOT + s2];
        bool fresh = !t.valid || (!from_global && row_words_fresh(wds, past)) || past;
        if (__builtin_amdgcn_ballot_w64(!fresh)) {
            const uint64_t t0 = wall_clock64();
            // Buffer loads with the cache policy of an agent-scope atomic
            // load (sc1), a wave-uniform descriptor and the lane's row in a
            // 32-bit offset (no 64-bit lane address held across the tile
            // loop); the empty asm with a memory clobber keeps them in the
            // loop.
            const auto rs = wide_rsrc(a.part + (t.m0 + 64 * wm + 32 * i) * NSLOT, 32 * NSLOT * 8);
            while (!fresh) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int s2 = 0; s2 < NSLOT; ++s2)
                    wds[s2] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                               rs, (chain_lane() & 31) * NSLOT * 8 + 8 * s2, 0, kChainXcdCpol));
                fresh = row_words_fresh(wds, past);
                if (!fresh && static_cast<int64_t>(wall_clock64() - t0) > a.spin_limit) {
                    __hip_atomic_store(a.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    fresh = true;
                }
            }
        }
        uint32_t mb = 0;
#pragma unroll
        for (int s2 = 0; s2 < NSLOT; ++s2)
            if (s2 < n_tiles_n) mb = static_cast<uint32_t>(wds[s2]) > mb ? static_cast<uint32_t>(wds[s2]) : mb;
        const float mx = __builtin_bit_cast(float, mb);
        const float so = (mx == 0.0f) ? 1.0f : mx / 127.0f;
        s_out[i] = so;
        inv_out[i] = 1.0f / so;
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const bool mine = wn == 0 && t.n0 == 0;
        // The row in the VGPR offset (the range check sees it).
        const int r0 = 64 * wm + 32 * i;
        const auto rs = wide_rsrc(mine ? static_cast<void*>(a.scale_out + t.m0) : nullptr, rows * 4);
        const int ln = chain_lane();
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, so), rs, (ln >= 32 ? 0x40000000 : 4 * ln) + 4 * r0,
                                              0, 0);
    };
    // Unit B(i, j): codes of y / s_out.  Group g of lane (lg, lr) packs the
    // codes of columns 8 g + 4 lg .. + 3 of row lr into dword D[g]; two
    // exchanges with the other lane half give lane lg = 0 columns 0 .. 15
    // of the unit's 32 and lane lg = 1 columns 16 .. 31, so one 16-byte
    // store per lane writes 32 rows x 32 bytes (as dword stores, 32 rows x
    // 8 bytes each: 4x the L2 write requests; measured at 65536 x 1024 x
    // 1024: 118-126 us against 123-129).
    auto b_unit = [&](Acc& acc, int i, int j, const WideTile& t) {
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const auto rs = wide_rsrc(a.Cq + t.m0 * N, rows * N);
        // The row in the VGPR offset (the range check sees it), the column
        // within the row in the scalar offset.
        const int soff = t.n0 + 32 * TJ * wn + 32 * j;   // wave-uniform
        const int ln = chain_lane();
        const int voff = ((ln & 31) + 64 * wm + 32 * i) * N + 16 * (ln >> 5);
        if (!t.valid) {
            __builtin_amdgcn_raw_buffer_store_b128(v4u{0u, 0u, 0u, 0u}, rs, voff, soff, 0);
            return;
        }
        const float inv = inv_out[i];
        uint32_t D[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // Through a scalar: clang's __builtin_bit_cast of an
                // ext-vector element reads the vector's element 0.
                const int32_t bits = acc[i][j][4 * g + e];
                y[e] = __builtin_bit_cast(float, bits);
            }
            uint64_t slow = 0;
            int32_t q[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = quant_i8_chain(y[e], inv, slow);
            if (slow) {
#pragma unroll
                for (int e = 0; e < 4; ++e) q[e] = quant_i8_token(y[e], s_out[i], inv);
            }
            D[g] = pack4(q[0], q[1], q[2], q[3]);
        }
        // v_permlane32_swap(D0, D2): lanes 0..31 keep D0 in the first result
        // and get their partner's D0 in the second; lanes 32..63 get their
        // partner's D2 in the first and keep D2 in the second -- columns
        // 0..7 and 16..23 in order, and likewise (D1, D3) for 8..15 and 24..31.
        const auto r02 = __builtin_amdgcn_permlane32_swap(D[0], D[2], false, false);
        const auto r13 = __builtin_amdgcn_permlane32_swap(D[1], D[3], false, false);
        const v4u out = {r02[0], r02[1], r13[0], r13[1]};
        __builtin_amdgcn_raw_buffer_store_b128(out, rs, voff, soff, kChainCodeCpol);
    };

    // ---- the step schedule ---------------------------------------------------
    WideTile cur = wide_tile<BM, BN>(0, ntiles, n_tiles_n);
    if (!cur.valid) return;
    {
        // The last LEAD steps of a tile before the first: their non-stage
        // instructions on zero-byte ranges, then the first tile's loads.
        const v4u none = wide_desc(nullptr, 0);
#pragma unroll
        for (int k = 0; k < Cf::LEAD; ++k) {
            const int j = NK - Cf::LEAD + k;
            for (int q = 0; q < S::pre(j); ++q) wide_null_store(none, 4 * lane);
            dma_step(st_base + Cf::STAGE * k, cur, k);
            for (int q = 0; q < S::post(j); ++q) wide_null_store(none, 4 * q);
        }
    }
    WideTile prev{0, 0, false};
    int sc = 0;

    auto tile_pass = [&](Acc& acc, Acc& pacc, int par, const WideTile& t, const WideTile& nxt, const WideTile& pt) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = v16i_w_t{};
        wide_static_for(std::make_integer_sequence<int, NK>{}, [&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int sl = sc + Cf::LEAD >= Cf::NS ? sc + Cf::LEAD - Cf::NS : sc + Cf::LEAD;
            __builtin_amdgcn_s_waitcnt(wide_waitcnt_imm(chain_wait<TJ>(k, NK, NL, NTAB, Cf::LEAD)));
            asm volatile("s_barrier" ::: "memory");
            // Before the stage loads.
            if constexpr (k == S::PUB0) publish(pt, 0);
            if constexpr (k == S::FETCH0) {
                fetch(pt, 0, par);
                publish(pt, 1);
            }
            if constexpr (k == S::USE0) row_scale(pt, 0, false);
            if constexpr (k == S::FETCH1) fetch(pt, 1, par);
            if constexpr (k == S::USE1) row_scale(pt, 1, false);
            // The stage loads of step k + LEAD (the next tile's past the end).
            constexpr int ks = k + Cf::LEAD;
            if constexpr (ks < NK) dma_step(st_base + Cf::STAGE * sl, t, ks);
            else dma_step(st_base + Cf::STAGE * sl, nxt, ks - NK);
            if constexpr (k == 0) dma_tables(par, t);
            // The step's drain unit, a group after each MFMA part.
            // (Nothing to drain before the first tile: its stores still go
            // out, on zero-byte ranges, for the counts.)
            auto unit = [&]() {
                if constexpr (k == 0) a_unit(pacc, 0, 1, par ^ 1, pt.valid);
                if constexpr (k == 1) a_unit(pacc, 1, 0, par ^ 1, pt.valid);
                if constexpr (k == 2) a_unit(pacc, 1, 1, par ^ 1, pt.valid);
                if constexpr (k == 4) b_unit(pacc, 0, 0, pt);
                if constexpr (k == 5) b_unit(pacc, 0, 1, pt);
                if constexpr (k == 6) b_unit(pacc, 1, 0, pt);
                if constexpr (k == 7) b_unit(pacc, 1, 1, pt);
            };
            const uint32_t st = st_base + Cf::STAGE * sc;
            v4i xf[4][TI], wf[4][TJ];
#pragma unroll
            for (int hh = 0; hh < 4; ++hh) {
                frag_read(st, hh, xf[hh], wf[hh]);
                __builtin_amdgcn_sched_group_barrier(0x0100, TI + TJ, 0);
#pragma unroll
                for (int i = 0; i < TI; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[hh][j], xf[hh][i], acc[i][j], 0, 0, 0);
                // The group's VALU work between the part's MFMAs.
#pragma unroll
                for (int q = 0; q < TI * TJ; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x0002, 8, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (TJ == 2 || (k != 0 && k != 2 && k != 5 && k != 7)) unit();
            // This tile's first unit, once its accumulators are final.
            if constexpr (k == NK - 1) a_unit(acc, 0, 0, par);
            if constexpr (k == 0 || k == 2) put_wave_max(k == 0 ? 0 : 1);
            sc = sc + 1 == Cf::NS ? 0 : sc + 1;
        });
    };
    // The last tile: the rest of its drain in sequence (A(0,0) ran in its
    // step 7), reading the others' words from global memory.
    auto final_drain = [&](Acc& acc, int par, const WideTile& t) {
        __builtin_amdgcn_s_waitcnt(0x070);
        asm volatile("s_barrier" ::: "memory");
        if constexpr (TJ == 2) a_unit(acc, 0, 1, par);
        put_wave_max(0);
        a_unit(acc, 1, 0, par);
        if constexpr (TJ == 2) a_unit(acc, 1, 1, par);
        put_wave_max(1);
        __syncthreads();
        publish(t, 0);
        publish(t, 1);
        row_scale(t, 0, true);
        for (int j = 0; j < TJ; ++j) b_unit(acc, 0, j, t);
        row_scale(t, 1, true);
        for (int j = 0; j < TJ; ++j) b_unit(acc, 1, j, t);
    };

#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) accB[i][j] = v16i_w_t{};
    int it = 0;
    for (;;) {
        WideTile nxt = wide_tile<BM, BN>(it + 1, ntiles, n_tiles_n);
        tile_pass(accA, accB, 0, cur, nxt, prev);
        prev = cur;
        cur = nxt;
        ++it;
        if (!cur.valid) {
            final_drain(accA, 0, prev);
            return;
        }
        nxt = wide_tile<BM, BN>(it + 1, ntiles, n_tiles_n);
        tile_pass(accB, accA, 1, cur, nxt, prev);
        prev = cur;
        cur = nxt;
        ++it;
        if (!cur.valid) {
            final_drain(accB, 1, prev);
            return;
        }
    }
}

}  // namespace nfq
