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
//    blocks of one row tile run in the same round of the tile deal, on the
//    same XCD; each publishes its 128 row maxima to global memory as 64-bit
//    words (epoch << 32 | bits of the max), written through to memory (sc1),
//    and reads the others' two steps later.  The epoch of the launch tells a
//    fresh word from a stale one, so nothing needs clearing between
//    launches; a stale word means a block of the row tile is late, and the
//    wave re-reads (bounded: after spin_limit ticks of the 100 MHz clock it
//    sets *fault and goes on, so the kernel always ends).
//  - Drain of tile t during tile t + 1, by step: 0 -> y of row block i = 0
//    (dequantise + bias + activation, kept in the accumulator registers as
//    float bits) and its row maxima; 1 -> the same for i = 1, then the
//    wave's row maxima into LDS; 2 -> the block's maxima (max over the four
//    column waves) published; 5 -> the row tile's published words DMA'd
//    into LDS; 6 -> checked, the row scales formed (and stored by the
//    column-tile-0 block), codes of i = 0 stored; 7 -> codes of i = 1.
//  - Every wave issues the same memory instructions in every step (null
//    ranges where it has nothing to move), so each wait's vmcnt is a
//    compile-time count, as in k_gemm_wide.
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

// Cache policy of the published words: written through to memory and read
// past the L2 (sc1), the coherence point of the CUs of different XCDs.
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

// Memory instructions of step k of a tile issued before its stage loads
// (right after the barrier) and after them (with the step's MFMAs).
template <int TJ>
struct ChainSteps {
    static constexpr int NSLOT = 1024 / WideCfg<TJ>::BN;        // published words per row
    static constexpr int PART_KB = WideCfg<TJ>::BM * NSLOT * 8 / 1024;   // 1 KB DMA loads per tile
    static constexpr int PUBLISH = 2, FETCH = 5, USE = 6;
    static constexpr int pre(int k) { return k == PUBLISH ? 1 : k == FETCH ? 1 : k == USE ? 1 : 0; }
    static constexpr int post(int k) { return k == USE || k == USE + 1 ? 4 * TJ : 0; }
};

// vmcnt at step k's wait: memory instructions issued after the stage loads
// of step k (issued in step k - LEAD of this or the previous tile).
template <int TJ>
constexpr int chain_wait(int k, int nk, int nl, int ntab, int lead) {
    using S = ChainSteps<TJ>;
    const int s = (k - lead + nk) % nk;
    int cnt = (s == 0 ? ntab : 0) + S::post(s);
    for (int d = lead - 1; d >= 1; --d) {
        const int j = (k - d + nk) % nk;
        cnt += S::pre(j) + nl + (j == 0 ? ntab : 0) + S::post(j);
    }
    // Step USE reads what step FETCH's first instruction DMA'd.
    if (k == S::USE) {
        const int j = S::FETCH;
        const int after = nl + (j == 0 ? ntab : 0) + S::post(j);
        cnt = cnt < after ? cnt : after;
    }
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
    static_assert(S::PART_KB <= W, "one published-word load per wave at most");
    using Acc = v16i_w_t[TI][TJ];
    constexpr int NTAB = 1;                       // sw, bias, row scales: one load each, waves 0..2
    static_assert(chain_wait<TJ>(0, NK, NL, NTAB, Cf::LEAD) < 64 && chain_wait<TJ>(6, NK, NL, NTAB, Cf::LEAD) < 64,
                  "vmcnt field");
    static_assert(Cf::LEAD < NK && Cf::NS == Cf::LEAD + 1, "stage ring");
    __shared__ __attribute__((aligned(16))) uint8_t stages[Cf::NS][Cf::STAGE];
    __shared__ __attribute__((aligned(16))) ChainTables tb[2];
    __shared__ __attribute__((aligned(16))) float pmax[Cf::WN][BM];          // wave row maxima
    __shared__ __attribute__((aligned(16))) uint64_t pub[BM * NSLOT];       // the row tile's published words

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid / Cf::WN, wn = wid % Cf::WN;
    const int K = a.K;
    const int64_t M = a.M;
    const int N = a.N;
    const int n_tiles_n = N / BN;
    const uint32_t st_base = wide_lds_addr(&stages[0][0]);
    const int lr = lane & 31, lg = lane >> 5;

    // ---- stage loads (as k_gemm_wide) ---------------------------------------
    int dvoff[NL];
#pragma unroll
    for (int c = 0; c < NL; ++c) {
        const int q = wid + W * c;
        const int row = 8 * q + (lane >> 3);
        const int grp = (lane & 7) ^ (row & 7);
        dvoff[c] = (q < BM / 8 ? row : row - BM) * K + 16 * grp;
    }
    auto dma_step = [&](uint32_t st, const WideTile& t, int step, int c0 = 0, int c1 = Cf::NL) {
        const int64_t rows_a = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const int64_t rows_w = t.valid ? (N - t.n0 < BN ? N - t.n0 : BN) : 0;
        const v4u ds_a = wide_desc(a.Aq + t.m0 * K, rows_a * K);
        const v4u ds_w = wide_desc(a.W + static_cast<int64_t>(t.n0) * K, rows_w * K);
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const int q = wid + W * c;
            if (c >= c0 && c < c1) wide_dma(q < BM / 8 ? ds_a : ds_w, st + 1024 * q, dvoff[c], ROW * step);
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
    auto mfma_part = [&](Acc& acc, const v4i (&xf)[TI], const v4i (&wf)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[j], xf[i], acc[i][j], 0, 0, 0);
    };

    // ---- the drain ---------------------------------------------------------
    // Value v of lane l in tile (i, j): row 64 wm + 32 i + l % 32 of the block
    // tile, column 32 TJ wn + 32 j + 8 (v / 4) + 4 (l / 32) + v % 4.
    float rmax[TI];
    float s_row = 1.0f, inv_row = 1.0f;     // this lane's row 64 wm + lane: scale and reciprocal
    // Phase A of row block i: y in place of the accumulators, row maxima.
    auto phase_a = [&](Acc& acc, int i, int par) {
        const ChainTables& T = tb[par];
        const float sa = T.sa[64 * wm + 32 * i + lr];
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < TJ; ++j)
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
        rmax[i] = fmaxf(mx, __shfl_xor(mx, 32));
    };
    // The wave's row maxima into LDS: lane (lg, lr) holds row 32 lg + lr.
    auto put_wave_max = [&]() { pmax[wn][64 * wm + lane] = lg ? rmax[1] : rmax[0]; };
    // Publish the block's row maxima (waves of column 0; the others store
    // into a zero-byte range).
    auto publish = [&](const WideTile& t) {
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const bool mine = wn == 0;
        float mx = pmax[0][64 * wm + lane];
#pragma unroll
        for (int w2 = 1; w2 < Cf::WN; ++w2) mx = fmaxf(mx, pmax[w2][64 * wm + lane]);
        const v2u_c word = {__builtin_bit_cast(uint32_t, mx), a.epoch};
        const auto rs = wide_rsrc(mine ? static_cast<void*>(a.part + t.m0 * NSLOT) : nullptr, rows * NSLOT * 8);
        const int ct = t.n0 / BN;
        __builtin_amdgcn_raw_buffer_store_b64(word, rs, ((64 * wm + lane) * NSLOT + ct) * 8, 0, kChainXcdCpol);
    };
    // DMA of the row tile's published words into `pub` (waves 0 ..
    // PART_KB - 1; the others zero bytes into the spare table).
    auto fetch = [&](const WideTile& t, int par) {
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const bool mine = wid < S::PART_KB;
        const v4u d = wide_desc(mine ? static_cast<const void*>(a.part + t.m0 * NSLOT + 128 * wid) : nullptr,
                                rows * NSLOT * 8 - 1024 * wid);
        const uint32_t dst = mine ? wide_lds_addr(pub) + 1024 * wid : wide_lds_addr(tb[par].spare);
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen sc1 lds"
                     :
                     : "s"(dst), "v"(16 * lane), "s"(d)
                     : "memory", "m0");
    };
    // Whether word s of row `row` (block-tile index) is this launch's.
    auto row_words_fresh = [&](const uint64_t* wds, int64_t grow) {
        bool ok = true;
#pragma unroll
        for (int s2 = 0; s2 < NSLOT; ++s2)
            if (s2 < n_tiles_n) ok &= static_cast<uint32_t>(wds[s2] >> 32) == a.epoch;
        return ok || grow >= M;
    };
    // The row scale from the published words of the lane's row 64 wm +
    // lane: from `pub` (or, with from_global, global memory), re-reading
    // global memory while any word is stale.
    auto row_scale = [&](const WideTile& t, bool from_global) {
        const int row = 64 * wm + lane;
        const int64_t grow = t.m0 + row;
        uint64_t wds[NSLOT];
#pragma unroll
        for (int s2 = 0; s2 < NSLOT; ++s2) wds[s2] = from_global ? 0 : pub[row * NSLOT + s2];
        bool fresh = !t.valid || (!from_global && row_words_fresh(wds, grow)) || grow >= M;
        if (__builtin_amdgcn_ballot_w64(!fresh)) {
            const uint64_t t0 = wall_clock64();
            while (!fresh) {
#pragma unroll
                for (int s2 = 0; s2 < NSLOT; ++s2)
                    wds[s2] = __hip_atomic_load(a.part + grow * NSLOT + s2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                fresh = row_words_fresh(wds, grow);
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
        s_row = (mx == 0.0f) ? 1.0f : mx / 127.0f;
        inv_row = 1.0f / s_row;
        // Column tile 0's wave of column 0 stores the scales.
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const bool mine = wn == 0 && t.n0 == 0;
        const auto rs = wide_rsrc(mine ? static_cast<void*>(a.scale_out + t.m0) : nullptr, rows * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s_row), rs, 4 * row, 0, 0);
    };
    // Phase B of row block i: codes of y / s_out, four per dword.
    auto phase_b = [&](Acc& acc, int i, const WideTile& t) {
        const float s = __shfl(s_row, 32 * i + lr);
        const float inv = __shfl(inv_row, 32 * i + lr);
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const auto rs = wide_rsrc(a.Cq + t.m0 * N, rows * N);
        const int rbase = (64 * wm + 32 * i + lr) * N + t.n0;
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = 32 * TJ * wn + 32 * j + 8 * g + 4 * lg;
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
                for (int e = 0; e < 4; ++e) q[e] = quant_i8_near(y[e], inv, slow);
                if (slow) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) q[e] = quant_i8_token(y[e], s, inv);
                }
                __builtin_amdgcn_raw_buffer_store_b32(pack4(q[0], q[1], q[2], q[3]), rs, rbase + col, 0, kChainCodeCpol);
            }
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
            if (S::pre(j) == 1) {
                if (j == S::FETCH) wide_dma(none, wide_lds_addr(tb[0].spare), 16 * lane, 0);
                else wide_null_store(none, 4 * lane);
            }
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
            // Instructions before the stage loads.
            if constexpr (k == S::PUBLISH) publish(pt);
            if constexpr (k == S::FETCH) fetch(pt, par);
            if constexpr (k == S::USE) row_scale(pt, false);
            constexpr int ks = k + Cf::LEAD;
            constexpr int NLP = (NL + 2) / 3;
            auto dma_group = [&](int hh) {
                if (hh * NLP >= NL) return;
                if constexpr (ks < NK) dma_step(st_base + Cf::STAGE * sl, t, ks, hh * NLP, hh * NLP + NLP);
                else dma_step(st_base + Cf::STAGE * sl, nxt, ks - NK, hh * NLP, hh * NLP + NLP);
                if (k == 0 && hh * NLP + NLP >= NL) dma_tables(par, t);
            };
            const uint32_t st = st_base + Cf::STAGE * sc;
            v4i xf[4][TI], wf[4][TJ];
            frag_read(st, 0, xf[0], wf[0]);
            frag_read(st, 1, xf[1], wf[1]);
            __builtin_amdgcn_sched_group_barrier(0x0100, 2 * (TI + TJ), 0);
#pragma unroll
            for (int hh = 0; hh < 4; ++hh) {
                dma_group(hh);
                if (hh + 2 < 4) {
                    frag_read(st, hh + 2, xf[hh + 2], wf[hh + 2]);
                    __builtin_amdgcn_sched_group_barrier(0x0100, TI + TJ, 0);
                }
                mfma_part(acc, xf[hh], wf[hh]);
                __builtin_amdgcn_sched_group_barrier(0x0008, TI * TJ, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            // Instructions after the stage loads.
            if constexpr (k == 0) phase_a(pacc, 0, par ^ 1);
            if constexpr (k == 1) {
                phase_a(pacc, 1, par ^ 1);
                put_wave_max();
            }
            if constexpr (k == S::USE) phase_b(pacc, 0, pt);
            if constexpr (k == S::USE + 1) phase_b(pacc, 1, pt);
            sc = sc + 1 == Cf::NS ? 0 : sc + 1;
        });
    };
    // The last tile: the whole drain in sequence.
    auto final_drain = [&](Acc& acc, int par, const WideTile& t) {
        __builtin_amdgcn_s_waitcnt(0x070);
        asm volatile("s_barrier" ::: "memory");
        phase_a(acc, 0, par);
        phase_a(acc, 1, par);
        put_wave_max();
        __syncthreads();
        publish(t);
        // Every wave reads the row tile's words from global memory.
        row_scale(t, true);
        phase_b(acc, 0, t);
        phase_b(acc, 1, t);
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
