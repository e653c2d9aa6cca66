// wide_kernel.h -- the persistent INT8 GEMM for the 1024-wide per-token
// layers (K = 128 NK): C[m][n] = act((scale_W[n] * s[m]) * float(t) + bias[n]),
// t = sum_k A_q[m][k] W_q[n][k] plus the zero-point terms of the formula.
//
// Why a second GEMM kernel: with fp32 output a 1024-wide layer writes 4 bytes
// per output for 2K = 2048 int8 operations.  A non-persistent kernel stores a
// tile only after its K loop, so the output stream and the MFMAs alternate
// instead of overlapping.  Here each CU runs one block of eight waves (two per
// SIMD) that walks its tiles in sequence with two accumulator sets per wave:
// while the MFMAs of tile t accumulate into one set, the epilogue of tile
// t - 1 (dequantise, bias, activation, stores) drains from the other, an
// eighth per K step, so the stores spread over the K loop, and each SIMD's
// second wave covers the first's LDS waits and epilogue work.
//
// Layout and schedule:
//  - Block tile 128 x 256 (or 128 x 128 for small M); wave (wm, wn) of the
//    2 x 4 grid owns a 64 x 64 (64 x 32) tile as 2 x 2 (2 x 1) tiles of
//    v_mfma_i32_32x32x32_i8 with the activation codes as the A operand, so
//    value v of lane l in tile (i, j) is row 32 i + 8 (v / 4) + 4 (l / 32) +
//    v % 4, column 32 j + l % 32: a store of one value per lane writes two
//    whole 128-byte row segments.  (The 16 x 16 x 64 form measured slower:
//    97-104 us against 91-97 us at 65536 x 1024 x 1024.)
//  - K advances 128 per step.  A stage holds the step's BM + BN rows of 128
//    bytes, with 16-byte group g of row r at slot g ^ ((r >> 1) & 7).  A
//    ds_read_b128 is served 16 lanes (256 bytes, 64 banks) at a time, and a
//    fragment read of one group takes 16 consecutive rows per phase: two
//    rows share their banks exactly when they share row parity and slot, so
//    the slot follows r / 2.  (With slot g ^ (r & 7), rows r and r + 8
//    collided: 43% of the LDS's active cycles were bank-conflict stalls at
//    65536 x 1024 x 1024, none now.)  The loads are buffer_load ... lds (16 bytes per
//    lane straight into LDS); 8 lanes cover one row's whole 128-byte line, so
//    every instruction reads 8 full cache lines (with 64-byte steps each
//    instruction read 16 half lines, and the loads alone took 50 us of a
//    65536 x 1024 x 1024 GEMM).  Three stages loaded two steps ahead (four,
//    three ahead, with 128 x 128 tiles); the load stream runs across tile
//    boundaries.
//  - Per-tile tables (scale_W, bias, row scales and the integer-epilogue
//    inputs) arrive by LDS DMA with the tile's first step, double-buffered
//    by tile parity; they are read one tile later, by the drain.
//  - One barrier per step.  Every wave issues the same memory instructions in
//    every step (a tile past the last, or the slice of a tile before the
//    first, gets a buffer range of zero bytes: its loads return zeros and its
//    stores are dropped), so each wait's vmcnt is a compile-time count.  The
//    loads are inline asm, which the compiler does not track; it would
//    otherwise also wait for the drain's stores before reading a stage.
//  - Output stores are non-temporal and written through the L2 (nt | sc1):
//    the 256 MiB of a trunk layer's output would otherwise displace the
//    L2-resident weight and code lines the loads reuse (measured: 146 -> 114
//    us at 65536 x 1024 x 1024 with nt; 81 us now, with sc1 too).
//  - Tiles are dealt so that at any time each XCD works on a contiguous
//    range of tiles: the BN-column tiles of one row tile share that XCD's L2.
#pragma once

#include <type_traits>
#include <utility>

#include "common.h"
#include "rows_kernel.h"

namespace nfq {

// Cache policy of the output stores: nt | sc1 (non-temporal, written
// through the L2).  Measured at 65536 x 1024 x 1024: 81.0 us, against 84-86
// with nt alone, 113 with sc1 alone and 119 with neither; at 4096 x 1024 x
// 1024: 11.0 us against 11.3-11.6 / 11.0 / 12.5.
constexpr int kWideStoreCpol = 2 | 16;

typedef int v16i_w_t __attribute__((ext_vector_type(16)));

// Block shapes: eight waves in a 2 x 4 grid, each wave 2 x TJ tiles of
// v_mfma_i32_32x32x32_i8 (64 x 32 TJ outputs), so the block tile is
// 128 x 128 TJ.  TJ = 2 for large M (fewer loads per product); TJ = 1 when
// 128 x 256 tiles would leave CUs idle (M = 4096: 128 tiles for 256 CUs).
template <int TJ>
struct WideCfg {
    static constexpr int WM = 2, WN = 4;                     // wave grid
    static constexpr int WAVES = WM * WN;                    // two per SIMD
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int TI = 2;                             // 32 x 32 tiles per wave, rows
    static constexpr int BM = 32 * TI * WM, BN = 32 * TJ * WN;
    static constexpr int ROW = 128;                          // bytes of K per stage row
    static constexpr int STAGE = (BM + BN) * ROW;            // 48 KB / 32 KB
    // LDS stages and the load lead in steps: three stages two steps ahead
    // fill the LDS at 128 x 256 (144 KB with the tables); 128 x 128 tiles
    // take a fourth stage, three steps ahead (a CU's L2 -> LDS rate grows
    // with the loads in flight).
    static constexpr int NS = TJ == 1 ? 4 : 3;
    static constexpr int LEAD = NS - 1;
    static constexpr int NL = (BM + BN) / 8 / WAVES;         // 1 KB loads per wave per step (8 rows each)
    static constexpr int VALS = TI * TJ * 16;                // accumulator values per lane
};
constexpr int kWideThreads = 512;

typedef const __attribute__((address_space(3))) v4i* lds_v4i_ptr;

// Byte offset of 16-byte group g of stage row `row` (128-byte rows).
__device__ __forceinline__ int wide_lds_off(int row, int g) {
    return row * 128 + 16 * (g ^ ((row >> 1) & 7));
}

// Raw buffer descriptor as four dwords (base, stride 0, num_records, the
// flags __builtin_amdgcn_make_buffer_rsrc is given elsewhere in this
// library); a null base or a negative size gives a zero-byte range.
__device__ __forceinline__ v4u wide_desc(const void* p, int64_t bytes) {
    const uint64_t base = reinterpret_cast<uint64_t>(p);
    const int64_t b = p ? (bytes < 0 ? 0 : bytes) : 0;
    return v4u{static_cast<uint32_t>(base), static_cast<uint32_t>(base >> 32) & 0xFFFFu, static_cast<uint32_t>(b),
               0x00020000u};
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wide_rsrc(const void* p, int64_t bytes) {
    const int64_t b = p ? (bytes < 0 ? 0 : bytes) : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(b), 0x00020000);
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t wide_lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 16 bytes per lane from the buffer at voff + soff into LDS at lds + 16 lane
// (buffer_load_dwordx4 ... lds; M0 holds the LDS base, one wait state after
// writing it).
__device__ __forceinline__ void wide_dma(v4u desc, uint32_t lds, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(desc), "s"(soff)
                 : "memory", "m0");
}

// One dword store of zero to a zero-byte range (dropped by the hardware):
// asm, so that the compiler cannot merge a run of them into one wider store,
// which would change the count the waits rely on.
__device__ __forceinline__ void wide_null_store(v4u desc, int voff) {
    asm volatile("buffer_store_dword %0, %1, %2, 0 offen" : : "v"(0), "v"(voff), "s"(desc) : "memory");
}

struct WideTile {
    int64_t m0;
    int n0;
    bool valid;
};

// Tile k of block b: at each k the grid covers tiles [k G, (k + 1) G), and
// block b (on XCD b % 8 when G % 8 == 0) takes tile k G + (b % 8) (G / 8) + b / 8,
// so each XCD holds a contiguous range.
template <int BM, int BN>
__device__ __forceinline__ WideTile wide_tile(int k, int ntiles, int n_tiles_n) {
    const int G = gridDim.x, b = blockIdx.x;
    const int local = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
    const int t = k * G + local;
    WideTile w;
    w.valid = t < ntiles;
    const int tt = w.valid ? t : 0;
    w.m0 = static_cast<int64_t>(tt / n_tiles_n) * BM;
    w.n0 = (tt % n_tiles_n) * BN;
    return w;
}

// LDS tables of one tile: each filled by one 1 KB load (lanes past the
// source range write zeros).
struct WideTables {
    float sw[256];                // scale_W (BN used)
    float bias[256];
    float sa[256];                // row scales (BM used)
    int32_t sum_a[256];           // row code sums (INT_EPI)
    int32_t zpw[256];             // weight zero points (INT_EPI)
    int32_t c0a[256];             // weight-row byte sums (INT_EPI, row-VNNI formula with sum_W)
    int32_t c0b[256];             // the caller's sum_W (same)
    int32_t spare[256];           // target of the zero-byte loads
};

// Calls f(std::integral_constant<int, k>) for k = 0 .. sizeof...(Ks) - 1.
template <typename F, int... Ks>
__device__ __forceinline__ void wide_static_for(std::integer_sequence<int, Ks...>, F&& f) {
    (f(std::integral_constant<int, Ks>{}), ...);
}

// Memory instructions a wave has issued after the loads of step k when it
// reaches step k's wait.  Those loads were issued in step k - LEAD of this or
// the previous tile, and every step j issues, in order, NL loads (of step
// j + LEAD), NTAB table loads if j == 0 and `stores` stores.
constexpr int wide_wait(int k, int nk, int nl, int ntab, int stores, int lead) {
    int cnt = 0;
    for (int d = lead; d >= 1; --d) {
        const int j = (k - d + nk) % nk;
        if (d != lead) cnt += nl;
        cnt += (j == 0 ? ntab : 0) + stores;
    }
    return cnt;
}

// s_waitcnt with vmcnt = n (gfx9 split field), expcnt off, lgkmcnt = 0.
constexpr int wide_waitcnt_imm(int n) { return 0x070 | (n & 15) | ((n >> 4) << 14); }

template <int ACT, bool INT_EPI, int NK, int TJ>
__global__ __launch_bounds__(kWideThreads, 1) void k_gemm_wide(RowsArgs a, int ntiles, int c0_mode) {
    using Cf = WideCfg<TJ>;
    constexpr int BM = Cf::BM, BN = Cf::BN, NL = Cf::NL, ROW = Cf::ROW, TI = Cf::TI;
    constexpr int W = Cf::WAVES;
    static_assert(Cf::THREADS == kWideThreads, "block size");
    using Acc = v16i_w_t[TI][TJ];
    constexpr int NTABLES = INT_EPI ? 7 : 3;             // tables per tile
    constexpr int NTAB = (NTABLES + W - 1) / W;          // table loads per wave
    // Epilogue per K step: VALS / NK values per lane in groups of four (one
    // q of a tile), one dword store each.
    constexpr int PER_STEP = Cf::VALS / NK / 4;
    constexpr int STORES = 4 * PER_STEP;
    static_assert(Cf::VALS % (4 * NK) == 0 && PER_STEP >= 1 && NK >= 2, "epilogue split over the K steps");
    static_assert(wide_wait(0, NK, NL, NTAB, STORES, Cf::LEAD) < 64 &&
                  wide_wait(1, NK, NL, NTAB, STORES, Cf::LEAD) < 64 &&
                  wide_wait(2, NK, NL, NTAB, STORES, Cf::LEAD) < 64, "vmcnt field");
    static_assert(Cf::LEAD < NK && Cf::NS == Cf::LEAD + 1, "stage ring");
    __shared__ __attribute__((aligned(16))) uint8_t stages[Cf::NS][Cf::STAGE];
    __shared__ __attribute__((aligned(16))) WideTables tb[2];

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid / Cf::WN, wn = wid % Cf::WN;
    const int K = a.K;   // == 128 NK
    const int64_t M = a.M;
    const int N = a.N;
    const int n_tiles_n = (N + BN - 1) / BN;
    const uint32_t st_base = wide_lds_addr(&stages[0][0]);

    // ---- loads of one K step of a tile into a stage ------------------------
    // Load c of this wave fills 8-row region q = wid + W c (A rows first, then
    // W rows); lane l fills slot l of the region's 1 KB: row 8 q + l / 8,
    // slot l % 8, which holds group (l % 8) ^ ((row >> 1) & 7) of that row.  The
    // offset within the tile's rows is fixed per load; the step enters as the
    // scalar offset 128 step.
    int dvoff[NL];
#pragma unroll
    for (int c = 0; c < NL; ++c) {
        const int q = wid + W * c;
        const int row = 8 * q + (lane >> 3);
        const int grp = (lane & 7) ^ ((row >> 1) & 7);
        dvoff[c] = (q < BM / 8 ? row : row - BM) * K + 16 * grp;
    }
    // Loads c0 .. c1 - 1 of the step (all of them by default).
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
    // Tables of tile t into tb[par]: table e is loaded by wave e % W; a wave
    // with none left loads zero bytes into the spare table, so every wave
    // issues NTAB loads.  (Selects, not arrays: an indexed local array would
    // live in scratch memory, whose accesses count in vmcnt.)
    auto dma_tables = [&](int par, const WideTile& t) {
        WideTables& T = tb[par];
        const int64_t cols = t.valid ? (N - t.n0 < BN ? N - t.n0 : BN) : 0;
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
#pragma unroll
        for (int c = 0; c < NTAB; ++c) {
            const int e = wid + W * c;
            const void* src = e == 0 ? static_cast<const void*>(a.sW + t.n0)
                            : e == 1 ? static_cast<const void*>(a.bias ? a.bias + t.n0 : nullptr)
                            : e == 2 ? static_cast<const void*>(a.scale_in + t.m0)
                            : (INT_EPI && e == 3) ? static_cast<const void*>(a.sum_in ? a.sum_in + t.m0 : nullptr)
                            : (INT_EPI && e == 4) ? static_cast<const void*>(a.zpW ? a.zpW + t.n0 : nullptr)
                            : (INT_EPI && e == 5) ? static_cast<const void*>(c0_mode ? a.colsum_in + t.n0 : nullptr)
                            : (INT_EPI && e == 6) ? static_cast<const void*>(c0_mode ? a.sumW + t.n0 : nullptr)
                            : nullptr;
            const int64_t len = (e == 2 || e == 3) ? 4 * rows : 4 * cols;
            const int32_t* dst = e == 0 ? reinterpret_cast<const int32_t*>(T.sw)
                               : e == 1 ? reinterpret_cast<const int32_t*>(T.bias)
                               : e == 2 ? reinterpret_cast<const int32_t*>(T.sa)
                               : (INT_EPI && e == 3) ? T.sum_a
                               : (INT_EPI && e == 4) ? T.zpw
                               : (INT_EPI && e == 5) ? T.c0a
                               : (INT_EPI && e == 6) ? T.c0b : T.spare;
            wide_dma(wide_desc(src, len), wide_lds_addr(dst), 16 * lane, 0);
        }
    };

    // ---- accumulators and the MFMA operand reads ----------------------------
    // K part hh (32 bytes) of a step: lane l reads row l % 32 of each 32-row
    // fragment, 16-byte group 2 hh + l / 32 (the same k order for both
    // operands).
    Acc accA, accB;
    const int lr = lane & 31, lg = lane >> 5;
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
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xf[i], wf[j], acc[i][j], 0, 0, 0);
    };

    // ---- epilogue slice sl of a finished accumulator set --------------------
    // Values 4 (sl PER_STEP + qq) + e of the lane's TI x TJ x 16, tile (i, j)
    // = value index / 16, its rows 8 q + e.  Rows past M, columns past N and
    // tiles that do not exist fall outside the store range (an offset past it
    // for the columns), so there is no branch.  t = D + c0 + c1 SA (zp_A = 0:
    // c1 = -2 zp_W and, for the row-VNNI formula with a caller's sum_W,
    // c0 = 128 (W-row byte sum - sum_W): the forms of int_epi_consts), then
    // the reference's dequantise order.
    //
    // The lane's TJ columns' constants are read from the tables once per tile
    // (slice 0) into registers.
    struct ColC {
        float sw[TJ], bb[TJ];
        int32_t c0[TJ], c1[TJ];
    };
    auto col_consts = [&](const WideTables& T_, ColC& cc) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = 32 * TJ * wn + 32 * j + lr;
            cc.sw[j] = T_.sw[col];
            cc.bb[j] = T_.bias[col];
            if constexpr (INT_EPI) {
                cc.c1[j] = static_cast<int32_t>(0u - 2u * static_cast<uint32_t>(T_.zpw[col]));
                cc.c0[j] = static_cast<int32_t>(128u * (static_cast<uint32_t>(T_.c0a[col]) -
                                                        static_cast<uint32_t>(T_.c0b[col])));
            }
        }
    };
    // Groups q0 .. q1 - 1 of slice sl (all of it by default).
    auto drain = [&](const Acc& acc, int par, const WideTile& t, ColC& cc, auto slc, int q0 = 0,
                     int q1 = Cf::VALS / NK / 4) {
        constexpr int sl = decltype(slc)::value;
        const WideTables& T_ = tb[par];
        if (sl == 0 && q0 == 0) col_consts(T_, cc);
        const int64_t rows = t.valid ? (M - t.m0 < BM ? M - t.m0 : BM) : 0;
        const auto rs = wide_rsrc(static_cast<float*>(a.C) + t.m0 * N, rows * N * 4);
#pragma unroll
        for (int qq = 0; qq < PER_STEP; ++qq) {
            if (qq < q0 || qq >= q1) continue;
            const int vi = 4 * (sl * PER_STEP + qq);
            const int i = vi / (16 * TJ), j = (vi / 16) % TJ, q = (vi % 16) / 4;
            const int col = 32 * TJ * wn + 32 * j + lr;       // within the block tile
            const int row0 = 32 * TI * wm + 32 * i + 4 * lg + 8 * q;
            const uint32_t voff0 = t.n0 + col < N ? static_cast<uint32_t>((row0 * N + t.n0 + col) * 4) : 0x80000000u;
            const v4f sa = *reinterpret_cast<const v4f*>(T_.sa + row0);
            v4i sa_i = {0, 0, 0, 0};
            if constexpr (INT_EPI) sa_i = *reinterpret_cast<const v4i*>(T_.sum_a + row0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int32_t d = acc[i][j][4 * q + e];
                float tv;
                if constexpr (INT_EPI)
                    tv = static_cast<float>(static_cast<int32_t>(static_cast<uint32_t>(d) + static_cast<uint32_t>(cc.c0[j]) +
                                                                 static_cast<uint32_t>(cc.c1[j]) * static_cast<uint32_t>(sa_i[e])));
                else
                    tv = static_cast<float>(d);
                const float y = activate<ACT>(dequant_bias(cc.sw[j], sa[e], tv, cc.bb[j]));
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), rs,
                                                      static_cast<int>(voff0 + static_cast<uint32_t>(e * N * 4)), 0, kWideStoreCpol);
            }
        }
    };

    // ---- the step schedule -------------------------------------------------
    // Step k of a tile: wait for this wave's loads of step k, barrier (every
    // wave's loads of step k have landed, and every wave has finished reading
    // the stage that step k + LEAD overwrites), the loads of step k + LEAD
    // (the next tile's past the end), the tile's own tables at k = 0, the
    // MFMAs, then slice k of the previous tile's epilogue.  The prologue
    // issues steps 0 .. LEAD - 1, each followed by STORES stores to a
    // zero-byte range: the instruction sequence of a tile's last LEAD steps,
    // so that the first tile's waits count right.  (Every wait counts this wave's vector
    // memory instructions exactly; the drain's stores go to rows N floats
    // apart, N unknown at compile time, so they cannot be merged either.)
    WideTile cur = wide_tile<BM, BN>(0, ntiles, n_tiles_n);
    if (!cur.valid) return;
    {
        const v4u none = wide_desc(nullptr, 0);
#pragma unroll
        for (int k = 0; k < Cf::LEAD; ++k) {
            dma_step(st_base + Cf::STAGE * k, cur, k);
#pragma unroll
            for (int q = 0; q < STORES; ++q) wide_null_store(none, 4 * q);
        }
    }
    WideTile prev{0, 0, false};
    int sc = 0;   // stage of the current step: the global step number mod NS

    auto tile_pass = [&](Acc& acc, const Acc& pacc, int par, const WideTile& t, const WideTile& nxt,
                         const WideTile& pt) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = v16i_w_t{};
        ColC cc;
        wide_static_for(std::make_integer_sequence<int, NK>{}, [&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int sl = sc + Cf::LEAD >= Cf::NS ? sc + Cf::LEAD - Cf::NS : sc + Cf::LEAD;
            __builtin_amdgcn_s_waitcnt(wide_waitcnt_imm(wide_wait(k, NK, NL, NTAB, STORES, Cf::LEAD)));
            asm volatile("s_barrier" ::: "memory");
            constexpr int ks = k + Cf::LEAD;
            // The step's loads go out in groups of NLP, one group ahead of
            // each K part's MFMAs, then the tables: the same instruction
            // order as one burst (the waits count the same), spread over the
            // step.
            constexpr int NLP = (NL + 2) / 3;
            auto dma_group = [&](int hh) {
                if (hh * NLP >= NL) return;
                if constexpr (ks < NK) dma_step(st_base + Cf::STAGE * sl, t, ks, hh * NLP, hh * NLP + NLP);
                else dma_step(st_base + Cf::STAGE * sl, nxt, ks - NK, hh * NLP, hh * NLP + NLP);
                if (k == 0 && hh * NLP + NLP >= NL) dma_tables(par, t);
            };
            // Parts 0 and 1 are read first; each later part is read while the
            // MFMAs of the part two before it run.  The scheduling groups pin
            // that order: left to itself the scheduler moves each read next to
            // its MFMA (fewer live registers) and every MFMA then waits for a
            // whole LDS round trip.
            const uint32_t st = st_base + Cf::STAGE * sc;
            v4i xf[4][TI], wf[4][TJ];
            frag_read(st, 0, xf[0], wf[0]);
            frag_read(st, 1, xf[1], wf[1]);
            __builtin_amdgcn_sched_group_barrier(0x0100, 2 * (TI + TJ), 0);   // DS reads
#pragma unroll
            for (int hh = 0; hh < 4; ++hh) {
                dma_group(hh);
                if (hh + 2 < 4) {
                    frag_read(st, hh + 2, xf[hh + 2], wf[hh + 2]);
                    __builtin_amdgcn_sched_group_barrier(0x0100, TI + TJ, 0);
                }
                mfma_part(acc, xf[hh], wf[hh]);
                __builtin_amdgcn_sched_group_barrier(0x0008, TI * TJ, 0);     // MFMA
                // Half of the slice's stores after part 2's MFMAs, the rest
                // after part 3's: after the step's last loads either way, so
                // the waits count the same.
                if constexpr (PER_STEP >= 2) {
                    if (hh == 2) {
                        __builtin_amdgcn_sched_barrier(0);
                        drain(pacc, par ^ 1, pt, cc, kc, 0, PER_STEP / 2);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            drain(pacc, par ^ 1, pt, cc, kc, PER_STEP >= 2 ? PER_STEP / 2 : 0, PER_STEP);
            sc = sc + 1 == Cf::NS ? 0 : sc + 1;
        });
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
            // accA holds the last tile (parity 0).
            __builtin_amdgcn_s_waitcnt(0x070);
            asm volatile("s_barrier" ::: "memory");
            ColC cc;
            wide_static_for(std::make_integer_sequence<int, NK>{}, [&](auto sc2) { drain(accA, 0, prev, cc, sc2); });
            return;
        }
        nxt = wide_tile<BM, BN>(it + 1, ntiles, n_tiles_n);
        tile_pass(accB, accA, 1, cur, nxt, prev);
        prev = cur;
        cur = nxt;
        ++it;
        if (!cur.valid) {
            __builtin_amdgcn_s_waitcnt(0x070);
            asm volatile("s_barrier" ::: "memory");
            ColC cc;
            wide_static_for(std::make_integer_sequence<int, NK>{}, [&](auto sc2) { drain(accB, 1, prev, cc, sc2); });
            return;
        }
    }
}

}  // namespace nfq
