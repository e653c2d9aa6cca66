// launch_rows.h -- the row-tile kernel launchers (rows_kernel.h); included by
// the rows_*.hip units, each instantiating its own input / output modes.
#pragma once

#include "launch.h"
#include "rows_kernel.h"

namespace nfq {

// Persistent launch: one wave per resident slot, each looping over row tiles.
template <int KB, bool FP8, int IN, int OUT, int ACT, bool HOIST, bool KFULL>
static void launch_rows_k(const RowsArgs& a, hipStream_t st) {
    auto kern = k_rows<KB, FP8, IN, OUT, ACT, HOIST, KFULL>;
    static const int per_cu = resident_blocks(kern);
    const int64_t tiles = (a.M + 15) / 16;
    const unsigned grid = grid_for(tiles, 4, per_cu);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, st, a);
}

template <int KB, bool FP8, int IN, int OUT, int ACT, bool KFULL>
static void launch_rows_h(const RowsArgs& a, hipStream_t st) {
    if constexpr (rows_hoist_fits(KB, FP8)) {
        if (a.N <= 64) {
            launch_rows_k<KB, FP8, IN, OUT, ACT, true, KFULL>(a, st);
            return;
        }
    }
    launch_rows_k<KB, FP8, IN, OUT, ACT, false, KFULL>(a, st);
}

template <int KB, bool FP8, int IN, int OUT, int ACT>
static void launch_rows_kb(const RowsArgs& a, hipStream_t st) {
    // The fixed-scale paths (LinearForward / LinearForwardBatched) are not
    // the hot loop: one instantiation with range checks serves every K.
    if (IN != IN_F32_FIXED && a.K == KB * 64) launch_rows_h<KB, FP8, IN, OUT, ACT, true>(a, st);
    else launch_rows_h<KB, FP8, IN, OUT, ACT, false>(a, st);
}

template <bool FP8, int IN, int OUT, int ACT>
static void launch_rows_act(const RowsArgs& a, hipStream_t st) {
    const int kb = (a.K + 63) / 64;
    if (kb <= 1) launch_rows_kb<1, FP8, IN, OUT, ACT>(a, st);
    else if (kb <= 2) launch_rows_kb<2, FP8, IN, OUT, ACT>(a, st);
    else if (kb <= 4) launch_rows_kb<4, FP8, IN, OUT, ACT>(a, st);
    else if constexpr (IN == IN_CODES) {
        if (kb <= 8) launch_rows_kb<8, FP8, IN, OUT, ACT>(a, st);
        else launch_rows_kb<16, FP8, IN, OUT, ACT>(a, st);
    }
}

template <bool FP8, int IN, int OUT>
void launch_rows(const RowsArgs& a, int act, hipStream_t st) {
    if constexpr (OUT == OUT_RAW) {
        launch_rows_act<FP8, IN, OUT, ACT_NONE>(a, st);
    } else {
        if (act == ACT_RELU) launch_rows_act<FP8, IN, OUT, ACT_RELU>(a, st);
        else if (act == ACT_GELU_TANH) launch_rows_act<FP8, IN, OUT, ACT_GELU_TANH>(a, st);
        else launch_rows_act<FP8, IN, OUT, ACT_NONE>(a, st);
    }
}

}  // namespace nfq
