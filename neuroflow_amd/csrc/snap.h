// snap.h -- the exponent of the runtime's log2 "FP8" snap (fno.cpp:579-606):
// e = int(std::round(std::log2(a) * 8) / 8) for 2^-6 <= a <= FLT_MAX, read
// off a table thr of the 15 step points (thr[j] the smallest float with
// e >= j - 5, located with the host's libm when the runtime is created).
//
// Each step lies within 512 ulps of 2^(j - 6 + 1/16) (steps to e <= 0) or
// 2^(j - 5 - 1/16) (steps to e >= 1), so step j lies in the binade
// [2^(j-6), 2^(j-5)) and every binade B = -6 .. 8 holds exactly one step.
// For a in binade B the count of steps <= a is then (B + 6) plus the one
// compare with the step in its own binade.  Usable from host and device code.
#pragma once

#include "gelu_exact.h"

namespace nfq {

// -6 + #{j : thr[j] <= a}: the definition.
NFQ_HD inline int snap_exponent_count(float a, const float* thr) {
    int e = -6;
#pragma unroll
    for (int j = 0; j < 15; ++j) e += a >= thr[j] ? 1 : 0;
    return e;
}

// The same from a's binade and one compare (one table read, any index).
NFQ_HD inline int snap_exponent_binade(float a, const float* thr) {
    const int b = static_cast<int>((gx_bits(a) >> 23) & 0xffu) - 127;
    const int j = b + 6 < 14 ? b + 6 : 14;
    return b >= 9 ? 9 : b + (a >= thr[j] ? 1 : 0);
}

// Whether thr has one step per binade as snap_exponent_binade assumes.
NFQ_HD inline bool snap_table_binned(const float* thr) {
    for (int j = 0; j < 15; ++j)
        if (static_cast<int>((gx_bits(thr[j]) >> 23) & 0xffu) - 127 != j - 6) return false;
    return true;
}

}  // namespace nfq
