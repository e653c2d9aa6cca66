// gemm.hip -- launchers of the tiled INT8 MFMA GEMM (gemm_kernel.h).
#include "gemm_kernel.h"
#include "launch.h"
#include "wide_kernel.h"

namespace nfq {

bool gemm_ok(const RowsArgs& a) {
    // K <= 65536 keeps a 256-row tile's byte count inside the 32-bit buffer range.
    return a.K % 64 == 0 && a.K >= 128 && a.K <= 65536 && a.N % 4 == 0 && a.kb_dot * 64 >= a.K &&
           aligned(a.Aq, 16) && aligned(a.W, 16) && aligned(a.C, 16);
}

template <int TM, int TN, int OUT, int ACT>
static void launch_gemm_t(const RowsArgs& a, hipStream_t st) {
    auto kern = k_gemm<TM, TN, OUT, ACT>;
    constexpr size_t lds = gemm_lds_bytes<TM, TN>();
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)attr;  // a failure surfaces as a launch error
    using S = GemmShape<TM, TN>;
    const int64_t blocks = ((a.M + S::BM - 1) / S::BM) * ((a.N + S::BN - 1) / S::BN);
    // MI355X deals blocks round-robin to 8 XCDs of 32 CUs.
    const int groups = num_cus() % 8 == 0 ? 8 : 1;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(256), lds, st, a, groups);
}

// Tile shape: 128 x 256 for large M and N (two blocks per CU); 64 x 128 for
// M <= 4096 with N >= 512 (twice the blocks of 128 x 128: at C5's branch,
// M = 4096, K = N = 1024, 12.6 us against 13.7 us, and 14.2 us at 64 x 64);
// else 128 x 128.  Measured on MI355X: 256 x 256 (one wave per SIMD) never
// beats 128 x 256, 64 x 128 loses at the trunk (173 us against 139 us).
static int gemm_shape(const RowsArgs& a) {
    // A gemm_tile override of 88|48|44|24|22 forces a shape (for tile sweeps;
    // 22 and 24 only on the LDS-DMA kernel).
    const int t = kernel_path().gemm_tile.load(std::memory_order_relaxed);
    if (t == 88 || t == 48 || t == 44 || t == 22 || t == 24) return t;
    if (a.M >= 16384 && a.N >= 1024) return 48;
    return (a.M <= 4096 && a.N >= 512) ? 24 : 44;
}

template <int TM, int TN, int OUT, int ACT>
static void launch_pipe_t(const RowsArgs& a, hipStream_t st) {
    using S = GemmShape<TM, TN>;
    const int64_t blocks = ((a.M + S::BM - 1) / S::BM) * ((a.N + S::BN - 1) / S::BN);
    const int groups = num_cus() % 8 == 0 ? 8 : 1;
    const int mf = kernel_path().gemm_mfma.load(std::memory_order_relaxed);
    if (mf == 32)
        hipLaunchKernelGGL((k_gemm_pipe<TM, TN, OUT, ACT, 32>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           a, groups);
    else
        hipLaunchKernelGGL((k_gemm_pipe<TM, TN, OUT, ACT, 16>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           a, groups);
}

// The LDS-DMA kernel takes every case whose epilogue needs no byte sums of
// its own: zp_A = 0, row sums given when zero points may be nonzero, and
// weight-row sums given when the row-VNNI formula has a caller's sum_W.
bool gemm_pipe_ok(const RowsArgs& a, int out) {
    if (a.zp_A != 0 || path_flag(kernel_path().gemm_reg)) return false;
    if (out == OUT_RAW) return true;
    const bool need_colsum = a.formula == F_ROW_VNNI && a.sumW;
    return (!a.zpW || a.sum_in) && (!need_colsum || a.colsum_in);
}

// The persistent GEMM (wide_kernel.h): the fused epilogue with zp_A = 0 and
// K = 512 or 1024, per-row scales given, and the byte sums the formula needs
// given (row code sums with zero points, weight-row sums with a caller's
// sum_W in the row-VNNI formula), as for the LDS-DMA kernel.
static bool wide_ok(const RowsArgs& a, int out) {
    if (out != OUT_EPI || a.zp_A != 0 || path_flag(kernel_path().no_wide) || path_flag(kernel_path().gemm_reg))
        return false;
    if (kernel_path().gemm_tile.load(std::memory_order_relaxed) != 0) return false;
    if ((a.K != 512 && a.K != 1024) || a.N % 4 != 0 || !a.scale_in) return false;
    if (a.formula == F_ROW_SCALAR || static_cast<int64_t>(128) * a.N * 4 >= (int64_t(1) << 31)) return false;
    const bool c0_mode = a.formula == F_ROW_VNNI && a.sumW;
    return (!a.zpW || a.sum_in) && (!c0_mode || a.colsum_in) && aligned(a.Aq, 16) && aligned(a.W, 16) &&
           aligned(a.C, 4);
}

template <int ACT, bool INT_EPI, int NK, int TJ>
static void launch_wide_t(const RowsArgs& a, hipStream_t st) {
    using Cf = WideCfg<TJ>;
    const int64_t ntiles = ((a.M + Cf::BM - 1) / Cf::BM) * ((a.N + Cf::BN - 1) / Cf::BN);
    const int grid = static_cast<int>(std::min<int64_t>(ntiles, num_cus()));
    const int c0_mode = a.formula == F_ROW_VNNI && a.sumW ? 1 : 0;
    hipLaunchKernelGGL((k_gemm_wide<ACT, INT_EPI, NK, TJ>), dim3(grid), dim3(kWideThreads), 0, st, a,
                       static_cast<int>(ntiles), c0_mode);
}

// 128 x 256 tiles when they give every CU at least two (fewer loads per
// product, and the epilogue of one tile overlaps the next); else 128 x 128.
// Measured on MI355X at K = N = 1024: M = 65536 91-110 us (128 x 128:
// 107-116), M = 4096 11.2 us (128 x 256: 14.2), M = 10000, N = 1000 23 us
// (31).
template <int ACT, bool INT_EPI, int NK>
static void launch_wide_k(const RowsArgs& a, hipStream_t st) {
    const int64_t t256 = ((a.M + 127) / 128) * ((a.N + 255) / 256);
    if (t256 >= 2 * static_cast<int64_t>(num_cus())) launch_wide_t<ACT, INT_EPI, NK, 2>(a, st);
    else launch_wide_t<ACT, INT_EPI, NK, 1>(a, st);
}

template <int ACT>
static void launch_wide(const RowsArgs& a, hipStream_t st) {
    const bool int_epi = a.zpW || (a.formula == F_ROW_VNNI && a.sumW);
    if (int_epi) {
        if (a.K == 1024) launch_wide_k<ACT, true, 8>(a, st);
        else launch_wide_k<ACT, true, 4>(a, st);
    } else {
        if (a.K == 1024) launch_wide_k<ACT, false, 8>(a, st);
        else launch_wide_k<ACT, false, 4>(a, st);
    }
}

template <int OUT, int ACT>
static void launch_gemm_act(const RowsArgs& a, hipStream_t st) {
    if constexpr (OUT == OUT_EPI) {
        if (wide_ok(a, OUT)) {
            launch_wide<ACT>(a, st);
            return;
        }
    }
    const int shape = gemm_shape(a);
    if (shape != 88 && gemm_pipe_ok(a, OUT)) {
        if (shape == 48) launch_pipe_t<4, 8, OUT, ACT>(a, st);
        else if (shape == 22) launch_pipe_t<2, 2, OUT, ACT>(a, st);
        else if (shape == 24) launch_pipe_t<2, 4, OUT, ACT>(a, st);
        else launch_pipe_t<4, 4, OUT, ACT>(a, st);
        return;
    }
    switch (shape) {
        case 88: launch_gemm_t<8, 8, OUT, ACT>(a, st); break;
        case 48: launch_gemm_t<4, 8, OUT, ACT>(a, st); break;
        default: launch_gemm_t<4, 4, OUT, ACT>(a, st); break;
    }
}

template <int OUT>
void launch_gemm(const RowsArgs& a, int act, hipStream_t st) {
    if constexpr (OUT == OUT_RAW) {
        launch_gemm_act<OUT, ACT_NONE>(a, st);
    } else {
        if (act == ACT_RELU) launch_gemm_act<OUT, ACT_RELU>(a, st);
        else if (act == ACT_GELU_TANH) launch_gemm_act<OUT, ACT_GELU_TANH>(a, st);
        else launch_gemm_act<OUT, ACT_NONE>(a, st);
    }
}

template void launch_gemm<OUT_EPI>(const RowsArgs&, int, hipStream_t);
template void launch_gemm<OUT_RAW>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
