// launch.h -- host-side launch helpers and the launcher declarations shared
// by the translation units of libnflow_quant (one unit per kernel family, so
// the device code of each compiles in parallel).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <mutex>

#include "nflow_quant.h"
#include "rows_kernel.h"

namespace nfq {

inline int num_cus() {
    static int cached = 0;
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    if (cached == 0) {
        int dev = 0;
        int cu = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            cu > 0)
            cached = cu;
        else
            cached = 256;
    }
    return cached;
}

inline unsigned grid_for(int64_t work_items, int64_t per_block, int max_blocks_per_cu) {
    const int64_t want = (work_items + per_block - 1) / per_block;
    const int64_t cap = static_cast<int64_t>(num_cus()) * max_blocks_per_cu;
    return static_cast<unsigned>(std::max<int64_t>(1, std::min(want, cap)));
}

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Kernel-selection overrides, for A/B timing and for tests that pin one of
// two kernels computing the same bits.  They are read from the environment
// once, at the first launch (NFLOW_NO_GEMM, NFLOW_NO_ROWS64,
// NFLOW_NO_TOKEN_GEMM, NFLOW_GEMM_REG, NFLOW_GEMM_TILE, NFLOW_GEMM_MFMA,
// NFLOW_NO_WIDE, NFLOW_NO_ROWS64_QUEUE, NFLOW_NO_LAYER_TAIL), and afterwards
// change only through nflow_debug_set_kernel_path; a launch reads relaxed
// atomics, never the environment.
struct KernelPath {
    std::atomic<int> no_gemm{0};
    std::atomic<int> no_rows64{0};
    std::atomic<int> no_token_gemm{0};
    std::atomic<int> gemm_reg{0};
    std::atomic<int> gemm_tile{0};   // 0: the launcher's choice
    std::atomic<int> gemm_mfma{0};   // 0: the launcher's choice, else 16 or 32
    std::atomic<int> no_wide{0};
    std::atomic<int> no_rows64_queue{0};
    std::atomic<int> no_layer_tail{0};   // the FNO runtime's layer + tail and projection head unfused
    std::atomic<int> generic_fft{0};     // the FNO runtime's row FFTs and channel mix on the any-size kernels
};
KernelPath& kernel_path();

inline bool path_flag(const std::atomic<int>& f) { return f.load(std::memory_order_relaxed) != 0; }

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Row-tile kernel eligibility for the given input mode.
inline bool rows_ok(const RowsArgs& a, int in_mode) {
    if (a.K % 4 != 0 || a.N % 4 != 0) return false;
    if (in_mode == IN_CODES) {
        if (a.K > 1024 || !aligned(a.Aq, 4)) return false;
    } else {
        if (a.K > 256 || !aligned(a.A, 16)) return false;
    }
    return aligned(a.W, 4) && aligned(a.C, 16);
}

// Resident blocks per CU of a kernel (cached per instantiation).
template <typename Kernel>
inline int resident_blocks(Kernel k) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, 256, 0) != hipSuccess || n < 1) n = 1;
    return n;
}

// Row-tile kernel launchers, explicitly instantiated in rows_*.hip.
template <bool FP8, int IN, int OUT>
void launch_rows(const RowsArgs& a, int act, hipStream_t st);

// The K = N = 64 per-token layer (rows64.hip).
bool rows64_ok(const RowsArgs& a);
template <bool FP8>
void launch_rows64(const RowsArgs& a, int act, hipStream_t st);
// Its fixed-scale INT8 form (one scale_A / zp_A for every row, no activation).
void launch_rows64_fixed(const RowsArgs& a, hipStream_t st);

// The one-pass per-token INT8 layer for K = 128 / 256 / 512, N % 64 == 0
// (token_gemm.hip): quantise into LDS, then the whole N range.
bool token_gemm_ok(const RowsArgs& a);
void launch_token_gemm(const RowsArgs& a, int act, hipStream_t st);

// The tiled MFMA GEMM on INT8 codes for K a multiple of 64, K >= 128 (gemm.hip).
bool gemm_ok(const RowsArgs& a);
// Whether launch_gemm takes the LDS-DMA kernel for `a` (out: OUT_EPI / OUT_RAW).
bool gemm_pipe_ok(const RowsArgs& a, int out);
template <int OUT>
void launch_gemm(const RowsArgs& a, int act, hipStream_t st);

// The 8-bit-output 1024-wide layer (chain.hip): codes + row scales in, the
// next layer's per-token codes + row scales out.
struct ChainArgs;
bool chain_ok(const ChainArgs& a);
void launch_chain(const ChainArgs& a, int act, hipStream_t st);

}  // namespace nfq
