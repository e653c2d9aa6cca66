// rows64.hip -- launchers of the K = N = 64 per-token layer (rows64_kernel.h).
#include "launch.h"
#include "rows64_kernel.h"

namespace nfq {

// The K = N = 64 per-token layer (rows64_kernel.h).
bool rows64_ok(const RowsArgs& a) {
    return a.K == 64 && a.N == 64 && aligned(a.A, 16) && aligned(a.C, 16) && aligned(a.W, 4);
}

// Tiles of 16 rows each loaded this many tiles ahead by every wave.
#ifndef NFQ_ROWS64_PF
#define NFQ_ROWS64_PF 1
#endif

template <bool FP8, int ACT, bool RES, int XQ, bool FIXED = false>
static void launch_rows64_act(const RowsArgs& a, hipStream_t st) {
    // With at least two tiles per wave at one 16-wave block per CU: the
    // tile queue (one block per CU, its waves taking tiles as they go).  Not
    // for the FNO layer with a residual and the per-position x2 fake-quant:
    // in a 1024-thread block (128 VGPRs per lane) that form spills (64 bytes
    // per lane for INT8, 20 for FP8), so it keeps the 4-wave blocks.
    const int64_t ntiles = (a.M + 15) / 16;
    if constexpr (!(RES && XQ == 2)) {
        if (ntiles >= 32 * static_cast<int64_t>(num_cus()) && !path_flag(kernel_path().no_rows64_queue)) {
            hipLaunchKernelGGL((k_rows64<FP8, ACT, 1, RES, XQ, FIXED, 16>), dim3(static_cast<unsigned>(num_cus())),
                               dim3(1024), 0, st, a);
            return;
        }
    }
    auto kern = k_rows64<FP8, ACT, NFQ_ROWS64_PF, RES, XQ, FIXED>;
    static const int per_cu = resident_blocks(kern);
    // Waves that all take the same number of tiles (to within one): the
    // fewest tiles per wave that a full grid of resident waves allows, but at
    // most 4 -- larger layers launch more waves than are resident, and the
    // later ones start as earlier ones finish.  Measured at K = N = 64 with
    // GELU, 1 Mi rows: 4 tiles per wave 85.4 us, 7 (a full grid doubled)
    // 89.0 us, 8 86.8 us; 256 Ki rows: 4 -> 23.8-24.1 us, 2 -> 25.3 us,
    // 6 -> 26.0 us; 32 Ki rows: 1 -> 7.5 us.  Fewer tiles per wave pay the
    // per-wave weight and constant setup more often; more leave a longer tail.
    const int64_t tiles = (a.M + 15) / 16;
    const int64_t slots = static_cast<int64_t>(num_cus()) * per_cu * 4;
    const int64_t per_wave = std::min<int64_t>(4, (tiles + slots - 1) / slots);
    const int64_t waves = (tiles + per_wave - 1) / per_wave;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, st, a);
}

template <bool FP8, bool RES, int XQ>
static void launch_rows64_res(const RowsArgs& a, int act, hipStream_t st) {
    if (act == ACT_RELU) launch_rows64_act<FP8, ACT_RELU, RES, XQ>(a, st);
    else if (act == ACT_GELU_TANH) launch_rows64_act<FP8, ACT_GELU_TANH, RES, XQ>(a, st);
    else launch_rows64_act<FP8, ACT_NONE, RES, XQ>(a, st);
}

template <bool FP8, int XQ>
static void launch_rows64_xq(const RowsArgs& a, int act, hipStream_t st) {
    if (a.residual) launch_rows64_res<FP8, true, XQ>(a, act, st);
    else launch_rows64_res<FP8, false, XQ>(a, act, st);
}

// a.residual (M x 64, 16-byte aligned) selects the FNO layer form act(x1 + x2),
// a.xq_kind the x2 fake-quant.
template <bool FP8>
void launch_rows64(const RowsArgs& a, int act, hipStream_t st) {
    if (a.xq_kind == 1) launch_rows64_xq<FP8, 1>(a, act, st);
    else if (a.xq_kind == 2) launch_rows64_xq<FP8, 2>(a, act, st);
    else launch_rows64_xq<FP8, 0>(a, act, st);
}

// The fixed-scale INT8 layer (LinearForwardBatched / LinearForward rows at
// K = N = 64): no activation, a.scale_A / a.zp_A for every row.
void launch_rows64_fixed(const RowsArgs& a, hipStream_t st) {
    launch_rows64_act<false, ACT_NONE, false, 0, true>(a, st);
}

template void launch_rows64<false>(const RowsArgs&, int, hipStream_t);
template void launch_rows64<true>(const RowsArgs&, int, hipStream_t);

}  // namespace nfq
