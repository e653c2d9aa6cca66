// chain.hip -- launcher of the 8-bit-output 1024-wide layer (chain_kernel.h).
#include "chain_kernel.h"
#include "launch.h"

namespace nfq {

bool chain_ok(const ChainArgs& a) {
    // The drain's schedule is written for K = 1024 (eight K steps); the
    // published words hold up to 1024 / BN column tiles per row.
    return a.K == 1024 && a.N >= 256 && a.N <= 1024 && a.N % 256 == 0 && a.M > 0 && aligned(a.Aq, 16) &&
           aligned(a.W, 16) && aligned(a.Cq, 4) && a.scale_in && a.scale_out && a.part && a.fault && a.epoch != 0;
}

int chain_grid(const ChainArgs& a, int tj, int64_t* ntiles_out) {
    const int bn = 128 * tj;
    const int64_t ntiles = ((a.M + 127) / 128) * (a.N / bn);
    // Every block of a row tile must work in the same round of the deal (a
    // block waits for the others' row maxima), so the grid is a multiple of
    // the column tiles per row, and of 8 for the XCD-contiguous deal.
    int g = num_cus();
    g -= g % 8;
    if (g < 8) g = 8;
    *ntiles_out = ntiles;
    return static_cast<int>(std::min<int64_t>(ntiles, g));
}

template <int ACT, int TJ>
static void launch_chain_t(const ChainArgs& a, hipStream_t st) {
    int64_t ntiles = 0;
    const int grid = chain_grid(a, TJ, &ntiles);
    hipLaunchKernelGGL((k_chain_wide<ACT, 8, TJ>), dim3(grid), dim3(kWideThreads), 0, st, a, static_cast<int>(ntiles));
}

// 128 x 256 tiles when every CU gets at least two, else 128 x 128 (as the
// fp32-output kernel).
template <int ACT>
static void launch_chain_act(const ChainArgs& a, hipStream_t st) {
    const int64_t t256 = ((a.M + 127) / 128) * (a.N / 256);
    if (t256 >= 2 * static_cast<int64_t>(num_cus())) launch_chain_t<ACT, 2>(a, st);
    else launch_chain_t<ACT, 1>(a, st);
}

void launch_chain(const ChainArgs& a, int act, hipStream_t st) {
    switch (act) {
        case ACT_RELU: launch_chain_act<ACT_RELU>(a, st); break;
        case ACT_GELU_TANH: launch_chain_act<ACT_GELU_TANH>(a, st); break;
        default: launch_chain_act<ACT_NONE>(a, st); break;
    }
}

}  // namespace nfq
