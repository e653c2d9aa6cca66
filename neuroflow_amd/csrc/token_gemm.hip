// token_gemm.hip -- launchers of the one-pass per-token INT8 layer for
// K = 128 / 256 / 512 (token_gemm_kernel.h).
#include "launch.h"
#include "token_gemm_kernel.h"

namespace nfq {

bool token_gemm_ok(const RowsArgs& a) {
    // N <= 2^24 keeps a 16-row output strip's byte count inside a buffer range.
    return (a.K == 128 || a.K == 256 || a.K == 512) && a.N % 64 == 0 && a.N > 0 && a.N <= (1 << 24) &&
           aligned(a.A, 16) &&
           aligned(a.C, 16) && aligned(a.W, 16);
}

template <int KB, int ACT>
static void launch_kb_act(const RowsArgs& a, hipStream_t st) {
    auto kern = k_token_gemm<KB, ACT>;
    static const int per_cu = resident_blocks(kern);
    const int64_t tiles = (a.M + 63) / 64;
    const int64_t grid = std::min<int64_t>(tiles, static_cast<int64_t>(num_cus()) * per_cu);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, a);
}

template <int KB>
static void launch_kb(const RowsArgs& a, int act, hipStream_t st) {
    if (act == ACT_RELU) launch_kb_act<KB, ACT_RELU>(a, st);
    else if (act == ACT_GELU_TANH) launch_kb_act<KB, ACT_GELU_TANH>(a, st);
    else launch_kb_act<KB, ACT_NONE>(a, st);
}

void launch_token_gemm(const RowsArgs& a, int act, hipStream_t st) {
    if (a.K == 128) launch_kb<2>(a, act, st);
    else if (a.K == 256) launch_kb<4>(a, act, st);
    else launch_kb<8>(a, act, st);
}

}  // namespace nfq
