// gelu_device_check.hip -- exhaustive device checks of two rewrites in the
// runtime's kernels, built as a test library (libgelu_device_check.so):
//   * gelu_fast<R> (reciprocal-step divisions) against gelu_ref (IEEE
//     divisions; equal to glibc on all 2^32 inputs on the host), bit for bit
//     on every float, for R = 0 and 1;
//   * snap_exponent_binade against snap_exponent_count on every float a in
//     [2^-6, FLT_MAX], for a step table given by the caller.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gelu_exact.h"
#include "snap.h"

namespace {

__global__ __launch_bounds__(256) void k_check(const float* thr, unsigned long long* cnt, uint32_t* first) {
    __shared__ float t[16];
    if (threadIdx.x < 15) t[threadIdx.x] = thr[threadIdx.x];
    __syncthreads();
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < (1ull << 32); i += stride) {
        const uint32_t u = static_cast<uint32_t>(i);
        const float x = nfq::gx_float(u);
        const uint32_t want = nfq::gx_bits(nfq::gelu_ref(x));
        if (nfq::gx_bits(nfq::gelu_fast<0>(x)) != want) {
            atomicAdd(&cnt[0], 1ull);
            atomicMin(&first[0], u);
        }
        if (nfq::gx_bits(nfq::gelu_fast<1>(x)) != want) {
            atomicAdd(&cnt[1], 1ull);
            atomicMin(&first[1], u);
        }
        if (u >= 0x3c800000u && u <= 0x7f7fffffu &&
            nfq::snap_exponent_binade(x, t) != nfq::snap_exponent_count(x, t)) {
            atomicAdd(&cnt[2], 1ull);
            atomicMin(&first[2], u);
        }
    }
}

}  // namespace

extern "C" int nfq_gelu_refine() { return nfq::kGeluRefine; }

// counts[0..2]: differing inputs of gelu_fast<0>, gelu_fast<1> and the snap
// exponent; first[0..2]: the smallest such bit pattern (0xffffffff if none).
extern "C" int nfq_check_gelu_snap(const float* thr_host, unsigned long long* counts, uint32_t* first) {
    float* thr = nullptr;
    unsigned long long* cnt = nullptr;
    uint32_t* fst = nullptr;
    hipError_t e = hipMalloc(&thr, 16 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&cnt, 3 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMalloc(&fst, 3 * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemcpy(thr, thr_host, 15 * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(cnt, 0, 3 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemset(fst, 0xff, 3 * sizeof(uint32_t));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_check, dim3(4096), dim3(256), 0, 0, thr, cnt, fst);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(counts, cnt, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(first, fst, 3 * sizeof(uint32_t), hipMemcpyDeviceToHost);
    hipFree(thr);
    hipFree(cnt);
    hipFree(fst);
    return static_cast<int>(e);
}
