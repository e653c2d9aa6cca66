// mfma_fp8_check.hip -- accumulation error of gfx950's FP8 MFMA against the
// bf16 MFMA on the same E4M3 values, built as a test library
// (libmfma_fp8_check.so).  This is the measurement behind the FP8 GEMM's use
// of v_mfma_f32_16x16x32_bf16 on exact E4M3 values instead of
// v_mfma_f32_16x16x32_fp8_fp8.
//
// One wave per trial.  Every row of the A operand is the same 32 E4M3 values
// a[t][0..31] and every column of B the same b[t][0..31]; both operands take
// k = 8 g .. 8 g + 7 from lane group g = lane / 16, so every one of the 256
// outputs is the dot product sum_k a_k b_k whatever the row / column
// mapping.  Each lane writes its 4 outputs of both instructions; the host
// checks they agree and compares them with the exact sum.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(64) void k_mfma_fp8(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
                                                 int trials, float* __restrict__ out_fp8,
                                                 float* __restrict__ out_bf16) {
    const int t = blockIdx.x;
    if (t >= trials) return;
    const int lane = threadIdx.x;
    const int g = lane >> 4;
    const uint8_t* pa = a + static_cast<int64_t>(t) * 32 + 8 * g;
    const uint8_t* pb = b + static_cast<int64_t>(t) * 32 + 8 * g;
    uint64_t av = 0, bv = 0;
    for (int i = 0; i < 8; ++i) {
        av |= static_cast<uint64_t>(pa[i]) << (8 * i);
        bv |= static_cast<uint64_t>(pb[i]) << (8 * i);
    }
    const nfq::v4f zero = {0.f, 0.f, 0.f, 0.f};
    const nfq::v4f d8 = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(static_cast<long>(av), static_cast<long>(bv),
                                                                    zero, 0, 0, 0);
    // The same values as bf16 (exact): 8 bf16 per lane in four dwords.
    nfq::v4i ab, bb;
    for (int i = 0; i < 4; ++i) {
        ab[i] = static_cast<int>(nfq::e4m3_to_bf16(pa[2 * i]) | (nfq::e4m3_to_bf16(pa[2 * i + 1]) << 16));
        bb[i] = static_cast<int>(nfq::e4m3_to_bf16(pb[2 * i]) | (nfq::e4m3_to_bf16(pb[2 * i + 1]) << 16));
    }
    const nfq::v4f d16 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ab),
                                                                  __builtin_bit_cast(v8bf, bb), zero, 0, 0, 0);
    for (int i = 0; i < 4; ++i) {
        out_fp8[static_cast<int64_t>(t) * 256 + lane * 4 + i] = d8[i];
        out_bf16[static_cast<int64_t>(t) * 256 + lane * 4 + i] = d16[i];
    }
}

}  // namespace

// a, b: trials x 32 E4M3 bytes (host); out_fp8, out_bf16: trials x 256 floats
// (host).  Returns the hipError_t of the first failing call (0 = success).
extern "C" int nfq_mfma_fp8_outputs(const uint8_t* a, const uint8_t* b, int trials, float* out_fp8,
                                    float* out_bf16) {
    if (trials <= 0) return 0;
    const size_t nin = static_cast<size_t>(trials) * 32, nout = static_cast<size_t>(trials) * 256;
    uint8_t *da = nullptr, *db = nullptr;
    float *d8 = nullptr, *d16 = nullptr;
    hipError_t e = hipMalloc(&da, nin);
    if (e == hipSuccess) e = hipMalloc(&db, nin);
    if (e == hipSuccess) e = hipMalloc(&d8, nout * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d16, nout * sizeof(float));
    if (e == hipSuccess) e = hipMemcpy(da, a, nin, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, b, nin, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_mfma_fp8, dim3(trials), dim3(64), 0, 0, da, db, trials, d8, d16);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(out_fp8, d8, nout * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(out_bf16, d16, nout * sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(da);
    (void)hipFree(db);
    (void)hipFree(d8);
    (void)hipFree(d16);
    return static_cast<int>(e);
}
