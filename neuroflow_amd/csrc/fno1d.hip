// fno1d.hip -- device kernels of the FNO1d runtime around the quantised
// local-linear layer: the fp32 Linear of the lift / projection / fallback
// layers, the input fake-quant, the spectral convolution (radix-2 FFT,
// channel mix, inverse FFT) and the layer tail act(x1 + fq(x2)).
//
// Every element is computed by the float operations of the reference build
// (cpp/src/fno.cpp and fft.cpp compiled by g++ -O3 -mfma): products the
// build fuses are written as __builtin_fmaf, everything else rounds on its
// own (this library is compiled with -ffp-contract=off).  GELU is
// gelu_ref (gelu_exact.h), bit-exact with glibc's tanhf.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "fno1d.h"
#include "gelu_exact.h"
#include "launch.h"

namespace nfq {

__device__ __forceinline__ float rt_activate(float y, int act) {
    if (act == RT_ACT_RELU) return y < 0.0f ? 0.0f : y;  // fno.cpp:37-40
    if (act == RT_ACT_GELU) return gelu_ref(y);
    return y;
}

// LDS written by some lanes of a wave, read by others after this point.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Logical block of this launch when blocks are dealt round-robin to the 8
// XCDs: each XCD takes a contiguous range of logical blocks, so the blocks
// that share a sample's data share one L2.  Returns -1 for the padding
// blocks of the last range.
__device__ __forceinline__ int64_t xcd_block(int64_t nlogical) {
    const int64_t per = gridDim.x / 8;
    const int64_t b = static_cast<int64_t>(blockIdx.x);
    const int64_t logical = (b % 8) * per + b / 8;
    return logical < nlogical ? logical : -1;
}

// ---------------------------------------------------------------------------
// fp32 Linear (fno.cpp:69-79) in the reference build's summation order.
// ---------------------------------------------------------------------------
template <bool LDSW>
__global__ __launch_bounds__(256) void k_linear_ref(LinArgs a) {
    extern __shared__ float wt[];  // W transposed: wt[p * n + j] = W[j][p]
    const int k = a.k, n = a.n;
    if constexpr (LDSW) {
        for (int i = threadIdx.x; i < k * n; i += blockDim.x) wt[(i % k) * n + i / k] = a.W[i];
        __syncthreads();
    }
    const int64_t total = a.samples * a.rows_out * static_cast<int64_t>(n);
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int j = static_cast<int>(idx % n);
        const int64_t r = idx / n;
        const int64_t s = r / a.rows_out;
        const int t = static_cast<int>(r % a.rows_out);
        float out = 0.0f;
        if (t < a.rows_valid) {
            const float* xr = a.x + (s * a.rows_in + t) * static_cast<int64_t>(k);
            const float* wr = a.W + static_cast<int64_t>(j) * k;
            auto wv = [&](int p) { return LDSW ? wt[p * n + j] : wr[p]; };
            float acc = a.b ? a.b[j] : 0.0f;
            int p = 0;
            for (; p + 16 <= k; p += 16)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc = acc + xr[p + q] * wv(p + q);
            if (k - p >= 8) {
#pragma unroll
                for (int q = 0; q < 8; ++q) acc = acc + xr[p + q] * wv(p + q);
                p += 8;
            }
            for (; p < k; ++p) acc = __builtin_fmaf(xr[p], wv(p), acc);
            out = rt_activate(acc, a.act);
        }
        a.y[r * n + j] = out;
    }
}

// fno.cpp:488-501: q = std::round(v / s) + zp, clamped, then (q - zp) * s.
__global__ __launch_bounds__(256) void k_fake_quant(float* h, int64_t n, float s, float zpf) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        h[i] = x2_fake_quant(h[i], s, zpf);
}

// ---------------------------------------------------------------------------
// Radix-2 FFT of one channel held by one wave in LDS (fft.cpp:34-68).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int bit_rev(int i, int log2n) {
    return log2n == 0 ? 0 : static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(i)) >> (32 - log2n));
}

// std::complex<float> product as the reference build computes it.
__device__ __forceinline__ float2 cmul_ref(float2 x, float2 w) {
    return make_float2(__builtin_fmaf(x.x, w.x, -(x.y * w.y)), __builtin_fmaf(x.x, w.y, x.y * w.x));
}

// The stages of fft.cpp:50-64 on a (already in bit-reversed order); the
// butterflies of a stage are independent, spread over the wave's lanes.
__device__ __forceinline__ void fft_stages(float2* a, int n, int log2n, const float2* tw, int lane) {
    for (int lh = 0; lh < log2n; ++lh) {
        const int half = 1 << lh;
        const float2* twl = tw + (half - 1);
        for (int q = lane; q < (n >> 1); q += 64) {
            const int kk = q & (half - 1);
            const int i = ((q >> lh) << (lh + 1)) + kk;
            const float2 u = a[i];
            const float2 v = cmul_ref(a[i + half], twl[kk]);
            a[i] = make_float2(u.x + v.x, u.y + v.y);
            a[i + half] = make_float2(u.x - v.x, u.y - v.y);
        }
        wave_sync();
    }
}

// Forward FFT of channel c of sample s (token-major h), bins 0 .. modes-1 to spec.
template <int WPB>
__global__ __launch_bounds__(64 * WPB) void k_rfft_modes(SpecArgs a, int64_t nlogical) {
    extern __shared__ float2 fbuf[];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t lb = xcd_block(nlogical);
    if (lb < 0) return;
    const int64_t item = lb * WPB + wid;
    if (item >= a.samples * a.w) return;
    const int64_t s = item / a.w;
    const int c = static_cast<int>(item % a.w);
    const int n = a.n;
    float2* buf = fbuf + static_cast<int64_t>(wid) * n;
    for (int t = lane; t < n; t += 64)
        buf[bit_rev(t, a.log2n)] = make_float2(a.h[(s * n + t) * a.w + c], 0.0f);
    wave_sync();
    fft_stages(buf, n, a.log2n, reinterpret_cast<const float2*>(a.tw_fwd), lane);
    float2* spec = reinterpret_cast<float2*>(a.spec) + (s * a.w + c) * a.modes;
    for (int m = lane; m < a.modes; m += 64) spec[m] = buf[m];
}

// Channel mix (fno.cpp:176-198) and inverse FFT (fft.cpp:86-100) for output
// channel wo of sample s, written token-major to x1.
template <int WPB>
__global__ __launch_bounds__(64 * WPB) void k_mix_irfft(SpecArgs a, int64_t nlogical) {
    extern __shared__ float2 fbuf[];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t lb = xcd_block(nlogical);
    if (lb < 0) return;
    const int64_t item = lb * WPB + wid;
    if (item >= a.samples * a.w) return;
    const int64_t s = item / a.w;
    const int wo = static_cast<int>(item % a.w);
    const int n = a.n, w = a.w, modes = a.modes, nh = n >> 1;
    float2* buf = fbuf + static_cast<int64_t>(wid) * n;
    // Bins the mix leaves at zero: (0, 0) up to n/2, their conjugate
    // mirrors (0, -0) above it.
    for (int i = lane; i < n; i += 64) buf[bit_rev(i, a.log2n)] = make_float2(0.0f, i > nh ? -0.0f : 0.0f);
    wave_sync();
    const float2* spec = reinterpret_cast<const float2*>(a.spec) + s * w * modes;
    for (int m = lane; m < modes; m += 64) {
        float sr = 0.0f, si = 0.0f;
        for (int k = 0; k < w; ++k) {
            const float2 hv = spec[static_cast<int64_t>(k) * modes + m];
            const int64_t wi = (static_cast<int64_t>(k) * w + wo) * modes + m;
            const float wr = a.w_real[wi], wim = a.w_imag[wi];
            sr = sr + __builtin_fmaf(-wim, hv.y, hv.x * wr);
            si = si + __builtin_fmaf(wr, hv.y, hv.x * wim);
        }
        buf[bit_rev(m, a.log2n)] = make_float2(sr, si);
        if (m >= 1 && m <= nh - 1) buf[bit_rev(n - m, a.log2n)] = make_float2(sr, -si);
    }
    wave_sync();
    fft_stages(buf, n, a.log2n, reinterpret_cast<const float2*>(a.tw_inv), lane);
    for (int t = lane; t < n; t += 64) a.x1[(s * n + t) * w + wo] = buf[t].x * a.inv_n;
}

// ---------------------------------------------------------------------------
// Layer tail.
// ---------------------------------------------------------------------------

// fno.cpp:579-606 with the exponent e = int(std::round(log2|v| * 8) / 8)
// read off the step points of the reference's libm (thr: the smallest float
// of each exponent from -5 to 9, computed on the host with that libm):
// e = -6 + #{thr <= |v|} for 2^-6 <= |v| <= FLT_MAX; NaN and Inf give
// ldexp(1, INT_MIN) = 0; 2^e for e >= 9 is capped at 448.
__device__ __forceinline__ float log2_snap(float x, float s, const float* thr) {
    const float v = x / s;
    const float av = fabsf(v);
    const float sign = v < 0.0f ? -1.0f : 1.0f;
    float qv;
    if (av < 0.015625f) {
        qv = av;
    } else if (!(av <= 0x1.fffffep+127f)) {
        qv = 0.0f;
    } else {
        int e = -6;
#pragma unroll
        for (int j = 0; j < 15; ++j) e += av >= thr[j] ? 1 : 0;
        qv = e >= 9 ? 448.0f : __builtin_bit_cast(float, static_cast<uint32_t>(127 + e) << 23);
    }
    const float clamped = (448.0f < qv) ? 448.0f : qv;
    return (sign * clamped) * s;
}

__global__ __launch_bounds__(256) void k_post_rt(PostArgs a) {
    const int64_t total = a.M * a.w;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        float x2 = a.x2[idx];
        if (a.kind == 1) {
            x2 = x2_fake_quant(x2, a.scale, a.zpf);
        } else if (a.kind == 2) {
            const int64_t m = idx / a.w;
            const int j = static_cast<int>(idx % a.w);
            const int64_t p = static_cast<int64_t>(j) * a.points + m % a.points;
            x2 = x2_fake_quant(x2, a.pos_scales[p], static_cast<float>(a.pos_zps[p]));
        } else if (a.kind == 3) {
            x2 = log2_snap(x2, a.scale, a.thr);
        }
        a.h[idx] = rt_activate(a.x1[idx] + x2, a.act);
    }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------

hipError_t launch_linear_ref(const LinArgs& a, hipStream_t st) {
    const int64_t total = a.samples * a.rows_out * static_cast<int64_t>(a.n);
    if (total <= 0) return hipSuccess;
    const unsigned grid = grid_for(total, 256, 8);
    const size_t wbytes = static_cast<size_t>(a.k) * a.n * sizeof(float);
    if (wbytes <= 48 * 1024)
        hipLaunchKernelGGL(k_linear_ref<true>, dim3(grid), dim3(256), wbytes, st, a);
    else
        hipLaunchKernelGGL(k_linear_ref<false>, dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_fake_quant(float* h, int64_t n, float scale, int32_t zp, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fake_quant, dim3(grid_for(n, 256, 8)), dim3(256), 0, st, h, n, scale,
                       static_cast<float>(zp));
    return hipGetLastError();
}

hipError_t launch_spectral(const SpecArgs& a, hipStream_t st) {
    const int64_t items = a.samples * a.w;
    if (items <= 0) return hipSuccess;
    const int wpb = a.n <= 2048 ? 4 : 1;
    const int64_t nlogical = (items + wpb - 1) / wpb;
    const unsigned grid = static_cast<unsigned>(8 * ((nlogical + 7) / 8));
    const size_t lds = static_cast<size_t>(wpb) * a.n * sizeof(float2);
    if (wpb == 4) {
        hipLaunchKernelGGL(k_rfft_modes<4>, dim3(grid), dim3(256), lds, st, a, nlogical);
        hipLaunchKernelGGL(k_mix_irfft<4>, dim3(grid), dim3(256), lds, st, a, nlogical);
    } else {
        hipLaunchKernelGGL(k_rfft_modes<1>, dim3(grid), dim3(64), lds, st, a, nlogical);
        hipLaunchKernelGGL(k_mix_irfft<1>, dim3(grid), dim3(64), lds, st, a, nlogical);
    }
    return hipGetLastError();
}

hipError_t launch_post(const PostArgs& a, hipStream_t st) {
    const int64_t total = a.M * a.w;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_post_rt, dim3(grid_for(total, 256, 8)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace nfq
