// fno1d.h -- launchers of the FNO1d runtime's device kernels (fno1d.hip),
// called by the host runtime (runtime.cpp).  Every launcher is stream-ordered
// and returns hipError_t of the launch.
//
// Layout: activations are token-major, (samples, points, width) with width
// contiguous -- the layout the local-linear kernels read -- where the
// reference keeps (samples, width, points) and permutes around its Linear
// (fno.cpp:437-445, 523-556).  Only the layout differs: every element is
// computed by the same float operations as the reference build.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace nfq {

enum RtAct { RT_ACT_NONE = 0, RT_ACT_RELU = 1, RT_ACT_GELU = 2 };

// Largest power-of-two grid length the LDS-resident FFT takes (one wave per
// channel, n complex values = 8n bytes of LDS per wave).
constexpr int kFftMaxPoints = 8192;

// y (samples, rows_out, n) = act(b + x W^T) in the reference Linear's
// summation order (fno.cpp:69-79 as compiled: blocks of 16 / 8 rounded
// products, the last k % 8 terms fused).  Row t of sample s reads input row
// s * rows_in + t; rows t >= rows_valid are written as 0 (the zero padding
// of fno.cpp:449-466).  W is (n, k) row-major, b may be null.
struct LinArgs {
    const float* x;
    const float* W;
    const float* b;
    float* y;
    int64_t samples;
    int rows_out;
    int rows_valid;
    int rows_in;
    int k;
    int n;
    int act;
};
hipError_t launch_linear_ref(const LinArgs& a, hipStream_t st);

// In-place INT8 fake-quant round trip of n elements (fno.cpp:488-501).
hipError_t launch_fake_quant(float* h, int64_t n, float scale, int32_t zp, hipStream_t st);

// Spectral convolution of fno.cpp:164-207 on token-major h (samples, n, w):
// forward FFT of every channel (radix-2, fft.cpp:48-84) keeping bins
// 0 .. modes-1 in spec (samples, w, modes) complex, then per output channel
// the channel mix (in, out, modes weights) and the inverse FFT
// (fft.cpp:86-100), written token-major to x1.  tw_fwd / tw_inv hold the
// stage twiddles: stage of length len at entries len/2 - 1 .. len - 2
// (n - 1 complex values per table).
struct SpecArgs {
    const float* h;
    float* spec;
    float* x1;
    const float* w_real;
    const float* w_imag;
    const float* tw_fwd;
    const float* tw_inv;
    int64_t samples;
    int n;
    int log2n;
    int w;
    int modes;
    float inv_n;
};
hipError_t launch_spectral(const SpecArgs& a, hipStream_t st);

// The layer tail h = act(x1 + fq(x2)) (fno.cpp:558-660) on token-major
// (M, w) buffers.  kind 0 none, 1 per-tensor INT8, 2 per-position INT8
// (index column * points + row % points, the reference's indexing),
// 3 the log2 snap of fno.cpp:579-606 with its exponent step points in thr.
struct PostArgs {
    const float* x2;
    const float* x1;
    float* h;
    int64_t M;
    int w;
    int points;
    int kind;
    float scale;
    float zpf;
    const float* pos_scales;
    const int32_t* pos_zps;
    float thr[15];
    int act;
};
hipError_t launch_post(const PostArgs& a, hipStream_t st);

}  // namespace nfq
