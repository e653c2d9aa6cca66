// fno_rt.h -- launchers of the FNO1d / FNO2d runtime's device kernels
// (fno_rt.hip), called by the host runtime (runtime.cpp).  Every launcher is
// stream-ordered and returns hipError_t of the launch.
//
// Layouts: the local-linear layers read and write token-major activations,
// (samples, points, width) with width contiguous; the spectral convolution
// reads and writes channel-major ones, (samples, width, points) with points
// contiguous -- the reference's layout (fno.cpp:437-445, 523-556; for FNO2d
// the points are the H x W grid, row-major, fno.cpp:855-865, 906-932).  The
// layer tail writes the new activation in both.  Only the layout differs
// from the reference: every element is computed by the same float
// operations as its x86 build.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

struct nflow_layer;

namespace nfq {

enum RtAct { RT_ACT_NONE = 0, RT_ACT_RELU = 1, RT_ACT_GELU = 2 };

// Largest power-of-two grid length the LDS-resident FFT takes (one wave per
// channel, n complex values = 8n bytes of LDS per wave).
constexpr int kFftMaxPoints = 8192;

// y (samples, rows_out, n) = act(b + x W^T) in the reference Linear's
// summation order (fno.cpp:69-79 as its build computes it: the first
// k - k % 8 products rounded and added in order, the last k % 8 fused).
// Row t of sample s reads input row s * rows_in + t; rows t >= rows_valid
// are written as 0 (the zero padding of fno.cpp:449-466).  W is (n, k)
// row-major, b may be null.
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

// An activation fake-quant: on = 0 none, 1 the INT8 per-tensor round trip
// (fno.cpp:488-501, 637-646, 830-842), 3 the log2 "FP8" snap (fno.cpp:579-606,
// 813-829) with its exponent step points in thr (see PostArgs).
struct FakeQuant {
    int on;
    float scale;
    float zpf;
    float thr[15];
};

// Token-major h (samples, n, w) to channel-major hc (samples, w, n), with the
// input fake-quant fq applied to both when on.
hipError_t launch_to_channel_major(float* h, float* hc, int64_t samples, int n, int w, FakeQuant fq,
                                   hipStream_t st);
// The lift with one input channel (LinArgs with k = 1, unpadded rows, no
// activation) followed by launch_to_channel_major, in one pass: h and hc
// as the two launches write them.
hipError_t launch_lift_layout(const float* x, const float* W, const float* b, float* h, float* hc, int64_t samples,
                              int n, int w, FakeQuant fq, hipStream_t st);

// Spectral convolution of fno.cpp:164-207 on channel-major hc: forward FFT
// of every channel (radix-2, fft.cpp:48-84) keeping bins 0 .. modes-1 in
// spec (samples, w, modes) complex, the channel mix into spec_mixed, and per
// output channel the inverse FFT (fft.cpp:86-100) into channel-major x1c.
// tw_fwd / tw_inv: the stage twiddles, stage of length len at entries
// len/2 - 1 .. len - 2 (n - 1 complex values per table).
struct SpecArgs {
    const float* hc;
    float* spec;          // forward bins (samples, w, modes) complex
    float* spec_mixed;    // mixed bins (samples, w, modes) complex
    float* x1c;
    const float* mix_real;  // the spectral weights held (modes, in, out)
    const float* mix_imag;
    const float* tw_fwd;
    const float* tw_inv;
    int64_t samples;
    int n;
    int log2n;
    int w;
    int modes;
    float inv_n;
    // Inverse FFT only: the value of the bins modes .. n/2 of item r is
    // fill[r % fill_period] (their mirrors its conjugate); null: (0, 0).
    const float2* fill;
    int fill_period;
};
hipError_t launch_spectral(const SpecArgs& a, hipStream_t st);

// The pieces of launch_spectral one at a time, for the 2-D convolution
// (fno.cpp:717-771 over fft.cpp:101-148).  Items are samples * w rows of n
// points (hc / x1c), each with `modes` kept bins (spec / spec_mixed).
hipError_t launch_rfft_rows(const SpecArgs& a, hipStream_t st);   // hc -> spec
hipError_t launch_spec_mix(const SpecArgs& a, hipStream_t st);    // spec -> spec_mixed
hipError_t launch_irfft_rows(const SpecArgs& a, hipStream_t st);  // spec_mixed (+ fill) -> x1c

// Column FFTs of the 2-D transform: `planes` planes of complex values with
// row stride mw (mw columns, j < mw); a radix-2 complex FFT of length h
// (fft.cpp:48-68) down each column.  Forward: in (planes, h, mw) -> rows
// 0 .. mh - 1 of the result to out (planes, mh, mw).  Inverse: in
// (planes, mh, mw), rows mh .. h - 1 taken as (0, 0) -> out (planes, h, mw),
// scaled by 1/h.  tw: the forward or inverse stage twiddles of length h.
struct ColArgs {
    const float* in;
    float* out;
    const float* tw;
    int64_t planes;
    int h;
    int log2h;
    int mw;
    int mh;
    float inv_h;
};
hipError_t launch_cfft_cols(const ColArgs& a, bool inverse, hipStream_t st);

// Token-major (samples, h, w, c) <-> (samples, hp, wp, c): pad copies the
// grid into the top-left corner of the larger one and zeroes the rest
// (fno.cpp:867-891); trim copies the corner back out (fno.cpp:946-964).
hipError_t launch_pad2d(const float* src, float* dst, int64_t samples, int h, int w, int hp, int wp, int c,
                        bool trim, hipStream_t st);

// y[i] = act(fq(y[i])) in place over n elements (fno.cpp:980-993).
hipError_t launch_fq_act(float* y, int64_t n, FakeQuant fq, int act, hipStream_t st);

// The layer tail h = act(x1 + fq(x2)) (fno.cpp:558-660) from token-major x2
// and channel-major x1c, written to token-major h and channel-major hc, with
// the next layer's input fake-quant (fq_next) applied.  kind 0 none,
// 1 per-tensor INT8, 2 per-position INT8 (index column * points + position,
// the reference's indexing), 3 the log2 snap of fno.cpp:579-606 with its
// exponent step points in thr.
struct PostArgs {
    const float* x2;
    const float* x1c;
    float* h;
    float* hc;
    int64_t samples;
    int n;
    int w;
    int kind;
    float scale;
    float zpf;
    const float* pos_scales;
    const int32_t* pos_zps;
    float thr[15];
    int act;
    FakeQuant fq_next;
};
hipError_t launch_post(const PostArgs& a, hipStream_t st);

// The INT8 local-linear layer (LinearForwardBatched + bias, int8_gemm.cpp:530-580,
// as fno.cpp:529-536 runs it) and the layer tail in one pass at width 64:
// x2 = (sW * sA) * D + b from the codes of h quantised with the per-tensor
// scale sA / zero point zpA, then the tail of PostArgs (p.x2 unused), h
// overwritten in place.  Taken when layer_tail_ok holds; the unfused pair
// computes the same bits.
struct LayerTailArgs {
    PostArgs p;
    const int8_t* W;         // (64, 64) codes, row per output channel
    const float* sW;         // (64)
    const float* bias;       // (64) or null
    const int32_t* zpW;      // (64) or null
    const int32_t* sumW;     // (64) or null
    float sA;
    int32_t zpA;
};
bool layer_tail_ok(const PostArgs& p, int in_features, int out_features);
// The fp32 local linear (64 x 64, launch_linear_ref's sums) and the tail in
// one pass, on the same conditions; W (64, 64) and b (64 or null) fp32.
bool linear_tail_ok(const PostArgs& p, const float* W);
hipError_t launch_linear_tail(const PostArgs& a, const float* W, const float* b, hipStream_t st);

// The projection head (fno.cpp:662-698, :966-993) in one pass: y = fq_o(
// proj_out(act(fq_q(proj_q(h))))) for width 64 and one output channel, with
// the sums and forms of launch_linear_ref and launch_fq_act.  h is
// token-major with rows_in rows per sample, of which the first n are read;
// y is (samples, n).
struct ProjArgs {
    const float* h;
    float* y;
    const float* Wq;
    const float* bq;
    const float* Wo;
    const float* bo;
    int64_t samples;
    int n;
    int rows_in;
    int w;
    int out_ch;
    int act;
    FakeQuant fq_q;
    FakeQuant fq_o;
};
bool proj_tail_ok(const ProjArgs& p);
hipError_t launch_proj_tail(const ProjArgs& a, hipStream_t st);
// The device arrays of an INT8 layer handle into a (layer.cpp): false for
// another format.
bool layer_int8_arrays(const nflow_layer* layer, LayerTailArgs* a, int* in_features, int* out_features);
hipError_t launch_layer_tail(const LayerTailArgs& a, hipStream_t st);

}  // namespace nfq
