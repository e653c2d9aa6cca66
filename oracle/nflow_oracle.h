/*
 * nflow_oracle.h -- CPU restatement of NeuroFlow's quantised inference GEMM
 * path, used ONLY as the reference results in tests.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library.  The product
 * (neuroflow_amd/, libnflow_quant.so) never links or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the NeuroFlow source tree).  Each function is pinned
 * by tests/test_oracle_*.py against the reference's known-answer tests, its
 * own build (oracle/_ref) or fixtures written by it, and closed forms.
 *
 * Build: plain C99, gcc -O2 -ffp-contract=off (no fast-math), so every
 * float expression rounds exactly as the reference's `-std=c++20` build does.
 */
#ifndef NFLOW_ORACLE_H
#define NFLOW_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: cpp/include/neuroflow/tensor.h:29-37. */
enum { ORC_OK = 0, ORC_INVALID_ARG = 1, ORC_INTERNAL = 99 };

/* Activation selector for the epilogue: none / relu / gelu (tanh form). */
enum { ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_GELU_TANH = 2 };

/* ---- INT8 activation quantisation ------------------------------------ */

/* One element: clamp(int32(std::round(a / scale)) + zp, -128, 127), with the
 * x86 conversion result (INT32_MIN) for NaN / out-of-range quotients.
 * int8_gemm.cpp:513-518 (QuantiseActivation), :233-238 (LinearForward). */
int8_t orc_quantise_one(float a, float scale, int32_t zp);

/* int8_gemm.cpp:507-520.  Null pointers: silent no-op (the reference is void). */
void orc_quantise_activation(const float* A, int8_t* A_q, int64_t bsz,
                             int in_features, float scale_A, int32_t zp_A);

/* Per-token (per-row) symmetric scale: absmax(row) / qmax, 1.0f for an
 * all-zero row (static_quant.py:349-350 convention).  NaN elements are
 * ignored by the max, matching `a > m ? a : m`. */
void orc_per_token_scales(const float* A, int64_t M, int K, float qmax,
                          float* scales);

/* Per-token INT8 quantisation: scales = absmax/127, codes as
 * orc_quantise_one(x, scale_row, 0).  Optional sum_a[m] = sum of codes. */
void orc_quantise_per_token_i8(const float* A, int64_t M, int K,
                               int8_t* A_q, float* scales, int32_t* sum_a);

/* ---- weights ---------------------------------------------------------- */

/* fno.cpp:325-358 QuantiseWeight2D: q = clamp(std::round(W/s_c) + zp_c)
 * computed in float; sum_w[c] = sum_i (q - zp_c). */
void orc_quantise_weight_2d(const float* W, int out_f, int in_f,
                            const float* scales, const int32_t* zps,
                            int8_t* W_q, int32_t* sum_w);

/* Per-channel symmetric scales: absmax(row c)/qmax, 1.0f for an all-zero row. */
void orc_per_channel_scales(const float* W, int out_f, int in_f, float qmax,
                            float* scales);

/* int8_gemm.cpp:479-496 PrecomputeSumW, written into caller memory. */
void orc_precompute_sum_w(const int8_t* W_q, const int32_t* zp_W, int in_f,
                          int out_f, int32_t* out);

/* ---- INT8 GEMM -------------------------------------------------------- */

/* Brute force C[m][n] = sum_k A[m][k] * W[n][k] (int64 accumulate, stored
 * as int32; |C| < 2^31 for K < 133000). */
void orc_gemm_i8_i32(const int8_t* A_q, const int8_t* W_q, int64_t M, int N,
                     int K, int32_t* C);

/* Parameter block: int8_gemm.h:45-65 (host pointers). */
typedef struct {
    const int8_t* W_int8;
    const float* scale_W;
    const int32_t* zp_W;
    const float* bias;
    int in_features;
    int out_features;
    float scale_A;
    int32_t zp_A;
    const int32_t* sum_W_per_row;
} orc_int8_linear_params;

/* int8_gemm.cpp:530-580 LinearForwardBatched. */
int orc_linear_forward_batched(const orc_int8_linear_params* p, int64_t bsz,
                               const float* A, float* C);

/* int8_gemm.cpp:201-470 LinearForward, as compiled with the reference's
 * AVX-512 VNNI flags (CMakeLists.txt:78): one activation row. */
int orc_linear_forward(const orc_int8_linear_params* p, const float* A,
                       float* C);

/* Epilogue activation, fno.cpp:36-48 (relu; gelu tanh form). */
void orc_apply_activation(float* y, int64_t n, int act);

/* fno.cpp:572-648: the FNO layer's INT8 fake-quant of x2 (token-major), per
 * tensor (scales NULL) or per position (the reference's indexing). */
int orc_x2_fake_quant(const float* x2, float* out, int64_t M, int N, float scale, int32_t zp,
                      const float* scales, const int32_t* zps, int points);

/* The per-token INT8 layer: for each row m, LinearForward with
 * scale_A = absmax(row)/127 (1.0f for a zero row), zp_A = 0, and the given
 * sum_W_per_row; then the activation.  scale_A_out (nullable) receives the
 * per-row scales. */
int orc_layer_per_token_i8(const orc_int8_linear_params* p, int64_t M,
                           const float* A, float* C, int act,
                           float* scale_A_out);

/* ---- FP8 E4M3 codec: fp8_e4m3.h:106-334 ------------------------------- */

uint8_t orc_e4m3_encode(float v);                 /* :106-215 */
float orc_e4m3_decode(uint8_t b);                  /* :223-275 */
void orc_e4m3_encode_array(const float* in, uint8_t* out, size_t n); /* :286-290 */
void orc_e4m3_decode_array(const uint8_t* in, float* out, size_t n); /* :295-299 */
void orc_fp8_fake_quant(const float* in, float scale, float* out, size_t n); /* :312-334 */

/* Encode every float whose bit pattern lies in [start, start + count). */
void orc_e4m3_encode_bits_range(uint32_t start, uint32_t count, uint8_t* out);

/* Encode the floats with bit patterns start + i * stride (mod 2^32), i < count. */
void orc_e4m3_encode_bits_stride(uint32_t start, uint32_t stride, uint32_t count,
                                 uint8_t* out);

/* Encode with the fake-quant scale-down (x * (1/scale), clamp +-448);
 * fp8_e4m3.h:319-329. */
uint8_t orc_fp8_quantise_one(float x, float inv_scale);

/* Per-token FP8: scales = absmax/448 (1.0f for zero rows), codes as
 * orc_fp8_quantise_one(x, 1/scale). */
void orc_quantise_per_token_fp8(const float* A, int64_t M, int K,
                                uint8_t* A_q, float* scales);

/* Per-channel FP8 weights: scales = absmax/448 per row, same encoding. */
void orc_quantise_weight_fp8(const float* W, int out_f, int in_f,
                             uint8_t* W_q, float* scales);

/* Exact FP8 GEMM: C[m][n] = sum_k dec(A[m][k]) * dec(W[n][k]) in double
 * (every product is exact in double and, for K <= 512, so is the sum). */
void orc_gemm_fp8_exact(const uint8_t* A_q, const uint8_t* W_q, int64_t M,
                        int N, int K, double* C);

/* The reference composition for an FP8 layer (no FP8 GEMM exists in the
 * reference): per-row fake-quant of A with s_a[m] and per-channel fake-quant
 * of W with s_w[n] (fp8_e4m3.h:312-334), then the FP32 Linear loop with the
 * bias as the initial accumulator (fno.cpp:68-79), then the activation. */
void orc_layer_fp8_composed(const float* A, const float* W, const float* bias,
                            int64_t M, int N, int K, int act, float* C,
                            float* scale_A_out, float* scale_W_out);

/* Exact-sum variant of the FP8 layer: y = (s_w[n]*s_a[m]) * (float)exact_sum
 * + bias, then the activation -- the tight pin for an fp32-accumulating GEMM. */
void orc_layer_fp8_exact(const uint8_t* A_q, const float* scale_A,
                         const uint8_t* W_q, const float* scale_W,
                         const float* bias, int64_t M, int N, int K, int act,
                         float* C);


/* ---- FNO1d forward pieces (nflow_oracle_fno.c) --------------------------- */

/* fft.cpp:48-68: in-place complex FFT of n (a power of two) interleaved
 * complex values; inverse != 0 runs the inverse with the 1/n scaling. */
void orc_cfft(float* a, int n, int inverse);
/* fft.cpp:72-84 / :86-100. */
void orc_rfft(const float* x, int n, float* out_complex);
void orc_irfft(const float* x_complex, int n, float* out);
/* fft.cpp:101-124 / :126-148: 2-D real FFT of an (H, W) plane to (H, W/2+1)
 * interleaved bins, and its inverse. */
void orc_rfft2(const float* x, int H, int W, float* out_complex);
void orc_irfft2(const float* x_complex, int H, int W, float* out);
/* fno.cpp:717-771: h, out (bsz, w, H, W); w_real / w_imag (w, w, mh, mw). */
void orc_spectral_conv2d(const float* h, int bsz, int w, int H, int W, int mh, int mw,
                         const float* w_real, const float* w_imag, float* out);
/* fno.cpp:164-207: h, out (bsz, w, n); w_real / w_imag (w, w, modes). */
void orc_spectral_conv1d(const float* h, int bsz, int w, int n, int modes,
                         const float* w_real, const float* w_imag, float* out);
/* fno.cpp:69-79: y (rows, n) = b + x (rows, k) @ W^T, summed in order the way the
 * reference build does (blocks of 16 / 8 rounded products, fused tail). */
void orc_linear_f32(const float* x, const float* W, const float* b, int64_t rows, int k, int n,
                    float* y);
/* The INT8 fake-quant round trip with one (scale, zero point) per element. */
void orc_fake_quant_arr(const float* in, const float* scales, const int32_t* zps, float* out,
                        int64_t n);
/* fno.cpp:579-606: the log2 "FP8" snap of x2 (per-tensor scale s). */
float orc_log2_snap_one(float x, float s);
void orc_log2_snap(const float* in, float s, float* out, int64_t n);
int orc_log2_snap_exponent(float a);

#ifdef __cplusplus
}
#endif
#endif /* NFLOW_ORACLE_H */
