/*
 * nflow_quant.h -- C-ABI of the MI355X (gfx950) quantised inference GEMM.
 *
 * This library replaces NeuroFlow's CPU INT8 GEMM (`nflow::int8_gemm`,
 * cpp/include/neuroflow/int8_gemm.h) and FP8 E4M3 codec
 * (cpp/include/neuroflow/fp8_e4m3.h) with hand-written HIP kernels.  Every
 * entry point is `extern "C"`, takes plain pointers and sizes, and returns a
 * status code with the values of `nflow::StatusCode`
 * (cpp/include/neuroflow/tensor.h:29-37).  The message of the last failing
 * call on the calling thread is available from nflow_last_error().
 *
 * Memory: every array argument of a device entry point is a DEVICE pointer
 * (hipMalloc'd, or a torch CUDA tensor's data_ptr()), unless the function
 * name starts with nflow_host_.  Kernels are enqueued on `stream` (a
 * hipStream_t; NULL = the default stream) and the call returns without
 * synchronising; results are ready once the stream has been synchronised.
 * Calls on one stream execute in order.  State kept between calls: device
 * properties and kernel-path flags (process-wide); per (device, stream), the
 * workspace buffers of the entry points that stage codes between launches and
 * the row-maxima words of the 8-bit-output layer, kept at the largest size
 * asked for until nflow_release_stream_workspace or the end of the process;
 * per device, the static scratch of
 * nflow_int8_linear_forward_per_token_noalloc.
 *
 * Numerics (the reference's x86 build is the specification):
 *   - activation codes: clamp(int32(roundf(a / scale)) + zp, -128, 127) with a
 *     correctly rounded division, half-away-from-zero rounding, and the x86
 *     conversion result INT32_MIN for NaN / |q| >= 2^31;
 *   - int32 accumulators are exact;
 *   - dequantise: (scale_W[o] * scale_A) * float(acc) + bias[o], no FMA;
 *   - FP8 E4M3 bytes reproduce fp32_to_e4m3_bits bit for bit;
 *   - GELU is the tanh form of fno.cpp:41-46.
 */
#ifndef NFLOW_QUANT_H
#define NFLOW_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NFLOW_QUANT_ABI_VERSION 3

/* nflow::StatusCode, cpp/include/neuroflow/tensor.h:29-37. */
enum nflow_status_code {
    NFLOW_OK = 0,
    NFLOW_INVALID_ARG = 1,
    NFLOW_FILE_NOT_FOUND = 2,
    NFLOW_PARSE_ERROR = 3,
    NFLOW_SHAPE_MISMATCH = 4,
    NFLOW_UNSUPPORTED_OP = 5,
    NFLOW_INTERNAL = 99
};

/* Epilogue activation (ApplyActivation, cpp/src/fno.cpp:36-48). */
enum nflow_activation {
    NFLOW_ACT_NONE = 0,
    NFLOW_ACT_RELU = 1,
    NFLOW_ACT_GELU_TANH = 2
};

/* nflow::int8_gemm::Int8LinearParams (cpp/include/neuroflow/int8_gemm.h:45-65),
 * field for field, with device pointers. */
typedef struct nflow_int8_linear_params {
    const int8_t* W_int8;         /* (out_features, in_features) row-major */
    const float* scale_W;         /* (out_features) per-channel scale */
    const int32_t* zp_W;          /* (out_features) per-channel zero point */
    const float* bias;            /* (out_features) or NULL */
    int in_features;
    int out_features;
    float scale_A;                /* per-tensor activation scale */
    int32_t zp_A;                 /* per-tensor activation zero point */
    const int32_t* sum_W_per_row; /* (out_features) or NULL */
} nflow_int8_linear_params;

/* FP8 E4M3 layer: per-channel symmetric weights (bytes as produced by
 * fp32_to_e4m3_bits, fp8_e4m3.h:106-215), no zero points. */
typedef struct nflow_fp8_linear_params {
    const uint8_t* W_e4m3;        /* (out_features, in_features) row-major */
    const float* scale_W;         /* (out_features) */
    const float* bias;            /* (out_features) or NULL */
    int in_features;
    int out_features;
} nflow_fp8_linear_params;

/* Weight format of a layer handle. */
enum nflow_format {
    NFLOW_FORMAT_INT8 = 0,       /* per-channel symmetric int8, per-token int8 activations */
    NFLOW_FORMAT_FP8_E4M3 = 1    /* per-channel E4M3, per-token E4M3 activations */
};

/* ---- library ------------------------------------------------------------ */

int nflow_quant_abi_version(void);

/* Message of the last non-OK status returned on this thread ("" if none). */
const char* nflow_last_error(void);

/* Kernel-path override for A/B timing and for tests that pin one of two
 * kernels computing the same bits (no counterpart in the reference, whose
 * SIMD path is fixed at compile time, int8_gemm.cpp:34-45).  Names:
 * "no_gemm", "no_rows64", "no_token_gemm", "gemm_reg" (0 / 1) and
 * "gemm_tile" (0 = the launcher's choice, else 88, 48, 44, 24 or 22) and
 * "gemm_mfma" (0 = the launcher's choice, else 16 or 32: the MFMA shape of
 * the LDS-DMA GEMM), "no_wide" (0 / 1: keep K = 512 / 1024 layers off the
 * persistent GEMM), "no_rows64_queue" (0 / 1: the K = N = 64 layer with
 * its static tile deal instead of the per-CU tile queue) and
 * "no_layer_tail" (0 / 1: the FNO runtime's width-64 local-linear layer and
 * its tail as two launches instead of one, and its projection head as two
 * to four instead of one) and "generic_fft" (0 / 1: the
 * FNO runtime's row FFTs of 64 .. 1024 points and its channel mix of up to
 * 64 channels on the any-size kernels instead of the fixed-size ones).  The
 * environment variables NFLOW_<NAME> set the initial values, read once at
 * the library's first launch.  Process-wide; *previous (if not NULL)
 * receives the value replaced.  Unknown names return NFLOW_INVALID_ARG. */
int nflow_debug_set_kernel_path(const char* name, int value, int* previous);

/* ---- nflow-quant kernel API (cpp/include/neuroflow/int8_gemm.h) ------------ */

/* Replaces int8_gemm::QuantiseActivation (int8_gemm.h:115-118,
 * int8_gemm.cpp:507-520).  A (bsz, in_features) fp32 -> A_q int8.  Null A or
 * A_q is a silent no-op returning NFLOW_OK, as the reference returns void. */
int nflow_int8_quantise_activation(const float* A, int8_t* A_q, int64_t bsz,
                                   int in_features, float scale_A, int32_t zp_A,
                                   void* stream);

/* Replaces int8_gemm::PrecomputeSumW (int8_gemm.h:74-76,
 * int8_gemm.cpp:479-496): sum_W_out[o] = sum_i (W_int8[o,i] - zp_W[o]).
 * The result goes to caller-owned device memory instead of a new[] array;
 * where the reference returns nullptr (null input, dims <= 0) this returns
 * NFLOW_INVALID_ARG. */
int nflow_int8_precompute_sum_w(const int8_t* W_int8, const int32_t* zp_W,
                                int in_features, int out_features,
                                int32_t* sum_W_out, void* stream);

/* Replaces int8_gemm::LinearForward (int8_gemm.h:90-91,
 * int8_gemm.cpp:201-470) as built with the reference's AVX-512 VNNI flags:
 * one activation row A (in_features) -> C (out_features).  Errors as the
 * reference: null W_int8/scale_W/zp_W/A/C or dims <= 0 -> NFLOW_INVALID_ARG. */
int nflow_int8_linear_forward(const nflow_int8_linear_params* p, const float* A,
                              float* C, void* stream);

/* LinearForward applied to each of `rows` rows of A with the same params
 * (the reference's per-row calling pattern, fno.cpp:87-110), in one launch. */
int nflow_int8_linear_forward_rows(const nflow_int8_linear_params* p, int64_t rows,
                                   const float* A, float* C, void* stream);

/* Replaces int8_gemm::LinearForwardBatched (int8_gemm.h:102-104,
 * int8_gemm.cpp:530-580).  bsz <= 0 -> NFLOW_OK with no work; null A or C ->
 * NFLOW_INVALID_ARG (the reference also dereferences W_int8/scale_W/zp_W
 * unchecked: here those are NFLOW_INVALID_ARG as well). */
int nflow_int8_linear_forward_batched(const nflow_int8_linear_params* p, int64_t bsz,
                                      const float* A, float* C, void* stream);

/* ---- per-token (dynamic) INT8 path ------------------------------------------
 * The reference's per-token path is LinearForward called once per row with
 * that row's scale_A (bench_int8_gemm.cpp:163, fno.cpp:87-110).  Here the
 * per-row scale is computed on the device: scale_A[m] = absmax(row m) / 127
 * (1.0f for an all-zero row), zp_A = 0. */

/* A (M, K) fp32 -> A_q (M, K) int8 codes, scale_A (M), optional sum_a (M) =
 * sum of each row's codes. */
int nflow_int8_quantise_per_token(const float* A, int64_t M, int K, int8_t* A_q,
                                  float* scale_A, int32_t* sum_a, void* stream);

/* The fused hot path: per-token quantise -> INT8 MFMA GEMM -> dequantise +
 * bias + activation, i.e. for every row m the result of LinearForward(p with
 * scale_A = absmax(row m)/127, zp_A = 0) followed by `activation`.  p->scale_A
 * and p->zp_A are ignored.  scale_A_out (nullable, M floats) receives the
 * per-row scales. */
int nflow_int8_linear_forward_per_token(const nflow_int8_linear_params* p, int64_t M,
                                        const float* A, float* C, float* scale_A_out,
                                        int activation, void* stream);

/* Size of the device scratch behind nflow_int8_linear_forward_per_token_noalloc. */
#define NFLOW_NOALLOC_SCRATCH_BYTES ((size_t)72 << 20)

/* nflow_int8_linear_forward_per_token that allocates nothing.  No
 * counterpart in the reference: it is for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments and results, bit for bit.  The
 * shapes the one-launch kernels do not take (e.g. K = 1024: per-token
 * quantise into codes, then the tiled GEMM) keep their codes, scales and
 * byte sums in a static device array of NFLOW_NOALLOC_SCRATCH_BYTES held by
 * each GPU the library runs on until the process ends, instead of a
 * stream-ordered allocation.  Workspace = M*K rounded up to 16, + 4M
 * (scales, unless scale_A_out is given), + 4M (row code sums, with zero
 * points), + 4N (weight-row sums, with a caller's sum_W); a call needing more
 * than the array returns NFLOW_INVALID_ARG before anything is launched.
 * Every call on one GPU shares that array and keeps nothing in it between
 * calls.  Host threads are safe when their calls share a stream: a
 * per-device lock is held from the array's lookup until the call's last
 * launch, so their launches do not interleave.  Calls on different streams
 * that the caller does not order race on the device. */
int nflow_int8_linear_forward_per_token_noalloc(const nflow_int8_linear_params* p, int64_t M,
                                                const float* A, float* C, float* scale_A_out,
                                                int activation, void* stream);

/* The FNO local-linear layer (cpp/src/fno.cpp:515-557, 650-654):
 * y = act(x1 + x2) with x2 = the per-token layer above (bias included) and
 * x1 (M, out_features) the spectral branch, in the operation order of the
 * reference (x2 = (scale_W * scale_A) * float(t) + bias, then x1 + x2, then
 * the activation).  x1 and y are device buffers that must not be the same. */
int nflow_int8_fno_layer_per_token(const nflow_int8_linear_params* p, int64_t M, const float* h,
                                   const float* x1, float* y, float* scale_A_out, int activation,
                                   void* stream);

/* Raw int32 accumulators: C[m][n] = sum_k A_q[m][k] * W_q[n][k]. */
int nflow_int8_gemm_i32(const int8_t* A_q, const int8_t* W_q, int64_t M, int N, int K,
                        int32_t* C, void* stream);

/* GEMM + epilogue on pre-quantised activations: for each row m, the
 * LinearForward result for codes A_q[m] with scale_A[m] and zp_A = 0, then
 * `activation`.  p->scale_A and p->zp_A are ignored. */
int nflow_int8_linear_forward_quantised(const nflow_int8_linear_params* p, int64_t M,
                                        const int8_t* A_q, const float* scale_A, float* C,
                                        int activation, void* stream);

/* nflow_int8_linear_forward_quantised with 8-bit output: the fp32 result of
 * that call (y, M x out_features) is quantised per token as
 * nflow_int8_quantise_per_token quantises it -- scale_C[m] = max_n |y[m][n]| /
 * 127 (1.0f for an all-zero row), C_q[m][n] = round-half-away(y[m][n] /
 * scale_C[m]) -- bit for bit, without y ever reaching memory when the layer
 * is symmetric (zp_W and sum_W_per_row NULL), in_features = 1024 and
 * out_features a multiple of 256 up to 1024, and the stream is not the
 * per-thread default stream; other calls compute y into a stream-ordered
 * buffer first (the same bits).  On a stream being captured into a graph it
 * returns NFLOW_UNSUPPORTED_OP and does nothing (the no-allocation entry
 * point below is the capturable form).  No single reference function: it is one
 * step of a chain of per-token layers (the DeepONet branch and trunk MLPs,
 * cpp/src/fno.cpp:1318-1341, 1364-1386, on the INT8 path of
 * int8_gemm.cpp:201-470), where the next layer's per-token quantise
 * (int8_gemm.cpp:507-520 with scale_A = absmax / 127) reads only codes. */
int nflow_int8_linear_forward_codes(const nflow_int8_linear_params* p, int64_t M, const int8_t* A_q,
                                    const float* scale_A, int8_t* C_q, float* scale_C, int activation,
                                    void* stream);

/* A chain of per-token INT8 layers (the MLPs of DeepONet::Forward,
 * cpp/src/fno.cpp:1318-1341 branch and 1364-1386 trunk, with each Linear on
 * the per-token INT8 path): h = x; h = nflow_int8_linear_forward_per_token(
 * layers[l], h, activations[l]) for l = 0 .. n_layers - 1; y = h.  Bit for
 * bit that sequence.  When every layer is symmetric (zp_W and sum_W_per_row
 * NULL), layers[0].in_features = 1024 and every hidden width is 1024 (the
 * last layer's out_features any), x is 16-byte aligned, M gives at least
 * two 128 x 256 tiles per CU, and the stream is not the per-thread default
 * stream, the hidden activations stay int8 codes + row scales
 * (nflow_int8_linear_forward_codes) and only y is fp32; else the layers run
 * one by one through fp32 buffers (the same bits).  On a stream being
 * captured into a graph: NFLOW_UNSUPPORTED_OP, nothing done.
 * layers[l + 1].in_features != layers[l].out_features ->
 * NFLOW_SHAPE_MISMATCH. */
int nflow_int8_mlp_forward_per_token(const nflow_int8_linear_params* layers, const int* activations,
                                     int n_layers, int64_t M, const float* x, float* y, void* stream);

/* Frees, in stream order, the buffers the library keeps for `stream` on
 * the current device (the workspaces of the per-token entry points and of
 * nflow_int8_mlp_forward_per_token, the 8-bit-output layer's row-maxima
 * words); the next call on the stream allocates anew.  For callers that
 * create and destroy streams: call it before hipStreamDestroy, or a later
 * stream with the same handle reuses the buffers.  No reference
 * counterpart (the reference allocates per call, int8_gemm.cpp:247, 539). */
int nflow_release_stream_workspace(void* stream);

/* Count of timed-out waits of the 8-bit-output kernel on `stream` since the
 * last query (it then resets it), after synchronising the stream.  The
 * kernel's blocks of one row tile wait for each other's row maxima; a wait
 * that lasts 2 s (blocks that could not run concurrently) gives up, leaves
 * wrong codes and counts here.  No reference counterpart (a diagnostic). */
int nflow_debug_chain_faults(void* stream, uint32_t* faults);

/* ---- FP8 E4M3 (cpp/include/neuroflow/fp8_e4m3.h) ---------------------------- */

/* Replaces fp32_array_to_e4m3_bits (fp8_e4m3.h:286-290). */
int nflow_fp8_e4m3_to_bits(const float* in, uint8_t* out, int64_t n, void* stream);

/* Replaces e4m3_bits_to_fp32_array (fp8_e4m3.h:295-299). */
int nflow_fp8_e4m3_from_bits(const uint8_t* in, float* out, int64_t n, void* stream);

/* Replaces fp8_e4m3_per_tensor_fake_quant (fp8_e4m3.h:312-334); in == out
 * is allowed. */
int nflow_fp8_e4m3_fake_quant(const float* in, float scale, float* out, int64_t n,
                              void* stream);

/* Per-token FP8: scale_A[m] = absmax(row m)/448 (1.0f for a zero row); codes
 * are fp32_to_e4m3_bits(clamp(a * (1/scale_A[m]), -448, 448)), the
 * scale-down of fp8_e4m3.h:319-327. */
int nflow_fp8_quantise_per_token(const float* A, int64_t M, int K, uint8_t* A_q,
                                 float* scale_A, void* stream);

/* The optional static fake-quant of x2 in the FNO layer (cpp/src/fno.cpp:
 * 572-648), INT8 forms: q = clamp(std::round(x2 / s) + zp, -128, 127) in
 * float, x2 = (q - zp) * s, applied after the bias and before x1 + x2.
 * PER_POSITION follows the reference's indexing: at that point x2 is laid
 * out (batch, width, points) but the loop addresses it as (batch, points,
 * width), so qparam p applies to flat offset p of a sample's (width, points)
 * plane.  For the token-major layer (row m = sample * points + position,
 * column j) that is index j * points + m % points.  The log2 "FP8" snap of
 * fno.cpp:579-606 is not an E4M3 operation and is not offered. */
enum nflow_x2_quant_kind {
    NFLOW_X2_NONE = 0,
    NFLOW_X2_PER_TENSOR = 1,
    NFLOW_X2_PER_POSITION = 2,
    NFLOW_X2_FP8_LOG2 = 3 /* reported by nflow_ir_fno_x2_quant; the layers reject it */
};

typedef struct nflow_x2_quant {
    int kind;                   /* enum nflow_x2_quant_kind */
    float scale;                /* PER_TENSOR (and FP8_LOG2) */
    int32_t zero_point;         /* PER_TENSOR */
    const float* scales;        /* PER_POSITION: n_positions scales (device memory for the layers) */
    const int32_t* zero_points; /* PER_POSITION: n_positions zero points */
    int64_t n_positions;        /* PER_POSITION: at least out_features * points */
    int32_t width;              /* PER_POSITION: the qparam's width; must equal out_features */
    int32_t points;             /* PER_POSITION: grid points per sample (rows per sample) */
} nflow_x2_quant;

/* nflow_int8_fno_layer_per_token with the x2 fake-quant x2q (NULL or kind
 * NONE: none); x1 may be NULL (no residual term). */
int nflow_int8_fno_layer_per_token_x2q(const nflow_int8_linear_params* p, int64_t M, const float* h,
                                       const float* x1, float* y, float* scale_A_out, int activation,
                                       const nflow_x2_quant* x2q, void* stream);

/* Fused FP8 layer: per-token FP8 quantise -> GEMM on the matrix cores with
 * fp32 accumulation (E4M3 values are exact in bfloat16, so the product runs
 * as bf16 MFMA on exact operands) -> (scale_W[n] * scale_A[m]) * acc +
 * bias[n] -> activation.
 * No FP8 GEMM exists in the reference; its FP8 path is fake-quant followed by
 * the FP32 Linear loop (fp8_e4m3.h:312-334, fno.cpp:68-79). */
int nflow_fp8_linear_forward_per_token(const nflow_fp8_linear_params* p, int64_t M,
                                       const float* A, float* C, float* scale_A_out,
                                       int activation, void* stream);

/* The FNO local-linear layer on the FP8 path: y = act(x1 + x2), x2 the
 * per-token FP8 layer above (see nflow_int8_fno_layer_per_token). */
int nflow_fp8_fno_layer_per_token(const nflow_fp8_linear_params* p, int64_t M, const float* h,
                                  const float* x1, float* y, float* scale_A_out, int activation,
                                  void* stream);

/* nflow_fp8_fno_layer_per_token with the x2 fake-quant (see nflow_x2_quant). */
int nflow_fp8_fno_layer_per_token_x2q(const nflow_fp8_linear_params* p, int64_t M, const float* h,
                                      const float* x1, float* y, float* scale_A_out, int activation,
                                      const nflow_x2_quant* x2q, void* stream);

/* fp32 accumulators of the FP8 GEMM: C[m][n] = sum_k dec(A_q[m][k]) * dec(W_q[n][k]). */
int nflow_fp8_gemm_f32(const uint8_t* A_q, const uint8_t* W_q, int64_t M, int N, int K,
                       float* C, void* stream);

/* GEMM + epilogue on pre-quantised FP8 activations with per-row scales. */
int nflow_fp8_linear_forward_quantised(const nflow_fp8_linear_params* p, int64_t M,
                                       const uint8_t* A_q, const float* scale_A, float* C,
                                       int activation, void* stream);

/* ---- one-time weight blob preparation (HOST pointers, CPU) ------------------
 * Run once per layer when the blobs are built (EnableInt8Gemm, runtime.cpp:
 * 155-166); the results are then uploaded to device memory by the caller. */

/* Replaces fno::QuantiseWeight2D (cpp/src/fno.cpp:325-358): W_q =
 * clamp(std::round(W / s_c) + zp_c) computed in float, and
 * sum_w[c] = sum_i (W_q[c,i] - zp_c).  sum_w may be NULL. */
int nflow_host_quantise_weight_2d(const float* W, int out_features, int in_features,
                                  const float* scales, const int32_t* zero_points,
                                  int8_t* W_q, int32_t* sum_w);

/* Per-channel symmetric scales: absmax(row c) / qmax (1.0f for a zero row);
 * qmax = 127 for INT8, 448 for FP8 E4M3. */
int nflow_host_per_channel_scales(const float* W, int out_features, int in_features,
                                  float qmax, float* scales);

/* Per-channel FP8 E4M3 weights: scales[c] = absmax(row c)/448 (1.0f for a
 * zero row), W_q = fp32_to_e4m3_bits(clamp(W * (1/scales[c]), -448, 448)). */
int nflow_host_fp8_quantise_weight(const float* W, int out_features, int in_features,
                                   uint8_t* W_q, float* scales);

/* ---- device-resident layers ---------------------------------------------
 * The Int8GemmLayer cache of fno::FNO1d::EnableInt8Gemm (cpp/src/fno.cpp:
 * 325-406, cpp/include/neuroflow/fno.h:66-87) as an opaque handle whose weight
 * blob lives in device memory: built and uploaded once, then used by every
 * forward call.  Creation allocates on the current device (hipMalloc) and is
 * not stream-ordered; forward is.  A handle must not be destroyed while work
 * that uses it is pending. */
typedef struct nflow_layer nflow_layer;

/* From host fp32 weights W (out_features, in_features) and an optional host
 * bias: INT8 builds scales = absmax/127 per channel and codes by
 * QuantiseWeight2D with zero points 0 (plus sum_W_per_row); FP8 builds
 * scales = absmax/448 and E4M3 codes. */
int nflow_layer_create(const float* W, const float* bias, int out_features, int in_features,
                       int format, nflow_layer** layer);

/* From an existing INT8 blob (host pointers): codes, per-channel scales and
 * zero points, optional bias and sum_W_per_row -- the per-channel qparams a
 * NIRQ file carries (cpp/include/neuroflow/ir_loader.h:556-650). */
int nflow_layer_create_int8(const int8_t* W_q, const float* scale_W, const int32_t* zp_W,
                            const float* bias, const int32_t* sum_W_per_row, int out_features,
                            int in_features, nflow_layer** layer);

/* The fused per-token layer on device buffers x (M, in_features) and
 * y (M, out_features): nflow_int8_linear_forward_per_token or
 * nflow_fp8_linear_forward_per_token with the handle's blob. */
int nflow_layer_forward(const nflow_layer* layer, int64_t M, const float* x, float* y,
                        float* scale_A_out, int activation, void* stream);

/* The FNO layer form act(x1 + x2) on a handle (see nflow_int8_fno_layer_per_token). */
int nflow_layer_forward_residual(const nflow_layer* layer, int64_t M, const float* x, const float* x1,
                                 float* y, float* scale_A_out, int activation, void* stream);

/* The FNO layer on a handle with the x2 fake-quant; x1 may be NULL. */
int nflow_layer_forward_fno(const nflow_layer* layer, int64_t M, const float* x, const float* x1, float* y,
                            float* scale_A_out, int activation, const nflow_x2_quant* x2q, void* stream);

/* The per-tensor INT8 layer of the IR-driven FNO path: LinearForwardBatched
 * with the handle's blob and the input's per-tensor (scale_A, zp_A), bias
 * added after the dequantisation (cpp/src/fno.cpp:135-156, 541-549);
 * INT8 handles only, M <= INT32_MAX. */
int nflow_layer_forward_per_tensor(const nflow_layer* layer, int64_t M, const float* x, float* y,
                                   float scale_A, int32_t zp_A, void* stream);

int nflow_layer_shape(const nflow_layer* layer, int* out_features, int* in_features, int* format);

/* Frees the handle and its device memory (NULL is allowed). */
int nflow_layer_destroy(nflow_layer* layer);

/* ---- NeuroIR binary + NIRQ block (HOST memory) -------------------------
 * Replaces ir_native::LoadBinary (cpp/include/neuroflow/ir_loader.h:58-654)
 * for what the device path needs: the header, every weight record and the
 * NIRQ qparams (kinds 0-3, ir_loader.h:556-650).  Status codes as the
 * reference: FileNotFound, ParseError, UnsupportedOp (unknown op code).
 * Weight names are not checked against the op's fixed order.  Pointers
 * returned by the accessors live until nflow_ir_close. */
typedef struct nflow_ir nflow_ir;

enum nflow_qparam_kind {
    NFLOW_QPARAM_PER_TENSOR = 0,
    NFLOW_QPARAM_PER_CHANNEL = 1,
    NFLOW_QPARAM_PER_TOKEN = 2,
    NFLOW_QPARAM_FP8_E4M3 = 3
};

int nflow_ir_open(const char* path, nflow_ir** ir);
int nflow_ir_open_memory(const void* data, size_t bytes, nflow_ir** ir);
int nflow_ir_close(nflow_ir* ir);

/* version 1-3; op_code 1-8 (FNO1d, FNO2d, FNO3d, DeepONet, TokenMixer,
 * GraphOp, TokenMixer2D, GraphOp2D); config8: the 7 or 8 config int32s, zero
 * padded; activation 0 gelu / 1 relu; quant_enabled: a NIRQ block was read.
 * Any output pointer may be NULL. */
int nflow_ir_header(const nflow_ir* ir, int* version, int* op_code, int32_t* config8, int* activation,
                    int* quant_enabled);
int nflow_ir_num_weights(const nflow_ir* ir, int* n);
/* Weight record `index` in file order; dims8 holds up to 8 dims. */
int nflow_ir_weight_at(const nflow_ir* ir, int index, const char** name, int* ndim, int64_t* dims8,
                       const float** data);
/* Weight by name (the first record of that name); InvalidArg if absent. */
int nflow_ir_weight(const nflow_ir* ir, const char* name, int* ndim, int64_t* dims8, const float** data);

/* Qparam records in file order (duplicates included) ... */
int nflow_ir_num_qparams(const nflow_ir* ir, int* n);
int nflow_ir_qparam_at(const nflow_ir* ir, int index, const char** name, int* kind);
/* ... and lookups by name, as the reference's maps (the last record of a
 * name wins; a per-tensor name ending in ".output" is an activation qparam,
 * any other a weight qparam).  *found = 0 when absent. */
int nflow_ir_per_tensor_qparam(const nflow_ir* ir, const char* name, int* found, float* scale, int32_t* zp);
int nflow_ir_per_channel_qparam(const nflow_ir* ir, const char* name, int* found, int* n_channels, int* axis,
                                const float** scales, const int32_t** zero_points);
int nflow_ir_per_token_qparam(const nflow_ir* ir, const char* name, int* found, int* n_tokens, int* width,
                              const float** scales, const int32_t** zero_points);
int nflow_ir_fp8_qparam(const nflow_ir* ir, const char* name, int* found, float* scale);

/* EnableInt8Gemm for one weight (cpp/src/fno.cpp:325-406): QuantiseWeight2D
 * with the IR's per-channel scales and zero points of `weight_name` (a 2-D
 * weight, channel axis 0), uploaded once with the IR weight `bias_name`
 * (NULL: no bias) as a device-resident INT8 layer handle. */
int nflow_ir_layer_create(const nflow_ir* ir, const char* weight_name, const char* bias_name,
                          nflow_layer** layer);

/* LinearDispatchTryInt8's decision for the FNO layer locs.{layer_index}
 * once EnableInt8Gemm has run (cpp/src/fno.cpp:125-159, 529-536): INT8 iff
 * its input key (lift.output for layer 0, else locs.{i-1}.output) has no
 * per-token or FP8 qparam, locs.{i}.weight would be cached, and the input
 * key has a per-tensor qparam, whose scale / zero point are returned. */
int nflow_ir_fno_int8_dispatch(const nflow_ir* ir, int layer_index, int* use_int8, float* scale_A,
                               int32_t* zp_A);

/* The x2 fake-quant the reference applies to locs.{layer_index}'s output
 * when the IR carries a qparam for "locs.{i}.output" (fno.cpp:572-648), with
 * its precedence: FP8 (kind FP8_LOG2, scale only), else per-token (kind
 * PER_POSITION; scales / zero_points point into the IR, host memory; points
 * is left 0 for the caller), else per-tensor, else NONE. */
int nflow_ir_fno_x2_quant(const nflow_ir* ir, int layer_index, nflow_x2_quant* x2q);

#ifdef __cplusplus
}
#endif
#endif /* NFLOW_QUANT_H */
