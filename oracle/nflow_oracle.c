/*
 * nflow_oracle.c -- CPU restatement of NeuroFlow's quantised inference GEMM
 * path.  TEST INFRASTRUCTURE ONLY (see nflow_oracle.h): the reference results
 * the HIP path is compared against, never the thing measured or shipped.
 *
 * Citations are file:line in the NeuroFlow source tree.  The arithmetic is
 * written so that gcc -O2 -ffp-contract=off rounds every float operation in
 * the same order as the reference C++.
 */
#include "nflow_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* x86 cvttss2si: NaN and |f| >= 2^31 give the "integer indefinite" value
 * INT32_MIN.  The reference's static_cast<int32_t>(float) compiles to it
 * (int8_gemm.cpp:234, :446, :514), so NaN / Inf / huge quotients quantise
 * through INT32_MIN + zp before the clamp. */
static int32_t cvt_f32_i32_x86(float f)
{
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int32_t)f;
}

static int32_t wrap_add_i32(int32_t a, int32_t b)
{
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

static int32_t wrap_sub_i32(int32_t a, int32_t b)
{
    return (int32_t)((uint32_t)a - (uint32_t)b);
}

static int32_t wrap_mul_i32(int32_t a, int32_t b)
{
    return (int32_t)((uint32_t)a * (uint32_t)b);
}

/* int8_gemm.cpp:513-518. */
int8_t orc_quantise_one(float a, float scale, int32_t zp)
{
    const float quot = a / scale;             /* true IEEE division */
    const float rounded = roundf(quot);       /* half away from zero */
    int32_t q = wrap_add_i32(cvt_f32_i32_x86(rounded), zp);
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    return (int8_t)q;
}

/* int8_gemm.cpp:507-520. */
void orc_quantise_activation(const float* A, int8_t* A_q, int64_t bsz,
                             int in_features, float scale_A, int32_t zp_A)
{
    if (!A || !A_q) return;
    const int64_t n = bsz * (int64_t)in_features;
    for (int64_t i = 0; i < n; ++i) A_q[i] = orc_quantise_one(A[i], scale_A, zp_A);
}

static float row_absmax(const float* x, int K)
{
    float m = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float a = fabsf(x[k]);
        if (a > m) m = a;
    }
    return m;
}

void orc_per_token_scales(const float* A, int64_t M, int K, float qmax,
                          float* scales)
{
    for (int64_t m = 0; m < M; ++m) {
        const float mx = row_absmax(A + m * K, K);
        scales[m] = (mx == 0.0f) ? 1.0f : mx / qmax;
    }
}

void orc_quantise_per_token_i8(const float* A, int64_t M, int K,
                               int8_t* A_q, float* scales, int32_t* sum_a)
{
    orc_per_token_scales(A, M, K, 127.0f, scales);
    for (int64_t m = 0; m < M; ++m) {
        int32_t s = 0;
        for (int k = 0; k < K; ++k) {
            const int8_t q = orc_quantise_one(A[m * K + k], scales[m], 0);
            A_q[m * K + k] = q;
            s += q;
        }
        if (sum_a) sum_a[m] = s;
    }
}

/* fno.cpp:340-356: the code is computed in float (round, + zp, clamp) and
 * then narrowed with static_cast<int8_t>; a NaN survives the clamps and
 * narrows through cvttss2si to 0x80000000, whose low byte is 0. */
void orc_quantise_weight_2d(const float* W, int out_f, int in_f,
                            const float* scales, const int32_t* zps,
                            int8_t* W_q, int32_t* sum_w)
{
    for (int c = 0; c < out_f; ++c) {
        const float s = scales[c];
        const float zp = (float)zps[c];
        int32_t row_sum = 0;
        for (int i = 0; i < in_f; ++i) {
            const int64_t off = (int64_t)c * in_f + i;
            float q = roundf(W[off] / s) + zp;
            if (q < -128.0f) q = -128.0f;
            if (q > 127.0f) q = 127.0f;
            const int8_t q8 = (int8_t)(uint8_t)(uint32_t)cvt_f32_i32_x86(q);
            W_q[off] = q8;
            row_sum += (int32_t)q8 - zps[c];
        }
        if (sum_w) sum_w[c] = row_sum;
    }
}

void orc_per_channel_scales(const float* W, int out_f, int in_f, float qmax,
                            float* scales)
{
    orc_per_token_scales(W, out_f, in_f, qmax, scales);
}

/* int8_gemm.cpp:479-496. */
void orc_precompute_sum_w(const int8_t* W_q, const int32_t* zp_W, int in_f,
                          int out_f, int32_t* out)
{
    for (int o = 0; o < out_f; ++o) {
        int32_t acc = 0;
        for (int i = 0; i < in_f; ++i) acc += (int32_t)W_q[(int64_t)o * in_f + i] - zp_W[o];
        out[o] = acc;
    }
}

void orc_gemm_i8_i32(const int8_t* A_q, const int8_t* W_q, int64_t M, int N,
                     int K, int32_t* C)
{
    for (int64_t m = 0; m < M; ++m) {
        const int8_t* a = A_q + m * K;
        for (int n = 0; n < N; ++n) {
            const int8_t* w = W_q + (int64_t)n * K;
            int64_t acc = 0;
            for (int k = 0; k < K; ++k) acc += (int64_t)a[k] * (int64_t)w[k];
            C[m * N + n] = (int32_t)acc;
        }
    }
}

/* The shared dequantise + bias step: (scale_W[o] * scale_A) * float(t) + b,
 * int8_gemm.cpp:464-467 and :573-576. */
static float dequant_bias(float sw, float sa, int64_t t, const float* bias, int o)
{
    const float y = sw * sa * (float)t;
    return y + (bias ? bias[o] : 0.0f);
}

/* int8_gemm.cpp:530-580. */
int orc_linear_forward_batched(const orc_int8_linear_params* p, int64_t bsz,
                               const float* A, float* C)
{
    if (bsz <= 0) return ORC_OK;
    if (!A || !C) return ORC_INVALID_ARG;
    const int K = p->in_features;
    const int N = p->out_features;
    int8_t* Aq = (int8_t*)malloc((size_t)(bsz * K > 0 ? bsz * K : 1));
    if (!Aq) return ORC_INTERNAL;
    orc_quantise_activation(A, Aq, bsz, K, p->scale_A, p->zp_A);
    for (int64_t r = 0; r < bsz; ++r) {
        const int8_t* a = Aq + r * K;
        int32_t sa = 0;
        for (int i = 0; i < K; ++i) sa = wrap_add_i32(sa, a[i]);
        for (int o = 0; o < N; ++o) {
            const int8_t* w = p->W_int8 + (int64_t)o * K;
            const int32_t zpw = p->zp_W[o];
            int32_t acc = 0;
            for (int i = 0; i < K; ++i)
                acc = wrap_add_i32(acc, wrap_mul_i32(a[i], (int32_t)w[i] - zpw));
            const int32_t sw_sum = p->sum_W_per_row ? p->sum_W_per_row[o] : 0;
            const int32_t t32 = wrap_sub_i32(wrap_sub_i32(acc, wrap_mul_i32(zpw, sa)),
                                             wrap_mul_i32(p->zp_A, sw_sum));
            const int64_t t = (int64_t)t32 + (int64_t)K * zpw * p->zp_A;
            C[r * N + o] = dequant_bias(p->scale_W[o], p->scale_A, t, p->bias, o);
        }
    }
    free(Aq);
    return ORC_OK;
}

/* int8_gemm.cpp:201-470 in its AVX-512 VNNI build.  For in_features <= 4096
 * the row is quantised once (:231-240); the per-output dot product runs
 * over the first in_f - in_f % 64 elements with a pre-shift of +128
 * (:365-376, :178-183) and is corrected with the per-row weight sum
 * (:386-393); the tail products of :378-385 are overwritten by :388 and so
 * do not reach the output.  Above 4096 the scalar loop of :444-456 runs. */
int orc_linear_forward(const orc_int8_linear_params* p, const float* A,
                       float* C)
{
    if (!p->W_int8 || !p->scale_W || !p->zp_W || !A || !C) return ORC_INVALID_ARG;
    if (p->in_features <= 0 || p->out_features <= 0) return ORC_INVALID_ARG;
    const int K = p->in_features;
    const int N = p->out_features;
    const float sA = p->scale_A;
    const int32_t zpA = p->zp_A;

    if (K <= 4096) {
        int8_t aq[4096];
        int32_t sum_a_int8 = 0;
        for (int i = 0; i < K; ++i) {
            aq[i] = orc_quantise_one(A[i], sA, zpA);
            sum_a_int8 += aq[i];
        }
        const int vec_end = K - K % 64;
        for (int o = 0; o < N; ++o) {
            const int8_t* w = p->W_int8 + (int64_t)o * K;
            const int32_t zpw = p->zp_W[o];
            int32_t sw_row;
            if (p->sum_W_per_row) {
                sw_row = p->sum_W_per_row[o];
            } else {
                sw_row = 0;
                for (int i = 0; i < K; ++i) sw_row += w[i];
            }
            int32_t dot = 0;
            for (int i = 0; i < vec_end; ++i)
                dot = wrap_add_i32(dot, ((int32_t)aq[i] + 128) * (int32_t)w[i]);
            const int32_t raw_dot = wrap_sub_i32(dot, wrap_mul_i32(128, sw_row));
            int32_t acc = wrap_sub_i32(raw_dot, wrap_mul_i32(zpA, sw_row));
            acc = wrap_sub_i32(acc, wrap_mul_i32(zpw, sum_a_int8));
            acc = wrap_add_i32(acc, wrap_mul_i32(wrap_mul_i32(K, zpA), zpw));
            const int32_t sum_a = wrap_sub_i32(sum_a_int8, wrap_mul_i32(K, zpA));
            const int32_t sum_w = wrap_sub_i32(sw_row, wrap_mul_i32(K, zpw));
            const int32_t t32 = wrap_sub_i32(wrap_sub_i32(acc, wrap_mul_i32(zpw, sum_a)),
                                             wrap_mul_i32(zpA, sum_w));
            const int64_t t = (int64_t)t32 + (int64_t)K * zpw * zpA;
            C[o] = dequant_bias(p->scale_W[o], sA, t, p->bias, o);
        }
        return ORC_OK;
    }

    for (int o = 0; o < N; ++o) {
        const int8_t* w = p->W_int8 + (int64_t)o * K;
        const int32_t zpw = p->zp_W[o];
        int32_t acc = 0, sum_a = 0, sum_w = 0;
        for (int i = 0; i < K; ++i) {
            const int32_t a_eff = (int32_t)orc_quantise_one(A[i], sA, zpA) - zpA;
            const int32_t w_eff = (int32_t)w[i] - zpw;
            acc = wrap_add_i32(acc, wrap_mul_i32(w_eff, a_eff));
            sum_a = wrap_add_i32(sum_a, a_eff);
            sum_w = wrap_add_i32(sum_w, w_eff);
        }
        const int32_t t32 = wrap_sub_i32(wrap_sub_i32(acc, wrap_mul_i32(zpw, sum_a)),
                                         wrap_mul_i32(zpA, sum_w));
        const int64_t t = (int64_t)t32 + (int64_t)K * zpw * zpA;
        C[o] = dequant_bias(p->scale_W[o], sA, t, p->bias, o);
    }
    return ORC_OK;
}

/* fno.cpp:36-48.  c = std::sqrt(2.0f / static_cast<float>(M_PI)).  The
 * reference build (g++ -O3 -mfma) fuses the last product of
 * z + 0.044715f * z * z * z with the addition: fma((0.044715f * z) * z, z, z);
 * the other operations round one by one. */
void orc_apply_activation(float* y, int64_t n, int act)
{
    if (act == ORC_ACT_RELU) {
        for (int64_t i = 0; i < n; ++i)
            if (y[i] < 0.0f) y[i] = 0.0f;
    } else if (act == ORC_ACT_GELU_TANH) {
        const float pi_f = (float)3.14159265358979323846;
        const float c = sqrtf(2.0f / pi_f);
        for (int64_t i = 0; i < n; ++i) {
            const float z = y[i];
            const float inner = fmaf((0.044715f * z) * z, z, z);
            y[i] = (0.5f * z) * (1.0f + tanhf(c * inner));
        }
    }
}

int orc_layer_per_token_i8(const orc_int8_linear_params* p, int64_t M,
                           const float* A, float* C, int act,
                           float* scale_A_out)
{
    const int K = p->in_features;
    const int N = p->out_features;
    for (int64_t m = 0; m < M; ++m) {
        orc_int8_linear_params row = *p;
        const float mx = row_absmax(A + m * K, K);
        row.scale_A = (mx == 0.0f) ? 1.0f : mx / 127.0f;
        row.zp_A = 0;
        if (scale_A_out) scale_A_out[m] = row.scale_A;
        const int rc = orc_linear_forward(&row, A + m * K, C + m * N);
        if (rc != ORC_OK) return rc;
        orc_apply_activation(C + m * N, N, act);
    }
    return ORC_OK;
}

/* fno.cpp:572-648, INT8 forms of the fake-quant of x2, on x2 held
 * token-major (M = batch * points rows, N = width columns), as this library
 * holds it.  The reference holds x2 as (batch, width, points) at that point
 * (fno.cpp:550-556) and indexes it in its per-token loop (fno.cpp:615-633) as
 * (batch, points, width); this restatement rebuilds the (batch, width,
 * points) buffer, runs that loop as written, and maps back.  Per tensor
 * (scales == NULL): every element with (scale, zp) (fno.cpp:634-646).
 * M must be a multiple of points for the per-position form. */
static float orc_fq1(float v, float scale, float zpf)
{
    float q = roundf(v / scale) + zpf;
    if (q < -128.0f) q = -128.0f;
    if (q > 127.0f) q = 127.0f;
    return (q - zpf) * scale;
}

int orc_x2_fake_quant(const float* x2, float* out, int64_t M, int N, float scale, int32_t zp,
                      const float* scales, const int32_t* zps, int points)
{
    if (!scales) {
        const float zpf = (float)zp;
        for (int64_t i = 0; i < M * (int64_t)N; ++i) out[i] = orc_fq1(x2[i], scale, zpf);
        return ORC_OK;
    }
    if (points <= 0 || M % points != 0) return ORC_INVALID_ARG;
    const int64_t n = points, w = N, bsz = M / points;
    float* buf = (float*)malloc(sizeof(float) * (size_t)(n * w));
    if (!buf) return ORC_INTERNAL;
    for (int64_t bi = 0; bi < bsz; ++bi) {
        /* x2 of sample bi as the reference holds it: [wi * n + ni]. */
        for (int64_t wi = 0; wi < w; ++wi)
            for (int64_t ni = 0; ni < n; ++ni) buf[wi * n + ni] = x2[(bi * n + ni) * w + wi];
        /* fno.cpp:620-632: qp_idx = ni * w_axis + wi, off = ni * w_axis + wi. */
        for (int64_t ni = 0; ni < n; ++ni)
            for (int64_t wi = 0; wi < w; ++wi) {
                const int64_t qp_idx = ni * w + wi;
                buf[qp_idx] = orc_fq1(buf[qp_idx], scales[qp_idx], (float)zps[qp_idx]);
            }
        for (int64_t wi = 0; wi < w; ++wi)
            for (int64_t ni = 0; ni < n; ++ni) out[(bi * n + ni) * w + wi] = buf[wi * n + ni];
    }
    free(buf);
    return ORC_OK;
}

/* ---- FP8 E4M3 ---------------------------------------------------------- */

/* fp8_e4m3.h:106-215.  The byte is assembled from the top three mantissa
 * bits with round-to-nearest-even on the 20-bit residue; exponents above 15
 * saturate to +-448; and -- on the exponent taken BEFORE rounding -- values
 * below the normal range go through nearbyint(|x| * 2^9) clamped to 0..7
 * (so [7.5*2^-9, 2^-6) encodes as 0x07, and (464, 496) encodes as NaN). */
uint8_t orc_e4m3_encode(float v)
{
    if (isnan(v)) return 0x7F;
    if (isinf(v)) return v < 0.0f ? 0xFE : 0x7E;
    uint32_t u;
    memcpy(&u, &v, sizeof u);
    const uint32_t sign = u >> 31;
    const uint32_t mag = u & 0x7FFFFFFFu;
    if (mag == 0) return (uint8_t)(sign << 7);
    const int32_t exp_pre = (int32_t)(mag >> 23) - 127 + 7;
    int32_t exp = exp_pre;
    uint32_t man = (mag >> 20) & 0x7u;
    const uint32_t rest = mag & 0xFFFFFu;
    if (rest > 0x80000u || (rest == 0x80000u && (man & 1u))) man += 1u;
    if (man & 0x8u) {
        man &= 0x7u;
        exp += 1;
    }
    if (exp > 15) return (uint8_t)((sign << 7) | 0x7Eu);
    if (exp_pre < 1) {
        float fmag;
        memcpy(&fmag, &mag, sizeof fmag);
        long long r = llrint((double)fmag * 512.0);   /* default mode: RNE */
        if (r < 0) r = 0;
        if (r > 7) r = 7;
        man = (uint32_t)r;
        exp = 0;
    }
    return (uint8_t)((sign << 7) | ((uint32_t)exp << 3) | man);
}

/* fp8_e4m3.h:223-275. */
float orc_e4m3_decode(uint8_t b)
{
    const uint32_t sign = (b >> 7) & 1u;
    const uint32_t e = (b >> 3) & 0xFu;
    const uint32_t m = b & 0x7u;
    float out;
    if (e == 0xFu && m == 0x7u) {
        const uint32_t q = 0x7FC00000u | (sign << 31);
        memcpy(&out, &q, sizeof out);
        return out;
    }
    if (e == 0) {
        if (m == 0) return sign ? -0.0f : 0.0f;
        out = ldexpf((float)m, -9);
        return sign ? -out : out;
    }
    const uint32_t bits = (sign << 31) | ((e + 120u) << 23) | (m << 20);
    memcpy(&out, &bits, sizeof out);
    return out;
}

void orc_e4m3_encode_array(const float* in, uint8_t* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = orc_e4m3_encode(in[i]);
}

void orc_e4m3_decode_array(const uint8_t* in, float* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = orc_e4m3_decode(in[i]);
}

void orc_e4m3_encode_bits_range(uint32_t start, uint32_t count, uint8_t* out)
{
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t u = start + i;
        float f;
        memcpy(&f, &u, sizeof f);
        out[i] = orc_e4m3_encode(f);
    }
}

void orc_e4m3_encode_bits_stride(uint32_t start, uint32_t stride, uint32_t count,
                                 uint8_t* out)
{
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t u = start + i * stride;
        float f;
        memcpy(&f, &u, sizeof f);
        out[i] = orc_e4m3_encode(f);
    }
}

/* fp8_e4m3.h:319-329: scale down with a reciprocal multiply, clamp +-448. */
uint8_t orc_fp8_quantise_one(float x, float inv_scale)
{
    const float xs = x * inv_scale;
    const float xc = (xs > 448.0f) ? 448.0f : (xs < -448.0f) ? -448.0f : xs;
    return orc_e4m3_encode(xc);
}

/* fp8_e4m3.h:312-334. */
void orc_fp8_fake_quant(const float* in, float scale, float* out, size_t n)
{
    const float inv = (scale == 0.0f) ? 1.0f : (1.0f / scale);
    for (size_t i = 0; i < n; ++i) out[i] = orc_e4m3_decode(orc_fp8_quantise_one(in[i], inv)) * scale;
}

void orc_quantise_per_token_fp8(const float* A, int64_t M, int K,
                                uint8_t* A_q, float* scales)
{
    orc_per_token_scales(A, M, K, 448.0f, scales);
    for (int64_t m = 0; m < M; ++m) {
        const float inv = (scales[m] == 0.0f) ? 1.0f : (1.0f / scales[m]);
        for (int k = 0; k < K; ++k) A_q[m * K + k] = orc_fp8_quantise_one(A[m * K + k], inv);
    }
}

void orc_quantise_weight_fp8(const float* W, int out_f, int in_f,
                             uint8_t* W_q, float* scales)
{
    orc_quantise_per_token_fp8(W, out_f, in_f, W_q, scales);
}

void orc_gemm_fp8_exact(const uint8_t* A_q, const uint8_t* W_q, int64_t M,
                        int N, int K, double* C)
{
    float lut[256];
    for (int b = 0; b < 256; ++b) lut[b] = orc_e4m3_decode((uint8_t)b);
    for (int64_t m = 0; m < M; ++m) {
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k)
                acc += (double)lut[A_q[m * K + k]] * (double)lut[W_q[(int64_t)n * K + k]];
            C[m * N + n] = acc;
        }
    }
}

void orc_layer_fp8_composed(const float* A, const float* W, const float* bias,
                            int64_t M, int N, int K, int act, float* C,
                            float* scale_A_out, float* scale_W_out)
{
    float* sw = (float*)malloc(sizeof(float) * (size_t)N);
    float* wf = (float*)malloc(sizeof(float) * (size_t)N * (size_t)K);
    float* af = (float*)malloc(sizeof(float) * (size_t)K);
    orc_per_channel_scales(W, N, K, 448.0f, sw);
    for (int n = 0; n < N; ++n) orc_fp8_fake_quant(W + (int64_t)n * K, sw[n], wf + (int64_t)n * K, (size_t)K);
    for (int64_t m = 0; m < M; ++m) {
        float sa;
        orc_per_token_scales(A + m * K, 1, K, 448.0f, &sa);
        if (scale_A_out) scale_A_out[m] = sa;
        orc_fp8_fake_quant(A + m * K, sa, af, (size_t)K);
        for (int n = 0; n < N; ++n) {
            const float* wj = wf + (int64_t)n * K;
            float acc = bias ? bias[n] : 0.0f;          /* fno.cpp:72 */
            for (int k = 0; k < K; ++k) acc += af[k] * wj[k];   /* fno.cpp:74 */
            C[m * N + n] = acc;
        }
        orc_apply_activation(C + m * N, N, act);
    }
    if (scale_W_out) memcpy(scale_W_out, sw, sizeof(float) * (size_t)N);
    free(sw);
    free(wf);
    free(af);
}

void orc_layer_fp8_exact(const uint8_t* A_q, const float* scale_A,
                         const uint8_t* W_q, const float* scale_W,
                         const float* bias, int64_t M, int N, int K, int act,
                         float* C)
{
    double* acc = (double*)malloc(sizeof(double) * (size_t)N);
    for (int64_t m = 0; m < M; ++m) {
        orc_gemm_fp8_exact(A_q + m * K, W_q, 1, N, K, acc);
        for (int n = 0; n < N; ++n) {
            const float y = scale_W[n] * scale_A[m] * (float)acc[n];
            C[m * N + n] = y + (bias ? bias[n] : 0.0f);
        }
        orc_apply_activation(C + m * N, N, act);
    }
    free(acc);
}
