/*
 * nflow_oracle_fno.c -- CPU restatement of the pieces of NeuroFlow's FNO1d
 * and FNO2d forwards (InferenceRuntime::Run, cpp/src/runtime.cpp:79-101, over
 * FNO1d::Forward, cpp/src/fno.cpp:408-700, and FNO2d::Forward, :777-995)
 * that surround the quantised
 * local-linear layer: the radix-2 FFT (cpp/src/fft.cpp), the spectral
 * convolution, the fp32 Linear loop, the weight and activation fake-quants
 * and the log2 "FP8" snap.  TEST INFRASTRUCTURE ONLY (see nflow_oracle.h).
 *
 * Every float operation is written in the reference build's order and
 * rounding: g++ -O3 -mfma (cpp/CMakeLists.txt:15-17, 68, 78) contracts some
 * products into fused multiply-adds in fft.cpp and fno.cpp (none in
 * int8_gemm.cpp).  This file is compiled with -ffp-contract=off and writes
 * each of those fusions as an explicit fmaf, in the form the reference's
 * compiled code takes (read from the x86 code of a reference build made here
 * from its sources):
 *   complex product a * b (std::complex<float>, fft.cpp:57, :61):
 *     re = fma(a.re, b.re, -(a.im * b.im)),  im = fma(a.re, b.im, a.im * b.re);
 *   spectral mix (fno.cpp:184-195): re term fma(-wi, hi, hr * wr),
 *     im term fma(wr, hi, hr * wi), each then added to its sum;
 *   Linear (fno.cpp:75): vectorised in blocks of 16 and 8 with rounded
 *     products, the last k % 8 terms as acc = fma(x, w, acc);
 *   GELU (fno.cpp:44): z + 0.044715 z^3 as fma((0.044715 * z) * z, z, z).
 * libm calls are the reference's: cosf / sinf for the twiddles, tanhf for
 * GELU, log2f and roundf for the snap.
 */
#include "nflow_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_PI_F 3.14159265358979323846f

/* fft.cpp:34-46: in-place bit-reversal permutation of n complex values. */
static void bit_reverse(float* a, int n)
{
    int j = 0;
    for (int i = 1; i < n; ++i) {
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) {
            float tr = a[2 * i], ti = a[2 * i + 1];
            a[2 * i] = a[2 * j];
            a[2 * i + 1] = a[2 * j + 1];
            a[2 * j] = tr;
            a[2 * j + 1] = ti;
        }
    }
}

/* fft.cpp:48-68: iterative radix-2 complex FFT.  The stage twiddle starts at
 * (1, 0) and is advanced by w *= wlen, wlen = (cosf(ang), sinf(ang)) with
 * ang = (+-2 * pi) / len in float; complex products are
 * the fused forms above.  The inverse scales both parts by 1.0f / n. */
void orc_cfft(float* a, int n, int inverse)
{
    bit_reverse(a, n);
    for (int len = 2; len <= n; len <<= 1) {
        const float ang = (inverse ? 2.0f : -2.0f) * ORC_PI_F / (float)len;
        const float wlr = cosf(ang), wli = sinf(ang);
        const int h = len / 2;
        for (int i = 0; i < n; i += len) {
            float wr = 1.0f, wi = 0.0f;
            for (int k = 0; k < h; ++k) {
                float* u = a + 2 * (i + k);
                float* x = a + 2 * (i + k + h);
                const float vr = fmaf(x[0], wr, -(x[1] * wi));
                const float vi = fmaf(x[0], wi, x[1] * wr);
                const float ur = u[0], ui = u[1];
                u[0] = ur + vr;
                u[1] = ui + vi;
                x[0] = ur - vr;
                x[1] = ui - vi;
                const float nr = fmaf(wr, wlr, -(wi * wli));
                const float ni = fmaf(wr, wli, wi * wlr);
                wr = nr;
                wi = ni;
            }
        }
    }
    if (inverse) {
        const float inv = 1.0f / (float)n;
        for (int i = 0; i < 2 * n; ++i) a[i] *= inv;
    }
}

/* fft.cpp:72-84: real input -> n/2 + 1 interleaved complex bins. */
void orc_rfft(const float* x, int n, float* out_complex)
{
    float* buf = (float*)malloc(sizeof(float) * 2 * (size_t)n);
    for (int i = 0; i < n; ++i) {
        buf[2 * i] = x[i];
        buf[2 * i + 1] = 0.0f;
    }
    orc_cfft(buf, n, 0);
    memcpy(out_complex, buf, sizeof(float) * 2 * (size_t)(n / 2 + 1));
    free(buf);
}

/* fft.cpp:86-100: n/2 + 1 bins, the upper half mirrored as conjugates
 * (-im, so a zero bin gives -0.0f), inverse FFT, real part. */
void orc_irfft(const float* xc, int n, float* out)
{
    float* buf = (float*)calloc(2 * (size_t)n, sizeof(float));
    const int half = n / 2 + 1;
    for (int i = 0; i < half; ++i) {
        buf[2 * i] = xc[2 * i];
        buf[2 * i + 1] = xc[2 * i + 1];
    }
    for (int i = 1; i < n - half + 1; ++i) {
        buf[2 * (n - i)] = buf[2 * i];
        buf[2 * (n - i) + 1] = -buf[2 * i + 1];
    }
    orc_cfft(buf, n, 1);
    for (int i = 0; i < n; ++i) out[i] = buf[2 * i];
    free(buf);
}

/* fno.cpp:164-207: h and out (bsz, w, n); weights (in=w, out=w, modes). */
void orc_spectral_conv1d(const float* h, int bsz, int w, int n, int modes,
                         const float* w_real, const float* w_imag, float* out)
{
    const int half = n / 2 + 1;
    float* H = (float*)malloc(sizeof(float) * (size_t)w * half * 2);
    float* O = (float*)malloc(sizeof(float) * (size_t)w * half * 2);
    for (int bi = 0; bi < bsz; ++bi) {
        memset(O, 0, sizeof(float) * (size_t)w * half * 2);
        for (int wi = 0; wi < w; ++wi)
            orc_rfft(h + ((size_t)bi * w + wi) * n, n, H + (size_t)wi * half * 2);
        for (int mi = 0; mi < modes; ++mi) {
            for (int wo = 0; wo < w; ++wo) {
                float sr = 0.0f, si = 0.0f;
                for (int k = 0; k < w; ++k) {
                    const float hr = H[(size_t)k * half * 2 + 2 * mi];
                    const float hi = H[(size_t)k * half * 2 + 2 * mi + 1];
                    const float wr = w_real[((size_t)k * w + wo) * modes + mi];
                    const float wim = w_imag[((size_t)k * w + wo) * modes + mi];
                    sr += fmaf(-wim, hi, hr * wr);
                    si += fmaf(wr, hi, hr * wim);
                }
                O[(size_t)wo * half * 2 + 2 * mi] = sr;
                O[(size_t)wo * half * 2 + 2 * mi + 1] = si;
            }
        }
        for (int wo = 0; wo < w; ++wo)
            orc_irfft(O + (size_t)wo * half * 2, n, out + ((size_t)bi * w + wo) * n);
    }
    free(H);
    free(O);
}

/* fft.cpp:101-124: the real FFT of each of the H rows (W points each), then
 * the complex FFT of each of the W/2 + 1 columns; out (H, W/2 + 1)
 * interleaved complex. */
void orc_rfft2(const float* x, int H, int W, float* out)
{
    const int hw = W / 2 + 1;
    float* scratch = (float*)malloc(sizeof(float) * 2 * (size_t)H * hw);
    float* col = (float*)malloc(sizeof(float) * 2 * (size_t)H);
    for (int i = 0; i < H; ++i) orc_rfft(x + (size_t)i * W, W, scratch + (size_t)i * hw * 2);
    for (int j = 0; j < hw; ++j) {
        for (int i = 0; i < H; ++i) {
            col[2 * i] = scratch[((size_t)i * hw + j) * 2];
            col[2 * i + 1] = scratch[((size_t)i * hw + j) * 2 + 1];
        }
        orc_cfft(col, H, 0);
        for (int i = 0; i < H; ++i) {
            out[((size_t)i * hw + j) * 2] = col[2 * i];
            out[((size_t)i * hw + j) * 2 + 1] = col[2 * i + 1];
        }
    }
    free(col);
    free(scratch);
}

/* fft.cpp:126-148: the inverse complex FFT of each of the W/2 + 1 columns
 * (with its 1/H), then the inverse real FFT of each row (with its 1/W). */
void orc_irfft2(const float* xc, int H, int W, float* out)
{
    const int hw = W / 2 + 1;
    float* scratch = (float*)malloc(sizeof(float) * 2 * (size_t)H * hw);
    float* col = (float*)malloc(sizeof(float) * 2 * (size_t)H);
    for (int j = 0; j < hw; ++j) {
        for (int i = 0; i < H; ++i) {
            col[2 * i] = xc[((size_t)i * hw + j) * 2];
            col[2 * i + 1] = xc[((size_t)i * hw + j) * 2 + 1];
        }
        orc_cfft(col, H, 1);
        for (int i = 0; i < H; ++i) {
            scratch[((size_t)i * hw + j) * 2] = col[2 * i];
            scratch[((size_t)i * hw + j) * 2 + 1] = col[2 * i + 1];
        }
    }
    for (int i = 0; i < H; ++i) orc_irfft(scratch + (size_t)i * hw * 2, W, out + (size_t)i * W);
    free(col);
    free(scratch);
}

/* fno.cpp:717-771: h and out (bsz, w, H, W); weights (in=w, out=w, mh, mw);
 * the output spectrum is zero outside the (mh, mw) corner.  The channel
 * mix has the 1-D mix's fused terms (the same x86 code in the build). */
void orc_spectral_conv2d(const float* h, int bsz, int w, int H, int W, int mh, int mw,
                         const float* w_real, const float* w_imag, float* out)
{
    const int hw = W / 2 + 1;
    const size_t plane = (size_t)H * hw * 2;
    float* S = (float*)malloc(sizeof(float) * (size_t)w * plane);
    float* O = (float*)malloc(sizeof(float) * (size_t)w * plane);
    for (int bi = 0; bi < bsz; ++bi) {
        memset(O, 0, sizeof(float) * (size_t)w * plane);
        for (int wi = 0; wi < w; ++wi)
            orc_rfft2(h + ((size_t)bi * w + wi) * H * W, H, W, S + (size_t)wi * plane);
        for (int mi = 0; mi < mh; ++mi) {
            for (int mj = 0; mj < mw; ++mj) {
                for (int wo = 0; wo < w; ++wo) {
                    float sr = 0.0f, si = 0.0f;
                    for (int k = 0; k < w; ++k) {
                        const float* hv = S + (size_t)k * plane + ((size_t)mi * hw + mj) * 2;
                        const size_t wix = (((size_t)k * w + wo) * mh + mi) * mw + mj;
                        const float wr = w_real[wix], wim = w_imag[wix];
                        sr += fmaf(-wim, hv[1], hv[0] * wr);
                        si += fmaf(wr, hv[1], hv[0] * wim);
                    }
                    float* ov = O + (size_t)wo * plane + ((size_t)mi * hw + mj) * 2;
                    ov[0] = sr;
                    ov[1] = si;
                }
            }
        }
        for (int wo = 0; wo < w; ++wo)
            orc_irfft2(O + (size_t)wo * plane, H, W, out + ((size_t)bi * w + wo) * H * W);
    }
    free(S);
    free(O);
}

/* fno.cpp:69-79 (the non-Eigen Linear), as the reference build computes it:
 * g++ -O3 vectorises the k loop as an in-order ("fold-left") reduction, so
 * acc starts at the bias; each block of 16 products, then one block of 8
 * if at least 8 remain, is added product by product with every product
 * rounded; the last k % 8 terms are contracted, acc = fma(x[p], W[j][p],
 * acc). */
static float linear_dot(const float* x, const float* w, float acc, int k)
{
    int p = 0;
    for (; p + 16 <= k; p += 16)
        for (int t = 0; t < 16; ++t) acc += x[p + t] * w[p + t];
    if (k - p >= 8) {
        for (int t = 0; t < 8; ++t) acc += x[p + t] * w[p + t];
        p += 8;
    }
    for (; p < k; ++p) acc = fmaf(x[p], w[p], acc);
    return acc;
}

void orc_linear_f32(const float* x, const float* W, const float* b, int64_t rows, int k, int n,
                    float* y)
{
    for (int64_t i = 0; i < rows; ++i) {
        const float* xi = x + i * k;
        float* yi = y + i * n;
        for (int j = 0; j < n; ++j) yi[j] = linear_dot(xi, W + (size_t)j * k, b ? b[j] : 0.0f, k);
    }
}

/* The fake-quant round trip of fno.cpp:250-255 (weights), :494-499 (layer
 * input), :623-630 and :640-645 (x2): q = std::round(v / s) + zp in float,
 * clamped to [-128, 127], then (q - zp) * s.  Per element scales / zero
 * points (one per element; callers broadcast). */
void orc_fake_quant_arr(const float* in, const float* scales, const int32_t* zps, float* out,
                        int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        const float s = scales[i];
        const float zp = (float)zps[i];
        float q = roundf(in[i] / s) + zp;
        if (q < -128.0f) q = -128.0f;
        if (q > 127.0f) q = 127.0f;
        out[i] = (q - zp) * s;
    }
}

/* x86 cvttss2si (the float -> int conversion of the ldexp argument). */
static int cvt_i32_x86(float f)
{
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int)f;
}

/* fno.cpp:579-606: the log2 "FP8" snap of x2 with per-tensor scale s > 0:
 * v = x / s; |v| < 2^-6 passes; otherwise 2^e with
 * e = int(std::round(log2(|v|) * 8) / 8) (the float exponent argument of
 * std::ldexp(float, int) converts by truncation), then std::min(., 448)
 * (NaN stays NaN there), times the sign and s.  NaN / Inf give e =
 * INT_MIN, i.e. 0. */
float orc_log2_snap_one(float x, float s)
{
    const float v = x / s;
    const float abs_v = fabsf(v);
    const float sign = v < 0.0f ? -1.0f : 1.0f;
    const float qv = (abs_v < 0.015625f)
                         ? abs_v
                         : ldexpf(1.0f, cvt_i32_x86(roundf(log2f(abs_v) * 8.0f) / 8.0f));
    const float clamped = (448.0f < qv) ? 448.0f : qv;
    return sign * clamped * s;
}

void orc_log2_snap(const float* in, float s, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_log2_snap_one(in[i], s);
}

/* The std::round(log2(a) * 8) / 8 exponent of the snap, as the reference's
 * libm computes it (for locating its step points). */
int orc_log2_snap_exponent(float a)
{
    return cvt_i32_x86(roundf(log2f(a) * 8.0f) / 8.0f);
}
