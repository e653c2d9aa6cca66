// host_quant.cpp -- host-side parts of libnflow_quant: the last-error slot and
// the one-time weight blob preparation run when a layer's INT8 / FP8 weights
// are built (the reference does this on the CPU in fno::QuantiseWeight2D,
// cpp/src/fno.cpp:325-358, called from EnableInt8Gemm, runtime.cpp:155-166).
// The resulting codes are uploaded once; no per-call work happens here.
//
// Compiled without fast-math and with -ffp-contract=off, so std::round(W / s)
// rounds exactly as the reference's x86 build.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>

#include "nflow_quant.h"
#include "status.h"

namespace nfq {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

// x86 cvttss2si: NaN and out-of-range values give INT32_MIN.
static int32_t cvt_i32_x86(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return static_cast<int32_t>(f);
}

static float row_absmax(const float* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = std::fabs(x[i]);
        if (a > m) m = a;
    }
    return m;
}

// fp32_to_e4m3_bits (cpp/include/neuroflow/fp8_e4m3.h:106-215): the same
// bit-level rounding as the device encoder in common.h.
static uint8_t e4m3_encode_host(float v) {
    uint32_t u;
    std::memcpy(&u, &v, sizeof u);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t mag = u & 0x7FFFFFFFu;
    if (mag > 0x7F800000u) return 0x7Fu;
    if (mag == 0x7F800000u) return static_cast<uint8_t>(sign | 0x7Eu);
    if (mag == 0u) return static_cast<uint8_t>(sign);
    const int32_t exp_pre = static_cast<int32_t>(mag >> 23) - 120;
    uint32_t man = (mag >> 20) & 0x7u;
    const uint32_t rest = mag & 0xFFFFFu;
    man += (rest > 0x80000u || (rest == 0x80000u && (man & 1u))) ? 1u : 0u;
    const int32_t exp = exp_pre + static_cast<int32_t>(man >> 3);
    man &= 0x7u;
    if (exp > 15) return static_cast<uint8_t>(sign | 0x7Eu);
    if (exp_pre < 1) {
        float fm;
        std::memcpy(&fm, &mag, sizeof fm);
        const float r = std::nearbyint(fm * 512.0f);
        const uint32_t ri = static_cast<uint32_t>(r);
        return static_cast<uint8_t>(sign | (ri > 7u ? 7u : ri));
    }
    return static_cast<uint8_t>(sign | (static_cast<uint32_t>(exp) << 3) | man);
}

}  // namespace nfq

using namespace nfq;

extern "C" {

const char* nflow_last_error(void) { return g_last_error.c_str(); }

int nflow_host_quantise_weight_2d(const float* W, int out_features, int in_features,
                                  const float* scales, const int32_t* zero_points, int8_t* W_q,
                                  int32_t* sum_w) {
    clear_error();
    if (!W || !scales || !zero_points || !W_q)
        return set_error(NFLOW_INVALID_ARG, "QuantiseWeight2D: null pointer");
    if (out_features <= 0 || in_features <= 0)
        return set_error(NFLOW_INVALID_ARG, "QuantiseWeight2D: bad dims");
    for (int c = 0; c < out_features; ++c) {
        const float s = scales[c];
        const float zp = static_cast<float>(zero_points[c]);
        int32_t row_sum = 0;
        for (int i = 0; i < in_features; ++i) {
            const int64_t off = static_cast<int64_t>(c) * in_features + i;
            float q = std::round(W[off] / s) + zp;
            if (q < -128.0f) q = -128.0f;
            if (q > 127.0f) q = 127.0f;
            // static_cast<int8_t>(float) narrows through cvttss2si (NaN -> 0).
            const int8_t q8 = static_cast<int8_t>(static_cast<uint8_t>(static_cast<uint32_t>(cvt_i32_x86(q))));
            W_q[off] = q8;
            row_sum += static_cast<int32_t>(q8) - zero_points[c];
        }
        if (sum_w) sum_w[c] = row_sum;
    }
    return NFLOW_OK;
}

int nflow_host_per_channel_scales(const float* W, int out_features, int in_features, float qmax,
                                  float* scales) {
    clear_error();
    if (!W || !scales) return set_error(NFLOW_INVALID_ARG, "per_channel_scales: null pointer");
    if (out_features <= 0 || in_features <= 0 || !(qmax > 0.0f))
        return set_error(NFLOW_INVALID_ARG, "per_channel_scales: bad dims or qmax");
    for (int c = 0; c < out_features; ++c) {
        const float m = row_absmax(W + static_cast<int64_t>(c) * in_features, in_features);
        scales[c] = (m == 0.0f) ? 1.0f : m / qmax;
    }
    return NFLOW_OK;
}

int nflow_host_fp8_quantise_weight(const float* W, int out_features, int in_features, uint8_t* W_q,
                                   float* scales) {
    clear_error();
    if (!W || !W_q || !scales) return set_error(NFLOW_INVALID_ARG, "fp8_quantise_weight: null pointer");
    if (out_features <= 0 || in_features <= 0)
        return set_error(NFLOW_INVALID_ARG, "fp8_quantise_weight: bad dims");
    for (int c = 0; c < out_features; ++c) {
        const float* w = W + static_cast<int64_t>(c) * in_features;
        const float m = row_absmax(w, in_features);
        const float s = (m == 0.0f) ? 1.0f : m / 448.0f;
        scales[c] = s;
        const float inv = (s == 0.0f) ? 1.0f : (1.0f / s);
        for (int i = 0; i < in_features; ++i) {
            const float xs = w[i] * inv;
            const float xc = (xs > 448.0f) ? 448.0f : ((xs < -448.0f) ? -448.0f : xs);
            W_q[static_cast<int64_t>(c) * in_features + i] = e4m3_encode_host(xc);
        }
    }
    return NFLOW_OK;
}

}  // extern "C"
