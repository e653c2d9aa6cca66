// common.h -- device helpers shared by the gfx950 kernels of libnflow_quant.
//
// Compiled with -ffp-contract=off: every float expression below rounds in
// the order written, which is what makes the dequantise step bit-exact with
// the reference's x86 build (int8_gemm.cpp:464-467, :573-576).  FMA is used
// only where written explicitly (__builtin_fmaf), never in a step that has to
// match the reference bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nfq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU_TANH = 2 };

// Which reference entry point's integer formula the epilogue reproduces.
//   BATCHED    int8_gemm.cpp:559-577 (LinearForwardBatched)
//   ROW_VNNI   int8_gemm.cpp:354-396, :461-467 (LinearForward, K <= 4096)
//   ROW_SCALAR int8_gemm.cpp:441-467 (LinearForward, K > 4096)
enum Formula { F_BATCHED = 0, F_ROW_VNNI = 1, F_ROW_SCALAR = 2 };

// ---------------------------------------------------------------------------
// INT8 activation code of one element, exactly as the reference's x86 build:
// correctly rounded a / s, half-away-from-zero rounding, cvttss2si semantics
// (NaN or |q| >= 2^31 -> INT32_MIN), wrapping + zp, clamp to [-128, 127].
// ---------------------------------------------------------------------------
__device__ __forceinline__ int32_t cvt_i32_x86(float r) {
    return (r >= -2147483648.0f && r < 2147483648.0f) ? static_cast<int32_t>(r)
                                                       : INT32_MIN;
}

__device__ __forceinline__ int32_t clamp_i8(int32_t q) {
    return q < -128 ? -128 : (q > 127 ? 127 : q);
}

__device__ __forceinline__ int32_t quant_i8_exact(float a, float s, int32_t zp) {
    const float r = roundf(a / s);
    const int32_t q = static_cast<int32_t>(static_cast<uint32_t>(cvt_i32_x86(r)) +
                                           static_cast<uint32_t>(zp));
    return clamp_i8(q);
}

// Per-token variant (zp = 0) with a reciprocal fast path.  t = a * inv_s
// (inv_s the correctly rounded 1/s, a normal number for every finite
// per-token scale) differs from the correctly rounded quotient q = fl(a / s)
// by at most 1.5 * 2^-23 |t|.  Rounding half away from zero and rounding
// half to even differ only at k + 0.5, so whenever the distance of |t| from
// the nearest half-integer, |fract(|t|) - 0.5|, exceeds |t| * 2^-20,
// rint(t) == round(q) (and |t| < 2^31, so the conversion is exact).
// quant_i8_fast returns false when that test fails -- about one element in
// 10^4, and every NaN / Inf / overflowing quotient -- and the caller then
// uses quant_i8_exact(a, s, 0) for that element.
__device__ __forceinline__ bool quant_i8_fast(float a, float inv_s, int32_t& q) {
    const float t = a * inv_s;
    const float at = fabsf(t);
    const float dist = fabsf(__builtin_amdgcn_fractf(at) - 0.5f);
    q = clamp_i8(static_cast<int32_t>(rintf(t)));
    return dist > __builtin_fmaf(at, 0x1p-20f, 0x1p-40f);
}

// Scalar form: per-token code of one element.
__device__ __forceinline__ int32_t quant_i8_token(float a, float s, float inv_s) {
    int32_t q;
    if (!quant_i8_fast(a, inv_s, q)) q = quant_i8_exact(a, s, 0);
    return q;
}

// Per-token INT8 code of t = a * inv_s for the fast path, and whether it may
// differ from the reference's.  With s = fl(amax / 127) normal, |a| <= amax
// and inv_s within 1 ulp of 1 / s (v_rcp_f32), t differs from q = fl(a / s)
// by at most 2^-22 |t|, and |t| < 127.5.  If the distance of t from
// r = rint(t) (exact: t and r are within a factor 2) is below
// 0.5 - 2^-21 |t|, q is closer than 0.5 to r, so round-half-away(q) == r and
// no clamp is needed.  NaN / Inf elements give a NaN distance and fail.
__device__ __forceinline__ int32_t quant_i8_near(float a, float inv_s, uint64_t& slow) {
    const float t = a * inv_s;
    const float r = rintf(t);
    const float lim = __builtin_fmaf(fabsf(t), -0x1p-21f, 0.5f);
    slow |= __builtin_amdgcn_ballot_w64(!(fabsf(t - r) < lim));
    return static_cast<int32_t>(r);
}

// Pack four int8 codes (low byte first) into one dword: two v_perm_b32
// select the low bytes (selector 0x0c zeroes a byte).
__device__ __forceinline__ uint32_t pack4(int32_t a, int32_t b, int32_t c, int32_t d) {
    const uint32_t lo = __builtin_amdgcn_perm(static_cast<uint32_t>(b), static_cast<uint32_t>(a),
                                              0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(static_cast<uint32_t>(d), static_cast<uint32_t>(c),
                                              0x04000c0cu);
    return lo | hi;
}

// DPP row moves (16-lane rows): the lane pattern CTRL of v within each row.
template <int CTRL>
__device__ __forceinline__ int dpp_movi(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, dpp_movi<CTRL>(__builtin_bit_cast(int, v)));
}

// Sum of the four signed bytes of a dword (v_dot4_i32_i8 against ones).
__device__ __forceinline__ int32_t sum_bytes_i8(uint32_t v, int32_t acc) {
    return __builtin_amdgcn_sdot4(static_cast<int>(v), 0x01010101, acc, false);
}

// ---------------------------------------------------------------------------
// FP8 E4M3 codec, bit-exact with fp8_e4m3.h:106-215 / :223-275 (including
// its choices: subnormal branch selected on the exponent before rounding and
// clamped to mantissa 7; (464, 496) -> NaN byte unless pre-clamped; any NaN
// -> 0x7F; +-Inf -> +-448).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t e4m3_encode(float v) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t mag = u & 0x7FFFFFFFu;
    if (mag > 0x7F800000u) return 0x7Fu;
    if (mag == 0x7F800000u) return sign | 0x7Eu;
    if (mag == 0u) return sign;
    const int32_t exp_pre = static_cast<int32_t>(mag >> 23) - 120;
    uint32_t man = (mag >> 20) & 0x7u;
    const uint32_t rest = mag & 0xFFFFFu;
    man += (rest > 0x80000u || (rest == 0x80000u && (man & 1u))) ? 1u : 0u;
    const int32_t exp = exp_pre + static_cast<int32_t>(man >> 3);
    man &= 0x7u;
    if (exp > 15) return sign | 0x7Eu;
    if (exp_pre < 1) {
        // |v| < 2^-6: |v| * 2^9 < 8 is exact in fp32; rint is round-half-even
        // like nearbyint in the default rounding mode.
        const float r = rintf(__uint_as_float(mag) * 512.0f);
        const uint32_t ri = static_cast<uint32_t>(r);
        return sign | (ri > 7u ? 7u : ri);
    }
    return sign | (static_cast<uint32_t>(exp) << 3) | man;
}

__device__ __forceinline__ float e4m3_decode(uint32_t b) {
    const uint32_t sign = (b & 0x80u) << 24;
    const uint32_t e = (b >> 3) & 0xFu;
    const uint32_t m = b & 0x7u;
    if (e == 0xFu && m == 0x7u) return __uint_as_float(sign | 0x7FC00000u);
    if (e == 0u) return __uint_as_float(sign | __float_as_uint(static_cast<float>(m) * 0x1p-9f));
    return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

// The fake-quant scale-down of fp8_e4m3.h:319-329: x * inv, clamp +-448, encode.
__device__ __forceinline__ uint32_t fp8_quant(float x, float inv) {
    const float xs = x * inv;
    const float xc = (xs > 448.0f) ? 448.0f : ((xs < -448.0f) ? -448.0f : xs);
    return e4m3_encode(xc);
}

// The value e4m3_decode(fp8_quant(x, inv)) computed without forming the byte
// (same result for every input; NaN stays NaN).  After the clamp |xc| <= 448:
//   |xc| >= 2^-6  round the fp32 mantissa to 3 bits, ties to even: adding
//                 0x7FFFF + lsb carries into bit 20 exactly when the 20-bit
//                 residue is above half, or equal to half with an odd lsb
//                 (the rule of fp8_e4m3.h:166-185, carry included);
//   |xc| <  2^-6  multiples of 2^-9 with ties to even, capped at 7 * 2^-9
//                 (fp8_e4m3.h:192-211): (|xc| + 2^14) - 2^14 rounds to the
//                 2^-9 grid because ulp(2^14) = 2^-9.
__device__ __forceinline__ float fp8_value_of(float xs) {
    const float xc = __builtin_amdgcn_fmed3f(xs, -448.0f, 448.0f);  // xs not NaN
    const uint32_t u = __float_as_uint(xc);
    const uint32_t nrm = (u + 0x7FFFFu + ((u >> 20) & 1u)) & 0xFFF00000u;
    const float sub = fminf((fabsf(xc) + 0x1p14f) - 0x1p14f, 7.0f * 0x1p-9f);
    const uint32_t subb = __float_as_uint(sub) | (u & 0x80000000u);
    return __uint_as_float(fabsf(xc) < 0x1p-6f ? subb : nrm);
}

__device__ __forceinline__ float fp8_value(float x, float inv) {
    const float xs = x * inv;
    const float v = fp8_value_of(xs);
    return __builtin_isnan(xs) ? xs : v;
}

// bfloat16 bits of two E4M3 values held as fp32, low half first (one v_perm).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}


// bfloat16 bits of the E4M3 byte b (the value of e4m3_decode, exactly).
__device__ __forceinline__ uint32_t e4m3_to_bf16(uint32_t b) {
    const uint32_t sign = (b & 0x80u) << 8;
    const uint32_t em = b & 0x7Fu;
    uint32_t r = (em < 8u) ? (__float_as_uint(static_cast<float>(em) * 0x1p-9f) >> 16)
                           : ((em << 4) + 0x3C00u);
    if (em == 0x7Fu) r = 0x7FC0u;
    return sign | r;
}

// ---------------------------------------------------------------------------
// Epilogue activation.  GELU uses the tanh form of fno.cpp:41-46,
//   0.5 z (1 + tanh(u)),  u = c (z + 0.044715 z^3),  c = sqrt(2/pi),
// evaluated through the identity 0.5 (1 + tanh u) = 1 / (1 + e^{-2u}):
//   gelu(z) = z / (1 + 2^(z (k1 + k3 z^2))),  k1 = -2 c log2(e), k3 = 0.044715 k1,
// with the hardware exp2 and reciprocal.  No cancellation occurs for z << 0
// (the tanh form computes 1 + tanh(u) ~ 0 there), and the relative error
// stays within a few ulp.  ReLU is `y < 0 ? 0 : y` as in fno.cpp:37-40.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gelu_tanh(float z) {
    const float k1 = -0x1.26aec2p+1f;  // -2 * sqrtf(2/pi) * log2(e)
    const float k3 = -0x1.a5a7cep-4f;  // 0.044715 * k1
    const float e = __builtin_amdgcn_exp2f(z * __builtin_fmaf(k3, z * z, k1));
    return z * __builtin_amdgcn_rcpf(1.0f + e);
}

template <int ACT>
__device__ __forceinline__ float activate(float y) {
    if constexpr (ACT == ACT_RELU) {
        return y < 0.0f ? 0.0f : y;
    } else if constexpr (ACT == ACT_GELU_TANH) {
        return gelu_tanh(y);
    } else {
        return y;
    }
}

__device__ __forceinline__ float activate_rt(float y, int act) {
    if (act == ACT_RELU) return y < 0.0f ? 0.0f : y;
    if (act == ACT_GELU_TANH) return gelu_tanh(y);
    return y;
}

// ---------------------------------------------------------------------------
// Integer epilogue: the reference formulas written as
//   t32 = D + c0 + c1 * SA   (mod 2^32),   t = int64(t32) + c2,
// with D the dot product of the raw codes (over the first Kd elements), SA the
// sum of a row's codes and per-channel constants:
//   BATCHED:    c0 = -zpA*SWp,                       c1 = -2 zpw, c2 = K zpw zpA
//   ROW_VNNI:   c0 = 128 Wd - 128 SWr - 2 zpA SWr + 3 K zpA zpw, (same c1, c2)
//   ROW_SCALAR: c0 = -2 zpA Sfull + 3 K zpw zpA,                (same c1, c2)
// where Sfull = sum of the weight row, Wd = its sum over the first Kd
// elements, SWp = sum_W_per_row[o] (0 if absent) and SWr = sum_W_per_row[o]
// (Sfull if absent).  Expanding int8_gemm.cpp:386-393 + :464-466 (VNNI),
// :444-456 + :464-466 (scalar) and :566-575 (batched) gives these forms.
// ---------------------------------------------------------------------------
struct IntEpi {
    int32_t c0;
    int32_t c1;
    int64_t c2;
};

__device__ __forceinline__ IntEpi int_epi_consts(int formula, int32_t K, int32_t zpA,
                                                 int32_t zpw, int32_t sum_w_given,
                                                 bool has_sum_w, int32_t Sfull, int32_t Wd) {
    IntEpi e;
    const uint32_t uK = static_cast<uint32_t>(K), uzpA = static_cast<uint32_t>(zpA),
                   uzpw = static_cast<uint32_t>(zpw);
    e.c1 = static_cast<int32_t>(0u - 2u * uzpw);
    e.c2 = static_cast<int64_t>(K) * zpw * zpA;
    if (formula == F_BATCHED) {
        const uint32_t swp = has_sum_w ? static_cast<uint32_t>(sum_w_given) : 0u;
        e.c0 = static_cast<int32_t>(0u - uzpA * swp);
    } else if (formula == F_ROW_VNNI) {
        const uint32_t swr = has_sum_w ? static_cast<uint32_t>(sum_w_given)
                                       : static_cast<uint32_t>(Sfull);
        e.c0 = static_cast<int32_t>(128u * static_cast<uint32_t>(Wd) - 128u * swr -
                                    2u * uzpA * swr + 3u * uK * uzpA * uzpw);
    } else {
        e.c0 = static_cast<int32_t>(0u - 2u * uzpA * static_cast<uint32_t>(Sfull) +
                                    3u * uK * uzpw * uzpA);
    }
    return e;
}

__device__ __forceinline__ float int_epi_value(const IntEpi& e, int32_t D, int32_t SA) {
    const uint32_t t32 = static_cast<uint32_t>(D) + static_cast<uint32_t>(e.c0) +
                         static_cast<uint32_t>(e.c1) * static_cast<uint32_t>(SA);
    if (e.c2 == 0) return static_cast<float>(static_cast<int32_t>(t32));
    return static_cast<float>(static_cast<int64_t>(static_cast<int32_t>(t32)) + e.c2);
}

// The FNO layer's INT8 fake-quant of x2 (fno.cpp:626-646 per-position,
// :637-646 per-tensor): q = std::round(v / s) + zp in float (true division,
// half away from zero), clamped to [-128, 127] (a NaN passes), then
// (q - zp) * s.
__device__ __forceinline__ float x2_fake_quant(float v, float s, float zpf) {
    float q = roundf(v / s) + zpf;
    q = q < -128.0f ? -128.0f : q;
    q = q > 127.0f ? 127.0f : q;
    return (q - zpf) * s;
}

// (scale_W[o] * scale_A) * float(t) + bias: the reference's operation order.
__device__ __forceinline__ float dequant_bias(float sw, float sa, float t, float b) {
    const float s = sw * sa;
    const float y = s * t;
    return y + b;
}

}  // namespace nfq
