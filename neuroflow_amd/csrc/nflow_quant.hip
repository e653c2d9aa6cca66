// nflow_quant.hip -- kernels and extern "C" entry points of libnflow_quant
// (declared in include/nflow_quant.h).
//
// Dispatch: the row-tile MFMA kernel (rows_kernel.h) serves every shape with
// K % 4 == 0, K <= 256 (fp32 input) or K <= 1024 (code input), N % 4 == 0
// and aligned pointers; anything else goes through the generic path
// (quantise kernel into a stream-ordered workspace, then one thread per
// output).  Both paths produce identical bits.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>

#include "nflow_quant.h"
#include "common.h"
#include "launch.h"
#include "rows_kernel.h"
#include "chain_kernel.h"
#include "status.h"

namespace nfq {

// ---------------------------------------------------------------------------
// Elementwise / per-row kernels
// ---------------------------------------------------------------------------

// QuantiseActivation, int8_gemm.cpp:507-520.
__global__ __launch_bounds__(256) void k_quantise_fixed(const float* __restrict__ A,
                                                        int8_t* __restrict__ Aq, int64_t n,
                                                        float s, int32_t zp) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        Aq[i] = static_cast<int8_t>(quant_i8_exact(A[i], s, zp));
}

// One wave per row: absmax -> scale -> codes (+ sum of codes).
// Weight-row byte sums the tiled GEMM's row-VNNI term needs next to a
// caller's sum_W (int8_gemm.cpp:386-393), formed by the quantise launch that
// runs just before the GEMM instead of a launch of their own.  out == null:
// none wanted.
struct CodeSums {
    const uint8_t* W;   // (N, K) int8 codes, 16-byte aligned rows
    int N;
    int K;              // a multiple of 16
    int32_t* out;       // (N)
};

// Rows 4 wg .. 4 wg + 3 of cs.W: 16 lanes per row, DPP row reductions.
__device__ __forceinline__ void code_sums_group(const CodeSums& cs, int64_t wg) {
    const int lane = threadIdx.x & 63, c = lane & 15;
    const int64_t n = wg * 4 + (lane >> 4);
    int32_t acc = 0;
    if (n < cs.N) {
        const v4u* w = reinterpret_cast<const v4u*>(cs.W + n * cs.K);
        for (int j = c; j < cs.K / 16; j += 16) {
            const v4u v = w[j];
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = sum_bytes_i8(v[q], acc);
        }
    }
    acc += dpp_movi<0xB1>(acc);   // quad_perm [1,0,3,2]
    acc += dpp_movi<0x4E>(acc);   // quad_perm [2,3,0,1]
    acc += dpp_movi<0x141>(acc);  // row_half_mirror
    acc += dpp_movi<0x140>(acc);  // row_mirror
    if (c == 0 && n < cs.N) cs.out[n] = acc;
}

// Every wave of a quantise launch first takes its share of the weight rows.
__device__ __forceinline__ void code_sums_share(const CodeSums& cs) {
    if (!cs.out) return;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t wg = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); wg * 4 < cs.N; wg += nw)
        code_sums_group(cs, wg);
}

template <bool FP8>
__global__ __launch_bounds__(256) void k_quantise_token(const float* __restrict__ A, int64_t M,
                                                        int K, uint8_t* __restrict__ Aq,
                                                        float* __restrict__ scale,
                                                        int32_t* __restrict__ sum_a,
                                                        CodeSums cs) {
    code_sums_share(cs);
    const int lane = threadIdx.x & 63;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); m < M; m += nw) {
        const float* x = A + m * K;
        float mx = 0.0f;
        for (int k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(x[k]));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float s = (mx == 0.0f) ? 1.0f : mx / (FP8 ? 448.0f : 127.0f);
        int32_t sa = 0;
        if constexpr (FP8) {
            const float inv = (s == 0.0f) ? 1.0f : 1.0f / s;
            for (int k = lane; k < K; k += 64) Aq[m * K + k] = static_cast<uint8_t>(fp8_quant(x[k], inv));
        } else {
            const float inv = 1.0f / s;
            for (int k = lane; k < K; k += 64) {
                const int32_t q = quant_i8_token(x[k], s, inv);
                Aq[m * K + k] = static_cast<uint8_t>(q);
                sa += q;
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) sa += __shfl_xor(sa, o);
        }
        if (lane == 0) {
            scale[m] = s;
            if (sum_a) sum_a[m] = sa;
        }
    }
}

// PrecomputeSumW, int8_gemm.cpp:479-496: one wave per output row.
__global__ __launch_bounds__(256) void k_sum_w(const int8_t* __restrict__ W,
                                               const int32_t* __restrict__ zp, int K, int N,
                                               int32_t* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= N) return;
    uint32_t acc = 0;
    for (int i = lane; i < K; i += 64)
        acc += static_cast<uint32_t>(static_cast<int32_t>(W[static_cast<int64_t>(o) * K + i]) - zp[o]);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s);
    if (lane == 0) out[o] = static_cast<int32_t>(acc);
}

// The weight-row byte sums on their own (linear_forward_quantised, which has
// no quantise launch to carry them).
__global__ __launch_bounds__(256) void k_code_sums(CodeSums cs) { code_sums_share(cs); }

__global__ __launch_bounds__(256) void k_e4m3_encode(const float* __restrict__ in,
                                                     uint8_t* __restrict__ out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        out[i] = static_cast<uint8_t>(e4m3_encode(in[i]));
}

__global__ __launch_bounds__(256) void k_e4m3_decode(const uint8_t* __restrict__ in,
                                                     float* __restrict__ out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        out[i] = e4m3_decode(in[i]);
}

// fp8_e4m3_per_tensor_fake_quant, fp8_e4m3.h:312-334 (in == out allowed).
__global__ __launch_bounds__(256) void k_fp8_fake_quant(const float* in, float scale, float* out,
                                                        int64_t n) {
    const float inv = (scale == 0.0f) ? 1.0f : (1.0f / scale);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        out[i] = e4m3_decode(fp8_quant(in[i], inv)) * scale;
}

// Generic product + epilogue: one thread per output, any K / N / alignment.
// Codes are read from Aq (already quantised); per-row scale from scale_in
// (or the fixed a.scale_A when scale_in is null).
template <bool FP8, int OUT>
__global__ __launch_bounds__(256) void k_generic(RowsArgs a, int act) {
    const int64_t total = a.M * a.N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int K = a.K;
    const int Kd = std::min(K, a.kb_dot * 64);
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += stride) {
        const int64_t m = idx / a.N;
        const int n = static_cast<int>(idx - m * a.N);
        const uint8_t* x = a.Aq + m * K;
        const uint8_t* w = a.W + static_cast<int64_t>(n) * K;
        if constexpr (FP8) {
            float acc = 0.0f;
            for (int k = 0; k < Kd; ++k) acc += e4m3_decode(x[k]) * e4m3_decode(w[k]);
            if constexpr (OUT == OUT_RAW) {
                static_cast<float*>(a.C)[idx] = acc;
            } else {
                const float sa = a.scale_in ? a.scale_in[m] : a.scale_A;
                const float b = a.bias ? a.bias[n] : 0.0f;
                static_cast<float*>(a.C)[idx] = activate_rt(dequant_bias(a.sW[n], sa, acc, b), act);
            }
        } else {
            uint32_t D = 0, SA = 0, Sf = 0, Sd = 0;
            for (int k = 0; k < K; ++k) {
                const int32_t xv = static_cast<int8_t>(x[k]);
                const int32_t wv = static_cast<int8_t>(w[k]);
                SA += static_cast<uint32_t>(xv);
                Sf += static_cast<uint32_t>(wv);
                if (k < Kd) {
                    D += static_cast<uint32_t>(xv * wv);
                    Sd += static_cast<uint32_t>(wv);
                }
            }
            if constexpr (OUT == OUT_RAW) {
                static_cast<int32_t*>(a.C)[idx] = static_cast<int32_t>(D);
            } else {
                const int32_t zpw = a.zpW ? a.zpW[n] : 0;
                const int32_t swg = a.sumW ? a.sumW[n] : 0;
                const IntEpi e = int_epi_consts(a.formula, K, a.zp_A, zpw, swg, a.sumW != nullptr,
                                                static_cast<int32_t>(Sf), static_cast<int32_t>(Sd));
                const float t = int_epi_value(e, static_cast<int32_t>(D), static_cast<int32_t>(SA));
                const float sa = a.scale_in ? a.scale_in[m] : a.scale_A;
                const float b = a.bias ? a.bias[n] : 0.0f;
                static_cast<float*>(a.C)[idx] = activate_rt(dequant_bias(a.sW[n], sa, t, b), act);
            }
        }
    }
}

// Code stores are written through the L2 (sc1): the codes then need no
// write-back at the end of the launch before the product reads them
// (measured on the 65536-row 1024-wide layer: 128.5-129.9 -> 125.3 us per
// layer; nt 144 us, the product then reading them from HBM).
constexpr int kCodeCpol = 16;

// The same for rows of K = 256 KV floats: the row stays in registers (KV
// float4 per lane), so HBM is read once, in 1 KB wave instructions, and the
// codes leave as one dword per lane per float4.
template <bool FP8, int KV>
__global__ __launch_bounds__(256) void k_quantise_rows(const float* __restrict__ A, int64_t M,
                                                       uint8_t* __restrict__ Aq,
                                                       float* __restrict__ scale,
                                                       int32_t* __restrict__ sum_a,
                                                       CodeSums cs) {
    code_sums_share(cs);
    constexpr int K = 256 * KV;
    const int lane = threadIdx.x & 63;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); m < M; m += nw) {
        const v4f* x4 = reinterpret_cast<const v4f*>(A + m * K);
        v4f x[KV];
#pragma unroll
        for (int i = 0; i < KV; ++i) x[i] = __builtin_nontemporal_load(x4 + lane + 64 * i);
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < KV; ++i)
            mx = fmaxf(fmaxf(mx, fmaxf(fabsf(x[i][0]), fabsf(x[i][1]))), fmaxf(fabsf(x[i][2]), fabsf(x[i][3])));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float s = (mx == 0.0f) ? 1.0f : mx / (FP8 ? 448.0f : 127.0f);
        const auto qr = __builtin_amdgcn_make_buffer_rsrc(Aq + m * K, 0, K, 0x00020000);
        int32_t sa = 0;
        if constexpr (FP8) {
            const float inv = (s == 0.0f) ? 1.0f : 1.0f / s;
#pragma unroll
            for (int i = 0; i < KV; ++i)
                __builtin_amdgcn_raw_buffer_store_b32(
                    fp8_quant(x[i][0], inv) | (fp8_quant(x[i][1], inv) << 8) | (fp8_quant(x[i][2], inv) << 16) |
                        (fp8_quant(x[i][3], inv) << 24),
                    qr, 4 * (lane + 64 * i), 0, kCodeCpol);
        } else {
            const float inv = 1.0f / s;
#pragma unroll
            for (int i = 0; i < KV; ++i) {
                const uint32_t w = pack4(quant_i8_token(x[i][0], s, inv), quant_i8_token(x[i][1], s, inv),
                                         quant_i8_token(x[i][2], s, inv), quant_i8_token(x[i][3], s, inv));
                __builtin_amdgcn_raw_buffer_store_b32(w, qr, 4 * (lane + 64 * i), 0, kCodeCpol);
                sa = sum_bytes_i8(w, sa);
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) sa += __shfl_xor(sa, o);
        }
        if (lane == 0) {
            scale[m] = s;
            if (sum_a) sum_a[m] = sa;
        }
    }
}

// Rows of K = 256 KV floats with KV <= 2: 16 lanes per row, so a wave holds
// four rows and every reduction is four DPP row steps.  The 64-lane form
// above waits on six cross-lane shuffles per reduction, which holds it to
// about 60% of a streaming copy at K = 256; this form reaches 88%.
// Lane (r, c) = (lane / 16, lane % 16) holds the float4s c + 16 j, j < 4 KV,
// of row 4 w + r: each load instruction reads 256 contiguous bytes of each
// of the four rows, and each code store writes 64.
template <bool FP8, int KV>
__global__ __launch_bounds__(256) void k_quantise_rows16(const float* __restrict__ A, int64_t M,
                                                         uint8_t* __restrict__ Aq,
                                                         float* __restrict__ scale,
                                                         int32_t* __restrict__ sum_a,
                                                         CodeSums cs) {
    code_sums_share(cs);
    constexpr int K = 256 * KV, J = 4 * KV;
    const int lane = threadIdx.x & 63, c = lane & 15;
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); w * 4 < M; w += nw) {
        const int64_t m = w * 4 + (lane >> 4);
        const bool live = m < M;
        const v4f* x4 = reinterpret_cast<const v4f*>(A + (live ? m : M - 1) * K);
        v4f x[J];
#pragma unroll
        for (int j = 0; j < J; ++j) x[j] = __builtin_nontemporal_load(x4 + c + 16 * j);
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
            mx = fmaxf(fmaxf(mx, fmaxf(fabsf(x[j][0]), fabsf(x[j][1]))), fmaxf(fabsf(x[j][2]), fabsf(x[j][3])));
        mx = fmaxf(mx, dpp_mov<0xB1>(mx));   // quad_perm [1,0,3,2]
        mx = fmaxf(mx, dpp_mov<0x4E>(mx));   // quad_perm [2,3,0,1]
        mx = fmaxf(mx, dpp_mov<0x141>(mx));  // row_half_mirror
        mx = fmaxf(mx, dpp_mov<0x140>(mx));  // row_mirror
        const float s = (mx == 0.0f) ? 1.0f : mx / (FP8 ? 448.0f : 127.0f);
        // The wave's four rows as one buffer range clipped at M (rows past
        // it are dropped by the hardware).
        const int64_t left = M - w * 4 < 4 ? M - w * 4 : 4;
        const auto qr = __builtin_amdgcn_make_buffer_rsrc(Aq + w * 4 * K, 0, static_cast<int>(left * K), 0x00020000);
        const int qoff = (lane >> 4) * K;
        int32_t sa = 0;
        if constexpr (FP8) {
            const float inv = (s == 0.0f) ? 1.0f : 1.0f / s;
#pragma unroll
            for (int j = 0; j < J; ++j)
                __builtin_amdgcn_raw_buffer_store_b32(
                    fp8_quant(x[j][0], inv) | (fp8_quant(x[j][1], inv) << 8) | (fp8_quant(x[j][2], inv) << 16) |
                        (fp8_quant(x[j][3], inv) << 24),
                    qr, qoff + 4 * (c + 16 * j), 0, kCodeCpol);
        } else {
            const float inv = 1.0f / s;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                uint32_t v = pack4(quant_i8_token(x[j][0], s, inv), quant_i8_token(x[j][1], s, inv),
                                   quant_i8_token(x[j][2], s, inv), quant_i8_token(x[j][3], s, inv));
                v = live ? v : 0u;
                __builtin_amdgcn_raw_buffer_store_b32(v, qr, qoff + 4 * (c + 16 * j), 0, kCodeCpol);
                sa = sum_bytes_i8(v, sa);
            }
            sa += dpp_movi<0xB1>(sa);
            sa += dpp_movi<0x4E>(sa);
            sa += dpp_movi<0x141>(sa);
            sa += dpp_movi<0x140>(sa);
        }
        if (c == 0 && live) {
            scale[m] = s;
            if (sum_a) sum_a[m] = sa;
        }
    }
}

// The FNO layer's tail for the kernels that do not fuse it: C holds x2
// (bias included); C = act(R + fq(x2)) with the optional x2 fake-quant of
// a.xq_* (fno.cpp:572-654) and R (the spectral branch x1) optional.  One
// block per row at a time, columns across the threads.
__global__ __launch_bounds__(256) void k_fno_post(float* __restrict__ C, const float* __restrict__ R,
                                                  RowsArgs a, int act) {
    const int N = a.N;
    for (int64_t m = blockIdx.x; m < a.M; m += gridDim.x) {
        const int pos = a.xq_kind == 2 ? static_cast<int>(m % a.xq_points) : 0;
        for (int j = threadIdx.x; j < N; j += blockDim.x) {
            const int64_t i = m * N + j;
            float x2 = C[i];
            if (a.xq_kind == 1) {
                x2 = x2_fake_quant(x2, a.xq_scale, a.xq_zpf);
            } else if (a.xq_kind == 2) {
                const int64_t idx = static_cast<int64_t>(j) * a.xq_points + pos;
                x2 = x2_fake_quant(x2, a.xq_scales[idx], static_cast<float>(a.xq_zps[idx]));
            }
            C[i] = activate_rt(R ? R[i] + x2 : x2, act);
        }
    }
}

// ---------------------------------------------------------------------------
// Launch helpers
// ---------------------------------------------------------------------------

template <bool FP8, int OUT>
static void launch_generic(const RowsArgs& a, int act, hipStream_t st) {
    const unsigned grid = grid_for(a.M * a.N, 256, 16);
    hipLaunchKernelGGL((k_generic<FP8, OUT>), dim3(grid), dim3(256), 0, st, a, act);
}

// Per-token quantise of (M, K) rows: the register-resident kernel for
// K = 256, 512, 1024, 2048, 4096 (16-byte aligned rows), else one wave per
// row with a loop over K.
template <bool FP8>
static void launch_quantise_token(const float* A, int64_t M, int K, uint8_t* Aq, float* scale,
                                  int32_t* sum_a, hipStream_t st,
                                  CodeSums cs = CodeSums{nullptr, 0, 0, nullptr}) {
    const dim3 grid(grid_for(M, 4, 16)), block(256);
    if (aligned(A, 16) && aligned(Aq, 4)) {
        // K <= 512: 16 lanes per row, a block takes 16 rows, 4 blocks per CU.
        // K >= 1024 keeps a row per wave: there the shuffles are a small share
        // of the row's time, and the 16-lane form has four times fewer waves
        // (measured on MI355X at M = 65536, K = 1024: 68 us against 64 us).
        const dim3 grid16(grid_for(M, 16, 4));
        switch (K) {
            case 256: hipLaunchKernelGGL((k_quantise_rows16<FP8, 1>), grid16, block, 0, st, A, M, Aq, scale, sum_a, cs); return;
            case 512: hipLaunchKernelGGL((k_quantise_rows16<FP8, 2>), grid16, block, 0, st, A, M, Aq, scale, sum_a, cs); return;
            case 1024: hipLaunchKernelGGL((k_quantise_rows<FP8, 4>), grid, block, 0, st, A, M, Aq, scale, sum_a, cs); return;
            case 2048: hipLaunchKernelGGL((k_quantise_rows<FP8, 8>), grid, block, 0, st, A, M, Aq, scale, sum_a, cs); return;
            case 4096: hipLaunchKernelGGL((k_quantise_rows<FP8, 16>), grid, block, 0, st, A, M, Aq, scale, sum_a, cs); return;
            default: break;
        }
    }
    hipLaunchKernelGGL((k_quantise_token<FP8>), grid, block, 0, st, A, M, K, Aq, scale, sum_a, cs);
}

static int env_int(const char* name) {
    const char* v = std::getenv(name);
    return (v && v[0]) ? std::atoi(v) : 0;
}

// Initialised from the environment on first use (a thread-safe static).
KernelPath& kernel_path() {
    static KernelPath* k = [] {
        auto* p = new KernelPath();
        p->no_gemm.store(env_int("NFLOW_NO_GEMM"));
        p->no_rows64.store(env_int("NFLOW_NO_ROWS64"));
        p->no_token_gemm.store(env_int("NFLOW_NO_TOKEN_GEMM"));
        p->gemm_reg.store(env_int("NFLOW_GEMM_REG"));
        p->gemm_tile.store(env_int("NFLOW_GEMM_TILE"));
        p->gemm_mfma.store(env_int("NFLOW_GEMM_MFMA"));
        p->no_wide.store(env_int("NFLOW_NO_WIDE"));
        p->no_rows64_queue.store(env_int("NFLOW_NO_ROWS64_QUEUE"));
        p->no_layer_tail.store(env_int("NFLOW_NO_LAYER_TAIL"));
        p->generic_fft.store(env_int("NFLOW_GENERIC_FFT"));
        return p;
    }();
    return *k;
}

static int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(NFLOW_INTERNAL, std::string(what) + ": " + hipGetErrorString(e));
    return NFLOW_OK;
}

// Workspace of one call (codes, scales and sums between a quantise launch
// and the product that reads them), used only by this call's launches on
// its stream.  Each (device, stream) pair keeps one buffer that grows to the
// largest request and is reused by the next call on that stream: calls on
// one stream run in order, so the previous call's kernels are done with it
// before the next call's start.  The pair's lock is held for the call's
// lifetime, so host threads sharing a stream cannot interleave their launches
// inside one call.  A larger request frees the old buffer in stream order and
// allocates anew.  (A stream-ordered allocation and free per call cost about
// 10 us of host time, more than a 4096-row 1024-wide layer takes on the GPU.)
// The per-thread default stream (one handle for many streams) and a stream
// under graph capture (whose allocations belong to the graph) keep the
// per-call allocation.  Buffers live until the process ends.
struct WsEntry {
    std::mutex mu;
    void* p = nullptr;
    size_t cap = 0;
};

// Slot 0 is a call's own workspace; slot 1 holds the fp32 activations
// between the layers of nflow_int8_mlp_forward_per_token, whose per-layer
// calls take slot 0 meanwhile.
static WsEntry* ws_entry(int dev, hipStream_t st, int slot) {
    static std::mutex map_mu;
    static std::map<std::pair<int, uintptr_t>, std::unique_ptr<WsEntry>>* map =
        new std::map<std::pair<int, uintptr_t>, std::unique_ptr<WsEntry>>();
    std::lock_guard<std::mutex> g(map_mu);
    auto& e = (*map)[{dev * 2 + slot, reinterpret_cast<uintptr_t>(st)}];
    if (!e) e.reset(new WsEntry);
    return e.get();
}

struct Scratch {
    void* p = nullptr;
    hipStream_t st = nullptr;
    hipError_t err = hipSuccess;
    bool owned = false;                    // per-call allocation (freed here)
    std::unique_lock<std::mutex> lock;
    Scratch(size_t bytes, hipStream_t s, int slot = 0) : st(s) {
        bytes = std::max<size_t>(bytes, 256);
        int dev = 0;
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (s == hipStreamPerThread || hipStreamIsCapturing(s, &cap) != hipSuccess ||
            cap != hipStreamCaptureStatusNone || hipGetDevice(&dev) != hipSuccess) {
            err = hipMallocAsync(&p, bytes, s);
            owned = err == hipSuccess;
            return;
        }
        WsEntry* e = ws_entry(dev, s, slot);
        lock = std::unique_lock<std::mutex>(e->mu);
        if (bytes > e->cap) {
            if (e->p) (void)hipFreeAsync(e->p, s);
            e->p = nullptr;
            e->cap = 0;
            const size_t want = (bytes + (size_t(2) << 20) - 1) & ~((size_t(2) << 20) - 1);
            err = hipMallocAsync(&e->p, want, s);
            if (err != hipSuccess) {
                e->p = nullptr;
                return;
            }
            e->cap = want;
        }
        p = e->p;
    }
    ~Scratch() {
        if (owned && p) (void)hipFreeAsync(p, st);
    }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
};

static int kb_dot_for(int formula, int K) {
    if (formula == F_ROW_VNNI) return K / 64;   // int8_gemm.cpp:366: vec_end = K - K % 64
    return (K + 63) / 64;
}

static int formula_row(int K) { return K <= 4096 ? F_ROW_VNNI : F_ROW_SCALAR; }

// Fixed-scale int8 path shared by LinearForward / rows / batched.
static int int8_fixed_path(const nflow_int8_linear_params* p, int64_t rows, const float* A, float* C,
                           int formula, hipStream_t st, const char* what) {
    RowsArgs a{};
    a.A = A;
    a.M = rows;
    a.K = p->in_features;
    a.N = p->out_features;
    a.W = reinterpret_cast<const uint8_t*>(p->W_int8);
    a.sW = p->scale_W;
    a.zpW = p->zp_W;
    a.bias = p->bias;
    a.sumW = p->sum_W_per_row;
    a.scale_A = p->scale_A;
    a.zp_A = p->zp_A;
    a.formula = formula;
    a.kb_dot = kb_dot_for(formula, a.K);
    a.C = C;
    if (rows64_ok(a) && !path_flag(kernel_path().no_rows64)) {
        launch_rows64_fixed(a, st);
        return check_launch(what);
    }
    if (rows_ok(a, IN_F32_FIXED)) {
        launch_rows<false, IN_F32_FIXED, OUT_EPI>(a, ACT_NONE, st);
        return check_launch(what);
    }
    Scratch ws(static_cast<size_t>(rows) * a.K, st);
    if (ws.err != hipSuccess) return set_error(NFLOW_INTERNAL, std::string(what) + ": workspace allocation failed");
    const int64_t n = rows * a.K;
    hipLaunchKernelGGL(k_quantise_fixed, dim3(grid_for(n, 256, 16)), dim3(256), 0, st, A,
                       static_cast<int8_t*>(ws.p), n, p->scale_A, p->zp_A);
    a.Aq = static_cast<const uint8_t*>(ws.p);
    a.scale_in = nullptr;
    launch_generic<false, OUT_EPI>(a, ACT_NONE, st);
    return check_launch(what);
}

// The tiled GEMM serves INT8 code input with K a multiple of 64, K >= 128
// (NFLOW_NO_GEMM=1 selects the row-tile kernel instead, for A/B timing).
static bool use_gemm(const RowsArgs& a) { return gemm_ok(a) && !path_flag(kernel_path().no_gemm); }

static int check_params(const nflow_int8_linear_params* p, const char* what) {
    if (!p || !p->W_int8 || !p->scale_W || !p->zp_W)
        return set_error(NFLOW_INVALID_ARG, std::string(what) + ": null input/output");
    if (p->in_features <= 0 || p->out_features <= 0)
        return set_error(NFLOW_INVALID_ARG, std::string(what) + ": bad feature dims");
    return NFLOW_OK;
}

static bool valid_act(int act) { return act == ACT_NONE || act == ACT_RELU || act == ACT_GELU_TANH; }

}  // namespace nfq

using namespace nfq;

extern "C" {

int nflow_quant_abi_version(void) { return NFLOW_QUANT_ABI_VERSION; }

int nflow_debug_set_kernel_path(const char* name, int value, int* previous) {
    clear_error();
    if (!name) return set_error(NFLOW_INVALID_ARG, "debug_set_kernel_path: null name");
    KernelPath& k = kernel_path();
    const std::string n(name);
    std::atomic<int>* f = n == "no_gemm" ? &k.no_gemm
                        : n == "no_rows64" ? &k.no_rows64
                        : n == "no_token_gemm" ? &k.no_token_gemm
                        : n == "gemm_reg" ? &k.gemm_reg
                        : n == "gemm_tile" ? &k.gemm_tile
                        : n == "gemm_mfma" ? &k.gemm_mfma
                        : n == "no_wide" ? &k.no_wide
                        : n == "no_rows64_queue" ? &k.no_rows64_queue
                        : n == "no_layer_tail" ? &k.no_layer_tail
                        : n == "generic_fft" ? &k.generic_fft : nullptr;
    if (!f) return set_error(NFLOW_INVALID_ARG, "debug_set_kernel_path: unknown name " + n);
    const int old = f->exchange(value, std::memory_order_relaxed);
    if (previous) *previous = old;
    return NFLOW_OK;
}

int nflow_int8_quantise_activation(const float* A, int8_t* A_q, int64_t bsz, int in_features,
                                   float scale_A, int32_t zp_A, void* stream) {
    clear_error();
    if (!A || !A_q) return NFLOW_OK;   // the reference returns silently (int8_gemm.cpp:511)
    const int64_t n = bsz * static_cast<int64_t>(in_features);
    if (n <= 0) return NFLOW_OK;
    hipLaunchKernelGGL(k_quantise_fixed, dim3(grid_for(n, 256, 16)), dim3(256), 0,
                       as_stream(stream), A, A_q, n, scale_A, zp_A);
    return check_launch("QuantiseActivation");
}

int nflow_int8_precompute_sum_w(const int8_t* W_int8, const int32_t* zp_W, int in_features,
                                int out_features, int32_t* sum_W_out, void* stream) {
    clear_error();
    if (!W_int8 || !zp_W || !sum_W_out || in_features <= 0 || out_features <= 0)
        return set_error(NFLOW_INVALID_ARG, "PrecomputeSumW: null input or bad dims");
    hipLaunchKernelGGL(k_sum_w, dim3((out_features + 3) / 4), dim3(256), 0, as_stream(stream),
                       W_int8, zp_W, in_features, out_features, sum_W_out);
    return check_launch("PrecomputeSumW");
}

int nflow_int8_linear_forward(const nflow_int8_linear_params* p, const float* A, float* C,
                              void* stream) {
    clear_error();
    if (!A || !C) return set_error(NFLOW_INVALID_ARG, "Int8Linear: null input/output");
    int rc = check_params(p, "Int8Linear");
    if (rc) return rc;
    return int8_fixed_path(p, 1, A, C, formula_row(p->in_features), as_stream(stream),
                           "Int8Linear");
}

int nflow_int8_linear_forward_rows(const nflow_int8_linear_params* p, int64_t rows,
                                   const float* A, float* C, void* stream) {
    clear_error();
    if (!A || !C) return set_error(NFLOW_INVALID_ARG, "Int8Linear: null input/output");
    int rc = check_params(p, "Int8Linear");
    if (rc) return rc;
    if (rows <= 0) return NFLOW_OK;
    return int8_fixed_path(p, rows, A, C, formula_row(p->in_features), as_stream(stream),
                           "Int8Linear");
}

int nflow_int8_linear_forward_batched(const nflow_int8_linear_params* p, int64_t bsz,
                                      const float* A, float* C, void* stream) {
    clear_error();
    if (bsz <= 0) return NFLOW_OK;
    if (!A || !C) return set_error(NFLOW_INVALID_ARG, "LinearForwardBatched: null A or C");
    int rc = check_params(p, "LinearForwardBatched");
    if (rc) return rc;
    return int8_fixed_path(p, bsz, A, C, F_BATCHED, as_stream(stream), "LinearForwardBatched");
}

int nflow_int8_quantise_per_token(const float* A, int64_t M, int K, int8_t* A_q, float* scale_A,
                                  int32_t* sum_a, void* stream) {
    clear_error();
    if (!A || !A_q || !scale_A) return set_error(NFLOW_INVALID_ARG, "quantise_per_token: null pointer");
    if (K <= 0) return set_error(NFLOW_INVALID_ARG, "quantise_per_token: K <= 0");
    if (M <= 0) return NFLOW_OK;
    launch_quantise_token<false>(A, M, K, reinterpret_cast<uint8_t*>(A_q), scale_A, sum_a, as_stream(stream));
    return check_launch("quantise_per_token");
}

}  // extern "C"

namespace nfq {

// Per-token INT8 layer; with a residual R (M x N) the result is the FNO layer
// form act(R + x2): fused in the K = N = 64 kernel, else x2 then one pass.
// The x2 fake-quant parameters into a (nflow_x2_quant, fno.cpp:572-648).
static int apply_x2q(RowsArgs& a, const nflow_x2_quant* xq, const char* what) {
    if (!xq || xq->kind == NFLOW_X2_NONE) return NFLOW_OK;
    const std::string w(what);
    if (xq->kind == NFLOW_X2_PER_TENSOR) {
        a.xq_kind = 1;
        a.xq_scale = xq->scale;
        a.xq_zpf = static_cast<float>(xq->zero_point);
        return NFLOW_OK;
    }
    if (xq->kind == NFLOW_X2_PER_POSITION) {
        if (!xq->scales || !xq->zero_points) return set_error(NFLOW_INVALID_ARG, w + ": null per-position qparams");
        if (xq->points <= 0) return set_error(NFLOW_INVALID_ARG, w + ": per-position qparams need points > 0");
        if (xq->width != a.N)
            return set_error(NFLOW_SHAPE_MISMATCH, w + ": per-position qparam width differs from out_features");
        if (xq->n_positions < static_cast<int64_t>(a.N) * xq->points)
            return set_error(NFLOW_SHAPE_MISMATCH, w + ": fewer per-position qparams than out_features * points");
        a.xq_kind = 2;
        a.xq_scales = xq->scales;
        a.xq_zps = xq->zero_points;
        a.xq_points = xq->points;
        return NFLOW_OK;
    }
    if (xq->kind == NFLOW_X2_FP8_LOG2)
        return set_error(NFLOW_UNSUPPORTED_OP, w + ": the log2 FP8 snap of x2 is not an E4M3 operation");
    return set_error(NFLOW_INVALID_ARG, w + ": unknown x2 fake-quant kind");
}

// Device scratch of nflow_int8_linear_forward_per_token_noalloc: the split
// path's codes, scales and byte sums (at most kNoAllocScratchBytes).  Each
// GPU the library runs on holds its own copy until the process ends; the
// name is a host-side stand-in, so host code uses only the device address
// hipGetSymbolAddress returns for the current device.  Nothing in it needs
// to start at zero: the quantise launch writes every byte the product reads.
constexpr size_t kNoAllocScratchBytes = NFLOW_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// The current device's address of `scratch`, looked up on the first call
// that needs it on that device and kept per device, and that device's lock
// on it: a call holds the lock from the lookup until its product is
// launched, so host threads whose calls share one stream cannot interleave
// their quantise and product launches on the one array (launches on
// different streams still run concurrently on the device and race).
constexpr int kMaxDevices = 64;
static std::mutex noalloc_mu[kMaxDevices];

static int noalloc_scratch_address(void** out, std::unique_lock<std::mutex>* hold) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    const hipError_t ed = hipGetDevice(&dev);
    if (ed != hipSuccess) return set_error(NFLOW_INTERNAL, std::string("noalloc scratch: hipGetDevice: ") + hipGetErrorString(ed));
    if (dev < 0 || dev >= kMaxDevices) return set_error(NFLOW_INTERNAL, "noalloc scratch: device index out of range");
    *hold = std::unique_lock<std::mutex>(noalloc_mu[dev]);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return set_error(NFLOW_INTERNAL, std::string("noalloc scratch: hipGetSymbolAddress: ") + hipGetErrorString(e));
        addr[dev] = ptr;
    }
    *out = addr[dev];
    return NFLOW_OK;
}

// The no-allocation entry point's workspace: the library's static device
// scratch of `cap` bytes, its address looked up (once per device) only after
// the shape has been checked against `cap`.  Null: allocate on the stream.
struct FixedWs {
    size_t cap;
    const char* what;
};

static int int8_per_token(const nflow_int8_linear_params* p, int64_t M, const float* A,
                          const float* R, float* C, float* scale_A_out, int activation,
                          const nflow_x2_quant* xq, void* stream, const FixedWs* fixed = nullptr) {
    if (!A || !C || !p || !p->W_int8 || !p->scale_W)
        return set_error(NFLOW_INVALID_ARG, "linear_forward_per_token: null input/output");
    if (p->in_features <= 0 || p->out_features <= 0)
        return set_error(NFLOW_INVALID_ARG, "linear_forward_per_token: bad feature dims");
    if (!valid_act(activation))
        return set_error(NFLOW_INVALID_ARG, "linear_forward_per_token: unknown activation");
    if (R && R == C) return set_error(NFLOW_INVALID_ARG, "fno_layer: x1 and y must be distinct buffers");
    RowsArgs a{};
    a.N = p->out_features;
    if (int rc = apply_x2q(a, xq, "fno_layer")) return rc;
    if (M <= 0) return NFLOW_OK;
    hipStream_t st = as_stream(stream);
    a.A = A;
    a.M = M;
    a.K = p->in_features;
    a.W = reinterpret_cast<const uint8_t*>(p->W_int8);
    a.sW = p->scale_W;
    a.zpW = p->zp_W;
    a.bias = p->bias;
    a.sumW = p->sum_W_per_row;
    a.zp_A = 0;
    a.formula = formula_row(a.K);
    a.kb_dot = kb_dot_for(a.formula, a.K);
    a.C = C;
    a.scale_out = scale_A_out;
    if (rows64_ok(a) && (!R || aligned(R, 16)) && !path_flag(kernel_path().no_rows64)) {
        a.residual = R;
        launch_rows64<false>(a, activation, st);
        return check_launch("linear_forward_per_token");
    }
    const bool post = R || a.xq_kind;
    const int act_x2 = post ? static_cast<int>(ACT_NONE) : activation;
    auto finish = [&]() {
        if (post) hipLaunchKernelGGL(k_fno_post, dim3(grid_for(M, 1, 16)), dim3(256), 0, st, C, R, a, activation);
        return check_launch("linear_forward_per_token");
    };
    // K = 128 .. 512: the one-pass kernel (quantise into LDS, then all of N).
    if (token_gemm_ok(a) && !path_flag(kernel_path().no_token_gemm)) {
        launch_token_gemm(a, act_x2, st);
        return finish();
    }
    // Wide K: quantise into a workspace, then the tiled GEMM (below).
    RowsArgs g = a;
    g.Aq = nullptr;  // the codes go to the workspace, which is 256-byte aligned
    const bool wide = use_gemm(g);
    if (!wide && rows_ok(a, IN_F32_TOKEN)) {
        launch_rows<false, IN_F32_TOKEN, OUT_EPI>(a, act_x2, st);
        return finish();
    }
    // Split path: quantise into a workspace, then the product.
    // Workspace: codes, then M scales; for the tiled GEMM, M row code sums
    // from the same quantise pass when zero points may be nonzero, and N
    // weight-row byte sums when the formula takes a caller's sum_W.
    const size_t codes = static_cast<size_t>(M) * a.K;
    const bool want_sums = wide && a.zpW;
    const bool want_colsum = wide && a.formula == F_ROW_VNNI && a.sumW;
    const size_t n_sums = (want_sums ? static_cast<size_t>(M) : 0) + (want_colsum ? a.N : 0);
    const size_t codes16 = ((codes + 15) / 16) * 16;
    if (fixed) {
        // Codes, then (with no scale_A_out) M scales, then the sums; every
        // region is written by the quantise launch before the product reads it.
        const size_t need = codes16 + (scale_A_out ? 0 : static_cast<size_t>(M) * sizeof(float)) +
                            n_sums * sizeof(int32_t);
        if (need > fixed->cap)
            return set_error(NFLOW_INVALID_ARG, std::string(fixed->what) + ": this shape needs " +
                                                    std::to_string(need) + " bytes of scratch, more than the " +
                                                    std::to_string(fixed->cap) + " the library holds (split the rows)");
        void* base = nullptr;
        std::unique_lock<std::mutex> hold;   // until the product is launched (end of scope)
        if (int rc = noalloc_scratch_address(&base, &hold)) return rc;
        uint8_t* q = static_cast<uint8_t*>(base);
        float* sc = scale_A_out ? scale_A_out : reinterpret_cast<float*>(q + codes16);
        int32_t* sums0 = reinterpret_cast<int32_t*>(q + codes16 + (scale_A_out ? 0 : static_cast<size_t>(M) * sizeof(float)));
        int32_t* sums = want_sums ? sums0 : nullptr;
        int32_t* colsum = want_colsum ? sums0 + (want_sums ? M : 0) : nullptr;
        launch_quantise_token<false>(A, M, a.K, q, sc, sums, st, CodeSums{a.W, a.N, a.K, colsum});
        a.Aq = q;
        a.scale_in = sc;
        a.sum_in = sums;
        a.colsum_in = colsum;
        if (wide) launch_gemm<OUT_EPI>(a, act_x2, st);
        else if (rows_ok(a, IN_CODES)) launch_rows<false, IN_CODES, OUT_EPI>(a, act_x2, st);
        else launch_generic<false, OUT_EPI>(a, act_x2, st);
        return finish();
    }
    Scratch ws(codes + 16 + static_cast<size_t>(M) * sizeof(float) + n_sums * sizeof(int32_t), st);
    if (ws.err != hipSuccess) return set_error(NFLOW_INTERNAL, "linear_forward_per_token: workspace allocation failed");
    uint8_t* q = static_cast<uint8_t*>(ws.p);
    float* sc = reinterpret_cast<float*>(q + codes16);
    int32_t* sums = want_sums ? reinterpret_cast<int32_t*>(sc + M) : nullptr;
    int32_t* colsum = want_colsum ? reinterpret_cast<int32_t*>(sc + M) + (want_sums ? M : 0) : nullptr;
    launch_quantise_token<false>(A, M, a.K, q, sc, sums, st, CodeSums{a.W, a.N, a.K, colsum});
    if (scale_A_out) (void)hipMemcpyAsync(scale_A_out, sc, sizeof(float) * M, hipMemcpyDeviceToDevice, st);
    a.Aq = q;
    a.scale_in = sc;
    a.sum_in = sums;
    a.colsum_in = colsum;
    if (wide) launch_gemm<OUT_EPI>(a, act_x2, st);
    else if (rows_ok(a, IN_CODES)) launch_rows<false, IN_CODES, OUT_EPI>(a, act_x2, st);
    else launch_generic<false, OUT_EPI>(a, act_x2, st);
    return finish();
}

}  // namespace nfq

extern "C" {

int nflow_int8_linear_forward_per_token(const nflow_int8_linear_params* p, int64_t M,
                                        const float* A, float* C, float* scale_A_out,
                                        int activation, void* stream) {
    clear_error();
    return int8_per_token(p, M, A, nullptr, C, scale_A_out, activation, nullptr, stream);
}

int nflow_int8_linear_forward_per_token_noalloc(const nflow_int8_linear_params* p, int64_t M,
                                                const float* A, float* C, float* scale_A_out,
                                                int activation, void* stream) {
    clear_error();
    FixedWs fixed{kNoAllocScratchBytes, "linear_forward_per_token_noalloc"};
    return int8_per_token(p, M, A, nullptr, C, scale_A_out, activation, nullptr, stream, &fixed);
}

int nflow_int8_fno_layer_per_token(const nflow_int8_linear_params* p, int64_t M, const float* h,
                                   const float* x1, float* y, float* scale_A_out, int activation,
                                   void* stream) {
    clear_error();
    return int8_per_token(p, M, h, x1, y, scale_A_out, activation, nullptr, stream);
}

int nflow_int8_fno_layer_per_token_x2q(const nflow_int8_linear_params* p, int64_t M, const float* h,
                                       const float* x1, float* y, float* scale_A_out, int activation,
                                       const nflow_x2_quant* x2q, void* stream) {
    clear_error();
    return int8_per_token(p, M, h, x1, y, scale_A_out, activation, x2q, stream);
}

int nflow_int8_gemm_i32(const int8_t* A_q, const int8_t* W_q, int64_t M, int N, int K, int32_t* C,
                        void* stream) {
    clear_error();
    if (!A_q || !W_q || !C) return set_error(NFLOW_INVALID_ARG, "gemm_i32: null pointer");
    if (N <= 0 || K <= 0) return set_error(NFLOW_INVALID_ARG, "gemm_i32: bad dims");
    if (M <= 0) return NFLOW_OK;
    RowsArgs a{};
    a.Aq = reinterpret_cast<const uint8_t*>(A_q);
    a.M = M;
    a.K = K;
    a.N = N;
    a.W = reinterpret_cast<const uint8_t*>(W_q);
    a.kb_dot = (K + 63) / 64;
    a.C = C;
    if (use_gemm(a)) launch_gemm<OUT_RAW>(a, ACT_NONE, as_stream(stream));
    else if (rows_ok(a, IN_CODES)) launch_rows<false, IN_CODES, OUT_RAW>(a, ACT_NONE, as_stream(stream));
    else launch_generic<false, OUT_RAW>(a, ACT_NONE, as_stream(stream));
    return check_launch("gemm_i32");
}

int nflow_int8_linear_forward_quantised(const nflow_int8_linear_params* p, int64_t M,
                                        const int8_t* A_q, const float* scale_A, float* C,
                                        int activation, void* stream) {
    clear_error();
    if (!A_q || !scale_A || !C || !p || !p->W_int8 || !p->scale_W)
        return set_error(NFLOW_INVALID_ARG, "linear_forward_quantised: null input/output");
    if (p->in_features <= 0 || p->out_features <= 0)
        return set_error(NFLOW_INVALID_ARG, "linear_forward_quantised: bad feature dims");
    if (!valid_act(activation))
        return set_error(NFLOW_INVALID_ARG, "linear_forward_quantised: unknown activation");
    if (M <= 0) return NFLOW_OK;
    RowsArgs a{};
    a.Aq = reinterpret_cast<const uint8_t*>(A_q);
    a.scale_in = scale_A;
    a.M = M;
    a.K = p->in_features;
    a.N = p->out_features;
    a.W = reinterpret_cast<const uint8_t*>(p->W_int8);
    a.sW = p->scale_W;
    a.zpW = p->zp_W;
    a.bias = p->bias;
    a.sumW = p->sum_W_per_row;
    a.zp_A = 0;
    a.formula = formula_row(a.K);
    a.kb_dot = kb_dot_for(a.formula, a.K);
    a.C = C;
    hipStream_t st = as_stream(stream);
    if (use_gemm(a)) {
        // Without zero points a caller's sum_W only needs the weight-row
        // byte sums (a pre-pass) to keep the GEMM on its LDS-DMA kernel.
        if (!a.zpW && a.formula == F_ROW_VNNI && a.sumW) {
            Scratch ws(static_cast<size_t>(a.N) * sizeof(int32_t), st);
            if (ws.err != hipSuccess)
                return set_error(NFLOW_INTERNAL, "linear_forward_quantised: workspace allocation failed");
            int32_t* colsum = static_cast<int32_t*>(ws.p);
            hipLaunchKernelGGL(k_code_sums, dim3(grid_for(a.N, 16, 4)), dim3(256), 0, st, CodeSums{a.W, a.N, a.K, colsum});
            a.colsum_in = colsum;
            launch_gemm<OUT_EPI>(a, activation, st);
            return check_launch("linear_forward_quantised");
        }
        launch_gemm<OUT_EPI>(a, activation, st);
    } else if (rows_ok(a, IN_CODES)) {
        launch_rows<false, IN_CODES, OUT_EPI>(a, activation, st);
    } else {
        launch_generic<false, OUT_EPI>(a, activation, st);
    }
    return check_launch("linear_forward_quantised");
}

int nflow_fp8_e4m3_to_bits(const float* in, uint8_t* out, int64_t n, void* stream) {
    clear_error();
    if (!in || !out) return set_error(NFLOW_INVALID_ARG, "fp8_e4m3_to_bits: null pointer");
    if (n <= 0) return NFLOW_OK;
    hipLaunchKernelGGL(k_e4m3_encode, dim3(grid_for(n, 256, 16)), dim3(256), 0, as_stream(stream),
                       in, out, n);
    return check_launch("fp8_e4m3_to_bits");
}

int nflow_fp8_e4m3_from_bits(const uint8_t* in, float* out, int64_t n, void* stream) {
    clear_error();
    if (!in || !out) return set_error(NFLOW_INVALID_ARG, "fp8_e4m3_from_bits: null pointer");
    if (n <= 0) return NFLOW_OK;
    hipLaunchKernelGGL(k_e4m3_decode, dim3(grid_for(n, 256, 16)), dim3(256), 0, as_stream(stream),
                       in, out, n);
    return check_launch("fp8_e4m3_from_bits");
}

int nflow_fp8_e4m3_fake_quant(const float* in, float scale, float* out, int64_t n, void* stream) {
    clear_error();
    if (!in || !out) return set_error(NFLOW_INVALID_ARG, "fp8_e4m3_fake_quant: null pointer");
    if (n <= 0) return NFLOW_OK;
    hipLaunchKernelGGL(k_fp8_fake_quant, dim3(grid_for(n, 256, 16)), dim3(256), 0,
                       as_stream(stream), in, scale, out, n);
    return check_launch("fp8_e4m3_fake_quant");
}

int nflow_fp8_quantise_per_token(const float* A, int64_t M, int K, uint8_t* A_q, float* scale_A,
                                 void* stream) {
    clear_error();
    if (!A || !A_q || !scale_A) return set_error(NFLOW_INVALID_ARG, "fp8_quantise_per_token: null pointer");
    if (K <= 0) return set_error(NFLOW_INVALID_ARG, "fp8_quantise_per_token: K <= 0");
    if (M <= 0) return NFLOW_OK;
    launch_quantise_token<true>(A, M, K, A_q, scale_A, static_cast<int32_t*>(nullptr), as_stream(stream));
    return check_launch("fp8_quantise_per_token");
}

static int fp8_check(const nflow_fp8_linear_params* p, int act, const char* what) {
    if (!p || !p->W_e4m3 || !p->scale_W) return set_error(NFLOW_INVALID_ARG, std::string(what) + ": null input/output");
    if (p->in_features <= 0 || p->out_features <= 0)
        return set_error(NFLOW_INVALID_ARG, std::string(what) + ": bad feature dims");
    if (!valid_act(act)) return set_error(NFLOW_INVALID_ARG, std::string(what) + ": unknown activation");
    return NFLOW_OK;
}

}  // extern "C"

namespace nfq {

static int fp8_per_token(const nflow_fp8_linear_params* p, int64_t M, const float* A, const float* R,
                         float* C, float* scale_A_out, int activation, const nflow_x2_quant* xq,
                         void* stream) {
    if (!A || !C) return set_error(NFLOW_INVALID_ARG, "fp8_linear_forward_per_token: null input/output");
    int rc = fp8_check(p, activation, "fp8_linear_forward_per_token");
    if (rc) return rc;
    if (R && R == C) return set_error(NFLOW_INVALID_ARG, "fp8_fno_layer: x1 and y must be distinct buffers");
    RowsArgs a{};
    a.N = p->out_features;
    if (int rc2 = apply_x2q(a, xq, "fp8_fno_layer")) return rc2;
    if (M <= 0) return NFLOW_OK;
    hipStream_t st = as_stream(stream);
    a.A = A;
    a.M = M;
    a.K = p->in_features;
    a.W = p->W_e4m3;
    a.sW = p->scale_W;
    a.bias = p->bias;
    a.kb_dot = (a.K + 63) / 64;
    a.C = C;
    a.scale_out = scale_A_out;
    if (rows64_ok(a) && (!R || aligned(R, 16)) && !path_flag(kernel_path().no_rows64)) {
        a.residual = R;
        launch_rows64<true>(a, activation, st);
        return check_launch("fp8_linear_forward_per_token");
    }
    const bool post = R || a.xq_kind;
    const int act_x2 = post ? static_cast<int>(ACT_NONE) : activation;
    auto finish = [&]() {
        if (post) hipLaunchKernelGGL(k_fno_post, dim3(grid_for(M, 1, 16)), dim3(256), 0, st, C, R, a, activation);
        return check_launch("fp8_linear_forward_per_token");
    };
    if (rows_ok(a, IN_F32_TOKEN)) {
        launch_rows<true, IN_F32_TOKEN, OUT_EPI>(a, act_x2, st);
        return finish();
    }
    const size_t codes = static_cast<size_t>(M) * a.K;
    Scratch ws(codes + 16 + static_cast<size_t>(M) * sizeof(float), st);
    if (ws.err != hipSuccess) return set_error(NFLOW_INTERNAL, "fp8_linear_forward_per_token: workspace allocation failed");
    uint8_t* q = static_cast<uint8_t*>(ws.p);
    float* sc = reinterpret_cast<float*>(q + ((codes + 15) / 16) * 16);
    launch_quantise_token<true>(A, M, a.K, q, sc, static_cast<int32_t*>(nullptr), st);
    if (scale_A_out) (void)hipMemcpyAsync(scale_A_out, sc, sizeof(float) * M, hipMemcpyDeviceToDevice, st);
    a.Aq = q;
    a.scale_in = sc;
    if (rows_ok(a, IN_CODES)) launch_rows<true, IN_CODES, OUT_EPI>(a, act_x2, st);
    else launch_generic<true, OUT_EPI>(a, act_x2, st);
    return finish();
}

}  // namespace nfq

extern "C" {

int nflow_fp8_linear_forward_per_token(const nflow_fp8_linear_params* p, int64_t M, const float* A,
                                       float* C, float* scale_A_out, int activation, void* stream) {
    clear_error();
    return fp8_per_token(p, M, A, nullptr, C, scale_A_out, activation, nullptr, stream);
}

int nflow_fp8_fno_layer_per_token(const nflow_fp8_linear_params* p, int64_t M, const float* h,
                                  const float* x1, float* y, float* scale_A_out, int activation,
                                  void* stream) {
    clear_error();
    return fp8_per_token(p, M, h, x1, y, scale_A_out, activation, nullptr, stream);
}

int nflow_fp8_fno_layer_per_token_x2q(const nflow_fp8_linear_params* p, int64_t M, const float* h,
                                      const float* x1, float* y, float* scale_A_out, int activation,
                                      const nflow_x2_quant* x2q, void* stream) {
    clear_error();
    return fp8_per_token(p, M, h, x1, y, scale_A_out, activation, x2q, stream);
}

int nflow_fp8_gemm_f32(const uint8_t* A_q, const uint8_t* W_q, int64_t M, int N, int K, float* C,
                       void* stream) {
    clear_error();
    if (!A_q || !W_q || !C) return set_error(NFLOW_INVALID_ARG, "fp8_gemm_f32: null pointer");
    if (N <= 0 || K <= 0) return set_error(NFLOW_INVALID_ARG, "fp8_gemm_f32: bad dims");
    if (M <= 0) return NFLOW_OK;
    RowsArgs a{};
    a.Aq = A_q;
    a.M = M;
    a.K = K;
    a.N = N;
    a.W = W_q;
    a.kb_dot = (K + 63) / 64;
    a.C = C;
    if (rows_ok(a, IN_CODES)) launch_rows<true, IN_CODES, OUT_RAW>(a, ACT_NONE, as_stream(stream));
    else launch_generic<true, OUT_RAW>(a, ACT_NONE, as_stream(stream));
    return check_launch("fp8_gemm_f32");
}

int nflow_fp8_linear_forward_quantised(const nflow_fp8_linear_params* p, int64_t M,
                                       const uint8_t* A_q, const float* scale_A, float* C,
                                       int activation, void* stream) {
    clear_error();
    if (!A_q || !scale_A || !C) return set_error(NFLOW_INVALID_ARG, "fp8_linear_forward_quantised: null input/output");
    int rc = fp8_check(p, activation, "fp8_linear_forward_quantised");
    if (rc) return rc;
    if (M <= 0) return NFLOW_OK;
    RowsArgs a{};
    a.Aq = A_q;
    a.scale_in = scale_A;
    a.M = M;
    a.K = p->in_features;
    a.N = p->out_features;
    a.W = p->W_e4m3;
    a.sW = p->scale_W;
    a.bias = p->bias;
    a.kb_dot = (a.K + 63) / 64;
    a.C = C;
    if (rows_ok(a, IN_CODES)) launch_rows<true, IN_CODES, OUT_EPI>(a, activation, as_stream(stream));
    else launch_generic<true, OUT_EPI>(a, activation, as_stream(stream));
    return check_launch("fp8_linear_forward_quantised");
}

}  // extern "C"

namespace nfq {

// ---------------------------------------------------------------------------
// 8-bit-output layers and the per-token layer chain
// ---------------------------------------------------------------------------

// Row-maxima exchange state of the 8-bit-output kernel, per (device,
// stream): the published words (zeroed when allocated; every launch tags its
// words with a new epoch, so a word of an earlier launch never reads as
// fresh) and a fault word, set by a launch whose wait for the other blocks
// of a row tile timed out.  Calls on one stream run in order; calls on
// different streams use different words.  The words grow with the largest M
// (freed and reallocated in stream order) and live until the process ends.
struct ChainState {
    std::mutex mu;
    uint64_t* part = nullptr;
    int64_t rows_cap = 0;
    uint32_t* fault = nullptr;
};

static ChainState* chain_state(int dev, hipStream_t st) {
    static std::mutex map_mu;
    static std::map<std::pair<int, uintptr_t>, std::unique_ptr<ChainState>>* map =
        new std::map<std::pair<int, uintptr_t>, std::unique_ptr<ChainState>>();
    std::lock_guard<std::mutex> g(map_mu);
    auto& e = (*map)[{dev, reinterpret_cast<uintptr_t>(st)}];
    if (!e) e.reset(new ChainState);
    return e.get();
}

// A nonzero tag no earlier launch of this process used (wraps after 2^32 - 1
// launches).
static uint32_t next_chain_epoch() {
    static std::atomic<uint32_t> e{0};
    uint32_t v;
    do v = e.fetch_add(1, std::memory_order_relaxed) + 1; while (v == 0);
    return v;
}

// A wave waits at most this long (ticks of the 100 MHz clock: 2 s) for the
// other blocks of its row tile; they run concurrently, so a timeout means
// they could not be scheduled.
constexpr int64_t kChainSpinTicks = 200000000;
constexpr int kChainSlots = 8;   // published words per row, at most (128-column tiles, N <= 1024)

// Words for M rows (and the fault word) in cs, allocated on stream st.
static int chain_words(ChainState* cs, int64_t M, hipStream_t st) {
    const int64_t rows = ((M + 127) / 128) * 128;
    if (!cs->fault) {
        if (hipMallocAsync(reinterpret_cast<void**>(&cs->fault), 256, st) != hipSuccess) {
            cs->fault = nullptr;
            return set_error(NFLOW_INTERNAL, "chain: fault word allocation failed");
        }
        if (hipMemsetAsync(cs->fault, 0, 256, st) != hipSuccess) return set_error(NFLOW_INTERNAL, "chain: memset failed");
    }
    if (rows > cs->rows_cap) {
        if (cs->part) (void)hipFreeAsync(cs->part, st);
        cs->part = nullptr;
        cs->rows_cap = 0;
        const int64_t want = std::max<int64_t>(rows, 4096);
        const size_t bytes = static_cast<size_t>(want) * kChainSlots * sizeof(uint64_t);
        if (hipMallocAsync(reinterpret_cast<void**>(&cs->part), bytes, st) != hipSuccess) {
            cs->part = nullptr;
            return set_error(NFLOW_INTERNAL, "chain: row-maxima allocation failed");
        }
        if (hipMemsetAsync(cs->part, 0, bytes, st) != hipSuccess) return set_error(NFLOW_INTERNAL, "chain: memset failed");
        cs->rows_cap = want;
    }
    return NFLOW_OK;
}

// The chain entry points under graph capture: refused before any
// allocation or launch.  The fused kernel's row-maxima words would be
// allocated and cleared inside the graph and a replay would reuse its
// launch's epoch (an earlier replay's words reading as fresh); the
// layer-by-layer route allocates its buffers inside the graph, and a graph
// captured that way (both entry points, 20000 rows) took an illegal memory
// access on its first replay, for a reason not found in this library.
static bool stream_capturing(hipStream_t st) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
}

// Whether calls on stream st may use the fused 8-bit-output kernel: not on
// the per-thread default stream, whose one handle names a different stream
// in each host thread, so concurrent launches would share the row-maxima
// words.  Those calls take the layer-by-layer path (the same bits).
static bool chain_stream_ok(hipStream_t st) { return st != hipStreamPerThread; }

// Whether a layer takes the fused 8-bit-output kernel: symmetric weights
// (no zero points, no caller sum_W: the integer terms of the formula are 0),
// K = 1024, N a multiple of 256 up to 1024, 16-byte aligned codes.
static bool chain_layer_ok(const nflow_int8_linear_params* p) {
    return !p->zp_W && !p->sum_W_per_row && p->in_features == 1024 && p->out_features >= 256 &&
           p->out_features <= 1024 && p->out_features % 256 == 0 && aligned(p->W_int8, 16);
}

// One fused layer on stream st with cs's words (cs locked by the caller).
static void chain_launch(const nflow_int8_linear_params* p, int64_t M, const uint8_t* Aq, const float* sA,
                         uint8_t* Cq, float* sC, int act, hipStream_t st, ChainState* cs) {
    ChainArgs c{};
    c.Aq = Aq;
    c.scale_in = sA;
    c.M = M;
    c.K = p->in_features;
    c.N = p->out_features;
    c.W = reinterpret_cast<const uint8_t*>(p->W_int8);
    c.sW = p->scale_W;
    c.bias = p->bias;
    c.Cq = Cq;
    c.scale_out = sC;
    c.part = cs->part;
    c.fault = cs->fault;
    c.epoch = next_chain_epoch();
    c.spin_limit = kChainSpinTicks;
    launch_chain(c, act, st);
}

// Codes + row scales -> fp32 (M, N) through the LinearForward formula with
// zp_A = 0 (the product of nflow_int8_linear_forward_quantised for
// symmetric layers and for those the tiled kernel forms the byte sums of).
static void codes_to_f32(const nflow_int8_linear_params* p, int64_t M, const uint8_t* Aq, const float* sA,
                         float* C, int act, hipStream_t st) {
    RowsArgs a{};
    a.Aq = Aq;
    a.scale_in = sA;
    a.M = M;
    a.K = p->in_features;
    a.N = p->out_features;
    a.W = reinterpret_cast<const uint8_t*>(p->W_int8);
    a.sW = p->scale_W;
    a.zpW = p->zp_W;
    a.bias = p->bias;
    a.sumW = p->sum_W_per_row;
    a.zp_A = 0;
    a.formula = formula_row(a.K);
    a.kb_dot = kb_dot_for(a.formula, a.K);
    a.C = C;
    if (use_gemm(a)) launch_gemm<OUT_EPI>(a, act, st);
    else if (rows_ok(a, IN_CODES)) launch_rows<false, IN_CODES, OUT_EPI>(a, act, st);
    else launch_generic<false, OUT_EPI>(a, act, st);
}

static int check_layer(const nflow_int8_linear_params* p, int act, const char* what) {
    if (!p || !p->W_int8 || !p->scale_W) return set_error(NFLOW_INVALID_ARG, std::string(what) + ": null layer parameters");
    if (p->in_features <= 0 || p->out_features <= 0)
        return set_error(NFLOW_INVALID_ARG, std::string(what) + ": bad feature dims");
    if (!valid_act(act)) return set_error(NFLOW_INVALID_ARG, std::string(what) + ": unknown activation");
    return NFLOW_OK;
}

}  // namespace nfq

extern "C" {

int nflow_int8_linear_forward_codes(const nflow_int8_linear_params* p, int64_t M, const int8_t* A_q,
                                    const float* scale_A, int8_t* C_q, float* scale_C, int activation,
                                    void* stream) {
    clear_error();
    if (int rc = check_layer(p, activation, "linear_forward_codes")) return rc;
    if (!A_q || !scale_A || !C_q || !scale_C) return set_error(NFLOW_INVALID_ARG, "linear_forward_codes: null input/output");
    if (M <= 0) return NFLOW_OK;
    hipStream_t st = as_stream(stream);
    if (stream_capturing(st))
        return set_error(NFLOW_UNSUPPORTED_OP, "linear_forward_codes: not available under graph capture (use "
                                               "nflow_int8_linear_forward_per_token_noalloc)");
    const uint8_t* aq = reinterpret_cast<const uint8_t*>(A_q);
    uint8_t* cq = reinterpret_cast<uint8_t*>(C_q);
    if (chain_layer_ok(p) && aligned(aq, 16) && aligned(cq, 4) && chain_stream_ok(st)) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return set_error(NFLOW_INTERNAL, "linear_forward_codes: hipGetDevice failed");
        ChainState* cs = chain_state(dev, st);
        std::lock_guard<std::mutex> lock(cs->mu);
        if (int rc = chain_words(cs, M, st)) return rc;
        chain_launch(p, M, aq, scale_A, cq, scale_C, activation, st, cs);
        return check_launch("linear_forward_codes");
    }
    // Other layers: the fp32 output into a stream-ordered buffer, then the
    // per-token quantise (the same bits).
    float* tmp = nullptr;
    const size_t bytes = static_cast<size_t>(M) * p->out_features * sizeof(float);
    if (hipMallocAsync(reinterpret_cast<void**>(&tmp), bytes, st) != hipSuccess)
        return set_error(NFLOW_INTERNAL, "linear_forward_codes: workspace allocation failed");
    int rc = nflow_int8_linear_forward_quantised(p, M, A_q, scale_A, tmp, activation, stream);
    if (rc == NFLOW_OK) {
        launch_quantise_token<false>(tmp, M, p->out_features, cq, scale_C, nullptr, st);
        rc = check_launch("linear_forward_codes");
    }
    (void)hipFreeAsync(tmp, st);
    return rc;
}

int nflow_int8_mlp_forward_per_token(const nflow_int8_linear_params* layers, const int* activations,
                                     int n_layers, int64_t M, const float* x, float* y, void* stream) {
    clear_error();
    if (!layers || !activations || n_layers <= 0) return set_error(NFLOW_INVALID_ARG, "mlp_forward_per_token: no layers");
    if (!x || !y) return set_error(NFLOW_INVALID_ARG, "mlp_forward_per_token: null input/output");
    for (int l = 0; l < n_layers; ++l) {
        if (int rc = check_layer(&layers[l], activations[l], "mlp_forward_per_token")) return rc;
        if (l > 0 && layers[l].in_features != layers[l - 1].out_features)
            return set_error(NFLOW_SHAPE_MISMATCH, "mlp_forward_per_token: layer " + std::to_string(l) +
                                                       " in_features != the previous layer's out_features");
    }
    if (M <= 0) return NFLOW_OK;
    hipStream_t st = as_stream(stream);
    if (stream_capturing(st))
        return set_error(NFLOW_UNSUPPORTED_OP, "mlp_forward_per_token: not available under graph capture (use "
                                               "nflow_int8_linear_forward_per_token_noalloc per layer)");
    if (n_layers == 1) return int8_per_token(&layers[0], M, x, nullptr, y, nullptr, activations[0], nullptr, stream);
    // Fused: every layer symmetric, every layer but the last on the
    // 8-bit-output kernel (K = 1024, so every hidden width is 1024), and
    // rows enough for two 128 x 256 tiles per CU: with one tile per CU the
    // 8-bit-output kernel's last row-maxima exchange is not overlapped
    // (measured at 4096 rows, K = N = 1024: 17.9 us against 11.2 us for the
    // fp32-output product, more than the quantise launch it saves).
    bool fused = aligned(x, 16) && !layers[n_layers - 1].zp_W && !layers[n_layers - 1].sum_W_per_row &&
                 ((M + 127) / 128) * 4 >= 2 * static_cast<int64_t>(num_cus()) && chain_stream_ok(st);
    for (int l = 0; l < n_layers - 1; ++l) fused = fused && chain_layer_ok(&layers[l]);
    if (fused) {
        const size_t codes = static_cast<size_t>(M) * 1024;
        const size_t codes16 = ((codes + 255) / 256) * 256;
        const size_t sc = ((static_cast<size_t>(M) * sizeof(float) + 255) / 256) * 256;
        Scratch ws(2 * codes16 + 2 * sc, st);
        if (ws.err != hipSuccess) return set_error(NFLOW_INTERNAL, "mlp_forward_per_token: workspace allocation failed");
        uint8_t* q[2] = {static_cast<uint8_t*>(ws.p), static_cast<uint8_t*>(ws.p) + codes16};
        float* s[2] = {reinterpret_cast<float*>(q[1] + codes16), reinterpret_cast<float*>(q[1] + codes16 + sc)};
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return set_error(NFLOW_INTERNAL, "mlp_forward_per_token: hipGetDevice failed");
        ChainState* cs = chain_state(dev, st);
        std::lock_guard<std::mutex> lock(cs->mu);
        if (int rc = chain_words(cs, M, st)) return rc;
        launch_quantise_token<false>(x, M, 1024, q[0], s[0], nullptr, st);
        int cur = 0;
        for (int l = 0; l < n_layers - 1; ++l) {
            chain_launch(&layers[l], M, q[cur], s[cur], q[cur ^ 1], s[cur ^ 1], activations[l], st, cs);
            cur ^= 1;
        }
        codes_to_f32(&layers[n_layers - 1], M, q[cur], s[cur], y, activations[n_layers - 1], st);
        return check_launch("mlp_forward_per_token");
    }
    // Layer by layer through fp32 activations in two buffers of the stream's
    // second workspace slot (each layer's own workspace is slot 0).
    int width = 0;
    for (int l = 0; l < n_layers - 1; ++l) width = std::max(width, layers[l].out_features);
    const size_t hb = ((static_cast<size_t>(M) * width * sizeof(float) + 255) / 256) * 256;
    Scratch hs(2 * hb, st, 1);
    if (hs.err != hipSuccess) return set_error(NFLOW_INTERNAL, "mlp_forward_per_token: workspace allocation failed");
    float* h[2] = {static_cast<float*>(hs.p), reinterpret_cast<float*>(static_cast<uint8_t*>(hs.p) + hb)};
    int rc = NFLOW_OK;
    const float* in = x;
    for (int l = 0; l < n_layers && rc == NFLOW_OK; ++l) {
        float* out = l == n_layers - 1 ? y : h[l & 1];
        rc = int8_per_token(&layers[l], M, in, nullptr, out, nullptr, activations[l], nullptr, stream);
        in = out;
    }
    return rc;
}

int nflow_release_stream_workspace(void* stream) {
    clear_error();
    hipStream_t st = as_stream(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(NFLOW_INTERNAL, "release_stream_workspace: hipGetDevice failed");
    for (int slot = 0; slot < 2; ++slot) {
        WsEntry* e = ws_entry(dev, st, slot);
        std::lock_guard<std::mutex> lock(e->mu);
        if (e->p) (void)hipFreeAsync(e->p, st);
        e->p = nullptr;
        e->cap = 0;
    }
    ChainState* cs = chain_state(dev, st);
    std::lock_guard<std::mutex> lock(cs->mu);
    if (cs->part) (void)hipFreeAsync(cs->part, st);
    if (cs->fault) (void)hipFreeAsync(cs->fault, st);
    cs->part = nullptr;
    cs->fault = nullptr;
    cs->rows_cap = 0;
    return check_launch("release_stream_workspace");
}

int nflow_debug_chain_faults(void* stream, uint32_t* faults) {
    clear_error();
    if (!faults) return set_error(NFLOW_INVALID_ARG, "debug_chain_faults: null output");
    *faults = 0;
    hipStream_t st = as_stream(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(NFLOW_INTERNAL, "debug_chain_faults: hipGetDevice failed");
    ChainState* cs = chain_state(dev, st);
    std::lock_guard<std::mutex> lock(cs->mu);
    if (!cs->fault) return NFLOW_OK;
    uint32_t v = 0;
    if (hipMemcpyAsync(&v, cs->fault, sizeof(v), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess || hipMemsetAsync(cs->fault, 0, sizeof(uint32_t), st) != hipSuccess)
        return set_error(NFLOW_INTERNAL, "debug_chain_faults: copy failed");
    *faults = v;
    return NFLOW_OK;
}

}  // extern "C"
