// fno_rt.hip -- device kernels of the FNO1d / FNO2d runtime around the
// quantised local-linear layer: the fp32 Linear of the lift / projection /
// fallback layers, the activation fake-quants, the spectral convolution
// (radix-2 FFTs along rows and, in 2-D, columns; channel mix; inverse FFTs)
// and the layer tail act(x1 + fq(x2)).
//
// Every element is computed by the float operations of the reference build
// (cpp/src/fno.cpp and fft.cpp compiled by g++ -O3 -mfma): products the
// build fuses are written as __builtin_fmaf, everything else rounds on its
// own (this library is compiled with -ffp-contract=off).  GELU is
// gelu_fast (gelu_exact.h), bit-exact with glibc's tanhf.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "fno_rt.h"
#include "gelu_exact.h"
#include "launch.h"
#include "rows64_kernel.h"
#include "snap.h"

namespace nfq {

__device__ __forceinline__ float rt_activate(float y, int act) {
    if (act == RT_ACT_RELU) return y < 0.0f ? 0.0f : y;  // fno.cpp:37-40
    if (act == RT_ACT_GELU) return gelu_fast<kGeluRefine>(y);
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
// fp32 Linear (fno.cpp:69-79) in the reference build's summation order: the
// first k - k % 8 products rounded and added one by one, the rest fused.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lin_step(float acc, float x, float w, bool plain) {
    return plain ? acc + x * w : __builtin_fmaf(x, w, acc);
}

// k == 64, n >= 16: one wave per 4 output rows; lane j holds column j of W
// in registers (chunks of 64 columns), the rows' inputs go through LDS and
// are read back as broadcasts.
__global__ __launch_bounds__(256) void k_linear_rows64(LinArgs a) {
    __shared__ v4f xs[4][64];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int n = a.n;
    const int64_t rows = a.samples * a.rows_out;
    const int64_t quads = (rows + 3) / 4;
    const int64_t wave0 = static_cast<int64_t>(blockIdx.x) * 4 + wid;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
    const float* xsf = reinterpret_cast<const float*>(xs[wid]);
    for (int cc = 0; cc < n; cc += 64) {
        const int j = cc + lane;
        const bool jv = j < n;
        float wr[64];
        const float* wj = a.W + static_cast<int64_t>(jv ? j : 0) * 64;
#pragma unroll
        for (int p = 0; p < 64; p += 4) {
            const v4f q = *reinterpret_cast<const v4f*>(wj + p);
            wr[p] = q[0];
            wr[p + 1] = q[1];
            wr[p + 2] = q[2];
            wr[p + 3] = q[3];
        }
        const float bj = (jv && a.b) ? a.b[j] : 0.0f;
        for (int64_t qd = wave0; qd < quads; qd += nwaves) {
            // Lane l loads 4 inputs of row 4 qd + l / 16.
            {
                const int64_t r = qd * 4 + (lane >> 4);
                v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (r < rows) {
                    const int64_t s = r / a.rows_out;
                    const int t = static_cast<int>(r % a.rows_out);
                    if (t < a.rows_valid)
                        v = *reinterpret_cast<const v4f*>(a.x + (s * a.rows_in + t) * 64 + 4 * (lane & 15));
                }
                xs[wid][lane] = v;
            }
            wave_sync();
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int64_t r = qd * 4 + rr;
                if (r >= rows) break;
                const int t = static_cast<int>(r % a.rows_out);
                float out = 0.0f;
                if (t < a.rows_valid) {
                    float acc = bj;
#pragma unroll
                    for (int p = 0; p < 64; ++p) acc = acc + xsf[rr * 64 + p] * wr[p];
                    out = rt_activate(acc, a.act);
                }
                if (jv) a.y[r * n + j] = out;
            }
            wave_sync();
        }
    }
}

// k == 64, n <= NMAX, unpadded rows: a block's 256 rows are staged in LDS by
// coalesced loads (one thread per row reading its own 256-byte row touched
// 64 lines per load instruction), then one thread per row as below.
template <int NMAX>
__global__ __launch_bounds__(256) void k_linear_narrow64(LinArgs a) {
    __shared__ float xs[256][65];
    __shared__ float ws[NMAX * 64];
    const int n = a.n;
    for (int i = threadIdx.x; i < n * 64; i += 256) ws[i] = a.W[i];
    const int64_t rows = a.samples * a.rows_out;
    for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * 256; r0 < rows; r0 += static_cast<int64_t>(gridDim.x) * 256) {
        const int nr = rows - r0 < 256 ? static_cast<int>(rows - r0) : 256;
        const v4f* x4 = reinterpret_cast<const v4f*>(a.x + r0 * 64);
        if (nr == 256) {
            // A whole block of rows: every load issued before the first is
            // waited for (one at a time, each 16-byte load's latency stood in
            // front of the next).
            v4f v[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) v[q] = x4[threadIdx.x + 256 * q];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int i = threadIdx.x + 256 * q;
                float* d = &xs[i >> 4][(i & 15) * 4];
                d[0] = v[q][0];
                d[1] = v[q][1];
                d[2] = v[q][2];
                d[3] = v[q][3];
            }
        } else {
            for (int i = threadIdx.x; i < nr * 16; i += 256) {
                const v4f v = x4[i];
                float* d = &xs[i >> 4][(i & 15) * 4];
                d[0] = v[0];
                d[1] = v[1];
                d[2] = v[2];
                d[3] = v[3];
            }
        }
        __syncthreads();
        const int t = threadIdx.x;
        if (t < nr) {
            float acc[NMAX];
#pragma unroll
            for (int j = 0; j < NMAX; ++j) acc[j] = (j < n && a.b) ? a.b[j] : 0.0f;
            for (int p = 0; p < 64; ++p) {
                const float xv = xs[t][p];
#pragma unroll
                for (int j = 0; j < NMAX; ++j)
                    if (j < n) acc[j] = lin_step(acc[j], xv, ws[j * 64 + p], true);
            }
#pragma unroll
            for (int j = 0; j < NMAX; ++j)
                if (j < n) a.y[(r0 + t) * n + j] = rt_activate(acc[j], a.act);
        }
        __syncthreads();
    }
}

// n <= 16: one thread per output row, all n columns in registers, W from LDS.
template <int NMAX>
__global__ __launch_bounds__(256) void k_linear_narrow(LinArgs a) {
    extern __shared__ float ws[];   // W (n, k) row-major
    const int k = a.k, n = a.n, kplain = k - k % 8;
    for (int i = threadIdx.x; i < n * k; i += blockDim.x) ws[i] = a.W[i];
    __syncthreads();
    const bool vec4 = (k % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0);
    const int64_t rows = a.samples * a.rows_out;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; r < rows;
         r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const uint32_t ro = static_cast<uint32_t>(a.rows_out);
        const int64_t s = rows < (int64_t(1) << 32) ? static_cast<uint32_t>(r) / ro : r / a.rows_out;
        const int t = static_cast<int>(r - s * a.rows_out);
        float acc[NMAX];
#pragma unroll
        for (int j = 0; j < NMAX; ++j) acc[j] = (j < n && a.b) ? a.b[j] : 0.0f;
        if (t < a.rows_valid) {
            const float* xr = a.x + (s * a.rows_in + t) * static_cast<int64_t>(k);
            int p = 0;
            if (vec4) {
                for (; p + 4 <= k; p += 4) {
                    const v4f xv = *reinterpret_cast<const v4f*>(xr + p);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int j = 0; j < NMAX; ++j)
                            if (j < n) acc[j] = lin_step(acc[j], xv[q], ws[j * k + p + q], p + q < kplain);
                }
            }
            for (; p < k; ++p) {
                const float xv = xr[p];
                const bool plain = p < kplain;
#pragma unroll
                for (int j = 0; j < NMAX; ++j)
                    if (j < n) acc[j] = lin_step(acc[j], xv, ws[j * k + p], plain);
            }
#pragma unroll
            for (int j = 0; j < NMAX; ++j)
                if (j < n) a.y[r * n + j] = rt_activate(acc[j], a.act);
        } else {
#pragma unroll
            for (int j = 0; j < NMAX; ++j)
                if (j < n) a.y[r * n + j] = 0.0f;
        }
    }
}

// k == 1 (the FNO lift), unpadded rows, n a power of two from 4 to 1024:
// thread x makes outputs 4 (x mod n / 4) .. + 3 of each of its rows (the
// grid's stride in quads is a multiple of n / 4, so its columns' weights and
// bias stay in registers), one 16-byte store per row; each output is
// fma(x, w, b), k_linear_flat's one fused step.
__global__ __launch_bounds__(256) void k_linear_k1(LinArgs a) {
    const int nq = a.n >> 2, lq = __builtin_ctz(static_cast<unsigned>(nq));
    const int64_t quads = a.samples * a.rows_out * static_cast<int64_t>(nq);
    const int64_t q0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int j0 = 4 * static_cast<int>(q0 & (nq - 1));
    float wv[4], bv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        wv[e] = a.W[j0 + e];
        bv[e] = a.b ? a.b[j0 + e] : 0.0f;
    }
    for (int64_t qd = q0; qd < quads; qd += static_cast<int64_t>(gridDim.x) * 256) {
        const float x = a.x[qd >> lq];
        v4f y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = rt_activate(__builtin_fmaf(x, wv[e], bv[e]), a.act);
        *reinterpret_cast<v4f*>(a.y + (qd << 2)) = y;   // row (qd >> lq), column j0: index 4 qd
    }
}

// Any shape: one thread per output.
__global__ __launch_bounds__(256) void k_linear_flat(LinArgs a) {
    const int k = a.k, n = a.n, kplain = k - k % 8;
    const int64_t total = a.samples * a.rows_out * static_cast<int64_t>(n);
    if (a.rows_in == a.rows_out && a.rows_valid == a.rows_out && (n & (n - 1)) == 0) {
        // Unpadded rows and a power-of-two width: input row r is output row
        // r, and the indices are a shift and a mask.
        const int ln = __builtin_ctz(static_cast<unsigned>(n));
        for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
             idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
            const int64_t r = idx >> ln;
            const int j = static_cast<int>(idx & (n - 1));
            const float* xr = a.x + r * k;
            const float* wr = a.W + static_cast<int64_t>(j) * k;
            float acc = a.b ? a.b[j] : 0.0f;
            for (int p = 0; p < k; ++p) acc = lin_step(acc, xr[p], wr[p], p < kplain);
            a.y[idx] = rt_activate(acc, a.act);
        }
        return;
    }
    const bool narrow_idx = total < (int64_t(1) << 32);
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t r, s;
        if (narrow_idx) {
            const uint32_t r32 = static_cast<uint32_t>(idx) / static_cast<uint32_t>(n);
            r = r32;
            s = r32 / static_cast<uint32_t>(a.rows_out);
        } else {
            r = idx / n;
            s = r / a.rows_out;
        }
        const int j = static_cast<int>(idx - r * n);
        const int t = static_cast<int>(r - s * a.rows_out);
        float out = 0.0f;
        if (t < a.rows_valid) {
            const float* xr = a.x + (s * a.rows_in + t) * static_cast<int64_t>(k);
            const float* wr = a.W + static_cast<int64_t>(j) * k;
            float acc = a.b ? a.b[j] : 0.0f;
            for (int p = 0; p < k; ++p) acc = lin_step(acc, xr[p], wr[p], p < kplain);
            out = rt_activate(acc, a.act);
        }
        a.y[r * n + j] = out;
    }
}

// ---------------------------------------------------------------------------
// Layout change and the layer tail, on 64-point x 64-channel tiles.
// ---------------------------------------------------------------------------
struct Tile {
    int64_t s;
    int t0, c0;
};

// Tile `id` of TT tokens x 64 channels.
template <int TT>
__device__ __forceinline__ bool tile_of(int64_t id, int64_t samples, int n, int w, Tile& tl) {
    const int tt = (n + TT - 1) / TT, tc = (w + 63) / 64;
    const int64_t per_sample = static_cast<int64_t>(tt) * tc;
    if (id >= samples * per_sample) return false;
    tl.s = id / per_sample;
    const int rem = static_cast<int>(id % per_sample);
    tl.t0 = (rem / tc) * TT;
    tl.c0 = (rem % tc) * 64;
    return true;
}

// fno.cpp:579-606 with the exponent e = int(std::round(log2|v| * 8) / 8)
// read off the step points of the reference's libm (thr: the smallest float
// of each exponent from -5 to 9, computed on the host with that libm):
// e = -6 + #{thr <= |v|} for 2^-6 <= |v| <= FLT_MAX, taken from |v|'s binade
// and one compare (snap.h; thr in LDS); NaN and Inf give ldexp(1, INT_MIN)
// = 0; 2^e for e >= 9 is capped at 448.
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
        const int e = snap_exponent_binade(av, thr);
        qv = e >= 9 ? 448.0f : __builtin_bit_cast(float, static_cast<uint32_t>(127 + e) << 23);
    }
    const float clamped = (448.0f < qv) ? 448.0f : qv;
    return (sign * clamped) * s;
}

// x2_fake_quant with the per-tensor scale's reciprocal inv = fl(1 / s)
// computed once (inv_ok: inv a normal float).  t = v * inv is within
// 1.5 * 2^-23 |t| of the quotient fl(v / s), so while |t| is farther than
// 2^-20 |t| from the nearest half-integer, rint(t) equals round(fl(v / s))
// (the two rounding rules differ only on ties) and the rest of the
// fake-quant follows unchanged; otherwise (near a tie, |t| >= 2^22, NaN,
// Inf) the exact division.
__device__ __forceinline__ float x2_fake_quant_inv(float v, float s, float inv, bool inv_ok, float zpf) {
    const float t = v * inv;
    const float at = fabsf(t);
    const float dist = fabsf(__builtin_amdgcn_fractf(at) - 0.5f);
    if (!(inv_ok && dist > __builtin_fmaf(at, 0x1p-20f, 0x1p-40f))) return x2_fake_quant(v, s, zpf);
    float q = rintf(t) + zpf;
    q = q < -128.0f ? -128.0f : q;
    q = q > 127.0f ? 127.0f : q;
    return (q - zpf) * s;
}

// The reciprocal of a per-tensor scale and whether it is a normal float.
struct ScaleInv {
    float inv;
    bool ok;
};
__device__ __forceinline__ ScaleInv scale_inv(float s) {
    const float inv = 1.0f / s;
    const float a = fabsf(inv);
    return {inv, a >= 0x1p-126f && a <= 0x1.fffffep+127f};
}

// Copies a step table into LDS; every thread of the block must call it.
__device__ __forceinline__ void stage_steps(float* steps, const float* thr) {
    if (threadIdx.x < 15) steps[threadIdx.x] = thr[threadIdx.x];
    __syncthreads();
}

// The input fake-quant's form FQ (0 off, 1 per tensor, 3 log2 snap) is a
// template parameter and each thread's offsets are its fixed offset plus q
// times a per-launch stride, as in the layer tail below; thread x holds
// token-major elements (token x / 64 + 4 q, channel x % 64) and
// channel-major elements (channel x / TT + (256 / TT) q, token x % TT).
template <int TT, int FQ>
__global__ __launch_bounds__(256) void k_to_channel_major(float* h, float* hc, int64_t samples, int n, int w,
                                                          FakeQuant fq) {
    constexpr int PER = TT * 64 / 256;
    constexpr int CSTEP = 256 / TT;
    static_assert(PER * 256 == TT * 64 && CSTEP * TT == 256, "tile size");
    __shared__ float tile[64][TT + 1];
    __shared__ float steps[16];
    stage_steps(steps, fq.thr);
    const ScaleInv inv = scale_inv(fq.scale);
    const int cm = threadIdx.x / TT, tm = threadIdx.x % TT;
    const int tk = threadIdx.x / 64, ck = threadIdx.x % 64;
    const int64_t o1 = static_cast<int64_t>(cm) * n + tm, d1 = static_cast<int64_t>(CSTEP) * n;
    const int64_t o2 = static_cast<int64_t>(tk) * w + ck, d2 = 4 * static_cast<int64_t>(w);
    Tile tl;
    for (int64_t id = blockIdx.x; tile_of<TT>(id, samples, n, w, tl); id += gridDim.x) {
        const int nt = n - tl.t0 < TT ? n - tl.t0 : TT;
        const int nc = w - tl.c0 < 64 ? w - tl.c0 : 64;
        const bool full = nt == TT && nc == 64;
        const int64_t cb = (tl.s * w + tl.c0) * static_cast<int64_t>(n) + tl.t0 + o1;
        const int64_t tb = (tl.s * n + tl.t0) * static_cast<int64_t>(w) + tl.c0 + o2;
        auto c_ok = [&](int q) { return full || (cm + CSTEP * q < nc && tm < nt); };
        auto t_ok = [&](int q) { return full || (tk + 4 * q < nt && ck < nc); };
        float v[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = t_ok(q) ? h[tb + q * d2] : 0.0f;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if constexpr (FQ == 1) v[q] = x2_fake_quant_inv(v[q], fq.scale, inv.inv, inv.ok, fq.zpf);
            else if constexpr (FQ == 3) v[q] = log2_snap(v[q], fq.scale, steps);
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (t_ok(q)) {
                if constexpr (FQ != 0) h[tb + q * d2] = v[q];
                tile[ck][tk + 4 * q] = v[q];
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (c_ok(q)) hc[cb + q * d1] = tile[cm + CSTEP * q][tm];
        __syncthreads();
    }
}

// The lift with one input channel (h = fma(x, w, b), k_linear_k1's step)
// and the layout change with layer 0's input fake-quant in one pass: the
// lift's output is formed in registers, so h is written once and never
// read back.  Element roles as k_to_channel_major.
template <int TT, int FQ>
__global__ __launch_bounds__(256) void k_lift_layout(const float* x, const float* Wl, const float* bl, float* h,
                                                     float* hc, int64_t samples, int n, int w, FakeQuant fq) {
    constexpr int PER = TT * 64 / 256;
    constexpr int CSTEP = 256 / TT;
    static_assert(PER * 256 == TT * 64 && CSTEP * TT == 256, "tile size");
    __shared__ float tile[64][TT + 1];
    __shared__ float steps[16];
    stage_steps(steps, fq.thr);
    const ScaleInv inv = scale_inv(fq.scale);
    const int cm = threadIdx.x / TT, tm = threadIdx.x % TT;
    const int tk = threadIdx.x / 64, ck = threadIdx.x % 64;
    const int64_t o1 = static_cast<int64_t>(cm) * n + tm, d1 = static_cast<int64_t>(CSTEP) * n;
    const int64_t o2 = static_cast<int64_t>(tk) * w + ck, d2 = 4 * static_cast<int64_t>(w);
    Tile tl;
    for (int64_t id = blockIdx.x; tile_of<TT>(id, samples, n, w, tl); id += gridDim.x) {
        const int nt = n - tl.t0 < TT ? n - tl.t0 : TT;
        const int nc = w - tl.c0 < 64 ? w - tl.c0 : 64;
        const bool full = nt == TT && nc == 64;
        const int64_t cb = (tl.s * w + tl.c0) * static_cast<int64_t>(n) + tl.t0 + o1;
        const int64_t tb = (tl.s * n + tl.t0) * static_cast<int64_t>(w) + tl.c0 + o2;
        const int64_t xb = tl.s * static_cast<int64_t>(n) + tl.t0 + tk;
        auto c_ok = [&](int q) { return full || (cm + CSTEP * q < nc && tm < nt); };
        auto t_ok = [&](int q) { return full || (tk + 4 * q < nt && ck < nc); };
        const bool col = full || ck < nc;
        const float wv = col ? Wl[tl.c0 + ck] : 0.0f;
        const float bv = (col && bl) ? bl[tl.c0 + ck] : 0.0f;
        float v[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = t_ok(q) ? x[xb + 4 * q] : 0.0f;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            v[q] = __builtin_fmaf(v[q], wv, bv);
            if constexpr (FQ == 1) v[q] = x2_fake_quant_inv(v[q], fq.scale, inv.inv, inv.ok, fq.zpf);
            else if constexpr (FQ == 3) v[q] = log2_snap(v[q], fq.scale, steps);
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (t_ok(q)) {
                h[tb + q * d2] = v[q];
                tile[ck][tk + 4 * q] = v[q];
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (c_ok(q)) hc[cb + q * d1] = tile[cm + CSTEP * q][tm];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Radix-2 FFT of one channel held by one wave in LDS (fft.cpp:34-68).
// ---------------------------------------------------------------------------

// A wave's LDS buffer holds element e at slot e + e / 8: a pass's stores
// and the next pass's loads (groups spaced 1, 8 or 64 apart) then fall on
// distinct banks, where the unpadded layout put 4 to 8 lanes of a phase on
// one bank.
__device__ __forceinline__ int fft_slot(int e) { return e + (e >> 3); }
__host__ __device__ constexpr int fft_buf_len(int n) { return n + (n >> 3); }
__device__ __forceinline__ int bit_rev(int i, int log2n) {
    return log2n == 0 ? 0 : static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(i)) >> (32 - log2n));
}

// std::complex<float> product as the reference build computes it.
__device__ __forceinline__ float2 cmul_ref(float2 x, float2 w) {
    return make_float2(__builtin_fmaf(x.x, w.x, -(x.y * w.y)), __builtin_fmaf(x.x, w.y, x.y * w.x));
}

// The stages of fft.cpp:50-64, P at a time: a pass takes the G = 2^P
// elements of a group (spaced h0 apart in the bit-reversed array) into
// registers and runs the butterflies of the stages with halves h0 .. 2^(P-1)
// h0 on them -- the same butterflies, in the same order per element, as
// the radix-2 loop.  Element e of the group at position base + e h0 sits at
// local index kk + (e mod 2^(st+1)) h0 of its stage-st block, so its twiddle
// is tw[h - 1 + kk + (e mod 2^st) h0].
//   SRC 0: LDS buf; 1: the channel's real input, bit-reversed on load;
//          2: the mixed spectrum, bins above n/2 the conjugates of those
//             below (fft.cpp:86-96), bins >= modes the fill value below
//             n/2 and its conjugate above ((0, 0) and (0, -0) in 1-D);
//          3: a strided complex column, rows >= src_rows (0, 0);
//   DST 0: LDS buf; 1: bins < modes to the kept spectrum; 2: real parts
//          times 1/n to the channel's output; 3: rows < dst_rows to a
//          strided complex column, times 1/n when `scale`.
struct FftIo {
    float2* buf;
    const float2* tw;
    const float* src_real;
    const float2* src_spec;
    float2* dst_spec;
    float* dst_real;
    int n;
    int log2n;
    int modes;
    float inv_n;
    float fill_re, fill_im;
    int src_stride, src_rows;
    int dst_stride, dst_rows;
    bool scale;
    // Natural-order outputs the caller keeps (0: all).  After a stage of
    // block size B, position q feeds a kept output only if q mod B < keep, so
    // a pass skips its groups whose in-block offset is keep or more: the
    // kept outputs come from the same butterflies in the same order.
    int keep;
};

template <int SRC>
__device__ __forceinline__ float2 fft_load(const FftIo& io, int e) {
    if constexpr (SRC == 0) {
        return io.buf[fft_slot(e)];
    } else {
        const int k = bit_rev(e, io.log2n);
        if constexpr (SRC == 1) {
            return make_float2(io.src_real[k], 0.0f);
        } else if constexpr (SRC == 2) {
            const int nh = io.n >> 1;
            if (k <= nh) {
                if (k < io.modes) return io.src_spec[k];
                return make_float2(io.fill_re, io.fill_im);
            }
            const int kk = io.n - k;
            if (kk < io.modes) {
                const float2 v = io.src_spec[kk];
                return make_float2(v.x, -v.y);
            }
            return make_float2(io.fill_re, -io.fill_im);
        } else {
            return k < io.src_rows ? io.src_spec[static_cast<int64_t>(k) * io.src_stride] : make_float2(0.0f, 0.0f);
        }
    }
}

template <int DST>
__device__ __forceinline__ void fft_store(const FftIo& io, int e, float2 v) {
    if constexpr (DST == 0) {
        io.buf[fft_slot(e)] = v;
    } else if constexpr (DST == 1) {
        if (e < io.modes) io.dst_spec[e] = v;
    } else if constexpr (DST == 2) {
        io.dst_real[e] = v.x * io.inv_n;
    } else {
        if (e < io.dst_rows)
            io.dst_spec[static_cast<int64_t>(e) * io.dst_stride] = io.scale ? make_float2(v.x * io.inv_n, v.y * io.inv_n) : v;
    }
}

template <int P, int SRC, int DST>
__device__ __forceinline__ void fft_pass(const FftIo& io, int h0, int lane) {
    constexpr int G = 1 << P;
    const int ngroups = io.n >> P;
    const int lh0 = __builtin_ctz(static_cast<unsigned>(h0));
    // Offsets kept per block of h0 groups, and the groups that feed a kept
    // output (all of them unless io.keep < h0).
    const int kkn = (io.keep > 0 && io.keep < h0) ? io.keep : h0;
    const int nneed = (ngroups >> lh0) * kkn;
    for (int g = lane; g < nneed; g += 64) {
        const int gq = kkn == h0 ? g : (g / kkn) * h0 + g % kkn;
        const int kk = gq & (h0 - 1);
        const int base = ((gq >> lh0) << (lh0 + P)) + kk;
        float2 v[G];
#pragma unroll
        for (int e = 0; e < G; ++e) v[e] = fft_load<SRC>(io, base + e * h0);
#pragma unroll
        for (int st = 0; st < P; ++st) {
            const int span = 1 << st;
            const int h = h0 << st;
#pragma unroll
            for (int e = 0; e < G; ++e) {
                if (e & span) continue;
                const float2 w = io.tw[h - 1 + kk + (e & (span - 1)) * h0];
                const float2 t = cmul_ref(v[e + span], w);
                const float2 u = v[e];
                v[e] = make_float2(u.x + t.x, u.y + t.y);
                v[e + span] = make_float2(u.x - t.x, u.y - t.y);
            }
        }
#pragma unroll
        for (int e = 0; e < G; ++e) fft_store<DST>(io, base + e * h0, v[e]);
    }
}

template <int P, int SRC>
__device__ __forceinline__ void fft_pass_to(const FftIo& io, int h0, int lane, bool last, int dst_last) {
    if (!last) fft_pass<P, SRC, 0>(io, h0, lane);
    else if (dst_last == 1) fft_pass<P, SRC, 1>(io, h0, lane);
    else if (dst_last == 2) fft_pass<P, SRC, 2>(io, h0, lane);
    else fft_pass<P, SRC, 3>(io, h0, lane);
}

// The whole transform of one channel by one wave: the first pass reads the
// source (SRC), the last writes the destination (dst_last), the others go
// through the wave's LDS buffer.
template <int SRC>
__device__ __forceinline__ void fft_run(const FftIo& io, int lane, int dst_last) {
    const int L = io.log2n;
    if (L == 0) {
        if (lane != 0) return;
        const float2 v = fft_load<SRC>(io, 0);
        if (dst_last == 1) fft_store<1>(io, 0, v);
        else if (dst_last == 2) fft_store<2>(io, 0, v);
        else fft_store<3>(io, 0, v);
        return;
    }
    int done = 0, h0 = 1;
    while (done < L) {
        const int P = (L - done) >= 3 ? 3 : (L - done);
        const bool last = done + P == L;
        if (done == 0) {
            if (P == 3) fft_pass_to<3, SRC>(io, h0, lane, last, dst_last);
            else if (P == 2) fft_pass_to<2, SRC>(io, h0, lane, last, dst_last);
            else fft_pass_to<1, SRC>(io, h0, lane, last, dst_last);
        } else {
            if (P == 3) fft_pass_to<3, 0>(io, h0, lane, last, dst_last);
            else if (P == 2) fft_pass_to<2, 0>(io, h0, lane, last, dst_last);
            else fft_pass_to<1, 0>(io, h0, lane, last, dst_last);
        }
        wave_sync();
        done += P;
        h0 <<= P;
    }
}

// Stage the block's twiddle table in LDS (TWL) before any wave leaves.
template <bool TWL>
__device__ __forceinline__ const float2* block_twiddles(float2* smem, const float* tw, int n) {
    if constexpr (TWL) {
        const float2* src = reinterpret_cast<const float2*>(tw);
        for (int i = threadIdx.x; i < n - 1; i += blockDim.x) smem[i] = src[i];
        __syncthreads();
        return smem;
    } else {
        return reinterpret_cast<const float2*>(tw);
    }
}

// Forward FFT of channel c of sample s (channel-major hc), bins 0 .. modes-1 to spec.
template <int WPB, bool TWL>
__global__ __launch_bounds__(64 * WPB) void k_rfft_modes(SpecArgs a, int64_t nlogical) {
    extern __shared__ float2 fsm[];
    const int n = a.n;
    const float2* tw = block_twiddles<TWL>(fsm, a.tw_fwd, n);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t lb = xcd_block(nlogical);
    if (lb < 0) return;
    const int64_t item = lb * WPB + wid;
    if (item >= a.samples * a.w) return;
    FftIo io{};
    io.buf = fsm + (TWL ? n : 0) + static_cast<int64_t>(wid) * fft_buf_len(n);
    io.tw = tw;
    io.src_real = a.hc + item * n;
    io.dst_spec = reinterpret_cast<float2*>(a.spec) + item * a.modes;
    io.n = n;
    io.log2n = a.log2n;
    io.modes = a.modes;
    io.keep = a.modes;
    fft_run<1>(io, lane, 1);
}

// Channel mix (fno.cpp:176-198): out[s][wo][m] = sum over wi, in order, of
// H[s][wi][m] * W[wi][wo][m] with the reference build's fused terms; the
// weights are held (m, wi, wo) so a wave's 64 output channels read 256
// contiguous bytes per wi.
__global__ __launch_bounds__(256) void k_spec_mix(SpecArgs a, const float* mix_r, const float* mix_i,
                                                  float* spec_out) {
    const int m = blockIdx.z;
    const int w = a.w, modes = a.modes;
    const int wo = blockIdx.y * 64 + (threadIdx.x & 63);
    const int64_t s = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wo >= w || s >= a.samples) return;
    const float2* H = reinterpret_cast<const float2*>(a.spec) + s * w * modes + m;
    const float* Wr = mix_r + static_cast<int64_t>(m) * w * w + wo;
    const float* Wi = mix_i + static_cast<int64_t>(m) * w * w + wo;
    float sr = 0.0f, si = 0.0f;
    // The loads of 16 input channels are issued together (one at a time,
    // each would wait out an L2 round trip); the sums still take the
    // channels one by one, in order.
    constexpr int KU = 16;
    for (int k0 = 0; k0 < w; k0 += KU) {
        float2 hv[KU];
        float wr[KU], wim[KU];
#pragma unroll
        for (int j = 0; j < KU; ++j) {
            const int k = k0 + j < w ? k0 + j : w - 1;    // clamped: only read, never summed
            hv[j] = H[static_cast<int64_t>(k) * modes];
            wr[j] = Wr[static_cast<int64_t>(k) * w];
            wim[j] = Wi[static_cast<int64_t>(k) * w];
        }
#pragma unroll
        for (int j = 0; j < KU; ++j) {
            if (k0 + j < w) {
                sr = sr + __builtin_fmaf(-wim[j], hv[j].y, hv[j].x * wr[j]);
                si = si + __builtin_fmaf(wr[j], hv[j].y, hv[j].x * wim[j]);
            }
        }
    }
    reinterpret_cast<float2*>(spec_out)[(s * w + wo) * modes + m] = make_float2(sr, si);
}

// The same mix for w <= 64 with the operands staged in LDS first: a block
// takes mode m (blockIdx.y) for four samples (one per wave), loads the
// mode's w x w weights and the four samples' w input bins with all of its
// loads in flight at once, then sums from LDS in the same order and fused
// forms as k_spec_mix (lane = output channel).
// W: the channel count when fixed at compile time (64), else 0.
template <int W>
__global__ __launch_bounds__(256) void k_spec_mix_lds(SpecArgs a, const float* mix_r, const float* mix_i,
                                                      float* spec_out) {
    __shared__ float wr_s[64 * 64], wi_s[64 * 64];
    __shared__ float2 h_s[4][64];
    const int m = blockIdx.y;
    const int w = W ? W : a.w, modes = a.modes, ww = w * w;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t s0 = static_cast<int64_t>(blockIdx.x) * 4;
    const float* Wr = mix_r + static_cast<int64_t>(m) * ww;
    const float* Wi = mix_i + static_cast<int64_t>(m) * ww;
    // Every load of the stage is issued before the first is waited for.
    float vr[16], vi[16];
    float2 hin = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < ww) {
            vr[j] = Wr[i];
            vi[j] = Wi[i];
        }
    }
    const int64_t s = s0 + wid;
    const bool live = lane < w && s < a.samples;
    if (live) hin = reinterpret_cast<const float2*>(a.spec)[(s * w + lane) * modes + m];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < ww) {
            wr_s[i] = vr[j];
            wi_s[i] = vi[j];
        }
    }
    h_s[wid][lane] = hin;
    __syncthreads();
    if (!live) return;
    float sr = 0.0f, si = 0.0f;
#pragma unroll 16
    for (int k = 0; k < w; ++k) {
        const float2 hv = h_s[wid][k];
        const float wr = wr_s[k * w + lane], wim = wi_s[k * w + lane];
        sr = sr + __builtin_fmaf(-wim, hv.y, hv.x * wr);
        si = si + __builtin_fmaf(wr, hv.y, hv.x * wim);
    }
    reinterpret_cast<float2*>(spec_out)[(s * w + lane) * modes + m] = make_float2(sr, si);
}

// Inverse FFT (fft.cpp:86-100) of output channel wo of sample s from the
// mixed spectrum, written channel-major to x1c.
template <int WPB, bool TWL>
__global__ __launch_bounds__(64 * WPB) void k_irfft(SpecArgs a, const float* spec_mixed, int64_t nlogical) {
    extern __shared__ float2 fsm[];
    const int n = a.n;
    const float2* tw = block_twiddles<TWL>(fsm, a.tw_inv, n);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t lb = xcd_block(nlogical);
    if (lb < 0) return;
    const int64_t item = lb * WPB + wid;
    if (item >= a.samples * a.w) return;
    FftIo io{};
    io.buf = fsm + (TWL ? n : 0) + static_cast<int64_t>(wid) * fft_buf_len(n);
    io.tw = tw;
    io.src_spec = reinterpret_cast<const float2*>(spec_mixed) + item * a.modes;
    io.dst_real = a.x1c + item * n;
    io.n = n;
    io.log2n = a.log2n;
    io.modes = a.modes;
    io.inv_n = a.inv_n;
    if (a.fill) {
        const float2 f = a.fill[item % a.fill_period];
        io.fill_re = f.x;
        io.fill_im = f.y;
    }
    fft_run<2>(io, lane, 2);
}

// ---------------------------------------------------------------------------
// Row transforms of a fixed length n = 2^LOG2N (64 .. 1024): the butterflies
// of fft_pass, in the same order per element, with every index known at
// compile time.  A wave takes R = 64 G1 / n rows at a time, so that its
// first pass (G1 = 2^P1 elements per lane) fills all 64 lanes; it keeps
// taking row sets until the rows run out, and loads the next set's inputs
// before it transforms the current one.  Lane buffers in LDS hold element e
// of a row at slot e + (e >> SL), rows STRIDE slots apart (no bank
// conflicts at n = 256).
// ---------------------------------------------------------------------------
template <int LOG2N> struct RowFftPlan;
template <> struct RowFftPlan<6> { static constexpr int P1 = 3, P2 = 3, P3 = 0, SL = 3, STRIDE = 72, WPB = 4; };
template <> struct RowFftPlan<7> { static constexpr int P1 = 4, P2 = 3, P3 = 0, SL = 4, STRIDE = 136, WPB = 4; };
template <> struct RowFftPlan<8> { static constexpr int P1 = 4, P2 = 4, P3 = 0, SL = 4, STRIDE = 272, WPB = 4; };
template <> struct RowFftPlan<9> { static constexpr int P1 = 3, P2 = 3, P3 = 3, SL = 3, STRIDE = 576, WPB = 8; };
template <> struct RowFftPlan<10> { static constexpr int P1 = 4, P2 = 3, P3 = 3, SL = 4, STRIDE = 1088, WPB = 8; };

template <int LOG2N>
struct RowFft {
    using PL = RowFftPlan<LOG2N>;
    static constexpr int N = 1 << LOG2N, G1 = 1 << PL::P1, R = 64 * G1 / N;
    static constexpr int WAVE_SLOTS = R * PL::STRIDE;
    __device__ static __forceinline__ int slot(int row, int e) { return row * PL::STRIDE + e + (e >> PL::SL); }
};

constexpr int ilog2c(int v) { return v <= 1 ? 0 : 1 + ilog2c(v >> 1); }
constexpr int bitrevc(int v, int bits) { return bits == 0 ? 0 : ((v & 1) << (bits - 1)) | bitrevc(v >> 1, bits - 1); }

// The P stages of one group on registers (fft_pass's loop body).
template <int P, int H0>
__device__ __forceinline__ void row_stages(float2 (&v)[1 << P], const float2* tw, int kk) {
    constexpr int G = 1 << P;
#pragma unroll
    for (int st = 0; st < P; ++st) {
        const int span = 1 << st;
        const int h = H0 << st;
#pragma unroll
        for (int e = 0; e < G; ++e) {
            if (e & span) continue;
            const float2 w = tw[h - 1 + kk + (e & (span - 1)) * H0];
            const float2 t = cmul_ref(v[e + span], w);
            const float2 u = v[e];
            v[e] = make_float2(u.x + t.x, u.y + t.y);
            v[e + span] = make_float2(u.x - t.x, u.y - t.y);
        }
    }
}

// A pass after the first: groups of 2^P elements spaced H0 apart, read from
// and (unless LAST) written back to the wave's buffer.  PRUNE: groups whose
// offset kk in their block is io.keep or more feed no kept output and are
// skipped; E0 (io.keep <= H0): only element 0 of a group feeds one, and
// only it is kept.  LAST hands the kept outputs (position < io.keep when
// PRUNE) of item item0 + row to io.store.
template <int LOG2N, int P, int H0, bool PRUNE, bool E0, bool LAST, class IO>
__device__ __forceinline__ void row_pass(float2* buf, const float2* tw, int lane, int64_t item0, const IO& io) {
    using F = RowFft<LOG2N>;
    constexpr int G = 1 << P, GPR = F::N / G, TOT = F::R * GPR, LH0 = ilog2c(H0);
#pragma unroll
    for (int it = 0; it < (TOT + 63) / 64; ++it) {
        const int q = it * 64 + lane;
        if (TOT % 64 != 0 && q >= TOT) continue;
        const int row = q / GPR, g = q % GPR;
        const int kk = g & (H0 - 1);
        const int base = ((g >> LH0) << (LH0 + P)) + kk;
        if (PRUNE && kk >= io.keep) continue;
        float2 v[G];
#pragma unroll
        for (int e = 0; e < G; ++e) v[e] = buf[F::slot(row, base + e * H0)];
        row_stages<P, H0>(v, tw, kk);
        if constexpr (!LAST) {
            if constexpr (E0) {
                buf[F::slot(row, base)] = v[0];
            } else {
#pragma unroll
                for (int e = 0; e < G; ++e) buf[F::slot(row, base + e * H0)] = v[e];
            }
        } else {
            const int64_t item = item0 + row;
            if (item >= io.items) continue;
            const int64_t ob = io.out_base(item);
            if constexpr (E0) {
                io.store(ob, base, v[0]);
            } else {
#pragma unroll
                for (int e = 0; e < G; ++e)
                    if (!PRUNE || base + e * H0 < io.keep) io.store(ob, base + e * H0, v[e]);
            }
        }
    }
}

// Passes 2 (and 3) of a row set, after the first pass has filled the buffer.
template <int LOG2N, bool PRUNE, bool E0, class IO>
__device__ __forceinline__ void row_rest(float2* buf, const float2* tw, int lane, int64_t item0, const IO& io) {
    using PL = RowFftPlan<LOG2N>;
    constexpr int H2 = 1 << PL::P1;
    wave_sync();
    if constexpr (PL::P3 == 0) {
        row_pass<LOG2N, PL::P2, H2, PRUNE, E0, true>(buf, tw, lane, item0, io);
    } else {
        row_pass<LOG2N, PL::P2, H2, PRUNE, E0, false>(buf, tw, lane, item0, io);
        wave_sync();
        row_pass<LOG2N, PL::P3, (H2 << PL::P2), PRUNE, E0, true>(buf, tw, lane, item0, io);
    }
    wave_sync();
}

template <int N>
__device__ __forceinline__ const float2* stage_row_twiddles(float2* smem, const float* tw) {
    const float2* src = reinterpret_cast<const float2*>(tw);
    for (int i = threadIdx.x; i < N - 1; i += blockDim.x) smem[i] = src[i];
    __syncthreads();
    return smem;
}

// The persistent row-set loop: a wave loads the inputs of the set NB - 1
// ahead into one of NB register buffers while it transforms the set held in
// another (the buffers rotate, so no copy between them).  Every load is
// issued whether its set exists or not (past the end, the last set's rows
// are read again and dropped): loads under no branch let the compiler wait
// for one buffer's loads only, with the others' still in flight.
template <int NB, typename Buf, typename Load, typename Run>
__device__ __forceinline__ void row_sets(int64_t first, int64_t stride, int64_t nsets, Buf (&b)[NB],
                                         const Load& load, const Run& run) {
    const int64_t last = nsets - 1;
    int64_t set = first;
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) {
        const int64_t s = set + i * stride;
        load(s < last ? s : last, b[i]);
    }
    while (set < nsets) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int64_t pre = set + (NB - 1) * stride;
            load(pre < last ? pre : last, b[(i + NB - 1) % NB]);
            __builtin_amdgcn_sched_barrier(0);   // the loads go out before the transform
            run(set, b[i]);
            set += stride;
            if (set >= nsets) break;
        }
    }
}

// The fixed-length transform of `items` sequences, R per wave at a time.
// IO supplies the sequences and takes the results: IO::Lane, the lane's
// constants (from its first-pass row and bit-reversed group index);
// IO::In, one set's prefetched inputs; load(lane, set, item, in);
// first(lane, in, v), the first pass's G1 inputs (element e = input
// bitrev(g G1 + e) = bitrev_P1(e) 2^LB + bitrev_LB(g)); out_base(item) and
// store(base, position, value) for the kept outputs; DEPTH, the sets in
// flight (loaded DEPTH - 1 ahead).
template <int LOG2N, bool PRUNE, bool E0, class IO>
__global__ __launch_bounds__(64 * RowFftPlan<LOG2N>::WPB) void k_fft_fixed(IO io, int64_t nsets) {
    using F = RowFft<LOG2N>;
    constexpr int N = F::N, G1 = F::G1, R = F::R, GPR1 = N / G1, LB = LOG2N - RowFftPlan<LOG2N>::P1;
    extern __shared__ float2 fsm[];
    const float2* tw = stage_row_twiddles<N>(fsm, io.tw);
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    float2* buf = fsm + N + wid * F::WAVE_SLOTS;
    const int row1 = lane / GPR1, g1 = lane % GPR1;
    const int rb = static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(g1)) >> (32 - LB));
    const typename IO::Lane ln = io.lane_setup(row1, rb);
    using In = typename IO::In;
    auto load = [&](int64_t set, In& d) { io.load(ln, set, set * R + row1, d); };
    auto run = [&](int64_t set, const In& d) {
        float2 v[G1];
        io.first(ln, d, v, reinterpret_cast<float*>(buf), lane);
        row_stages<RowFftPlan<LOG2N>::P1, 1>(v, tw, 0);
#pragma unroll
        for (int e = 0; e < G1; ++e) buf[F::slot(row1, g1 * G1 + e)] = v[e];
        row_rest<LOG2N, PRUNE, E0>(buf, tw, lane, set * R, io);
    };
    In b[IO::DEPTH] = {};
    constexpr int WPB = RowFftPlan<LOG2N>::WPB;
    row_sets<IO::DEPTH>(static_cast<int64_t>(blockIdx.x) * WPB + wid, static_cast<int64_t>(gridDim.x) * WPB, nsets, b,
                        load, run);
}

template <int LOG2N> struct FftConsts {
    static constexpr int N = 1 << LOG2N, P1 = RowFftPlan<LOG2N>::P1, G1 = 1 << P1, LB = LOG2N - P1;
    __device__ static __forceinline__ int bin(int rb, int e) { return (bitrevc(e, P1) << LB) + rb; }
};

// Row FFTs of hc (k_rfft_modes's results): real rows of n points, bins
// < keep (= modes) to spec.
template <int LOG2N>
struct RowFwdIO {
    using C = FftConsts<LOG2N>;
    static constexpr int DEPTH = 2;
    const float* hc;
    float2* spec;
    const float* tw;
    int64_t items;
    int keep;
    struct Lane { int rb, row, c; };
    struct In { float v[C::G1]; };
    __device__ Lane lane_setup(int row1, int rb) const {
        // The natural-order load role: row1, and the lane's 16-byte column
        // within the row's first-pass lanes.
        return Lane{rb, row1, static_cast<int>(threadIdx.x & 63) % (C::N / C::G1)};
    }
    // The row is read in natural order, 16 bytes a lane (lane (r, c) of the
    // set's row r takes floats 64 q + 4 c .. + 3, q < G1 / 4: whole 256-byte
    // runs per instruction), and put in first-pass order through the wave's
    // buffer (rows RS floats apart, so that the four rows' gathers fall on
    // distinct banks).
    static constexpr int Q = C::G1 / 4, RS = C::N + 16;
    static_assert(C::G1 % 4 == 0 && RowFft<LOG2N>::R * RS <= 2 * RowFft<LOG2N>::WAVE_SLOTS, "row scratch");
    __device__ void load(const Lane& ln, int64_t, int64_t item, In& d) const {
        // A row past the end reads the last row: transformed, never stored.
        const v4f* src = reinterpret_cast<const v4f*>(hc + (item < items ? item : items - 1) * C::N) + ln.c;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const v4f x = src[q * (C::N / 4 / Q)];
            d.v[4 * q] = x[0];
            d.v[4 * q + 1] = x[1];
            d.v[4 * q + 2] = x[2];
            d.v[4 * q + 3] = x[3];
        }
    }
    __device__ void first(const Lane& ln, const In& d, float2 (&v)[C::G1], float* scratch, int) const {
        float* row = scratch + ln.row * RS;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            *reinterpret_cast<v4f*>(row + q * (C::N / Q) + 4 * ln.c) =
                v4f{d.v[4 * q], d.v[4 * q + 1], d.v[4 * q + 2], d.v[4 * q + 3]};
        wave_sync();
#pragma unroll
        for (int e = 0; e < C::G1; ++e) v[e] = make_float2(row[C::bin(ln.rb, e)], 0.0f);
        wave_sync();
    }
    __device__ int64_t out_base(int64_t item) const { return item * keep; }
    __device__ void store(int64_t ob, int pos, float2 v) const { spec[ob + pos] = v; }
};

// Inverse row FFTs (k_irfft's results): the bins of row item are its
// `modes` mixed bins, bins modes .. n/2 the item's fill value, bins above
// n/2 the conjugates of those below; real parts times 1 / n to x1c.  With
// FEW (modes <= 2^LB) only a lane's elements 0 and G1 - 1 can be mixed bins.
template <int LOG2N, bool FEW>
struct RowInvIO {
    using C = FftConsts<LOG2N>;
    static constexpr int G1 = C::G1, DEPTH = 2;
    const float2* spec;
    float* out;
    const float2* fill;
    const float* tw;
    int64_t items;
    int keep;              // unused (nothing pruned)
    int modes;
    int fill_period;
    float inv_n;
    static constexpr int R = RowFft<LOG2N>::R;
    // The lane's mixed elements (bit e) and the byte offsets of their bins
    // in the set's mixed bins.
    struct Lane { uint32_t off[G1]; uint32_t mixed; int rb; };
    struct In { float2 v[FEW ? 2 : G1]; float2 f; };
    __device__ Lane lane_setup(int row1, int rb) const {
        Lane ln{};
        ln.rb = rb;
#pragma unroll
        for (int e = 0; e < G1; ++e) {
            const int k = C::bin(rb, e);
            const bool up = k > C::N / 2;
            const bool mx = up ? C::N - k < modes : k < modes;
            ln.mixed |= mx ? 1u << e : 0u;
            ln.off[e] = static_cast<uint32_t>(row1 * modes + (mx ? (up ? C::N - k : k) : 0)) * 8u;
        }
        return ln;
    }
    __device__ void load(const Lane& ln, int64_t set, int64_t item, In& d) const {
        d.f = make_float2(0.0f, 0.0f);
        if (item >= items) return;    // a row past the end: transformed, never stored
        if (fill) {
            const bool pow2 = (fill_period & (fill_period - 1)) == 0;
            d.f = fill[pow2 ? (item & (fill_period - 1)) : item % fill_period];
        }
        const char* src = reinterpret_cast<const char*>(spec + set * R * modes);
        if constexpr (FEW) {
            if (ln.mixed & 1u) d.v[0] = *reinterpret_cast<const float2*>(src + ln.off[0]);
            if ((ln.mixed >> (G1 - 1)) & 1u) d.v[1] = *reinterpret_cast<const float2*>(src + ln.off[G1 - 1]);
        } else {
#pragma unroll
            for (int e = 0; e < G1; ++e)
                if ((ln.mixed >> e) & 1u) d.v[e] = *reinterpret_cast<const float2*>(src + ln.off[e]);
        }
    }
    __device__ void first(const Lane& ln, const In& d, float2 (&v)[G1], float*, int) const {
#pragma unroll
        for (int e = 0; e < G1; ++e) {
            float2 x = d.f;
            if constexpr (FEW) {
                if (e == 0 && (ln.mixed & 1u)) x = d.v[0];
                if (e == G1 - 1 && ((ln.mixed >> e) & 1u)) x = d.v[1];
            } else {
                if ((ln.mixed >> e) & 1u) x = d.v[e];
            }
            v[e] = C::bin(ln.rb, e) > C::N / 2 ? make_float2(x.x, -x.y) : x;
        }
    }
    __device__ int64_t out_base(int64_t item) const { return item * C::N; }
    __device__ void store(int64_t ob, int pos, float2 v) const { out[ob + pos] = v.x * inv_n; }
};

// Column FFTs (k_cfft_cols's results): item = plane * mw + j is column j of
// a plane of rows x mw complex values (fft.cpp:111-122, :131-141).  Forward:
// h rows in, rows < keep (= mh) out.  Inverse: rows < mh in (the rest
// zero), all h rows out times 1 / h; FEW (mh <= 2^LB): only a lane's
// element 0 can be a stored row.
template <int LOG2N, bool INV, bool FEW>
struct ColIO {
    using C = FftConsts<LOG2N>;
    static constexpr int G1 = C::G1, DEPTH = 2;
    const float2* in;
    float2* out;
    const float* tw;
    int64_t items;
    int keep;              // forward: mh
    int mw;
    int mh;
    float inv_h;
    struct Lane { int rb; };
    struct In { float2 v[INV && FEW ? 1 : G1]; };
    __device__ Lane lane_setup(int, int rb) const { return Lane{rb}; }
    // Column item's element (plane * rows + r) * mw + j for r = 0: plane =
    // item / mw, j = item % mw (items < 2^32, checked at launch).
    __device__ int64_t col_base(int64_t item, int rows) const {
        const uint32_t it = static_cast<uint32_t>(item), um = static_cast<uint32_t>(mw);
        const uint32_t plane = it / um, j = it - plane * um;
        return static_cast<int64_t>(plane) * rows * mw + j;
    }
    __device__ void load(const Lane& ln, int64_t, int64_t item, In& d) const {
        // A column past the end reads the last column: transformed, never stored.
        const float2* src = in + col_base(item < items ? item : items - 1, INV ? mh : C::N);
        if constexpr (INV && FEW) {
            d.v[0] = ln.rb < mh ? src[static_cast<int64_t>(ln.rb) * mw] : make_float2(0.0f, 0.0f);
        } else {
#pragma unroll
            for (int e = 0; e < G1; ++e) {
                const int k = C::bin(ln.rb, e);
                d.v[e] = (!INV || k < mh) ? src[static_cast<int64_t>(k) * mw] : make_float2(0.0f, 0.0f);
            }
        }
    }
    __device__ void first(const Lane&, const In& d, float2 (&v)[G1], float*, int) const {
#pragma unroll
        for (int e = 0; e < G1; ++e) {
            if constexpr (INV && FEW) v[e] = e == 0 ? d.v[0] : make_float2(0.0f, 0.0f);
            else v[e] = d.v[e];
        }
    }
    __device__ int64_t out_base(int64_t item) const { return col_base(item, INV ? C::N : mh); }
    __device__ void store(int64_t ob, int pos, float2 v) const {
        out[ob + static_cast<int64_t>(pos) * mw] = INV ? make_float2(v.x * inv_h, v.y * inv_h) : v;
    }
};

// Column FFT (fft.cpp:48-68 down column j of a plane, fft.cpp:111-122 /
// :131-141): item = plane * mw + j.
template <int WPB, bool TWL, bool INV>
__global__ __launch_bounds__(64 * WPB) void k_cfft_cols(ColArgs a, int64_t nlogical) {
    extern __shared__ float2 fsm[];
    const int n = a.h;
    const float2* tw = block_twiddles<TWL>(fsm, a.tw, n);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t lb = xcd_block(nlogical);
    if (lb < 0) return;
    const int64_t item = lb * WPB + wid;
    if (item >= a.planes * a.mw) return;
    const int64_t plane = item / a.mw;
    const int j = static_cast<int>(item % a.mw);
    const int in_rows = INV ? a.mh : a.h, out_rows = INV ? a.h : a.mh;
    FftIo io{};
    io.buf = fsm + (TWL ? n : 0) + static_cast<int64_t>(wid) * fft_buf_len(n);
    io.tw = tw;
    io.src_spec = reinterpret_cast<const float2*>(a.in) + plane * in_rows * a.mw + j;
    io.src_stride = a.mw;
    io.src_rows = in_rows;
    io.dst_spec = reinterpret_cast<float2*>(a.out) + plane * out_rows * a.mw + j;
    io.dst_stride = a.mw;
    io.dst_rows = out_rows;
    io.n = n;
    io.log2n = a.log2h;
    io.inv_n = a.inv_h;
    io.scale = INV;
    io.keep = INV ? 0 : out_rows;
    fft_run<3>(io, lane, 3);
}

// ---------------------------------------------------------------------------
// Layer tail.
// ---------------------------------------------------------------------------

// The snaps read their step tables from LDS, one entry per element
// (snap_exponent_binade); the runtime checks the one-step-per-binade layout
// of the table at creation.
//
// The tail of fno.cpp:572-660 (the x2 fake-quant, h = act(x1 + x2)) and the
// next layer's input fake-quant (fno.cpp:488-501).  The launch's forms are
// template parameters: KIND, the x2 fake-quant (0 none, 1 per tensor, 2 per
// position, 3 log2 snap); ACT (RT_ACT_NONE, RT_ACT_RELU or RT_ACT_GELU);
// FQN, the next layer's input fake-quant (0 off, 1 per tensor, 3 log2 snap).  Chosen per element at run time, they put every element's
// loads, stores and 64-bit index products behind uniform branches of their
// own.  Thread x holds, per tile, channel-major elements (channel x / TT +
// (256 / TT) q, token x % TT) and token-major elements (token x / 64 + 4 q,
// channel x % 64), q = 0 .. PER - 1: their offsets are the thread's fixed
// offset plus q times a per-launch stride.  Each thread's elements of a tile
// are loaded together (every load of a phase issued before the first is
// waited for); the stores follow all of the phase's results.
template <int KIND, int ACT, int FQN>
__device__ __forceinline__ float post_element(float x1, float x2, const PostArgs& a, const ScaleInv& inv_x2,
                                              const ScaleInv& inv_next, const float* thr_x2,
                                              const float* thr_next, float pscale, float pzp) {
    if constexpr (KIND == 1) x2 = x2_fake_quant_inv(x2, a.scale, inv_x2.inv, inv_x2.ok, a.zpf);
    else if constexpr (KIND == 2) x2 = x2_fake_quant(x2, pscale, pzp);
    else if constexpr (KIND == 3) x2 = log2_snap(x2, a.scale, thr_x2);
    float y = x1 + x2;
    if constexpr (ACT == RT_ACT_RELU) y = y < 0.0f ? 0.0f : y;   // fno.cpp:37-40
    else if constexpr (ACT == RT_ACT_GELU) y = gelu_fast<kGeluRefine>(y);
    if constexpr (FQN == 1) y = x2_fake_quant_inv(y, a.fq_next.scale, inv_next.inv, inv_next.ok, a.fq_next.zpf);
    else if constexpr (FQN == 3) y = log2_snap(y, a.fq_next.scale, thr_next);
    return y;
}

template <int TT, int KIND, int ACT, int FQN>
__global__ __launch_bounds__(256) void k_post_rt(PostArgs a) {
    constexpr int PER = TT * 64 / 256;   // elements per thread and tile
    constexpr int CSTEP = 256 / TT;      // channel rows per block pass (channel-major)
    static_assert(PER * 256 == TT * 64 && CSTEP * TT == 256, "tile size");
    __shared__ float tx1[64][TT + 1];  // x1, then (in place, same thread) the new h
    __shared__ float thr_x2[16], thr_next[16];
    const int n = a.n, w = a.w;
    if (threadIdx.x < 15) thr_x2[threadIdx.x] = a.thr[threadIdx.x];
    stage_steps(thr_next, a.fq_next.thr);
    const ScaleInv inv_x2 = scale_inv(a.scale), inv_next = scale_inv(a.fq_next.scale);
    const int cm = threadIdx.x / TT, tm = threadIdx.x % TT;    // channel-major: channel, token
    const int tk = threadIdx.x / 64, ck = threadIdx.x % 64;    // token-major: token, channel
    const int64_t o1 = static_cast<int64_t>(cm) * n + tm, d1 = static_cast<int64_t>(CSTEP) * n;
    const int64_t o2 = static_cast<int64_t>(tk) * w + ck, d2 = 4 * static_cast<int64_t>(w);
    Tile tl;
    for (int64_t id = blockIdx.x; tile_of<TT>(id, a.samples, n, w, tl); id += gridDim.x) {
        const int nt = n - tl.t0 < TT ? n - tl.t0 : TT;       // tokens and channels of the tile
        const int nc = w - tl.c0 < 64 ? w - tl.c0 : 64;
        const bool full = nt == TT && nc == 64;               // block-uniform
        const int64_t cb = (tl.s * w + tl.c0) * static_cast<int64_t>(n) + tl.t0 + o1;
        const int64_t tb = (tl.s * n + tl.t0) * static_cast<int64_t>(w) + tl.c0 + o2;
        auto c_ok = [&](int q) { return full || (cm + CSTEP * q < nc && tm < nt); };
        auto t_ok = [&](int q) { return full || (tk + 4 * q < nt && ck < nc); };
        // x1 (channel-major) into LDS.
        float v[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = c_ok(q) ? a.x1c[cb + q * d1] : 0.0f;
#pragma unroll
        for (int q = 0; q < PER; ++q) tx1[cm + CSTEP * q][tm] = v[q];
        __syncthreads();
        // x2 (token-major), then the tail of each element.  All results
        // before any store: a store is counted with the loads, so a wait for
        // a later load would also wait for every earlier store.
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = t_ok(q) ? a.x2[tb + q * d2] : 0.0f;
        float ps[PER], pz[PER];
        if constexpr (KIND == 2) {
            // Position (channel, token) of the reference's per-position
            // tables: index channel * n + token (rows past the tile read
            // position 0).
            const int64_t pb = static_cast<int64_t>(tl.c0 + ck) * n + tl.t0 + tk;
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int64_t p = t_ok(q) ? pb + 4 * q : 0;
                ps[q] = a.pos_scales[p];
                pz[q] = static_cast<float>(a.pos_zps[p]);
            }
        }
#pragma unroll
        for (int q = 0; q < PER; ++q)
            v[q] = post_element<KIND, ACT, FQN>(tx1[ck][tk + 4 * q], v[q], a, inv_x2, inv_next, thr_x2, thr_next,
                                                KIND == 2 ? ps[q] : 0.0f, KIND == 2 ? pz[q] : 0.0f);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (t_ok(q)) {
                a.h[tb + q * d2] = v[q];
                tx1[ck][tk + 4 * q] = v[q];
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (c_ok(q)) a.hc[cb + q * d1] = tx1[cm + CSTEP * q][tm];
        __syncthreads();
    }
}

// The INT8 local-linear layer and the tail in one pass (LayerTailArgs): on a
// 32-token x 64-channel tile, the h tile is read once (16 bytes per thread,
// token-major) and quantised with the per-tensor scale into LDS codes (the
// reciprocal fast path with the exact quotient where it is not certain, as
// k_rows64's fixed-scale form), each wave forms a 16-token x 32-channel
// block of D with two v_mfma_i32_16x16x64_i8 (weights in registers), and the
// dequantise + bias and the tail run in the MFMA result layout on x1 from
// the channel-major LDS tile, where the results replace x1 for the two
// stores.  x2 never reaches HBM: per layer 256 MB move instead of 402 MB at
// 256 x 1024 x 64.
template <int KIND, int ACT, int FQN, bool INT_EPI>
__global__ __launch_bounds__(256) void k_layer_tail(LayerTailArgs la) {
    constexpr int TT = 32, PER = TT * 64 / 256, CSTEP = 256 / TT, CODE_DW = 20;   // 64 code bytes + 16 of padding
    const PostArgs& a = la.p;
    __shared__ float tx1[64][TT + 1];   // x1, then (in place, same lane) the new h
    __shared__ uint32_t codes[TT * CODE_DW];
    __shared__ float thr_x2[16], thr_next[16];
    __shared__ float csw[64], cbias[64];
    __shared__ IntEpi cepi[INT_EPI ? 64 : 1];
    const int n = a.n;                  // w == 64, n % 32 == 0 (layer_tail_ok)
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (threadIdx.x < 15) thr_x2[threadIdx.x] = a.thr[threadIdx.x];
    if (threadIdx.x < 64) {
        const int c = threadIdx.x;
        csw[c] = la.sW[c];
        cbias[c] = la.bias ? la.bias[c] : 0.0f;
        if constexpr (INT_EPI) {
            const uint32_t* wr = reinterpret_cast<const uint32_t*>(la.W + 64 * c);
            int32_t sfull = 0;
#pragma unroll
            for (int q = 0; q < 16; ++q) sfull = sum_bytes_i8(wr[q], sfull);
            cepi[c] = int_epi_consts(F_BATCHED, 64, la.zpA, la.zpW ? la.zpW[c] : 0, la.sumW ? la.sumW[c] : 0,
                                     la.sumW != nullptr, sfull, sfull);
        }
    }
    stage_steps(thr_next, a.fq_next.thr);
    const ScaleInv inv_x2 = scale_inv(a.scale), inv_next = scale_inv(a.fq_next.scale);
    const float fixed_inv = 1.0f / la.sA;
    const bool fixed_exact = !(la.sA >= 0x1p-120f && la.sA <= 0x1p120f);
    // MFMA roles: wave wid takes tokens 16 (wid & 1) .. + 15 and channels
    // 32 (wid >> 1) .. + 31 (two 16-column tiles); lane (r, g) supplies
    // weight row 32 (wid >> 1) + 16 ct + r and code row 16 (wid & 1) + r,
    // bytes 16 g .. 16 g + 15, and receives token 16 (wid & 1) + r, channels
    // 32 (wid >> 1) + 16 ct + 4 g .. + 3.
    const int r = lane & 15, g = lane >> 4, tr = wid & 1, chh = wid >> 1;
    v4i wop[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(la.W + (32 * chh + 16 * ct + r) * 64 + 16 * g);
        wop[ct] = v4i{static_cast<int>(src[0]), static_cast<int>(src[1]), static_cast<int>(src[2]),
                      static_cast<int>(src[3])};
    }
    // Load and store roles as the tail's: channel-major (channel x / 32 +
    // 8 q, token x % 32), token-major (token x / 64 + 4 q, channel x % 64);
    // the h tile's loads: token x / 16 + 16 q, channels 4 (x % 16) .. + 3.
    const int cm = threadIdx.x / TT, tm = threadIdx.x % TT, tk = threadIdx.x / 64, ck = threadIdx.x % 64;
    const int hq_t = threadIdx.x / 16, hq_c = 4 * (threadIdx.x % 16);
    const int64_t o1 = static_cast<int64_t>(cm) * n + tm, d1 = static_cast<int64_t>(CSTEP) * n;
    Tile tl;
    for (int64_t id = blockIdx.x; tile_of<TT>(id, a.samples, n, 64, tl); id += gridDim.x) {
        const int64_t cb = tl.s * 64 * static_cast<int64_t>(n) + tl.t0 + o1;
        const int64_t tb = (tl.s * n + tl.t0) * 64;
        v4f hv[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) hv[q] = *reinterpret_cast<const v4f*>(a.h + tb + (hq_t + 16 * q) * 64 + hq_c);
        float xv[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) xv[q] = a.x1c[cb + q * d1];
#pragma unroll
        for (int q = 0; q < PER; ++q) tx1[cm + CSTEP * q][tm] = xv[q];
        // Codes of the h tile (QuantiseActivation with the layer's scale).
        uint32_t badm = 0;
        int32_t cq[2][4];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bool bad;
                cq[q][e] = quant_i8_fixed_near(hv[q][e], fixed_inv, la.zpA, bad);
                badm |= (bad || fixed_exact) ? (1u << (4 * q + e)) : 0u;
            }
        if (__builtin_amdgcn_ballot_w64(badm != 0)) {
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (badm & (1u << (4 * q + e))) cq[q][e] = quant_i8_exact(hv[q][e], la.sA, la.zpA);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
            codes[(hq_t + 16 * q) * CODE_DW + hq_c / 4] = pack4(cq[q][0], cq[q][1], cq[q][2], cq[q][3]);
        __syncthreads();
        // D, the dequantise + bias, and the tail of the lane's eight values.
        const uint32_t* crow = codes + (16 * tr + r) * CODE_DW + 4 * g;
        const v4i xo = v4i{static_cast<int>(crow[0]), static_cast<int>(crow[1]), static_cast<int>(crow[2]),
                           static_cast<int>(crow[3])};
        int32_t SA = 0;
        if constexpr (INT_EPI) {
#pragma unroll
            for (int q = 0; q < 4; ++q) SA = sum_bytes_i8(static_cast<uint32_t>(xo[q]), SA);
            SA = row_sum4(SA);
        }
        const int tok = 16 * tr + r;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wop[ct], xo, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int ch = 32 * chh + 16 * ct + 4 * g + v;
                float t;
                if constexpr (INT_EPI) t = int_epi_value(cepi[ch], acc[v], SA);
                else t = static_cast<float>(acc[v]);
                const float x2 = dequant_bias(csw[ch], la.sA, t, cbias[ch]);
                float ps = 0.0f, pz = 0.0f;
                if constexpr (KIND == 2) {
                    const int64_t pidx = static_cast<int64_t>(ch) * n + tl.t0 + tok;
                    ps = a.pos_scales[pidx];
                    pz = static_cast<float>(a.pos_zps[pidx]);
                }
                tx1[ch][tok] = post_element<KIND, ACT, FQN>(tx1[ch][tok], x2, a, inv_x2, inv_next, thr_x2, thr_next,
                                                            ps, pz);
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q) a.h[tb + (tk + 4 * q) * 64 + ck] = tx1[ck][tk + 4 * q];
#pragma unroll
        for (int q = 0; q < PER; ++q) a.hc[cb + q * d1] = tx1[cm + CSTEP * q][tm];
        __syncthreads();
    }
}

// The fp32 local-linear layer (k_linear_rows64's sums: bias, then the 64
// products rounded and added in order) and the tail in one pass, on the
// tail's 32-token tiles at width 64: lane j of every wave holds row j of W
// in registers, the h tile is staged in LDS (token-major) and read back as
// broadcasts, and the lane's eight outputs (tokens x / 64 + 4 q, channel
// x % 64) go through the tail as k_post_rt's token-major elements.
template <int KIND, int ACT, int FQN>
__global__ __launch_bounds__(256) void k_linear_tail(PostArgs a, const float* Wl, const float* bl) {
    constexpr int TT = 32, PER = TT * 64 / 256, CSTEP = 256 / TT, HS = 68;
    __shared__ float tx1[64][TT + 1];
    __shared__ __attribute__((aligned(16))) float th[TT * HS];
    __shared__ float thr_x2[16], thr_next[16];
    const int n = a.n;                  // w == 64, n % 32 == 0 (linear_tail_ok)
    if (threadIdx.x < 15) thr_x2[threadIdx.x] = a.thr[threadIdx.x];
    stage_steps(thr_next, a.fq_next.thr);
    const ScaleInv inv_x2 = scale_inv(a.scale), inv_next = scale_inv(a.fq_next.scale);
    const int cm = threadIdx.x / TT, tm = threadIdx.x % TT, tk = threadIdx.x / 64, ck = threadIdx.x % 64;
    const int hq_t = threadIdx.x / 16, hq_c = 4 * (threadIdx.x % 16);
    float wr[64];
#pragma unroll
    for (int p = 0; p < 64; p += 4) {
        const v4f q = *reinterpret_cast<const v4f*>(Wl + ck * 64 + p);
        wr[p] = q[0];
        wr[p + 1] = q[1];
        wr[p + 2] = q[2];
        wr[p + 3] = q[3];
    }
    const float bj = bl ? bl[ck] : 0.0f;
    const int64_t o1 = static_cast<int64_t>(cm) * n + tm, d1 = static_cast<int64_t>(CSTEP) * n;
    Tile tl;
    for (int64_t id = blockIdx.x; tile_of<TT>(id, a.samples, n, 64, tl); id += gridDim.x) {
        const int64_t cb = tl.s * 64 * static_cast<int64_t>(n) + tl.t0 + o1;
        const int64_t tb = (tl.s * n + tl.t0) * 64;
        v4f hv[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) hv[q] = *reinterpret_cast<const v4f*>(a.h + tb + (hq_t + 16 * q) * 64 + hq_c);
        float xv[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) xv[q] = a.x1c[cb + q * d1];
#pragma unroll
        for (int q = 0; q < 2; ++q) *reinterpret_cast<v4f*>(th + (hq_t + 16 * q) * HS + hq_c) = hv[q];
#pragma unroll
        for (int q = 0; q < PER; ++q) tx1[cm + CSTEP * q][tm] = xv[q];
        __syncthreads();
        float ps[PER], pz[PER];
        if constexpr (KIND == 2) {
            const int64_t pb = static_cast<int64_t>(ck) * n + tl.t0 + tk;
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                ps[q] = a.pos_scales[pb + 4 * q];
                pz[q] = static_cast<float>(a.pos_zps[pb + 4 * q]);
            }
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const float* hr = th + (tk + 4 * q) * HS;
            float acc = bj;
#pragma unroll
            for (int p = 0; p < 64; p += 4) {
                const v4f hp = *reinterpret_cast<const v4f*>(hr + p);
                acc = acc + hp[0] * wr[p];
                acc = acc + hp[1] * wr[p + 1];
                acc = acc + hp[2] * wr[p + 2];
                acc = acc + hp[3] * wr[p + 3];
            }
            tx1[ck][tk + 4 * q] = post_element<KIND, ACT, FQN>(tx1[ck][tk + 4 * q], acc, a, inv_x2, inv_next, thr_x2,
                                                               thr_next, KIND == 2 ? ps[q] : 0.0f,
                                                               KIND == 2 ? pz[q] : 0.0f);
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q) a.h[tb + (tk + 4 * q) * 64 + ck] = tx1[ck][tk + 4 * q];
#pragma unroll
        for (int q = 0; q < PER; ++q) a.hc[cb + q * d1] = tx1[cm + CSTEP * q][tm];
        __syncthreads();
    }
}

// The projection head in one pass (fno.cpp:662-698, :966-993): proj_q
// (64 -> 64, k_linear_rows64's sums), its fake-quant FQQ and the activation,
// then proj_out (64 -> 1, k_linear_narrow64's sums over the 64 activations
// in order) and its fake-quant FQO, on 32-token tiles.  Lane j of each wave
// holds row j of proj_q.weight in registers; the h tile and the activations
// are staged in LDS (token-major), and 32 threads take one token's proj_out
// each.
template <int ACT, int FQQ, int FQO>
__global__ __launch_bounds__(256) void k_proj_tail(ProjArgs a) {
    constexpr int TT = 32, HS = 68, QS = 65, PER = TT * 64 / 256;
    __shared__ __attribute__((aligned(16))) float th[TT * HS];
    __shared__ float tq[TT * QS];
    __shared__ float wo_s[64];
    __shared__ float steps_q[16], steps_o[16];
    if (threadIdx.x < 64) wo_s[threadIdx.x] = a.Wo[threadIdx.x];
    stage_steps(steps_q, a.fq_q.thr);
    stage_steps(steps_o, a.fq_o.thr);
    const ScaleInv inv_q = scale_inv(a.fq_q.scale), inv_o = scale_inv(a.fq_o.scale);
    const int tk = threadIdx.x / 64, ck = threadIdx.x % 64;
    const int hq_t = threadIdx.x / 16, hq_c = 4 * (threadIdx.x % 16);
    float wr[64];
#pragma unroll
    for (int p = 0; p < 64; p += 4) {
        const v4f q = *reinterpret_cast<const v4f*>(a.Wq + ck * 64 + p);
        wr[p] = q[0];
        wr[p + 1] = q[1];
        wr[p + 2] = q[2];
        wr[p + 3] = q[3];
    }
    const float bj = a.bq ? a.bq[ck] : 0.0f;
    const float bo = a.bo ? a.bo[0] : 0.0f;
    const int n = a.n;
    Tile tl;
    for (int64_t id = blockIdx.x; tile_of<TT>(id, a.samples, n, 64, tl); id += gridDim.x) {
        const float* hs = a.h + (tl.s * a.rows_in + tl.t0) * 64;
        v4f hv[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) hv[q] = *reinterpret_cast<const v4f*>(hs + (hq_t + 16 * q) * 64 + hq_c);
#pragma unroll
        for (int q = 0; q < 2; ++q) *reinterpret_cast<v4f*>(th + (hq_t + 16 * q) * HS + hq_c) = hv[q];
        __syncthreads();
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const float* hr = th + (tk + 4 * q) * HS;
            float acc = bj;
#pragma unroll
            for (int p = 0; p < 64; p += 4) {
                const v4f x = *reinterpret_cast<const v4f*>(hr + p);
                acc = acc + x[0] * wr[p];
                acc = acc + x[1] * wr[p + 1];
                acc = acc + x[2] * wr[p + 2];
                acc = acc + x[3] * wr[p + 3];
            }
            if constexpr (FQQ == 1) acc = x2_fake_quant_inv(acc, a.fq_q.scale, inv_q.inv, inv_q.ok, a.fq_q.zpf);
            else if constexpr (FQQ == 3) acc = log2_snap(acc, a.fq_q.scale, steps_q);
            if constexpr (ACT == RT_ACT_RELU) acc = acc < 0.0f ? 0.0f : acc;   // fno.cpp:37-40
            else if constexpr (ACT == RT_ACT_GELU) acc = gelu_fast<kGeluRefine>(acc);
            tq[(tk + 4 * q) * QS + ck] = acc;
        }
        __syncthreads();
        if (threadIdx.x < TT) {
            const float* qr = tq + threadIdx.x * QS;
            float acc = bo;
#pragma unroll
            for (int j = 0; j < 64; ++j) acc = acc + qr[j] * wo_s[j];
            if constexpr (FQO == 1) acc = x2_fake_quant_inv(acc, a.fq_o.scale, inv_o.inv, inv_o.ok, a.fq_o.zpf);
            else if constexpr (FQO == 3) acc = log2_snap(acc, a.fq_o.scale, steps_o);
            a.y[tl.s * n + tl.t0 + threadIdx.x] = acc;
        }
    }
}

// ---------------------------------------------------------------------------
// FNO2d padding and the projection fake-quants.
// ---------------------------------------------------------------------------

// One thread per element of the larger grid (samples, hp, wp, c).
__global__ __launch_bounds__(256) void k_pad2d(const float* src, float* dst, int64_t samples, int h, int w, int hp,
                                               int wp, int c, int trim) {
    const int64_t total = samples * hp * wp * c;
    for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int ch = static_cast<int>(i % c);
        const int64_t p = i / c;
        const int x = static_cast<int>(p % wp);
        const int64_t q = p / wp;
        const int y = static_cast<int>(q % hp);
        const int64_t s = q / hp;
        const bool in = y < h && x < w;
        const int64_t small = ((s * h + y) * w + x) * c + ch;
        if (trim) {
            if (in) dst[small] = src[i];
        } else {
            dst[i] = in ? src[small] : 0.0f;
        }
    }
}

// The fake-quant's form FQ (0 off, 1 per tensor, 3 log2 snap) and the
// activation are template parameters; four elements per thread and pass
// (16-byte accesses) when y is 16-byte aligned, the rest one by one.
template <int FQ, int ACT>
__global__ __launch_bounds__(256) void k_fq_act(float* y, int64_t n, FakeQuant fq, int vec) {
    __shared__ float steps[16];
    stage_steps(steps, fq.thr);
    const ScaleInv inv = scale_inv(fq.scale);
    auto f = [&](float v) {
        if constexpr (FQ == 1) v = x2_fake_quant_inv(v, fq.scale, inv.inv, inv.ok, fq.zpf);
        else if constexpr (FQ == 3) v = log2_snap(v, fq.scale, steps);
        if constexpr (ACT == RT_ACT_RELU) v = v < 0.0f ? 0.0f : v;   // fno.cpp:37-40
        else if constexpr (ACT == RT_ACT_GELU) v = gelu_fast<kGeluRefine>(v);
        return v;
    };
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t n4 = vec ? n / 4 : 0;
    v4f* y4 = reinterpret_cast<v4f*>(y);
    for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < n4; i += stride) {
        v4f v = y4[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f(v[e]);
        y4[i] = v;
    }
    for (int64_t i = 4 * n4 + blockIdx.x * 256LL + threadIdx.x; i < n; i += stride) y[i] = f(y[i]);
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------

hipError_t launch_linear_ref(const LinArgs& a, hipStream_t st) {
    const int64_t rows = a.samples * a.rows_out;
    if (rows <= 0 || a.n <= 0) return hipSuccess;
    if (a.k == 64 && a.n >= 16 && aligned(a.x, 16) && aligned(a.W, 16)) {
        hipLaunchKernelGGL(k_linear_rows64, dim3(grid_for((rows + 3) / 4, 4, 8)), dim3(256), 0, st, a);
    } else if (a.n <= 16 && static_cast<size_t>(a.n) * a.k * sizeof(float) <= 48 * 1024) {
        // Registers for as many columns as there are (each column's sum in
        // the same order whatever NMAX is).
        const size_t lds = static_cast<size_t>(a.n) * a.k * sizeof(float);
        if (a.k == 64 && a.rows_in == a.rows_out && a.rows_valid == a.rows_out && aligned(a.x, 16)) {
            if (a.n == 1)
                hipLaunchKernelGGL(k_linear_narrow64<1>, dim3(grid_for(rows, 256, 2)), dim3(256), 0, st, a);
            else if (a.n <= 4)
                hipLaunchKernelGGL(k_linear_narrow64<4>, dim3(grid_for(rows, 256, 2)), dim3(256), 0, st, a);
            else
                hipLaunchKernelGGL(k_linear_narrow64<16>, dim3(grid_for(rows, 256, 2)), dim3(256), 0, st, a);
        } else if (a.n == 1)
            hipLaunchKernelGGL(k_linear_narrow<1>, dim3(grid_for(rows, 256, 8)), dim3(256), lds, st, a);
        else if (a.n <= 4)
            hipLaunchKernelGGL(k_linear_narrow<4>, dim3(grid_for(rows, 256, 8)), dim3(256), lds, st, a);
        else
            hipLaunchKernelGGL(k_linear_narrow<16>, dim3(grid_for(rows, 256, 8)), dim3(256), lds, st, a);
    } else if (a.k == 1 && a.rows_in == a.rows_out && a.rows_valid == a.rows_out && a.n >= 4 && a.n <= 1024 &&
               (a.n & (a.n - 1)) == 0 && aligned(a.y, 16)) {
        hipLaunchKernelGGL(k_linear_k1, dim3(grid_for(rows * (a.n / 4), 256, 8)), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(k_linear_flat, dim3(grid_for(rows * a.n, 256, 8)), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

static int64_t tile_count(int64_t samples, int n, int w, int tt) {
    return samples * ((n + tt - 1) / tt) * static_cast<int64_t>((w + 63) / 64);
}

// Tiles of 64 tokens, or of 8 when 64-token tiles would give fewer than two
// blocks per CU (a small batch: one 1024-point sample of width 64 is 16
// tiles; the tail then ran 22.7 us, its threads each taking 16 exact GELUs
// in sequence on 16 CUs).
static bool small_tiles(int64_t samples, int n, int w) {
    return tile_count(samples, n, w, 64) < 2 * static_cast<int64_t>(num_cus());
}

template <int TT>
static void launch_channel_major_tt(float* h, float* hc, int64_t samples, int n, int w, const FakeQuant& fq,
                                    hipStream_t st) {
    const dim3 grid(grid_for(tile_count(samples, n, w, TT), 1, 8));
    if (fq.on == 1)
        hipLaunchKernelGGL((k_to_channel_major<TT, 1>), grid, dim3(256), 0, st, h, hc, samples, n, w, fq);
    else if (fq.on == 3)
        hipLaunchKernelGGL((k_to_channel_major<TT, 3>), grid, dim3(256), 0, st, h, hc, samples, n, w, fq);
    else
        hipLaunchKernelGGL((k_to_channel_major<TT, 0>), grid, dim3(256), 0, st, h, hc, samples, n, w, fq);
}

template <int TT>
static void launch_lift_layout_tt(const float* x, const float* W, const float* b, float* h, float* hc,
                                  int64_t samples, int n, int w, const FakeQuant& fq, hipStream_t st) {
    const dim3 grid(grid_for(tile_count(samples, n, w, TT), 1, 8));
    if (fq.on == 1)
        hipLaunchKernelGGL((k_lift_layout<TT, 1>), grid, dim3(256), 0, st, x, W, b, h, hc, samples, n, w, fq);
    else if (fq.on == 3)
        hipLaunchKernelGGL((k_lift_layout<TT, 3>), grid, dim3(256), 0, st, x, W, b, h, hc, samples, n, w, fq);
    else
        hipLaunchKernelGGL((k_lift_layout<TT, 0>), grid, dim3(256), 0, st, x, W, b, h, hc, samples, n, w, fq);
}

hipError_t launch_lift_layout(const float* x, const float* W, const float* b, float* h, float* hc, int64_t samples,
                              int n, int w, FakeQuant fq, hipStream_t st) {
    if (samples <= 0) return hipSuccess;
    if (small_tiles(samples, n, w))
        launch_lift_layout_tt<8>(x, W, b, h, hc, samples, n, w, fq, st);
    else
        launch_lift_layout_tt<64>(x, W, b, h, hc, samples, n, w, fq, st);
    return hipGetLastError();
}

hipError_t launch_to_channel_major(float* h, float* hc, int64_t samples, int n, int w, FakeQuant fq,
                                   hipStream_t st) {
    if (samples <= 0) return hipSuccess;
    if (small_tiles(samples, n, w))
        launch_channel_major_tt<8>(h, hc, samples, n, w, fq, st);
    else
        launch_channel_major_tt<64>(h, hc, samples, n, w, fq, st);
    return hipGetLastError();
}

// One wave per FFT of n points: 4 waves per block with the twiddle table
// (n - 1 values) in LDS when n <= 2048, else one wave reading it from L2.
// Blocks are dealt to the 8 XCDs in contiguous logical ranges (xcd_block).
struct FftLaunch {
    bool small;
    int64_t nlogical;
    unsigned grid;
    size_t lds;
};
static FftLaunch fft_launch(int64_t items, int n) {
    FftLaunch f{};
    f.small = n <= 2048;
    const int wpb = f.small ? 4 : 1;
    f.nlogical = (items + wpb - 1) / wpb;
    f.grid = static_cast<unsigned>(8 * ((f.nlogical + 7) / 8));
    f.lds = (static_cast<size_t>(wpb) * fft_buf_len(n) + (f.small ? n : 0)) * sizeof(float2);
    return f;
}

// The fixed-length kernels: lengths 64 .. 1024, a persistent grid of as
// many blocks as the CUs' LDS holds at once (160 KiB each; blocks of WPB
// waves sharing one twiddle table: 8 at 512 and 1024 points, whose tables
// are the largest), each wave taking R sequences at a time.
template <int LOG2N>
static bool fixed_launch(int64_t items, int keep, unsigned& grid, int64_t& nsets, size_t& lds) {
    if (path_flag(kernel_path().generic_fft) || keep < 1) return false;
    using F = RowFft<LOG2N>;
    nsets = (items + F::R - 1) / F::R;
    constexpr int WPB = RowFftPlan<LOG2N>::WPB;
    lds = (static_cast<size_t>(F::N) + WPB * static_cast<size_t>(F::WAVE_SLOTS)) * sizeof(float2);
    const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(8, (160 * 1024) / static_cast<int64_t>(lds)));
    const int64_t blocks = (nsets + WPB - 1) / WPB, cap = per_cu * static_cast<int64_t>(num_cus());
    grid = static_cast<unsigned>(blocks < cap ? blocks : cap);
    return true;
}

template <int LOG2N, bool PRUNE, bool E0, class IO>
static void launch_fixed(const IO& io, unsigned grid, int64_t nsets, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((k_fft_fixed<LOG2N, PRUNE, E0, IO>), dim3(grid), dim3(64 * RowFftPlan<LOG2N>::WPB), lds, st, io,
                       nsets);
}

template <int LOG2N>
static bool launch_rfft_fixed(const SpecArgs& a, int64_t items, hipStream_t st) {
    unsigned grid;
    int64_t nsets;
    size_t lds;
    if (!fixed_launch<LOG2N>(items, a.modes, grid, nsets, lds)) return false;
    const RowFwdIO<LOG2N> io{a.hc, reinterpret_cast<float2*>(a.spec), a.tw_fwd, items, a.modes};
    if (a.modes <= RowFft<LOG2N>::G1) launch_fixed<LOG2N, true, true>(io, grid, nsets, lds, st);
    else launch_fixed<LOG2N, true, false>(io, grid, nsets, lds, st);
    return true;
}

template <int LOG2N>
static bool launch_irfft_fixed(const SpecArgs& a, int64_t items, hipStream_t st) {
    unsigned grid;
    int64_t nsets;
    size_t lds;
    if (!fixed_launch<LOG2N>(items, a.modes, grid, nsets, lds)) return false;
    const float2* spec = reinterpret_cast<const float2*>(a.spec_mixed);
    if (a.modes <= RowFft<LOG2N>::N / RowFft<LOG2N>::G1) {
        const RowInvIO<LOG2N, true> io{spec, a.x1c, a.fill, a.tw_inv, items, 0, a.modes, a.fill_period, a.inv_n};
        launch_fixed<LOG2N, false, false>(io, grid, nsets, lds, st);
    } else {
        const RowInvIO<LOG2N, false> io{spec, a.x1c, a.fill, a.tw_inv, items, 0, a.modes, a.fill_period, a.inv_n};
        launch_fixed<LOG2N, false, false>(io, grid, nsets, lds, st);
    }
    return true;
}

template <int LOG2N>
static bool launch_cfft_fixed(const ColArgs& a, bool inverse, int64_t items, hipStream_t st) {
    unsigned grid;
    int64_t nsets;
    size_t lds;
    if (items > static_cast<int64_t>(UINT32_MAX) || !fixed_launch<LOG2N>(items, a.mh, grid, nsets, lds)) return false;
    const float2* in = reinterpret_cast<const float2*>(a.in);
    float2* out = reinterpret_cast<float2*>(a.out);
    if (inverse) {
        if (a.mh <= RowFft<LOG2N>::N / RowFft<LOG2N>::G1) {
            const ColIO<LOG2N, true, true> io{in, out, a.tw, items, 0, a.mw, a.mh, a.inv_h};
            launch_fixed<LOG2N, false, false>(io, grid, nsets, lds, st);
        } else {
            const ColIO<LOG2N, true, false> io{in, out, a.tw, items, 0, a.mw, a.mh, a.inv_h};
            launch_fixed<LOG2N, false, false>(io, grid, nsets, lds, st);
        }
    } else {
        const ColIO<LOG2N, false, false> io{in, out, a.tw, items, a.mh, a.mw, a.mh, a.inv_h};
        if (a.mh <= RowFft<LOG2N>::G1) launch_fixed<LOG2N, true, true>(io, grid, nsets, lds, st);
        else launch_fixed<LOG2N, true, false>(io, grid, nsets, lds, st);
    }
    return true;
}

hipError_t launch_rfft_rows(const SpecArgs& a, hipStream_t st) {
    const int64_t items = a.samples * a.w;
    if (items <= 0) return hipSuccess;
    bool fixed = false;
    switch (a.log2n) {
        case 6: fixed = launch_rfft_fixed<6>(a, items, st); break;
        case 7: fixed = launch_rfft_fixed<7>(a, items, st); break;
        case 8: fixed = launch_rfft_fixed<8>(a, items, st); break;
        case 9: fixed = launch_rfft_fixed<9>(a, items, st); break;
        case 10: fixed = launch_rfft_fixed<10>(a, items, st); break;
        default: break;
    }
    if (fixed) return hipGetLastError();
    const FftLaunch f = fft_launch(items, a.n);
    if (f.small)
        hipLaunchKernelGGL((k_rfft_modes<4, true>), dim3(f.grid), dim3(256), f.lds, st, a, f.nlogical);
    else
        hipLaunchKernelGGL((k_rfft_modes<1, false>), dim3(f.grid), dim3(64), f.lds, st, a, f.nlogical);
    return hipGetLastError();
}

hipError_t launch_spec_mix(const SpecArgs& a, hipStream_t st) {
    if (a.samples <= 0 || a.w <= 0 || a.modes <= 0) return hipSuccess;
    if (a.w <= 64 && a.modes <= 65535 && !path_flag(kernel_path().generic_fft)) {
        const dim3 mg(static_cast<unsigned>((a.samples + 3) / 4), static_cast<unsigned>(a.modes));
        if (a.w == 64)
            hipLaunchKernelGGL(k_spec_mix_lds<64>, mg, dim3(256), 0, st, a, a.mix_real, a.mix_imag, a.spec_mixed);
        else
            hipLaunchKernelGGL(k_spec_mix_lds<0>, mg, dim3(256), 0, st, a, a.mix_real, a.mix_imag, a.spec_mixed);
        return hipGetLastError();
    }
    const dim3 mg(static_cast<unsigned>((a.samples + 3) / 4), static_cast<unsigned>((a.w + 63) / 64),
                  static_cast<unsigned>(a.modes));
    hipLaunchKernelGGL(k_spec_mix, mg, dim3(256), 0, st, a, a.mix_real, a.mix_imag, a.spec_mixed);
    return hipGetLastError();
}

hipError_t launch_irfft_rows(const SpecArgs& a, hipStream_t st) {
    const int64_t items = a.samples * a.w;
    if (items <= 0) return hipSuccess;
    bool fixed = false;
    switch (a.log2n) {
        case 6: fixed = launch_irfft_fixed<6>(a, items, st); break;
        case 7: fixed = launch_irfft_fixed<7>(a, items, st); break;
        case 8: fixed = launch_irfft_fixed<8>(a, items, st); break;
        case 9: fixed = launch_irfft_fixed<9>(a, items, st); break;
        case 10: fixed = launch_irfft_fixed<10>(a, items, st); break;
        default: break;
    }
    if (fixed) return hipGetLastError();
    const FftLaunch f = fft_launch(items, a.n);
    if (f.small)
        hipLaunchKernelGGL((k_irfft<4, true>), dim3(f.grid), dim3(256), f.lds, st, a, a.spec_mixed, f.nlogical);
    else
        hipLaunchKernelGGL((k_irfft<1, false>), dim3(f.grid), dim3(64), f.lds, st, a, a.spec_mixed, f.nlogical);
    return hipGetLastError();
}

hipError_t launch_spectral(const SpecArgs& a, hipStream_t st) {
    if (hipError_t e = launch_rfft_rows(a, st)) return e;
    if (hipError_t e = launch_spec_mix(a, st)) return e;
    return launch_irfft_rows(a, st);
}

hipError_t launch_cfft_cols(const ColArgs& a, bool inverse, hipStream_t st) {
    const int64_t items = a.planes * a.mw;
    if (items <= 0) return hipSuccess;
    bool fixed = false;
    switch (a.log2h) {
        case 6: fixed = launch_cfft_fixed<6>(a, inverse, items, st); break;
        case 7: fixed = launch_cfft_fixed<7>(a, inverse, items, st); break;
        case 8: fixed = launch_cfft_fixed<8>(a, inverse, items, st); break;
        case 9: fixed = launch_cfft_fixed<9>(a, inverse, items, st); break;
        case 10: fixed = launch_cfft_fixed<10>(a, inverse, items, st); break;
        default: break;
    }
    if (fixed) return hipGetLastError();
    const FftLaunch f = fft_launch(items, a.h);
    if (inverse) {
        if (f.small)
            hipLaunchKernelGGL((k_cfft_cols<4, true, true>), dim3(f.grid), dim3(256), f.lds, st, a, f.nlogical);
        else
            hipLaunchKernelGGL((k_cfft_cols<1, false, true>), dim3(f.grid), dim3(64), f.lds, st, a, f.nlogical);
    } else {
        if (f.small)
            hipLaunchKernelGGL((k_cfft_cols<4, true, false>), dim3(f.grid), dim3(256), f.lds, st, a, f.nlogical);
        else
            hipLaunchKernelGGL((k_cfft_cols<1, false, false>), dim3(f.grid), dim3(64), f.lds, st, a, f.nlogical);
    }
    return hipGetLastError();
}

hipError_t launch_pad2d(const float* src, float* dst, int64_t samples, int h, int w, int hp, int wp, int c,
                        bool trim, hipStream_t st) {
    const int64_t total = samples * hp * wp * c;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pad2d, dim3(grid_for(total, 256, 8)), dim3(256), 0, st, src, dst, samples, h, w, hp, wp, c,
                       trim ? 1 : 0);
    return hipGetLastError();
}

template <int FQ>
static void launch_fq_act_fq(float* y, int64_t n, const FakeQuant& fq, int act, hipStream_t st) {
    const int vec = aligned(y, 16) ? 1 : 0;
    const dim3 grid(grid_for(vec ? (n + 3) / 4 : n, 256, 8));
    if (act == RT_ACT_GELU)
        hipLaunchKernelGGL((k_fq_act<FQ, RT_ACT_GELU>), grid, dim3(256), 0, st, y, n, fq, vec);
    else if (act == RT_ACT_RELU)
        hipLaunchKernelGGL((k_fq_act<FQ, RT_ACT_RELU>), grid, dim3(256), 0, st, y, n, fq, vec);
    else
        hipLaunchKernelGGL((k_fq_act<FQ, RT_ACT_NONE>), grid, dim3(256), 0, st, y, n, fq, vec);
}

hipError_t launch_fq_act(float* y, int64_t n, FakeQuant fq, int act, hipStream_t st) {
    if (n <= 0 || (fq.on == 0 && act == RT_ACT_NONE)) return hipSuccess;
    if (fq.on == 1) launch_fq_act_fq<1>(y, n, fq, act, st);
    else if (fq.on == 3) launch_fq_act_fq<3>(y, n, fq, act, st);
    else launch_fq_act_fq<0>(y, n, fq, act, st);
    return hipGetLastError();
}

// The tail on 32-token tiles (eight elements per thread, four waves per
// SIMD; 64-token tiles held 153 VGPRs, three waves per SIMD, and ran 96.8 us
// against 77.7 us at 256 x 1024 x 64, 359 us against 302 us for the FNO2d
// model's tail), or 8-token tiles for a small batch.
template <int TT, int KIND, int ACT>
static void launch_post_fqn(const PostArgs& a, unsigned grid, hipStream_t st) {
    if (a.fq_next.on == 1)
        hipLaunchKernelGGL((k_post_rt<TT, KIND, ACT, 1>), dim3(grid), dim3(256), 0, st, a);
    else if (a.fq_next.on == 3)
        hipLaunchKernelGGL((k_post_rt<TT, KIND, ACT, 3>), dim3(grid), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((k_post_rt<TT, KIND, ACT, 0>), dim3(grid), dim3(256), 0, st, a);
}

template <int TT, int KIND>
static void launch_post_act(const PostArgs& a, unsigned grid, hipStream_t st) {
    if (a.act == RT_ACT_GELU) launch_post_fqn<TT, KIND, RT_ACT_GELU>(a, grid, st);
    else if (a.act == RT_ACT_RELU) launch_post_fqn<TT, KIND, RT_ACT_RELU>(a, grid, st);
    else launch_post_fqn<TT, KIND, RT_ACT_NONE>(a, grid, st);
}

template <int TT>
static void launch_post_tt(const PostArgs& a, hipStream_t st) {
    const unsigned grid = grid_for(tile_count(a.samples, a.n, a.w, TT), 1, 8);
    switch (a.kind) {
        case 1: launch_post_act<TT, 1>(a, grid, st); break;
        case 2: launch_post_act<TT, 2>(a, grid, st); break;
        case 3: launch_post_act<TT, 3>(a, grid, st); break;
        default: launch_post_act<TT, 0>(a, grid, st); break;
    }
}

hipError_t launch_post(const PostArgs& a, hipStream_t st) {
    if (a.samples <= 0) return hipSuccess;
    if (tile_count(a.samples, a.n, a.w, 32) < 2 * static_cast<int64_t>(num_cus()))
        launch_post_tt<8>(a, st);
    else
        launch_post_tt<32>(a, st);
    return hipGetLastError();
}

// The fused layer + tail: width 64, whole 32-token tiles (n a multiple of
// 32), at least two tiles per CU, the runtime's activations (ReLU, GELU) and
// next-input fake-quants (off, per tensor), and the layer of 64 x 64.
bool layer_tail_ok(const PostArgs& p, int in_features, int out_features) {
    return !path_flag(kernel_path().no_layer_tail) && p.w == 64 && in_features == 64 && out_features == 64 &&
           p.n > 0 && p.n % 32 == 0 && tile_count(p.samples, p.n, p.w, 32) >= 2 * static_cast<int64_t>(num_cus()) &&
           (p.act == RT_ACT_RELU || p.act == RT_ACT_GELU) && (p.fq_next.on == 0 || p.fq_next.on == 1) &&
           p.kind >= 0 && p.kind <= 3 && aligned(p.h, 16);
}

template <int KIND, int ACT, int FQN>
static void launch_layer_tail_epi(const LayerTailArgs& a, unsigned grid, hipStream_t st) {
    if (a.zpA == 0 && !a.zpW)
        hipLaunchKernelGGL((k_layer_tail<KIND, ACT, FQN, false>), dim3(grid), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((k_layer_tail<KIND, ACT, FQN, true>), dim3(grid), dim3(256), 0, st, a);
}

template <int KIND, int ACT>
static void launch_layer_tail_fqn(const LayerTailArgs& a, unsigned grid, hipStream_t st) {
    if (a.p.fq_next.on == 1) launch_layer_tail_epi<KIND, ACT, 1>(a, grid, st);
    else launch_layer_tail_epi<KIND, ACT, 0>(a, grid, st);
}

template <int KIND>
static void launch_layer_tail_act(const LayerTailArgs& a, unsigned grid, hipStream_t st) {
    if (a.p.act == RT_ACT_GELU) launch_layer_tail_fqn<KIND, RT_ACT_GELU>(a, grid, st);
    else launch_layer_tail_fqn<KIND, RT_ACT_RELU>(a, grid, st);
}

hipError_t launch_layer_tail(const LayerTailArgs& a, hipStream_t st) {
    if (a.p.samples <= 0) return hipSuccess;
    const unsigned grid = grid_for(tile_count(a.p.samples, a.p.n, a.p.w, 32), 1, 8);
    switch (a.p.kind) {
        case 1: launch_layer_tail_act<1>(a, grid, st); break;
        case 2: launch_layer_tail_act<2>(a, grid, st); break;
        case 3: launch_layer_tail_act<3>(a, grid, st); break;
        default: launch_layer_tail_act<0>(a, grid, st); break;
    }
    return hipGetLastError();
}

// The fp32 local linear + tail: as layer_tail_ok, for a 64 x 64 fp32 layer
// whose rows are read as 16-byte vectors.
bool linear_tail_ok(const PostArgs& p, const float* W) { return layer_tail_ok(p, 64, 64) && aligned(W, 16); }

template <int KIND, int ACT>
static void launch_linear_tail_fqn(const PostArgs& a, const float* W, const float* b, unsigned grid, hipStream_t st) {
    if (a.fq_next.on == 1) hipLaunchKernelGGL((k_linear_tail<KIND, ACT, 1>), dim3(grid), dim3(256), 0, st, a, W, b);
    else hipLaunchKernelGGL((k_linear_tail<KIND, ACT, 0>), dim3(grid), dim3(256), 0, st, a, W, b);
}

template <int KIND>
static void launch_linear_tail_act(const PostArgs& a, const float* W, const float* b, unsigned grid, hipStream_t st) {
    if (a.act == RT_ACT_GELU) launch_linear_tail_fqn<KIND, RT_ACT_GELU>(a, W, b, grid, st);
    else launch_linear_tail_fqn<KIND, RT_ACT_RELU>(a, W, b, grid, st);
}

hipError_t launch_linear_tail(const PostArgs& a, const float* W, const float* b, hipStream_t st) {
    if (a.samples <= 0) return hipSuccess;
    const unsigned grid = grid_for(tile_count(a.samples, a.n, a.w, 32), 1, 8);
    switch (a.kind) {
        case 1: launch_linear_tail_act<1>(a, W, b, grid, st); break;
        case 2: launch_linear_tail_act<2>(a, W, b, grid, st); break;
        case 3: launch_linear_tail_act<3>(a, W, b, grid, st); break;
        default: launch_linear_tail_act<0>(a, W, b, grid, st); break;
    }
    return hipGetLastError();
}

// The projection head in one launch: proj_q 64 -> 64 and proj_out 64 -> 1,
// whole 32-token tiles, at least two tiles per CU, the fake-quant forms off /
// per tensor / log2 snap, 16-byte aligned h rows and proj_q weight.
bool proj_tail_ok(const ProjArgs& p) {
    const auto fq_ok = [](const FakeQuant& f) { return f.on == 0 || f.on == 1 || f.on == 3; };
    return !path_flag(kernel_path().no_layer_tail) && p.w == 64 && p.out_ch == 1 && p.n > 0 && p.n % 32 == 0 &&
           p.rows_in >= p.n && tile_count(p.samples, p.n, 64, 32) >= 2 * static_cast<int64_t>(num_cus()) &&
           fq_ok(p.fq_q) && fq_ok(p.fq_o) && (p.act == RT_ACT_NONE || p.act == RT_ACT_RELU || p.act == RT_ACT_GELU) &&
           aligned(p.h, 16) && aligned(p.Wq, 16);
}

template <int ACT, int FQQ>
static void launch_proj_tail_fqo(const ProjArgs& a, unsigned grid, hipStream_t st) {
    if (a.fq_o.on == 1) hipLaunchKernelGGL((k_proj_tail<ACT, FQQ, 1>), dim3(grid), dim3(256), 0, st, a);
    else if (a.fq_o.on == 3) hipLaunchKernelGGL((k_proj_tail<ACT, FQQ, 3>), dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_proj_tail<ACT, FQQ, 0>), dim3(grid), dim3(256), 0, st, a);
}

template <int ACT>
static void launch_proj_tail_fqq(const ProjArgs& a, unsigned grid, hipStream_t st) {
    if (a.fq_q.on == 1) launch_proj_tail_fqo<ACT, 1>(a, grid, st);
    else if (a.fq_q.on == 3) launch_proj_tail_fqo<ACT, 3>(a, grid, st);
    else launch_proj_tail_fqo<ACT, 0>(a, grid, st);
}

hipError_t launch_proj_tail(const ProjArgs& a, hipStream_t st) {
    if (a.samples <= 0) return hipSuccess;
    const unsigned grid = grid_for(tile_count(a.samples, a.n, 64, 32), 1, 8);
    if (a.act == RT_ACT_GELU) launch_proj_tail_fqq<RT_ACT_GELU>(a, grid, st);
    else if (a.act == RT_ACT_RELU) launch_proj_tail_fqq<RT_ACT_RELU>(a, grid, st);
    else launch_proj_tail_fqq<RT_ACT_NONE>(a, grid, st);
    return hipGetLastError();
}

}  // namespace nfq
