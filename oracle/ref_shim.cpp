// ref_shim.cpp -- C entry points over NeuroFlow's own INT8 GEMM and FP8 codec.
//
// TEST INFRASTRUCTURE.  Built by oracle/Makefile together with the reference's
// unmodified cpp/src/int8_gemm.cpp and header-only cpp/include/neuroflow/
// fp8_e4m3.h, straight from the reference tree, into oracle/_ref/.  Used to
// pin the C restatement (oracle/nflow_oracle.c) and as the CPU baseline timed
// by bench.py.  Nothing in the product links this.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "neuroflow/fp8_e4m3.h"
#include "neuroflow/int8_gemm.h"

namespace ig = nflow::int8_gemm;

extern "C" {

// Same layout as orc_int8_linear_params / nflow_int8_linear_params.
struct ref_params {
    const int8_t* W_int8;
    const float* scale_W;
    const int32_t* zp_W;
    const float* bias;
    int in_features;
    int out_features;
    float scale_A;
    int32_t zp_A;
    const int32_t* sum_W_per_row;
};

static ig::Int8LinearParams to_ref(const ref_params* p) {
    ig::Int8LinearParams q;
    q.W_int8 = p->W_int8;
    q.scale_W = p->scale_W;
    q.zp_W = p->zp_W;
    q.bias = p->bias;
    q.in_features = p->in_features;
    q.out_features = p->out_features;
    q.scale_A = p->scale_A;
    q.zp_A = p->zp_A;
    q.sum_W_per_row = p->sum_W_per_row;
    return q;
}

int ref_linear_forward(const ref_params* p, const float* A, float* C) {
    return static_cast<int>(ig::LinearForward(to_ref(p), A, C).code());
}

int ref_linear_forward_batched(const ref_params* p, int bsz, const float* A, float* C) {
    return static_cast<int>(ig::LinearForwardBatched(to_ref(p), bsz, A, C).code());
}

void ref_quantise_activation(const float* A, int8_t* A_q, int bsz, int in_features,
                             float scale_A, int32_t zp_A) {
    ig::QuantiseActivation(A, A_q, bsz, in_features, scale_A, zp_A);
}

// PrecomputeSumW returns new[]; copy out and free it here.  Returns 0 when
// the reference returned nullptr.
int ref_precompute_sum_w(const int8_t* W, const int32_t* zp, int in_f, int out_f,
                         int32_t* out) {
    const int32_t* s = ig::PrecomputeSumW(W, zp, in_f, out_f);
    if (!s) return 0;
    std::memcpy(out, s, sizeof(int32_t) * static_cast<size_t>(out_f));
    delete[] s;
    return 1;
}

void ref_e4m3_encode_array(const float* in, uint8_t* out, size_t n) {
    nflow::fp32_array_to_e4m3_bits(in, out, n);
}

void ref_e4m3_decode_array(const uint8_t* in, float* out, size_t n) {
    nflow::e4m3_bits_to_fp32_array(in, out, n);
}

void ref_fp8_fake_quant(const float* in, float scale, float* out, size_t n) {
    nflow::fp8_e4m3_per_tensor_fake_quant(in, scale, out, n);
}

// Encode every float whose bit pattern lies in [start, start + count).
void ref_e4m3_encode_bits_range(uint32_t start, uint32_t count, uint8_t* out) {
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t u = start + i;
        float f;
        std::memcpy(&f, &u, sizeof f);
        out[i] = nflow::fp32_to_e4m3_bits(f);
    }
}

// ---------------------------------------------------------------------------
// CPU baseline harness.  Times the reference's per-token INT8 layer: for each
// row, scale_A = absmax/127 and one LinearForward call with zp_A = 0 and the
// precomputed sum_W_per_row (the recommended production pattern,
// int8_gemm.h:54-64), followed by the tanh-form GELU of fno.cpp:41-46.  Rows
// are split across `threads` std::threads, each calling the unmodified
// reference function.  Returns the median wall time over `reps` passes.
// ---------------------------------------------------------------------------
static void gelu_row(float* y, int n) {
    const float c = std::sqrt(2.0f / static_cast<float>(3.14159265358979323846));
    for (int i = 0; i < n; ++i) {
        const float z = y[i];
        y[i] = 0.5f * z * (1.0f + std::tanh(c * (z + 0.044715f * z * z * z)));
    }
}

static void per_token_rows(const ref_params* p, const float* A, float* C, int64_t r0,
                           int64_t r1, int act_gelu) {
    ig::Int8LinearParams q = to_ref(p);
    const int K = p->in_features;
    const int N = p->out_features;
    for (int64_t r = r0; r < r1; ++r) {
        const float* a = A + r * K;
        float mx = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float v = std::fabs(a[k]);
            if (v > mx) mx = v;
        }
        q.scale_A = (mx == 0.0f) ? 1.0f : mx / 127.0f;
        q.zp_A = 0;
        (void)ig::LinearForward(q, a, C + r * N);
        if (act_gelu) gelu_row(C + r * N, N);
    }
}

double ref_time_per_token_layer(const ref_params* p, int64_t M, const float* A, float* C,
                                int act_gelu, int threads, int reps) {
    if (threads < 1) threads = 1;
    std::vector<double> times;
    for (int rep = 0; rep < reps; ++rep) {
        auto t0 = std::chrono::steady_clock::now();
        if (threads == 1) {
            per_token_rows(p, A, C, 0, M, act_gelu);
        } else {
            std::vector<std::thread> pool;
            const int64_t chunk = (M + threads - 1) / threads;
            for (int t = 0; t < threads; ++t) {
                const int64_t r0 = t * chunk;
                const int64_t r1 = std::min<int64_t>(M, r0 + chunk);
                if (r0 >= r1) break;
                pool.emplace_back(per_token_rows, p, A, C, r0, r1, act_gelu);
            }
            for (auto& th : pool) th.join();
        }
        auto t1 = std::chrono::steady_clock::now();
        times.push_back(std::chrono::duration<double>(t1 - t0).count());
    }
    std::sort(times.begin(), times.end());
    return times[times.size() / 2];
}

// Timing of LinearForwardBatched (one per-tensor scale; the FNO1d production
// path, fno.cpp:125-159), rows split across threads.
double ref_time_batched_layer(const ref_params* p, int64_t M, const float* A, float* C,
                              int threads, int reps) {
    if (threads < 1) threads = 1;
    const ig::Int8LinearParams q = to_ref(p);
    const int K = p->in_features;
    const int N = p->out_features;
    std::vector<double> times;
    for (int rep = 0; rep < reps; ++rep) {
        auto t0 = std::chrono::steady_clock::now();
        std::vector<std::thread> pool;
        const int64_t chunk = (M + threads - 1) / threads;
        for (int t = 0; t < threads; ++t) {
            const int64_t r0 = t * chunk;
            const int64_t r1 = std::min<int64_t>(M, r0 + chunk);
            if (r0 >= r1) break;
            pool.emplace_back([&q, A, C, K, N, r0, r1]() {
                (void)ig::LinearForwardBatched(q, static_cast<int>(r1 - r0), A + r0 * K,
                                               C + r0 * N);
            });
        }
        for (auto& th : pool) th.join();
        auto t1 = std::chrono::steady_clock::now();
        times.push_back(std::chrono::duration<double>(t1 - t0).count());
    }
    std::sort(times.begin(), times.end());
    return times[times.size() / 2];
}

// Timing of the FP8 composition the reference offers (it has no FP8 GEMM):
// per row, scale = absmax / 448 and the reference's
// fp8_e4m3_per_tensor_fake_quant (fp8_e4m3.h:312-334), then the fp32 Linear
// loop of fno.cpp:68-79 (bias first, products added in k order) against
// weights fake-quantised once per output channel with the same routine
// (outside the timed region, as weights are prepared once), then the tanh
// GELU.  Rows split across threads; median wall time over `reps` passes.
static void fp8_rows(const float* A, const float* Wq, const float* bias, int K, int N, float* C,
                     int64_t r0, int64_t r1, int act_gelu) {
    std::vector<float> xq(K);
    for (int64_t r = r0; r < r1; ++r) {
        const float* a = A + r * K;
        float mx = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float v = std::fabs(a[k]);
            if (v > mx) mx = v;
        }
        const float s = (mx == 0.0f) ? 1.0f : mx / 448.0f;
        nflow::fp8_e4m3_per_tensor_fake_quant(a, s, xq.data(), static_cast<size_t>(K));
        float* y = C + r * N;
        for (int j = 0; j < N; ++j) {
            float acc = bias ? bias[j] : 0.0f;
            const float* w = Wq + static_cast<int64_t>(j) * K;
            for (int k = 0; k < K; ++k) acc += xq[k] * w[k];
            y[j] = acc;
        }
        if (act_gelu) gelu_row(y, N);
    }
}

double ref_time_fp8_layer(const float* A, const float* W, const float* bias, int64_t M, int K, int N,
                          float* C, int act_gelu, int threads, int reps) {
    if (threads < 1) threads = 1;
    std::vector<float> Wq(static_cast<size_t>(N) * K);
    for (int j = 0; j < N; ++j) {
        const float* w = W + static_cast<int64_t>(j) * K;
        float mx = 0.0f;
        for (int k = 0; k < K; ++k) mx = std::max(mx, std::fabs(w[k]));
        const float s = (mx == 0.0f) ? 1.0f : mx / 448.0f;
        nflow::fp8_e4m3_per_tensor_fake_quant(w, s, Wq.data() + static_cast<int64_t>(j) * K,
                                              static_cast<size_t>(K));
    }
    std::vector<double> times;
    for (int rep = 0; rep < reps; ++rep) {
        auto t0 = std::chrono::steady_clock::now();
        std::vector<std::thread> pool;
        const int64_t chunk = (M + threads - 1) / threads;
        for (int t = 0; t < threads; ++t) {
            const int64_t r0 = t * chunk;
            const int64_t r1 = std::min<int64_t>(M, r0 + chunk);
            if (r0 >= r1) break;
            pool.emplace_back(fp8_rows, A, Wq.data(), bias, K, N, C, r0, r1, act_gelu);
        }
        for (auto& th : pool) th.join();
        auto t1 = std::chrono::steady_clock::now();
        times.push_back(std::chrono::duration<double>(t1 - t0).count());
    }
    std::sort(times.begin(), times.end());
    return times[times.size() / 2];
}

}  // extern "C"
