// ref_fno_run.cpp -- test infrastructure only: runs a NeuroIR file through
// the reference's own InferenceRuntime (cpp/src/runtime.cpp, fno.cpp,
// fft.cpp, tensor.cpp, int8_gemm.cpp, compiled from where they lie) on a raw
// float32 input, and writes the raw float32 output, so the tests can compare
// whole FNO1d runs -- and pieces of the layer exposed by crafted weights --
// and FNO2d runs -- with this library.
//
//   ref_fno_run <ir> <x.f32> <batch> <n> <in_ch> <out_ch> <y.f32> [int8|fp32] [reps] [threads]
//
// <n> is the grid: "n" for a 1-D model (shapes (batch, n, ch)) or "HxW" for
// FNO2d (shapes (batch, H, W, ch)).
// "int8" calls EnableInt8Gemm() before Run.  Prints "status <code>".  A
// <y.f32> of "-" skips the first (untimed, output-writing) run.  With
// reps > 0 it then times `reps` runs of the whole batch, split by samples
// over `threads` std::threads that each hold their own InferenceRuntime
// (FNO1d::Forward is single-threaded; one runtime per thread keeps its
// mutable caches private), and prints "us_per_run <median>".
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "neuroflow/runtime.h"

int main(int argc, char** argv) {
    if (argc < 8) return 2;
    const int64_t b = std::atoll(argv[3]), ci = std::atoll(argv[5]), co = std::atoll(argv[6]);
    // Grid: "n" or "HxW".
    std::vector<int64_t> grid;
    {
        const std::string g = argv[4];
        const size_t xpos = g.find('x');
        if (xpos == std::string::npos) grid = {std::atoll(g.c_str())};
        else grid = {std::atoll(g.substr(0, xpos).c_str()), std::atoll(g.substr(xpos + 1).c_str())};
    }
    int64_t n = 1;
    for (int64_t d : grid) n *= d;
    auto shape = [&](int64_t batch, int64_t ch) {
        std::vector<int64_t> sh{batch};
        sh.insert(sh.end(), grid.begin(), grid.end());
        sh.push_back(ch);
        return sh;
    };
    const bool int8 = argc > 8 && std::string(argv[8]) == "int8";
    const int reps = argc > 9 ? std::atoi(argv[9]) : 0;
    const int threads = argc > 10 ? std::max(1, std::atoi(argv[10])) : 1;
    std::vector<float> x(static_cast<size_t>(b * n * ci)), y(static_cast<size_t>(b * n * co), 0.0f);
    FILE* fx = std::fopen(argv[2], "rb");
    if (!fx || std::fread(x.data(), sizeof(float), x.size(), fx) != x.size()) return 3;
    std::fclose(fx);
    std::unique_ptr<nflow::InferenceRuntime> rt;
    nflow::Status s = nflow::InferenceRuntime::Create(argv[1], rt);
    if (s.ok() && int8) rt->EnableInt8Gemm();
    const bool write_y = std::string(argv[7]) != "-";
    if (s.ok() && write_y) s = rt->Run(x.data(), shape(b, ci), y.data(), shape(b, co));
    std::printf("status %d\n", static_cast<int>(s.code()));
    if (!s.ok()) return 0;
    if (write_y) {
        FILE* fy = std::fopen(argv[7], "wb");
        if (!fy || std::fwrite(y.data(), sizeof(float), y.size(), fy) != y.size()) return 4;
        std::fclose(fy);
    }
    if (reps <= 0) return 0;

    const int T = static_cast<int>(std::min<int64_t>(threads, b));
    std::vector<std::unique_ptr<nflow::InferenceRuntime>> rts(T);
    for (int t = 0; t < T; ++t) {
        if (!nflow::InferenceRuntime::Create(argv[1], rts[t]).ok()) return 5;
        if (int8) rts[t]->EnableInt8Gemm();
    }
    std::vector<double> us;
    for (int r = 0; r < reps; ++r) {
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<std::thread> pool;
        for (int t = 0; t < T; ++t) {
            const int64_t s0 = b * t / T, s1 = b * (t + 1) / T;
            pool.emplace_back([&, t, s0, s1] {
                if (s1 > s0)
                    (void)rts[t]->Run(x.data() + s0 * n * ci, shape(s1 - s0, ci), y.data() + s0 * n * co,
                                      shape(s1 - s0, co));
            });
        }
        for (auto& th : pool) th.join();
        us.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count());
    }
    std::sort(us.begin(), us.end());
    std::printf("us_per_run %.3f\n", us[us.size() / 2]);
    return 0;
}
