// ref_fno_run.cpp -- test infrastructure only: runs a NeuroIR file through
// the reference's own InferenceRuntime (cpp/src/runtime.cpp, fno.cpp,
// fft.cpp, tensor.cpp, int8_gemm.cpp, compiled from where they lie) on a raw
// float32 input, and writes the raw float32 output, so the tests can compare
// whole FNO1d runs -- and pieces of the layer exposed by crafted weights --
// with this library.
//
//   ref_fno_run <ir> <x.f32> <batch> <n> <in_ch> <out_ch> <y.f32> [int8]
//
// "int8" calls EnableInt8Gemm() before Run.  Prints "status <code>".
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <vector>

#include "neuroflow/runtime.h"

int main(int argc, char** argv) {
    if (argc < 8) return 2;
    const int64_t b = std::atoll(argv[3]), n = std::atoll(argv[4]), ci = std::atoll(argv[5]),
                  co = std::atoll(argv[6]);
    std::vector<float> x(static_cast<size_t>(b * n * ci)), y(static_cast<size_t>(b * n * co), 0.0f);
    FILE* fx = std::fopen(argv[2], "rb");
    if (!fx || std::fread(x.data(), sizeof(float), x.size(), fx) != x.size()) return 3;
    std::fclose(fx);
    std::unique_ptr<nflow::InferenceRuntime> rt;
    nflow::Status s = nflow::InferenceRuntime::Create(argv[1], rt);
    if (s.ok() && argc > 8 && std::string(argv[8]) == "int8") rt->EnableInt8Gemm();
    if (s.ok()) s = rt->Run(x.data(), {b, n, ci}, y.data(), {b, n, co});
    std::printf("status %d\n", static_cast<int>(s.code()));
    if (!s.ok()) return 0;
    FILE* fy = std::fopen(argv[7], "wb");
    if (!fy || std::fwrite(y.data(), sizeof(float), y.size(), fy) != y.size()) return 4;
    std::fclose(fy);
    return 0;
}
