// ref_ir_dump.cpp -- test infrastructure only: loads a NeuroIR binary with
// the reference's own ir_native::LoadBinary (cpp/include/neuroflow/
// ir_loader.h:58-654, compiled from where it lies with cpp/src/tensor.cpp)
// and prints what it read, one record per line, so the tests can compare
// libnflow_quant's reader with it.  FNO1d files only for the weights.
//
//   status <code>
//   op <name> activation <gelu|relu> quant <0|1>
//   cfg <in> <out> <width> <modes> <n_layers> <pad_factor>
//   weight <name> <ndim> <dims...> <fnv1a-64 of the float bytes, hex>
//   act_pt|w_pt <name> <scale bits, hex> <zp>
//   pc <name> <axis> <n> <scale bits...> <zps...>
//   pt <name> <width> <n> <scale bits...> <zps...>
//   fp8 <name> <scale bits>
// Map entries are sorted by name.
#include <algorithm>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "neuroflow/ir_loader.h"

namespace {

uint32_t bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

uint64_t fnv(const float* p, int64_t n) {
    uint64_t h = 1469598103934665603ull;
    const auto* b = reinterpret_cast<const unsigned char*>(p);
    for (int64_t i = 0; i < n * 4; ++i) h = (h ^ b[i]) * 1099511628211ull;
    return h;
}

void weight(const char* name, const nflow::Tensor& t) {
    std::printf("weight %s %zu", name, t.shape().size());
    for (auto d : t.shape()) std::printf(" %" PRId64, static_cast<int64_t>(d));
    std::printf(" %016" PRIx64 "\n", fnv(t.data(), t.numel()));
}

template <typename M>
std::vector<std::string> keys(const M& m) {
    std::vector<std::string> k;
    for (const auto& kv : m) k.push_back(kv.first);
    std::sort(k.begin(), k.end());
    return k;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) return 2;
    nflow::LoadedModel m;
    const auto st = nflow::ir_native::LoadBinary(argv[1], m);
    std::printf("status %d\n", static_cast<int>(st.code()));
    if (!st.ok()) return 0;
    const auto& c = m.fno1d_cfg;
    const std::string act = m.op == "FNO1d" ? c.activation : std::string("-");
    std::printf("op %s activation %s quant %d\n", m.op.c_str(), act.c_str(), m.quant_enabled ? 1 : 0);
    if (m.op == "FNO1d") {
        std::printf("cfg %d %d %d %d %d %d\n", c.in_channels, c.out_channels, c.width, c.modes, c.n_layers,
                    c.pad_factor);
        const auto& w = m.fno1d_weights;
        weight("lift.weight", w.lift_w);
        weight("lift.bias", w.lift_b);
        for (size_t i = 0; i < w.loc_w.size(); ++i) {
            const std::string p = std::to_string(i);
            weight(("specs." + p + ".weights_real").c_str(), w.spec_w_real[i]);
            weight(("specs." + p + ".weights_imag").c_str(), w.spec_w_imag[i]);
            weight(("locs." + p + ".weight").c_str(), w.loc_w[i]);
            weight(("locs." + p + ".bias").c_str(), w.loc_b[i]);
        }
        weight("proj_q.weight", w.proj_q_w);
        weight("proj_q.bias", w.proj_q_b);
        weight("proj_out.weight", w.proj_out_w);
        weight("proj_out.bias", w.proj_out_b);
    }
    for (const auto& k : keys(m.activation_qparams)) {
        const auto& q = m.activation_qparams.at(k);
        std::printf("act_pt %s %08x %d\n", k.c_str(), bits(q.scale), q.zero_point);
    }
    for (const auto& k : keys(m.weight_qparams)) {
        const auto& q = m.weight_qparams.at(k);
        std::printf("w_pt %s %08x %d\n", k.c_str(), bits(q.scale), q.zero_point);
    }
    for (const auto& k : keys(m.weight_per_channel_qparams)) {
        const auto& q = m.weight_per_channel_qparams.at(k);
        std::printf("pc %s %d %zu", k.c_str(), q.channel_axis, q.scales.size());
        for (float s : q.scales) std::printf(" %08x", bits(s));
        for (int32_t z : q.zero_points) std::printf(" %d", z);
        std::printf("\n");
    }
    for (const auto& k : keys(m.activation_per_token_qparams)) {
        const auto& q = m.activation_per_token_qparams.at(k);
        std::printf("pt %s %d %zu", k.c_str(), q.width, q.scales.size());
        for (float s : q.scales) std::printf(" %08x", bits(s));
        for (int32_t z : q.zero_points) std::printf(" %d", z);
        std::printf("\n");
    }
    for (const auto& k : keys(m.activation_fp8_qparams))
        std::printf("fp8 %s %08x\n", k.c_str(), bits(m.activation_fp8_qparams.at(k).scale));
    return 0;
}
