// runtime.cpp -- nflow::InferenceRuntime for FNO1d and FNO2d on the device
// (cpp/src/runtime.cpp:15-101, 150-173, cpp/include/neuroflow/runtime.h:
// 64-121): load a NeuroIR binary, apply the NIRQ weight fake-quant
// (fno.cpp:209-300, 997-1020), optionally build the INT8 local-linear blobs
// (EnableInt8Gemm, fno.cpp:325-406; FNO1d only, as in the reference), and
// run FNO1d::Forward (fno.cpp:408-700) or FNO2d::Forward (fno.cpp:777-995)
// with every stage on the GPU:
//   FNO1d: lift (fp32 Linear) -> channel-major copy (with layer 0's input
//   fake-quant) -> L x [spectral convolution (channel-major), local linear
//   (token-major; INT8 LinearForwardBatched when dispatched, fp32 Linear
//   otherwise), tail act(x1 + fq(x2)) written in both layouts with the next
//   layer's input fake-quant] -> proj_q + act -> proj_out.
//   FNO2d: lift (+ lift.output fake-quant) -> zero padding -> channel-major
//   copy -> L x [row FFTs, column FFTs of the kept columns, channel mix of
//   the (modes_h, modes_w) corner, inverse column FFTs, inverse row FFTs;
//   fp32 local linear; tail act(x1 + fq(x2))] -> trim -> proj_q + fake-quant
//   + act -> proj_out + fake-quant.
// The weights live in HBM from creation on; a run allocates nothing once
// its workspace (grown on demand) fits the shape.
#include <hip/hip_runtime_api.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "fno_rt.h"
#include "nflow_quant.h"
#include "nflow_runtime.h"
#include "snap.h"
#include "status.h"

namespace nfq {
namespace {

struct LayerQuant {
    bool in_fq = false;       // fake-quant of the layer input (fno.cpp:488-501)
    float in_scale = 1.0f;
    int32_t in_zp = 0;
    int x2_kind = 0;          // 0 none, 1 per tensor, 2 per position, 3 log2 snap
    float x2_scale = 1.0f;
    int32_t x2_zp = 0;
    int pos_width = 0;        // per position: the qparam's width
    int64_t pos_count = 0;    // and its number of entries
    size_t pos_off = 0;       // offset of its scales / zero points in the weight block
    bool int8 = false;        // LinearDispatchTryInt8 takes the INT8 path (fno.cpp:125-159)
    float sa = 1.0f;
    int32_t zpa = 0;
};

void host_fake_quant(float* v, size_t n, float s, float zpf) {
    // fno.cpp:250-255.
    for (size_t i = 0; i < n; ++i) {
        float q = std::round(v[i] / s) + zpf;
        if (q < -128.0f) q = -128.0f;
        if (q > 127.0f) q = 127.0f;
        v[i] = (q - zpf) * s;
    }
}

int snap_exponent_host(float a) {
    const float r = std::round(std::log2(a) * 8.0f) / 8.0f;
    return (r >= -2147483648.0f && r < 2147483648.0f) ? static_cast<int>(r) : INT_MIN;
}

uint32_t fbits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
float ffrom(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// The exponent steps of the log2 snap (fno.cpp:594-601) under this host's
// libm, which is the reference's: the exponent int(round(8 log2 a) / 8) goes
// from -6 (a = 2^-6) to 9 in 15 steps, at a = 2^(-m + 1/16) (m = 6 .. 1) and
// a = 2^(m - 1/16) (m = 1 .. 9).  Each step point is located exactly by
// scanning the floats around it; the scan also checks that the exponent is
// monotone there.
bool snap_thresholds(float thr[15]) {
    int j = 0;
    for (int m = -6; m <= 8; ++m) {
        const int after = m + 1;
        const double target = after <= 0 ? std::exp2(after - 1 + 1.0 / 16) : std::exp2(after - 1.0 / 16);
        const uint32_t u0 = fbits(static_cast<float>(target));
        uint32_t first = 0;
        int prev = INT_MIN;
        for (uint32_t u = u0 - 512; u <= u0 + 512; ++u) {
            const int e = snap_exponent_host(ffrom(u));
            if (e != m && e != after) return false;
            if (prev != INT_MIN && e < prev) return false;
            if (e == after && !first) first = u;
            prev = e;
        }
        if (!first || snap_exponent_host(ffrom(u0 - 512)) != m) return false;
        thr[j++] = ffrom(first);
    }
    return true;
}

// Stage twiddles of fft.cpp:50-63 (w starts at (1, 0), w *= wlen with
// wlen = (cos, sin) of (+-2 * pi) / len; the product in the reference
// build's fused form), stage len at entries len/2 - 1 .. len - 2.
void twiddles(int n, bool inverse, std::vector<float>& out) {
    out.assign(2 * static_cast<size_t>(n > 1 ? n - 1 : 1), 0.0f);
    for (int len = 2; len <= n; len <<= 1) {
        const float ang = (inverse ? 2.0f : -2.0f) * static_cast<float>(M_PI) / static_cast<float>(len);
        float sn, cs;
        sincosf(ang, &sn, &cs);
        float wr = 1.0f, wi = 0.0f;
        const int half = len / 2;
        for (int k = 0; k < half; ++k) {
            out[2 * static_cast<size_t>(half - 1 + k)] = wr;
            out[2 * static_cast<size_t>(half - 1 + k) + 1] = wi;
            const float nr = std::fma(wr, cs, -(wi * sn));
            const float ni = std::fma(wr, sn, wi * cs);
            wr = nr;
            wi = ni;
        }
    }
}

bool is_pow2(int64_t n) { return n > 0 && (n & (n - 1)) == 0; }

// The inverse complex FFT of n zeros (fft.cpp:48-68 with the table above):
// the reference's inverse 2-D transform runs it down every column it does
// not mix (fft.cpp:131-141), and its products can carry -0.0f, which the
// row transforms then read as those columns' bins.  out: n complex values.
void zero_column_ifft(int n, const std::vector<float>& tw_inv, std::vector<float>& out) {
    out.assign(2 * static_cast<size_t>(n), 0.0f);
    for (int len = 2; len <= n; len <<= 1) {
        const int half = len / 2;
        for (int i = 0; i < n; i += len) {
            for (int k = 0; k < half; ++k) {
                float* u = out.data() + 2 * static_cast<size_t>(i + k);
                float* v = out.data() + 2 * static_cast<size_t>(i + k + half);
                const float wr = tw_inv[2 * static_cast<size_t>(half - 1 + k)];
                const float wi = tw_inv[2 * static_cast<size_t>(half - 1 + k) + 1];
                const float tr = std::fma(v[0], wr, -(v[1] * wi));
                const float ti = std::fma(v[0], wi, v[1] * wr);
                const float ur = u[0], ui = u[1];
                u[0] = ur + tr;
                u[1] = ui + ti;
                v[0] = ur - tr;
                v[1] = ui - ti;
            }
        }
    }
    const float inv = 1.0f / static_cast<float>(n);
    for (float& f : out) f *= inv;
}

}  // namespace
}  // namespace nfq

using namespace nfq;

struct nflow_runtime {
    std::string op;
    int device = 0;
    int32_t cfg[7] = {};              // the IR's configuration block
    bool fno2d = false;
    int in_ch = 0, out_ch = 0, width = 0, modes = 0, n_layers = 0, pad_factor = 1;
    int modes_h = 0, modes_w = 0;     // FNO2d (modes = modes_h * modes_w there)
    int act = RT_ACT_GELU;
    bool quant_enabled = false;
    bool int8_enabled = false;
    // FNO2d's fake-quants outside the layers (lift / proj_q / proj_out .output).
    FakeQuant fq_lift{}, fq_projq{}, fq_projout{};

    // Host copies of the IR data the runtime needs after creation.
    nflow_ir* ir = nullptr;
    std::map<std::string, std::vector<float>> w;   // weights after the NIRQ fake-quant
    std::vector<LayerQuant> lq;
    float thr[15] = {};

    // Device: one block for every fp32 weight and per-position qparam.
    void* dblock = nullptr;
    std::map<std::string, size_t> off;  // float offsets into dblock
    std::vector<nflow_layer*> int8_layers;

    // Device twiddles per grid length, the zero-column pattern per column
    // length (FNO2d), workspace grown on demand.
    std::map<int, float*> tw;
    std::map<int, float*> zfill;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // Device copies of the host input and output of nflow_runtime_run,
    // grown on demand and kept (a device allocation and free per call cost
    // more than a small batch's whole forward).
    float* stage_x = nullptr;
    float* stage_y = nullptr;
    size_t stage_x_n = 0, stage_y_n = 0;
    // Pinned host copies for inputs and outputs up to kPinnedStageMax
    // floats: the caller's (pageable) arrays are copied into them on the host
    // and moved by DMA, which costs less per small call than a pageable copy.
    float* pin_x = nullptr;
    float* pin_y = nullptr;
    size_t pin_x_n = 0, pin_y_n = 0;

    // Runs on one handle share the tables and the workspace above.  `mu`
    // serialises the host side (table inserts, workspace growth, the INT8
    // cache); `done` is recorded on the stream of every run, and a run on a
    // different stream than the previous one first waits for it, so two runs
    // never use the workspace at the same time on the device.
    std::mutex mu;
    hipStream_t last_stream = nullptr;
    hipEvent_t done = nullptr;
    bool ran = false;

    const float* dw(const std::string& name) const {
        return static_cast<const float*>(dblock) + off.at(name);
    }
};

namespace nfq {
namespace {

void free_runtime(nflow_runtime* rt) {
    if (!rt) return;
    int cur = 0;
    const bool sw = hipGetDevice(&cur) == hipSuccess && cur != rt->device;
    if (sw) (void)hipSetDevice(rt->device);
    for (auto* l : rt->int8_layers) nflow_layer_destroy(l);
    for (auto& kv : rt->tw) (void)hipFree(kv.second);
    for (auto& kv : rt->zfill) (void)hipFree(kv.second);
    if (rt->dblock) (void)hipFree(rt->dblock);
    if (rt->ws) (void)hipFree(rt->ws);
    if (rt->stage_x) (void)hipFree(rt->stage_x);
    if (rt->stage_y) (void)hipFree(rt->stage_y);
    if (rt->pin_x) (void)hipHostFree(rt->pin_x);
    if (rt->pin_y) (void)hipHostFree(rt->pin_y);
    if (rt->done) (void)hipEventDestroy(rt->done);
    if (sw) (void)hipSetDevice(cur);
    if (rt->ir) nflow_ir_close(rt->ir);
    delete rt;
}

int parse_err(const std::string& m) { return set_error(NFLOW_PARSE_ERROR, "runtime: " + m); }

// The weight of the fixed FNO1d sequence (ir_loader.h:274-298) with the
// shape the configuration implies.
int take_weight(nflow_runtime* rt, const std::string& name, std::vector<int64_t> dims) {
    int ndim = 0;
    int64_t d8[8] = {};
    const float* data = nullptr;
    if (nflow_ir_weight(rt->ir, name.c_str(), &ndim, d8, &data) != NFLOW_OK)
        return parse_err("weight name mismatch: " + name + " is missing");
    if (ndim != static_cast<int>(dims.size()))
        return parse_err("weight " + name + " has the wrong rank for the configuration");
    int64_t numel = 1;
    for (int i = 0; i < ndim; ++i) {
        if (d8[i] != dims[i]) return parse_err("weight " + name + " has the wrong shape for the configuration");
        numel *= d8[i];
    }
    rt->w[name].assign(data, data + numel);
    return NFLOW_OK;
}

// EnablePerChannelWeightDequant (fno.cpp:209-300): per-channel qparams of a
// 2-D weight on axis 0 or a 3-D spectral weight on axis 1, else the weight's
// per-tensor qparam.
int dequantise_weight(nflow_runtime* rt, const std::string& name) {
    std::vector<float>& t = rt->w[name];
    int found = 0, n_ch = 0, axis = 0, ndim = 0;
    int64_t d8[8] = {};
    const float* sc = nullptr;
    const int32_t* zp = nullptr;
    (void)nflow_ir_weight(rt->ir, name.c_str(), &ndim, d8, nullptr);
    (void)nflow_ir_per_channel_qparam(rt->ir, name.c_str(), &found, &n_ch, &axis, &sc, &zp);
    if (found) {
        if (ndim == 2 && axis == 0) {
            if (n_ch > d8[0]) return set_error(NFLOW_SHAPE_MISMATCH, "runtime: more channel qparams than rows of " + name);
            for (int64_t c = 0; c < n_ch; ++c)
                host_fake_quant(t.data() + c * d8[1], static_cast<size_t>(d8[1]), sc[c], static_cast<float>(zp[c]));
            return NFLOW_OK;
        }
        if (ndim == 3 && axis == 1) {
            if (n_ch < d8[1]) return set_error(NFLOW_SHAPE_MISMATCH, "runtime: fewer channel qparams than channels of " + name);
            for (int64_t i = 0; i < d8[0]; ++i)
                for (int64_t c = 0; c < d8[1]; ++c)
                    host_fake_quant(t.data() + (i * d8[1] + c) * d8[2], static_cast<size_t>(d8[2]), sc[c],
                                    static_cast<float>(zp[c]));
            return NFLOW_OK;
        }
    }
    float s = 1.0f;
    int32_t z = 0;
    (void)nflow_ir_per_tensor_qparam(rt->ir, name.c_str(), &found, &s, &z);
    if (found) host_fake_quant(t.data(), t.size(), s, static_cast<float>(z));
    return NFLOW_OK;
}

std::vector<std::string> weight_names(const nflow_runtime* rt) {
    std::vector<std::string> names = {"lift.weight", "lift.bias"};
    for (int i = 0; i < rt->n_layers; ++i) {
        const std::string p = "specs." + std::to_string(i);
        names.push_back(p + ".weights_real");
        names.push_back(p + ".weights_imag");
    }
    for (int i = 0; i < rt->n_layers; ++i) {
        const std::string p = "locs." + std::to_string(i);
        names.push_back(p + ".weight");
        names.push_back(p + ".bias");
    }
    for (const char* s : {"proj_q.weight", "proj_q.bias", "proj_out.weight", "proj_out.bias"}) names.push_back(s);
    return names;
}

int init(nflow_runtime* rt) {
    int version = 0, op = 0, act = 0, quant = 0;
    int32_t cfg[8] = {};
    if (int rc = nflow_ir_header(rt->ir, &version, &op, cfg, &act, &quant)) return rc;
    static const char* kOps[] = {"", "FNO1d", "FNO2d", "FNO3d", "DeepONet", "TokenMixer", "GraphOp",
                                 "TokenMixer2D", "GraphOp2D"};
    rt->op = (op >= 1 && op <= 8) ? kOps[op] : "";
    if (op != 1 && op != 2)
        return set_error(NFLOW_UNSUPPORTED_OP,
                         "runtime: the device runtime serves FNO1d and FNO2d (the ops with the "
                         "local-linear layer path); this IR holds " + rt->op);
    std::memcpy(rt->cfg, cfg, sizeof(rt->cfg));
    rt->fno2d = op == 2;
    rt->in_ch = cfg[0];
    rt->out_ch = cfg[1];
    rt->width = cfg[2];
    if (rt->fno2d) {
        // [in_ch, out_ch, width, modes_h, modes_w, n_layers, pad_factor] (ir_loader.h:150-160).
        rt->modes_h = cfg[3];
        rt->modes_w = cfg[4];
        rt->n_layers = cfg[5];
        rt->pad_factor = cfg[6];
        rt->modes = rt->modes_h * rt->modes_w;
    } else {
        rt->modes = cfg[3];
        rt->n_layers = cfg[4];
        rt->pad_factor = cfg[5];
    }
    rt->act = act == 1 ? RT_ACT_RELU : RT_ACT_GELU;
    rt->quant_enabled = quant != 0;
    if (rt->in_ch <= 0 || rt->out_ch <= 0 || rt->width <= 0 || rt->modes_h < 0 || rt->modes_w < 0 || rt->modes < 0 ||
        rt->n_layers < 0)
        return parse_err(std::string("bad ") + rt->op + " configuration");
    const int64_t w = rt->width, m = rt->modes;
    if (int rc = take_weight(rt, "lift.weight", {w, rt->in_ch})) return rc;
    if (int rc = take_weight(rt, "lift.bias", {w})) return rc;
    for (int i = 0; i < rt->n_layers; ++i) {
        const std::string s = "specs." + std::to_string(i), l = "locs." + std::to_string(i);
        // (in, out, modes), or (in, out, modes_h, modes_w) for FNO2d.
        const std::vector<int64_t> sdims =
            rt->fno2d ? std::vector<int64_t>{w, w, rt->modes_h, rt->modes_w} : std::vector<int64_t>{w, w, m};
        if (int rc = take_weight(rt, s + ".weights_real", sdims)) return rc;
        if (int rc = take_weight(rt, s + ".weights_imag", sdims)) return rc;
        if (int rc = take_weight(rt, l + ".weight", {w, w})) return rc;
        if (int rc = take_weight(rt, l + ".bias", {w})) return rc;
    }
    if (int rc = take_weight(rt, "proj_q.weight", {w, w})) return rc;
    if (int rc = take_weight(rt, "proj_q.bias", {w})) return rc;
    if (int rc = take_weight(rt, "proj_out.weight", {rt->out_ch, w})) return rc;
    if (int rc = take_weight(rt, "proj_out.bias", {rt->out_ch})) return rc;
    if (rt->quant_enabled)
        for (const auto& name : weight_names(rt))
            if (int rc = dequantise_weight(rt, name)) return rc;
    // The spectral weights again, held (modes, in, out) for the channel mix.
    for (int i = 0; i < rt->n_layers; ++i) {
        for (const char* part : {"real", "imag"}) {
            const std::vector<float>& src = rt->w["specs." + std::to_string(i) + ".weights_" + part];
            std::vector<float> dst(src.size());
            for (int64_t a = 0; a < w; ++a)
                for (int64_t o = 0; o < w; ++o)
                    for (int64_t k = 0; k < m; ++k) dst[(k * w + a) * w + o] = src[(a * w + o) * m + k];
            rt->w["mix." + std::to_string(i) + "." + part] = std::move(dst);
        }
    }

    // Per-layer activation quantisation (fno.cpp:482-501, 571-648).
    rt->lq.assign(rt->n_layers, LayerQuant{});
    bool any_snap = false;
    std::vector<std::pair<std::vector<float>, std::vector<int32_t>>> pos(rt->n_layers);
    if (rt->fno2d && rt->quant_enabled) {
        // FNO2d's apply_fake_quant (fno.cpp:810-843): the FP8 qparam of the
        // key first (the snap when its scale is positive, else nothing),
        // then the per-tensor INT8 one; no per-token path.
        auto fq_of = [&](const std::string& key) {
            FakeQuant f{};
            int found = 0;
            float fs = 0.0f;
            (void)nflow_ir_fp8_qparam(rt->ir, key.c_str(), &found, &fs);
            if (found) {
                if (fs > 0.0f) {
                    f.on = 3;
                    f.scale = fs;
                    any_snap = true;
                }
                return f;
            }
            float s = 1.0f;
            int32_t z = 0;
            (void)nflow_ir_per_tensor_qparam(rt->ir, key.c_str(), &found, &s, &z);
            if (found) {
                f.on = 1;
                f.scale = s;
                f.zpf = static_cast<float>(z);
            }
            return f;
        };
        rt->fq_lift = fq_of("lift.output");
        rt->fq_projq = fq_of("proj_q.output");
        rt->fq_projout = fq_of("proj_out.output");
        for (int i = 0; i < rt->n_layers; ++i) {
            const FakeQuant f = fq_of("locs." + std::to_string(i) + ".output");
            rt->lq[i].x2_kind = f.on;
            rt->lq[i].x2_scale = f.scale;
            rt->lq[i].x2_zp = static_cast<int32_t>(f.zpf);
        }
    }
    for (int i = 0; i < rt->n_layers && rt->quant_enabled && !rt->fno2d; ++i) {
        LayerQuant& q = rt->lq[i];
        const std::string in_key = i == 0 ? "lift.output" : "locs." + std::to_string(i - 1) + ".output";
        int found = 0;
        (void)nflow_ir_per_tensor_qparam(rt->ir, in_key.c_str(), &found, &q.in_scale, &q.in_zp);
        q.in_fq = found != 0;
        const std::string key = "locs." + std::to_string(i) + ".output";
        float fs = 0.0f;
        (void)nflow_ir_fp8_qparam(rt->ir, key.c_str(), &found, &fs);
        if (found) {
            if (fs > 0.0f) {
                q.x2_kind = 3;
                q.x2_scale = fs;
                any_snap = true;
            }
            continue;
        }
        int n_tok = 0, width = 0;
        const float* ps = nullptr;
        const int32_t* pz = nullptr;
        (void)nflow_ir_per_token_qparam(rt->ir, key.c_str(), &found, &n_tok, &width, &ps, &pz);
        if (found) {
            q.x2_kind = 2;
            q.pos_width = width;
            q.pos_count = n_tok;
            pos[i].first.assign(ps, ps + n_tok);
            pos[i].second.assign(pz, pz + n_tok);
            continue;
        }
        (void)nflow_ir_per_tensor_qparam(rt->ir, key.c_str(), &found, &q.x2_scale, &q.x2_zp);
        if (found) q.x2_kind = 1;
    }
    if (any_snap && !snap_thresholds(rt->thr))
        return set_error(NFLOW_INTERNAL, "runtime: the host libm's log2 is not monotone at a snap step");
    if (any_snap && !nfq::snap_table_binned(rt->thr))
        return set_error(NFLOW_INTERNAL, "runtime: a snap step of the host libm lies outside its binade");
    for (FakeQuant* f : {&rt->fq_lift, &rt->fq_projq, &rt->fq_projout})
        std::memcpy(f->thr, rt->thr, sizeof(f->thr));

    // Upload: every weight, then the per-position qparams (scales, then zps).
    size_t total = 0;
    for (const auto& kv : rt->w) {
        rt->off[kv.first] = total;
        total += (kv.second.size() + 63) & ~size_t(63);
    }
    for (int i = 0; i < rt->n_layers; ++i) {
        if (rt->lq[i].x2_kind != 2) continue;
        rt->lq[i].pos_off = total;
        total += ((2 * pos[i].first.size()) + 63) & ~size_t(63);
    }
    std::vector<float> host(total ? total : 1, 0.0f);
    for (const auto& kv : rt->w) std::memcpy(host.data() + rt->off[kv.first], kv.second.data(), kv.second.size() * 4);
    for (int i = 0; i < rt->n_layers; ++i) {
        if (rt->lq[i].x2_kind != 2) continue;
        std::memcpy(host.data() + rt->lq[i].pos_off, pos[i].first.data(), pos[i].first.size() * 4);
        std::memcpy(host.data() + rt->lq[i].pos_off + pos[i].first.size(), pos[i].second.data(),
                    pos[i].second.size() * 4);
    }
    (void)hipGetDevice(&rt->device);
    if (hipMalloc(&rt->dblock, host.size() * 4) != hipSuccess) {
        rt->dblock = nullptr;
        return set_error(NFLOW_INTERNAL, "runtime: device allocation of the weights failed");
    }
    if (hipMemcpy(rt->dblock, host.data(), host.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
        return set_error(NFLOW_INTERNAL, "runtime: weight upload failed");
    return NFLOW_OK;
}

// Ensure `bytes` of workspace (not stream-ordered: waits for the device
// before freeing a smaller one).
int ensure_ws(nflow_runtime* rt, size_t bytes) {
    if (bytes <= rt->ws_bytes) return NFLOW_OK;
    if (rt->ws) {
        (void)hipDeviceSynchronize();
        (void)hipFree(rt->ws);
        rt->ws = nullptr;
        rt->ws_bytes = 0;
    }
    if (hipMalloc(&rt->ws, bytes) != hipSuccess) {
        rt->ws = nullptr;
        return set_error(NFLOW_INTERNAL, "runtime: workspace allocation failed");
    }
    rt->ws_bytes = bytes;
    return NFLOW_OK;
}

const float* twiddle_table(nflow_runtime* rt, int n) {
    auto it = rt->tw.find(n);
    if (it != rt->tw.end()) return it->second;
    std::vector<float> f, inv;
    twiddles(n, false, f);
    twiddles(n, true, inv);
    float* d = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d), (f.size() + inv.size()) * 4) != hipSuccess) return nullptr;
    if (hipMemcpy(d, f.data(), f.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d + f.size(), inv.data(), inv.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return nullptr;
    }
    rt->tw[n] = d;
    return d;
}

// The zero-column pattern of a column length, uploaded once (FNO2d).
const float2* zfill_table(nflow_runtime* rt, int n) {
    auto it = rt->zfill.find(n);
    if (it != rt->zfill.end()) return reinterpret_cast<const float2*>(it->second);
    std::vector<float> inv, z;
    twiddles(n, true, inv);
    zero_column_ifft(n, inv, z);
    float* d = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d), z.size() * 4) != hipSuccess) return nullptr;
    if (hipMemcpy(d, z.data(), z.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return nullptr;
    }
    rt->zfill[n] = d;
    return reinterpret_cast<const float2*>(d);
}

int check_shapes(const nflow_runtime* rt, const int64_t* xs, int xn, const int64_t* ys, int yn) {
    if (rt->fno2d) {
        // FNO2d::Forward's checks, in its order and with its messages (fno.cpp:778-795).
        if (!xs || xn != 4) return set_error(NFLOW_SHAPE_MISMATCH, "expected 4D input (batch, h, w, in_ch)");
        if (xs[3] != rt->in_ch) return set_error(NFLOW_SHAPE_MISMATCH, "input channels mismatch");
        if (!ys || yn != 4 || ys[0] != xs[0] || ys[1] != xs[1] || ys[2] != xs[2] || ys[3] != rt->out_ch)
            return set_error(NFLOW_SHAPE_MISMATCH, "output buffer shape mismatch");
        if (!is_pow2(xs[1]) || !is_pow2(xs[2]))
            return set_error(NFLOW_INVALID_ARG, "FNO2d: H and W must each be a power of two");
        return NFLOW_OK;
    }
    // FNO1d::Forward's checks, in its order and with its messages (fno.cpp:409-425).
    if (!xs || xn != 3) return set_error(NFLOW_SHAPE_MISMATCH, "expected 3D input (batch, n, in_ch)");
    if (xs[2] != rt->in_ch) return set_error(NFLOW_SHAPE_MISMATCH, "input channels mismatch");
    if (!ys || yn != 3 || ys[0] != xs[0] || ys[1] != xs[1] || ys[2] != rt->out_ch)
        return set_error(NFLOW_SHAPE_MISMATCH, "output buffer shape mismatch");
    if (!is_pow2(xs[1])) return set_error(NFLOW_INVALID_ARG, "Stage 1: input length n must be a power of two");
    return NFLOW_OK;
}

int launch_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        return set_error(NFLOW_INTERNAL, std::string("runtime: ") + what + ": " + hipGetErrorString(e));
    return NFLOW_OK;
}

// FNO1d::Forward on device buffers (fno.cpp:408-700).
int run_device(nflow_runtime* rt, const float* x, const int64_t* xs, float* y, hipStream_t st) {
    const int64_t b = xs[0], n = xs[1];
    const int w = rt->width;
    int64_t n_pad = n;
    if (rt->pad_factor > 1) {
        const int64_t r = n % rt->pad_factor;
        n_pad = n + (r == 0 ? 0 : rt->pad_factor - r);
    }
    if (!is_pow2(n_pad))
        return set_error(NFLOW_INVALID_ARG, "runtime: the padded length is not a power of two (the FFT needs one)");
    if (n_pad > kFftMaxPoints)
        return set_error(NFLOW_UNSUPPORTED_OP, "runtime: grids longer than 8192 points are not supported");
    if (rt->modes > n_pad / 2 + 1)
        return set_error(NFLOW_INVALID_ARG, "runtime: modes exceed the n/2 + 1 bins of the grid");
    if (b == 0) return NFLOW_OK;
    const int64_t M = b * n_pad;
    if (M > INT32_MAX) return set_error(NFLOW_INVALID_ARG, "runtime: batch * points exceeds the batched API's int");
    for (int i = 0; i < rt->n_layers; ++i) {
        const LayerQuant& q = rt->lq[i];
        if (q.x2_kind == 2 && (q.pos_width != w || q.pos_count < n_pad * w))
            return set_error(NFLOW_SHAPE_MISMATCH, "runtime: per-token qparams of locs." + std::to_string(i) +
                                                       ".output do not cover (points, width)");
    }
    const float* tw = twiddle_table(rt, static_cast<int>(n_pad));
    if (!tw) return set_error(NFLOW_INTERNAL, "runtime: twiddle upload failed");
    // Workspace: h (token-major), hc (channel-major), x1c, x2 (M x w each)
    // and the kept spectrum.
    const size_t act_elems = static_cast<size_t>(M) * w;
    const size_t spec_elems = static_cast<size_t>(b) * w * (rt->modes > 0 ? rt->modes : 1) * 2;
    const size_t a64 = (act_elems + 63) & ~size_t(63);
    if (int rc = ensure_ws(rt, (4 * a64 + 2 * spec_elems) * sizeof(float))) return rc;
    float* H = static_cast<float*>(rt->ws);
    float* HC = H + a64;
    float* X1C = HC + a64;
    float* X2 = X1C + a64;
    float* SPEC = X2 + a64;
    float* SPEC2 = SPEC + spec_elems;
    auto in_fq = [&](int i) {
        FakeQuant f{0, 1.0f, 0.0f};
        if (i < rt->n_layers && rt->lq[i].in_fq) f = FakeQuant{1, rt->lq[i].in_scale, static_cast<float>(rt->lq[i].in_zp)};
        return f;
    };

    if (rt->in_ch == 1 && n_pad == n && rt->n_layers > 0) {
        // The lift (one input channel) and the layout change in one pass.
        if (int rc = launch_check(launch_lift_layout(x, rt->dw("lift.weight"), rt->dw("lift.bias"), H, HC, b,
                                                     static_cast<int>(n), w, in_fq(0), st),
                                  "lift + layout change"))
            return rc;
    } else {
        LinArgs lift{x, rt->dw("lift.weight"), rt->dw("lift.bias"), H, b, static_cast<int>(n_pad), static_cast<int>(n),
                     static_cast<int>(n), rt->in_ch, w, RT_ACT_NONE};
        if (int rc = launch_check(launch_linear_ref(lift, st), "lift")) return rc;
        if (rt->n_layers > 0)
            if (int rc = launch_check(launch_to_channel_major(H, HC, b, static_cast<int>(n_pad), w, in_fq(0), st),
                                      "layout change"))
                return rc;
    }
    int log2n = 0;
    while ((int64_t(1) << log2n) < n_pad) ++log2n;
    for (int i = 0; i < rt->n_layers; ++i) {
        const LayerQuant& q = rt->lq[i];
        const std::string si = std::to_string(i);
        SpecArgs sp{HC, SPEC, SPEC2, X1C, rt->dw("mix." + si + ".real"), rt->dw("mix." + si + ".imag"),
                    tw, tw + 2 * (n_pad > 1 ? n_pad - 1 : 1), b, static_cast<int>(n_pad), log2n, w, rt->modes,
                    1.0f / static_cast<float>(n_pad)};
        if (int rc = launch_check(launch_spectral(sp, st), "spectral convolution")) return rc;
        PostArgs pa{};
        pa.x2 = X2;
        pa.x1c = X1C;
        pa.h = H;
        pa.hc = HC;
        pa.samples = b;
        pa.n = static_cast<int>(n_pad);
        pa.w = w;
        pa.kind = q.x2_kind;
        pa.scale = q.x2_scale;
        pa.zpf = static_cast<float>(q.x2_zp);
        if (q.x2_kind == 2) {
            pa.pos_scales = static_cast<const float*>(rt->dblock) + q.pos_off;
            pa.pos_zps = reinterpret_cast<const int32_t*>(pa.pos_scales + q.pos_count);
        }
        std::memcpy(pa.thr, rt->thr, sizeof(pa.thr));
        pa.act = rt->act;
        pa.fq_next = in_fq(i + 1);
        // The INT8 layer and the tail in one launch where it applies (the
        // same bits as the two launches below).
        LayerTailArgs lt{};
        int lin = 0, lout = 0;
        if (q.int8 && rt->int8_enabled && layer_int8_arrays(rt->int8_layers[i], &lt, &lin, &lout) &&
            layer_tail_ok(pa, lin, lout)) {
            lt.p = pa;
            lt.sA = q.sa;
            lt.zpA = q.zpa;
            if (int rc = launch_check(launch_layer_tail(lt, st), "layer + tail")) return rc;
            continue;
        }
        // Likewise the fp32 local linear and the tail.
        if (!(q.int8 && rt->int8_enabled) && linear_tail_ok(pa, rt->dw("locs." + si + ".weight"))) {
            if (int rc = launch_check(launch_linear_tail(pa, rt->dw("locs." + si + ".weight"),
                                                         rt->dw("locs." + si + ".bias"), st),
                                      "local linear + tail"))
                return rc;
            continue;
        }
        if (q.int8 && rt->int8_enabled) {
            if (int rc = nflow_layer_forward_per_tensor(rt->int8_layers[i], M, H, X2, q.sa, q.zpa, st)) return rc;
        } else {
            LinArgs loc{H, rt->dw("locs." + si + ".weight"), rt->dw("locs." + si + ".bias"), X2, b,
                        static_cast<int>(n_pad), static_cast<int>(n_pad), static_cast<int>(n_pad), w, w, RT_ACT_NONE};
            if (int rc = launch_check(launch_linear_ref(loc, st), "local linear")) return rc;
        }
        if (int rc = launch_check(launch_post(pa, st), "layer tail")) return rc;
    }
    // Trim, proj_q + act, proj_out (fno.cpp:662-698): one launch where it
    // applies (the same bits as the two below).
    ProjArgs pj{H, y, rt->dw("proj_q.weight"), rt->dw("proj_q.bias"), rt->dw("proj_out.weight"),
                rt->dw("proj_out.bias"), b, static_cast<int>(n), static_cast<int>(n_pad), w, rt->out_ch, rt->act,
                FakeQuant{}, FakeQuant{}};
    if (proj_tail_ok(pj)) return launch_check(launch_proj_tail(pj, st), "projection");
    LinArgs pq{H, rt->dw("proj_q.weight"), rt->dw("proj_q.bias"), X2, b, static_cast<int>(n), static_cast<int>(n),
               static_cast<int>(n_pad), w, w, rt->act};
    if (int rc = launch_check(launch_linear_ref(pq, st), "proj_q")) return rc;
    LinArgs po{X2, rt->dw("proj_out.weight"), rt->dw("proj_out.bias"), y, b, static_cast<int>(n), static_cast<int>(n),
               static_cast<int>(n), w, rt->out_ch, RT_ACT_NONE};
    return launch_check(launch_linear_ref(po, st), "proj_out");
}

// FNO2d::Forward on device buffers (fno.cpp:777-995).
int run_device_2d(nflow_runtime* rt, const float* x, const int64_t* xs, float* y, hipStream_t st) {
    const int64_t b = xs[0];
    const int H = static_cast<int>(xs[1]), W = static_cast<int>(xs[2]);
    const int w = rt->width, mh = rt->modes_h, mw = rt->modes_w;
    int Hp = H, Wp = W;
    if (rt->pad_factor > 1) {
        const int pf = rt->pad_factor;
        Hp = H + (pf - H % pf) % pf;
        Wp = W + (pf - W % pf) % pf;
    }
    const bool padded = Hp != H || Wp != W;
    if (!is_pow2(Hp) || !is_pow2(Wp))
        return set_error(NFLOW_INVALID_ARG, "runtime: the padded grid is not a power of two (the FFT needs one)");
    if (Hp > kFftMaxPoints || Wp > kFftMaxPoints)
        return set_error(NFLOW_UNSUPPORTED_OP, "runtime: grid sides longer than 8192 points are not supported");
    if (mh > Hp || mw > Wp / 2 + 1)
        return set_error(NFLOW_INVALID_ARG, "runtime: modes exceed the bins of the grid");
    if (b == 0) return NFLOW_OK;
    const int64_t pts = static_cast<int64_t>(Hp) * Wp, pts0 = static_cast<int64_t>(H) * W;
    if (pts > INT32_MAX) return set_error(NFLOW_INVALID_ARG, "runtime: the grid exceeds the Linear's int");
    const float* twW = twiddle_table(rt, Wp);
    const float* twH = twiddle_table(rt, Hp);
    const float2* zf = zfill_table(rt, Hp);
    if (!twW || !twH || !zf) return set_error(NFLOW_INTERNAL, "runtime: twiddle upload failed");
    const float* twW_inv = twW + 2 * (Wp > 1 ? Wp - 1 : 1);
    const float* twH_inv = twH + 2 * (Hp > 1 ? Hp - 1 : 1);
    // Workspace: h (token-major), hc (channel-major), x1c, x2 (b Hp Wp w each),
    // the row spectra (b w Hp mw complex; reused for the inverse), the kept
    // corner and its mix (b w mh mw complex each), and with padding the
    // unpadded grid (b H W w).
    auto r64 = [](size_t v) { return (v + 63) & ~size_t(63); };
    const size_t act_e = r64(static_cast<size_t>(b) * pts * w);
    const size_t row_e = r64(static_cast<size_t>(b) * w * Hp * (mw > 0 ? mw : 1) * 2);
    const size_t cor_e = r64(static_cast<size_t>(b) * w * (mh * mw > 0 ? mh * mw : 1) * 2);
    const size_t pad_e = padded ? r64(static_cast<size_t>(b) * pts0 * w) : 0;
    if (int rc = ensure_ws(rt, (4 * act_e + row_e + 2 * cor_e + pad_e) * sizeof(float))) return rc;
    float* Hb = static_cast<float*>(rt->ws);
    float* HC = Hb + act_e;
    float* X1C = HC + act_e;
    float* X2 = X1C + act_e;
    float* R = X2 + act_e;
    float* S = R + row_e;
    float* SM = S + cor_e;
    float* P = SM + cor_e;
    int log2W = 0, log2H = 0;
    while ((1 << log2W) < Wp) ++log2W;
    while ((1 << log2H) < Hp) ++log2H;

    // Lift (fno.cpp:848-852), padding (fno.cpp:867-891), layout change with
    // lift.output's fake-quant (fno.cpp:852-865; the pads are zeros, which
    // every fake-quant keeps at +0).
    const int ip0 = static_cast<int>(pts0);
    if (rt->in_ch == 1 && !padded && rt->n_layers > 0) {
        // The lift (one input channel) and the layout change in one pass.
        if (int rc = launch_check(launch_lift_layout(x, rt->dw("lift.weight"), rt->dw("lift.bias"), Hb, HC, b,
                                                     static_cast<int>(pts), w, rt->fq_lift, st),
                                  "lift + layout change"))
            return rc;
    } else {
        LinArgs lift{x, rt->dw("lift.weight"), rt->dw("lift.bias"), padded ? P : Hb, b, ip0, ip0, ip0, rt->in_ch, w,
                     RT_ACT_NONE};
        if (int rc = launch_check(launch_linear_ref(lift, st), "lift")) return rc;
        if (padded)
            if (int rc = launch_check(launch_pad2d(P, Hb, b, H, W, Hp, Wp, w, false, st), "padding")) return rc;
        if (rt->n_layers > 0) {
            if (int rc = launch_check(launch_to_channel_major(Hb, HC, b, static_cast<int>(pts), w, rt->fq_lift, st),
                                      "layout change"))
                return rc;
        } else if (int rc = launch_check(launch_fq_act(Hb, b * pts * w, rt->fq_lift, RT_ACT_NONE, st),
                                         "lift fake-quant")) {
            return rc;
        }
    }
    for (int i = 0; i < rt->n_layers; ++i) {
        const LayerQuant& q = rt->lq[i];
        const std::string si = std::to_string(i);
        // Spectral convolution (fno.cpp:717-771): rows, kept columns, mix, back.
        SpecArgs rows{};
        rows.hc = HC;
        rows.spec = R;
        rows.samples = b;
        rows.w = w * Hp;
        rows.n = Wp;
        rows.log2n = log2W;
        rows.modes = mw;
        rows.tw_fwd = twW;
        if (int rc = launch_check(launch_rfft_rows(rows, st), "row FFT")) return rc;
        ColArgs cf{R, S, twH, b * w, Hp, log2H, mw, mh, 1.0f};
        if (int rc = launch_check(launch_cfft_cols(cf, false, st), "column FFT")) return rc;
        SpecArgs mix{};
        mix.spec = S;
        mix.spec_mixed = SM;
        mix.mix_real = rt->dw("mix." + si + ".real");
        mix.mix_imag = rt->dw("mix." + si + ".imag");
        mix.samples = b;
        mix.w = w;
        mix.modes = mh * mw;
        if (int rc = launch_check(launch_spec_mix(mix, st), "channel mix")) return rc;
        ColArgs ci{SM, R, twH_inv, b * w, Hp, log2H, mw, mh, 1.0f / static_cast<float>(Hp)};
        if (int rc = launch_check(launch_cfft_cols(ci, true, st), "inverse column FFT")) return rc;
        SpecArgs irows{};
        irows.spec_mixed = R;
        irows.x1c = X1C;
        irows.samples = b;
        irows.w = w * Hp;
        irows.n = Wp;
        irows.log2n = log2W;
        irows.modes = mw;
        irows.tw_inv = twW_inv;
        irows.inv_n = 1.0f / static_cast<float>(Wp);
        irows.fill = zf;
        irows.fill_period = Hp;
        if (int rc = launch_check(launch_irfft_rows(irows, st), "inverse row FFT")) return rc;
        const int ip = static_cast<int>(pts);
        if (q.int8 && rt->int8_enabled && b * pts > INT32_MAX)
            return set_error(NFLOW_INVALID_ARG, "runtime: batch * points exceeds the batched API's int");
        // Tail (fno.cpp:934-945).
        PostArgs pa{};
        pa.x2 = X2;
        pa.x1c = X1C;
        pa.h = Hb;
        pa.hc = HC;
        pa.samples = b;
        pa.n = ip;
        pa.w = w;
        pa.kind = q.x2_kind;
        pa.scale = q.x2_scale;
        pa.zpf = static_cast<float>(q.x2_zp);
        std::memcpy(pa.thr, rt->thr, sizeof(pa.thr));
        pa.act = rt->act;
        // The INT8 layer and the tail in one launch where it applies (as FNO1d).
        LayerTailArgs lt{};
        int lin = 0, lout = 0;
        if (q.int8 && rt->int8_enabled && layer_int8_arrays(rt->int8_layers[i], &lt, &lin, &lout) &&
            layer_tail_ok(pa, lin, lout)) {
            lt.p = pa;
            lt.sA = q.sa;
            lt.zpA = q.zpa;
            if (int rc = launch_check(launch_layer_tail(lt, st), "layer + tail")) return rc;
            continue;
        }
        if (!(q.int8 && rt->int8_enabled) && linear_tail_ok(pa, rt->dw("locs." + si + ".weight"))) {
            if (int rc = launch_check(launch_linear_tail(pa, rt->dw("locs." + si + ".weight"),
                                                         rt->dw("locs." + si + ".bias"), st),
                                      "local linear + tail"))
                return rc;
            continue;
        }
        // Local linear (fno.cpp:906-932): fp32 as in the reference, or, after
        // the FNO2d INT8 opt-in, FNO1d's INT8 branch (LinearForwardBatched
        // with the input key's per-tensor qparam, then + bias).
        if (q.int8 && rt->int8_enabled) {
            if (int rc = nflow_layer_forward_per_tensor(rt->int8_layers[i], b * pts, Hb, X2, q.sa, q.zpa, st))
                return rc;
        } else {
            LinArgs loc{Hb, rt->dw("locs." + si + ".weight"), rt->dw("locs." + si + ".bias"), X2, b, ip, ip, ip, w,
                        w, RT_ACT_NONE};
            if (int rc = launch_check(launch_linear_ref(loc, st), "local linear")) return rc;
        }
        if (int rc = launch_check(launch_post(pa, st), "layer tail")) return rc;
    }
    // Trim (fno.cpp:946-964), proj_q + fake-quant + act, proj_out + fake-quant (fno.cpp:966-993).
    const float* hsrc = Hb;
    if (padded) {
        if (int rc = launch_check(launch_pad2d(Hb, P, b, H, W, Hp, Wp, w, true, st), "trim")) return rc;
        hsrc = P;
    }
    ProjArgs pj{hsrc, y, rt->dw("proj_q.weight"), rt->dw("proj_q.bias"), rt->dw("proj_out.weight"),
                rt->dw("proj_out.bias"), b, ip0, ip0, w, rt->out_ch, rt->act, rt->fq_projq, rt->fq_projout};
    if (proj_tail_ok(pj)) return launch_check(launch_proj_tail(pj, st), "projection");
    const bool pq_fq = rt->fq_projq.on != 0;
    LinArgs pq{hsrc, rt->dw("proj_q.weight"), rt->dw("proj_q.bias"), X2, b, ip0, ip0, ip0, w, w,
               pq_fq ? static_cast<int>(RT_ACT_NONE) : rt->act};
    if (int rc = launch_check(launch_linear_ref(pq, st), "proj_q")) return rc;
    if (pq_fq)
        if (int rc = launch_check(launch_fq_act(X2, b * pts0 * w, rt->fq_projq, rt->act, st), "proj_q fake-quant"))
            return rc;
    LinArgs po{X2, rt->dw("proj_out.weight"), rt->dw("proj_out.bias"), y, b, ip0, ip0, ip0, w, rt->out_ch,
               RT_ACT_NONE};
    if (int rc = launch_check(launch_linear_ref(po, st), "proj_out")) return rc;
    return launch_check(launch_fq_act(y, b * pts0 * rt->out_ch, rt->fq_projout, RT_ACT_NONE, st),
                        "proj_out fake-quant");
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        int cur = 0;
        if (hipGetDevice(&cur) == hipSuccess && cur != dev && hipSetDevice(dev) == hipSuccess) prev = cur;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Orders a run on `st` after the handle's previous run (called with rt->mu
// held) and, once the run is enqueued, marks its end.
int order_run(nflow_runtime* rt, hipStream_t st) {
    if (!rt->done && hipEventCreateWithFlags(&rt->done, hipEventDisableTiming) != hipSuccess) {
        rt->done = nullptr;
        return set_error(NFLOW_INTERNAL, "runtime_run: event creation failed");
    }
    if (rt->ran && st != rt->last_stream && hipStreamWaitEvent(st, rt->done, 0) != hipSuccess)
        return set_error(NFLOW_INTERNAL, "runtime_run: cross-stream wait failed");
    return NFLOW_OK;
}

// A failed run is marked too: kernels it queued before failing use the
// handle's workspace, and a later run on another stream must wait for them.
int mark_run(nflow_runtime* rt, hipStream_t st, int rc) {
    if (hipEventRecord(rt->done, st) != hipSuccess) {
        if (rc) return rc;   // the run's own error first
        return set_error(NFLOW_INTERNAL, "runtime_run: event record failed");
    }
    rt->last_stream = st;
    rt->ran = true;
    return rc;
}

int create_from(nflow_ir* ir, nflow_runtime** out) {
    nflow_runtime* rt = new (std::nothrow) nflow_runtime;
    if (!rt) {
        nflow_ir_close(ir);
        return set_error(NFLOW_INTERNAL, "runtime: out of host memory");
    }
    rt->ir = ir;
    if (int rc = init(rt)) {
        const std::string msg = nflow_last_error();
        free_runtime(rt);
        return set_error(rc, msg);
    }
    *out = rt;
    return NFLOW_OK;
}

}  // namespace
}  // namespace nfq

extern "C" {

int nflow_runtime_create(const char* ir_path, nflow_runtime** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "runtime_create: null handle pointer");
    *out = nullptr;
    if (!ir_path) return set_error(NFLOW_INVALID_ARG, "runtime_create: null path");
    nflow_ir* ir = nullptr;
    if (int rc = nflow_ir_open(ir_path, &ir)) return rc;
    return create_from(ir, out);
}

int nflow_runtime_create_memory(const void* data, size_t bytes, nflow_runtime** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "runtime_create_memory: null handle pointer");
    *out = nullptr;
    nflow_ir* ir = nullptr;
    if (int rc = nflow_ir_open_memory(data, bytes, &ir)) return rc;
    return create_from(ir, out);
}

int nflow_runtime_destroy(nflow_runtime* rt) {
    clear_error();
    free_runtime(rt);
    return NFLOW_OK;
}

const char* nflow_runtime_op(const nflow_runtime* rt) { return rt ? rt->op.c_str() : ""; }

int nflow_runtime_config(const nflow_runtime* rt, int32_t* config7, int* activation, int* quant_enabled) {
    clear_error();
    if (!rt) return set_error(NFLOW_INVALID_ARG, "runtime_config: null runtime");
    if (config7) std::memcpy(config7, rt->cfg, sizeof(rt->cfg));
    if (activation) *activation = rt->act == RT_ACT_RELU ? NFLOW_ACT_RELU : NFLOW_ACT_GELU_TANH;
    if (quant_enabled) *quant_enabled = rt->quant_enabled ? 1 : 0;
    return NFLOW_OK;
}

}  // extern "C"

namespace nfq {
namespace {
// EnableInt8Gemm's cache of the dispatched layers (fno.cpp:360-406) and the
// per-layer decision of LinearDispatchTryInt8 (fno.cpp:125-159).
int build_int8_layers(nflow_runtime* rt) {
    DeviceGuard g(rt->device);
    for (auto* l : rt->int8_layers) nflow_layer_destroy(l);
    rt->int8_layers.assign(rt->n_layers, nullptr);
    rt->int8_enabled = true;
    // fno.cpp:360-406 caches lift / proj blobs too, but only locs.{i} is
    // ever dispatched (fno.cpp:529-536); those are the ones built here.
    for (int i = 0; i < rt->n_layers; ++i) {
        LayerQuant& q = rt->lq[i];
        q.int8 = false;
        const std::string key = "locs." + std::to_string(i) + ".weight";
        int found = 0, n_ch = 0, axis = 0;
        const float* sc = nullptr;
        const int32_t* zp = nullptr;
        (void)nflow_ir_per_channel_qparam(rt->ir, key.c_str(), &found, &n_ch, &axis, &sc, &zp);
        if (!found || axis != 0) continue;
        const int w = rt->width;
        if (n_ch < w) return set_error(NFLOW_SHAPE_MISMATCH, "runtime: fewer channel qparams than rows of " + key);
        std::vector<int8_t> wq(static_cast<size_t>(w) * w);
        std::vector<int32_t> sum(w);
        if (int rc = nflow_host_quantise_weight_2d(rt->w[key].data(), w, w, sc, zp, wq.data(), sum.data())) return rc;
        if (int rc = nflow_layer_create_int8(wq.data(), sc, zp, rt->w["locs." + std::to_string(i) + ".bias"].data(),
                                             sum.data(), w, w, &rt->int8_layers[i]))
            return rc;
        // LinearDispatchTryInt8's conditions on the input key (fno.cpp:129-136).
        int use = 0;
        if (int rc = nflow_ir_fno_int8_dispatch(rt->ir, i, &use, &q.sa, &q.zpa)) return rc;
        q.int8 = use != 0;
    }
    return NFLOW_OK;
}
}  // namespace
}  // namespace nfq

extern "C" {

int nflow_runtime_enable_int8_gemm(nflow_runtime* rt) {
    clear_error();
    if (!rt) return set_error(NFLOW_INVALID_ARG, "runtime_enable_int8_gemm: null runtime");
    // runtime.cpp:155-166: a no-op for every model but FNO1d.
    if (rt->fno2d) return NFLOW_OK;
    std::lock_guard<std::mutex> lock(rt->mu);
    return build_int8_layers(rt);
}

int nflow_runtime_enable_int8_gemm_fno2d(nflow_runtime* rt) {
    clear_error();
    if (!rt) return set_error(NFLOW_INVALID_ARG, "runtime_enable_int8_gemm_fno2d: null runtime");
    if (!rt->fno2d)
        return set_error(NFLOW_UNSUPPORTED_OP, "runtime_enable_int8_gemm_fno2d: the model is " + rt->op +
                                                   " (FNO1d has EnableInt8Gemm)");
    std::lock_guard<std::mutex> lock(rt->mu);
    return build_int8_layers(rt);
}

int nflow_runtime_is_int8_gemm_enabled(const nflow_runtime* rt, int* enabled) {
    clear_error();
    if (!rt || !enabled) return set_error(NFLOW_INVALID_ARG, "runtime_is_int8_gemm_enabled: null argument");
    // Under the handle's lock: EnableInt8Gemm sets the flag while it builds.
    std::lock_guard<std::mutex> lock(const_cast<nflow_runtime*>(rt)->mu);
    *enabled = rt->int8_enabled ? 1 : 0;
    return NFLOW_OK;
}

int nflow_runtime_layer_dispatch(const nflow_runtime* rt, int layer_index, int* uses_int8) {
    clear_error();
    if (!rt || !uses_int8) return set_error(NFLOW_INVALID_ARG, "runtime_layer_dispatch: null argument");
    if (layer_index < 0 || layer_index >= rt->n_layers)
        return set_error(NFLOW_INVALID_ARG, "runtime_layer_dispatch: layer index out of range");
    std::lock_guard<std::mutex> lock(const_cast<nflow_runtime*>(rt)->mu);
    *uses_int8 = (rt->int8_enabled && rt->lq[layer_index].int8) ? 1 : 0;
    return NFLOW_OK;
}

int nflow_runtime_run_device(nflow_runtime* rt, const float* x, const int64_t* x_shape, int x_ndim, float* y,
                             const int64_t* y_shape, int y_ndim, void* stream) {
    clear_error();
    if (!rt) return set_error(NFLOW_INVALID_ARG, "runtime_run: null runtime");
    if (int rc = check_shapes(rt, x_shape, x_ndim, y_shape, y_ndim)) return rc;
    if (x_shape[0] > 0 && (!x || !y)) return set_error(NFLOW_INVALID_ARG, "runtime_run: null input/output");
    DeviceGuard g(rt->device);
    std::lock_guard<std::mutex> lock(rt->mu);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (int rc = order_run(rt, st)) return rc;
    const int rc = rt->fno2d ? run_device_2d(rt, x, x_shape, y, st) : run_device(rt, x, x_shape, y, st);
    return mark_run(rt, st, rc);
}

int nflow_runtime_run(nflow_runtime* rt, const float* x, const int64_t* x_shape, int x_ndim, float* y,
                      const int64_t* y_shape, int y_ndim) {
    clear_error();
    if (!rt) return set_error(NFLOW_INVALID_ARG, "runtime_run: null runtime");
    if (int rc = check_shapes(rt, x_shape, x_ndim, y_shape, y_ndim)) return rc;
    size_t nx = 1, ny = 1;
    for (int d = 0; d < x_ndim; ++d) nx *= static_cast<size_t>(x_shape[d]);
    for (int d = 0; d < y_ndim; ++d) ny *= static_cast<size_t>(y_shape[d]);
    if (nx == 0) return NFLOW_OK;
    if (!x || !y) return set_error(NFLOW_INVALID_ARG, "runtime_run: null input/output");
    DeviceGuard g(rt->device);
    std::unique_lock<std::mutex> lock(rt->mu);
    // The staging buffers are used only here, under the lock, and every call
    // returns after the work that reads them has finished, so growing them
    // never frees a buffer that a run still reads.
    auto grow = [](float*& p, size_t& cap, size_t n) {
        if (cap >= n) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        if (hipMalloc(reinterpret_cast<void**>(&p), n * 4) != hipSuccess) {
            p = nullptr;
            return false;
        }
        cap = n;
        return true;
    };
    if (!grow(rt->stage_x, rt->stage_x_n, nx) || !grow(rt->stage_y, rt->stage_y_n, ny))
        return set_error(NFLOW_INTERNAL, "runtime_run: allocation failed");
    auto grow_pinned = [](float*& p, size_t& cap, size_t n) {
        if (cap >= n) return true;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        if (hipHostMalloc(reinterpret_cast<void**>(&p), n * 4, hipHostMallocDefault) != hipSuccess) {
            p = nullptr;
            return false;
        }
        cap = n;
        return true;
    };
    constexpr size_t kPinnedStageMax = size_t(1) << 21;   // floats (8 MiB)
    const bool pinned = nx <= kPinnedStageMax && ny <= kPinnedStageMax &&
                        grow_pinned(rt->pin_x, rt->pin_x_n, nx) && grow_pinned(rt->pin_y, rt->pin_y_n, ny);
    float* dx = rt->stage_x;
    float* dy = rt->stage_y;
    int rc = NFLOW_OK;
    if (pinned) {
        std::memcpy(rt->pin_x, x, nx * 4);
        if (hipMemcpyAsync(dx, rt->pin_x, nx * 4, hipMemcpyHostToDevice, nullptr) != hipSuccess)
            rc = set_error(NFLOW_INTERNAL, "runtime_run: input copy failed");
    } else if (hipMemcpy(dx, x, nx * 4, hipMemcpyHostToDevice) != hipSuccess) {
        rc = set_error(NFLOW_INTERNAL, "runtime_run: input copy failed");
    }
    if (!rc) rc = order_run(rt, nullptr);
    if (!rc) rc = mark_run(rt, nullptr, rt->fno2d ? run_device_2d(rt, dx, x_shape, dy, nullptr)
                                                  : run_device(rt, dx, x_shape, dy, nullptr));
    if (!rc && pinned) {
        if (hipMemcpyAsync(rt->pin_y, dy, ny * 4, hipMemcpyDeviceToHost, nullptr) != hipSuccess ||
            hipStreamSynchronize(nullptr) != hipSuccess)
            rc = set_error(NFLOW_INTERNAL, "runtime_run: output copy failed");
        else
            std::memcpy(y, rt->pin_y, ny * 4);
    } else if (!rc && hipMemcpy(y, dy, ny * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        rc = set_error(NFLOW_INTERNAL, "runtime_run: output copy failed");
    }
    // The output copy (and, pinned, the stream synchronise after it) returns
    // once the forward queued before it on the null stream has finished; a
    // failed call may have left work queued on the staging buffers, so it
    // waits for the device before returning.
    if (rc) (void)hipDeviceSynchronize();
    return rc;
}

}  // extern "C"
