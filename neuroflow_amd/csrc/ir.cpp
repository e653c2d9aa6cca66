// ir.cpp -- the NeuroIR binary (.nneuroir) and its NIRQ quantisation block,
// read on the host, and the IR-driven device layers: what
// ir_native::LoadBinary (cpp/include/neuroflow/ir_loader.h:58-654) hands to
// FNO1d::EnableInt8Gemm (cpp/src/fno.cpp:360-406), with the per-channel
// weight blobs uploaded once as nflow_layer handles, and the per-layer INT8
// decision of LinearDispatchTryInt8 (cpp/src/fno.cpp:125-159, 529-536).
//
// Layout (little-endian; neuroflow/ir/export.py:export_to_binary):
//   "NIR0", u16 version (1..3), u8 op_code (1..8), u8 reserved,
//   i32 config[7 or 8] (8 for op codes 3, 5, 6, 7, 8), u8 activation
//   (1 = relu, anything else gelu), 3 reserved bytes, u32 n_weights, then
//   n_weights records {u8 name_len, name, u8 ndim, i32 dims[ndim],
//   f32 data[prod(dims)]}, then optionally "NIRQ", u8 quant_flag (must be 1),
//   u32 n_qparams and n_qparams records {u8 kind, u8 name_len, name, body}:
//     kind 0 per-tensor INT8: f32 scale, i32 zero_point
//     kind 1 per-channel INT8: u32 n, u8 axis, f32 scales[n], i32 zps[n]
//     kind 2 per-token INT8:   u32 n, u32 width, f32 scales[n], i32 zps[n]
//     kind 3 FP8 E4M3:         f32 scale
// Records are read generically (name, dims, data); the reference reads the
// op's fixed name sequence, which export_to_binary always writes, and fails
// on another order -- this reader accepts any names.  Errors follow the
// reference: FileNotFound for an unreadable file, UnsupportedOp for an
// unknown op code, ParseError for everything else (bad magic or version,
// truncation, quant_flag != 1, an unknown qparam kind).  Bytes after the
// block, or trailing bytes that do not start with "NIRQ", are ignored.
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iterator>
#include <map>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "nflow_quant.h"
#include "status.h"

struct nflow_ir {
    int version = 0;
    int op_code = 0;
    int32_t cfg[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int activation = 0;  // 0 gelu, 1 relu
    bool quant_enabled = false;

    struct Weight {
        std::string name;
        std::vector<int64_t> dims;
        std::vector<float> data;
    };
    std::vector<Weight> weights;
    std::unordered_map<std::string, size_t> weight_index;  // first record of a name

    struct PerTensor { float scale; int32_t zp; };
    struct PerChannel { int axis; std::vector<float> scales; std::vector<int32_t> zps; };
    struct PerToken { int width; std::vector<float> scales; std::vector<int32_t> zps; };
    // The reference's LoadedModel maps (runtime.h:37-62): per-tensor
    // qparams of names ending in ".output" are activation qparams, the rest
    // weight qparams; a later record of a name replaces an earlier one.
    std::map<std::string, PerTensor> act_tensor, weight_tensor;
    std::map<std::string, PerChannel> per_channel;
    std::map<std::string, PerToken> per_token;
    std::map<std::string, float> fp8;
    struct QRecord { std::string name; int kind; };
    std::vector<QRecord> qrecords;  // file order
};

namespace nfq {
namespace {

class Reader {
public:
    Reader(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    size_t off = 0;
    bool has(size_t bytes) const { return off + bytes <= n_ && off + bytes >= off; }
    bool u8(uint8_t& v) { if (!has(1)) return false; v = p_[off++]; return true; }
    template <typename T>
    bool pod(T& v) {
        if (!has(sizeof(T))) return false;
        std::memcpy(&v, p_ + off, sizeof(T));
        off += sizeof(T);
        return true;
    }
    bool bytes(void* dst, size_t len) {
        if (!has(len)) return false;
        std::memcpy(dst, p_ + off, len);
        off += len;
        return true;
    }
    bool str(size_t len, std::string& s) {
        if (!has(len)) return false;
        s.assign(reinterpret_cast<const char*>(p_ + off), len);
        off += len;
        return true;
    }
    bool magic(const char* m) const { return has(4) && std::memcmp(p_ + off, m, 4) == 0; }

private:
    const uint8_t* p_;
    size_t n_;
};

int parse_error(const std::string& what) { return set_error(NFLOW_PARSE_ERROR, "ir: " + what); }

bool ends_with_output(const std::string& s) {
    return s.size() >= 7 && s.compare(s.size() - 7, 7, ".output") == 0;
}

int parse(const uint8_t* p, size_t n, nflow_ir& ir) {
    Reader rd(p, n);
    if (!rd.magic("NIR0")) return parse_error("bad magic in IR file");
    rd.off = 4;
    uint16_t version = 0;
    if (!rd.pod(version)) return parse_error("truncated header");
    if (version < 1 || version > 3) return parse_error("unsupported IR binary version");
    uint8_t op = 0, reserved = 0;
    if (!rd.u8(op) || !rd.u8(reserved)) return parse_error("truncated header");
    if (op < 1 || op > 8) return set_error(NFLOW_UNSUPPORTED_OP, "ir: unknown op_code");
    ir.version = version;
    ir.op_code = op;
    const int cfg_len = (op == 3 || op >= 5) ? 8 : 7;
    for (int i = 0; i < cfg_len; ++i)
        if (!rd.pod(ir.cfg[i])) return parse_error("truncated config");
    uint8_t act = 0;
    if (!rd.u8(act)) return parse_error("truncated activation");
    ir.activation = act == 1 ? 1 : 0;
    rd.off += 3;  // reserved2 (the reference skips it unchecked; n_weights then fails)
    uint32_t n_weights = 0;
    if (!rd.pod(n_weights)) return parse_error("truncated n_weights");
    ir.weights.reserve(n_weights < 4096 ? n_weights : 4096);
    for (uint32_t w = 0; w < n_weights; ++w) {
        nflow_ir::Weight wt;
        uint8_t name_len = 0, ndim = 0;
        if (!rd.u8(name_len)) return parse_error("truncated name_len");
        if (!rd.str(name_len, wt.name)) return parse_error("truncated name");
        if (!rd.u8(ndim)) return parse_error("truncated ndim");
        int64_t numel = 1;
        for (int d = 0; d < ndim; ++d) {
            int32_t v = 0;
            if (!rd.pod(v)) return parse_error("truncated dim");
            if (v < 0) return parse_error("negative dim");
            wt.dims.push_back(v);
            numel *= v;
            if (numel > (int64_t(1) << 40)) return parse_error("truncated data");
        }
        const size_t bytes = static_cast<size_t>(numel) * sizeof(float);
        if (!rd.has(bytes)) return parse_error("truncated data");
        wt.data.resize(static_cast<size_t>(numel));
        rd.bytes(wt.data.data(), bytes);
        ir.weight_index.emplace(wt.name, ir.weights.size());
        ir.weights.push_back(std::move(wt));
    }
    if (!rd.magic("NIRQ")) return NFLOW_OK;
    rd.off += 4;
    uint8_t flag = 0;
    if (!rd.u8(flag)) return parse_error("truncated quant_flag");
    if (flag != 1) return parse_error("unsupported quant_flag");
    ir.quant_enabled = true;
    uint32_t nq = 0;
    if (!rd.pod(nq)) return parse_error("truncated n_qparams");
    for (uint32_t i = 0; i < nq; ++i) {
        uint8_t kind = 0, name_len = 0;
        std::string name;
        if (!rd.u8(kind)) return parse_error("truncated qparam kind");
        if (!rd.u8(name_len)) return parse_error("truncated qparam name_len");
        if (!rd.str(name_len, name)) return parse_error("truncated qparam name");
        if (kind == 0) {
            nflow_ir::PerTensor q{0.0f, 0};
            if (!rd.has(8)) return parse_error("truncated qparam scale/zp");
            rd.pod(q.scale);
            rd.pod(q.zp);
            (ends_with_output(name) ? ir.act_tensor : ir.weight_tensor)[name] = q;
        } else if (kind == 1 || kind == 2) {
            uint32_t cnt = 0;
            uint32_t extra = 0;
            if (kind == 1) {
                uint8_t axis = 0;
                if (!rd.has(5)) return parse_error("truncated per-channel header");
                rd.pod(cnt);
                rd.u8(axis);
                extra = axis;
            } else {
                if (!rd.has(8)) return parse_error("truncated per-token header");
                rd.pod(cnt);
                rd.pod(extra);
            }
            const size_t bytes = static_cast<size_t>(cnt) * 8;
            if (!rd.has(bytes))
                return parse_error(kind == 1 ? "truncated per-channel data" : "truncated per-token data");
            std::vector<float> scales(cnt);
            std::vector<int32_t> zps(cnt);
            rd.bytes(scales.data(), static_cast<size_t>(cnt) * 4);
            rd.bytes(zps.data(), static_cast<size_t>(cnt) * 4);
            if (kind == 1)
                ir.per_channel[name] = nflow_ir::PerChannel{static_cast<int>(extra), std::move(scales), std::move(zps)};
            else
                ir.per_token[name] = nflow_ir::PerToken{static_cast<int>(extra), std::move(scales), std::move(zps)};
        } else if (kind == 3) {
            float s = 0.0f;
            if (!rd.pod(s)) return parse_error("truncated fp8 scale");
            ir.fp8[name] = s;
        } else {
            return parse_error("unsupported qparam kind");
        }
        ir.qrecords.push_back({name, kind});
    }
    return NFLOW_OK;
}

int open_bytes(const uint8_t* p, size_t n, nflow_ir** out) {
    nflow_ir* ir = new (std::nothrow) nflow_ir;
    if (!ir) return set_error(NFLOW_INTERNAL, "ir: out of host memory");
    int rc;
    try {
        rc = parse(p, n, *ir);
    } catch (const std::bad_alloc&) {
        rc = set_error(NFLOW_INTERNAL, "ir: out of host memory");
    }
    if (rc != NFLOW_OK) {
        delete ir;
        return rc;
    }
    *out = ir;
    return NFLOW_OK;
}

const nflow_ir::Weight* find_weight(const nflow_ir* ir, const char* name) {
    auto it = ir->weight_index.find(name);
    return it == ir->weight_index.end() ? nullptr : &ir->weights[it->second];
}

}  // namespace
}  // namespace nfq

using namespace nfq;

extern "C" {

int nflow_ir_open(const char* path, nflow_ir** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "ir_open: null handle pointer");
    *out = nullptr;
    if (!path) return set_error(NFLOW_INVALID_ARG, "ir_open: null path");
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) return set_error(NFLOW_FILE_NOT_FOUND, std::string("cannot open IR file: ") + path);
    std::vector<uint8_t> buf((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    return open_bytes(buf.data(), buf.size(), out);
}

int nflow_ir_open_memory(const void* data, size_t bytes, nflow_ir** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "ir_open_memory: null handle pointer");
    *out = nullptr;
    if (!data && bytes) return set_error(NFLOW_INVALID_ARG, "ir_open_memory: null data");
    return open_bytes(static_cast<const uint8_t*>(data), bytes, out);
}

int nflow_ir_close(nflow_ir* ir) {
    clear_error();
    delete ir;
    return NFLOW_OK;
}

int nflow_ir_header(const nflow_ir* ir, int* version, int* op_code, int32_t* config8, int* activation,
                    int* quant_enabled) {
    clear_error();
    if (!ir) return set_error(NFLOW_INVALID_ARG, "ir_header: null ir");
    if (version) *version = ir->version;
    if (op_code) *op_code = ir->op_code;
    if (config8) std::memcpy(config8, ir->cfg, sizeof(ir->cfg));
    if (activation) *activation = ir->activation;
    if (quant_enabled) *quant_enabled = ir->quant_enabled ? 1 : 0;
    return NFLOW_OK;
}

int nflow_ir_num_weights(const nflow_ir* ir, int* n) {
    clear_error();
    if (!ir || !n) return set_error(NFLOW_INVALID_ARG, "ir_num_weights: null argument");
    *n = static_cast<int>(ir->weights.size());
    return NFLOW_OK;
}

static int weight_out(const nflow_ir::Weight& w, const char** name, int* ndim, int64_t* dims8,
                      const float** data) {
    if (w.dims.size() > 8) return set_error(NFLOW_UNSUPPORTED_OP, "ir: weight has more than 8 dims");
    if (name) *name = w.name.c_str();
    if (ndim) *ndim = static_cast<int>(w.dims.size());
    if (dims8)
        for (size_t d = 0; d < w.dims.size(); ++d) dims8[d] = w.dims[d];
    if (data) *data = w.data.data();
    return NFLOW_OK;
}

int nflow_ir_weight_at(const nflow_ir* ir, int index, const char** name, int* ndim, int64_t* dims8,
                       const float** data) {
    clear_error();
    if (!ir) return set_error(NFLOW_INVALID_ARG, "ir_weight_at: null ir");
    if (index < 0 || static_cast<size_t>(index) >= ir->weights.size())
        return set_error(NFLOW_INVALID_ARG, "ir_weight_at: index out of range");
    return weight_out(ir->weights[index], name, ndim, dims8, data);
}

int nflow_ir_weight(const nflow_ir* ir, const char* name, int* ndim, int64_t* dims8, const float** data) {
    clear_error();
    if (!ir || !name) return set_error(NFLOW_INVALID_ARG, "ir_weight: null argument");
    const auto* w = find_weight(ir, name);
    if (!w) return set_error(NFLOW_INVALID_ARG, std::string("ir_weight: no weight ") + name);
    return weight_out(*w, nullptr, ndim, dims8, data);
}

int nflow_ir_num_qparams(const nflow_ir* ir, int* n) {
    clear_error();
    if (!ir || !n) return set_error(NFLOW_INVALID_ARG, "ir_num_qparams: null argument");
    *n = static_cast<int>(ir->qrecords.size());
    return NFLOW_OK;
}

int nflow_ir_qparam_at(const nflow_ir* ir, int index, const char** name, int* kind) {
    clear_error();
    if (!ir) return set_error(NFLOW_INVALID_ARG, "ir_qparam_at: null ir");
    if (index < 0 || static_cast<size_t>(index) >= ir->qrecords.size())
        return set_error(NFLOW_INVALID_ARG, "ir_qparam_at: index out of range");
    if (name) *name = ir->qrecords[index].name.c_str();
    if (kind) *kind = ir->qrecords[index].kind;
    return NFLOW_OK;
}

int nflow_ir_per_tensor_qparam(const nflow_ir* ir, const char* name, int* found, float* scale, int32_t* zp) {
    clear_error();
    if (!ir || !name || !found) return set_error(NFLOW_INVALID_ARG, "ir_per_tensor_qparam: null argument");
    const auto& m = ends_with_output(name) ? ir->act_tensor : ir->weight_tensor;
    auto it = m.find(name);
    *found = it != m.end();
    if (*found) {
        if (scale) *scale = it->second.scale;
        if (zp) *zp = it->second.zp;
    }
    return NFLOW_OK;
}

int nflow_ir_per_channel_qparam(const nflow_ir* ir, const char* name, int* found, int* n_channels, int* axis,
                                const float** scales, const int32_t** zero_points) {
    clear_error();
    if (!ir || !name || !found) return set_error(NFLOW_INVALID_ARG, "ir_per_channel_qparam: null argument");
    auto it = ir->per_channel.find(name);
    *found = it != ir->per_channel.end();
    if (*found) {
        if (n_channels) *n_channels = static_cast<int>(it->second.scales.size());
        if (axis) *axis = it->second.axis;
        if (scales) *scales = it->second.scales.data();
        if (zero_points) *zero_points = it->second.zps.data();
    }
    return NFLOW_OK;
}

int nflow_ir_per_token_qparam(const nflow_ir* ir, const char* name, int* found, int* n_tokens, int* width,
                              const float** scales, const int32_t** zero_points) {
    clear_error();
    if (!ir || !name || !found) return set_error(NFLOW_INVALID_ARG, "ir_per_token_qparam: null argument");
    auto it = ir->per_token.find(name);
    *found = it != ir->per_token.end();
    if (*found) {
        if (n_tokens) *n_tokens = static_cast<int>(it->second.scales.size());
        if (width) *width = it->second.width;
        if (scales) *scales = it->second.scales.data();
        if (zero_points) *zero_points = it->second.zps.data();
    }
    return NFLOW_OK;
}

int nflow_ir_fp8_qparam(const nflow_ir* ir, const char* name, int* found, float* scale) {
    clear_error();
    if (!ir || !name || !found) return set_error(NFLOW_INVALID_ARG, "ir_fp8_qparam: null argument");
    auto it = ir->fp8.find(name);
    *found = it != ir->fp8.end();
    if (*found && scale) *scale = it->second;
    return NFLOW_OK;
}

int nflow_ir_layer_create(const nflow_ir* ir, const char* weight_name, const char* bias_name,
                          nflow_layer** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "ir_layer_create: null handle pointer");
    *out = nullptr;
    if (!ir || !weight_name) return set_error(NFLOW_INVALID_ARG, "ir_layer_create: null argument");
    const auto* w = find_weight(ir, weight_name);
    if (!w) return set_error(NFLOW_INVALID_ARG, std::string("ir_layer_create: no weight ") + weight_name);
    auto pc = ir->per_channel.find(weight_name);
    if (pc == ir->per_channel.end())
        return set_error(NFLOW_INVALID_ARG, std::string("ir_layer_create: no per-channel qparams for ") + weight_name);
    // QuantiseWeight2D's conditions (fno.cpp:329-331): a 2-D weight,
    // channel axis 0; one scale per output row.
    if (w->dims.size() != 2 || pc->second.axis != 0)
        return set_error(NFLOW_UNSUPPORTED_OP, "ir_layer_create: weight is not 2-D or channel axis is not 0");
    const int64_t n_out = w->dims[0], n_in = w->dims[1];
    if (n_out <= 0 || n_in <= 0 || n_out > INT32_MAX || n_in > INT32_MAX)
        return set_error(NFLOW_INVALID_ARG, "ir_layer_create: bad weight dims");
    if (static_cast<int64_t>(pc->second.scales.size()) < n_out)
        return set_error(NFLOW_INVALID_ARG, "ir_layer_create: fewer channel qparams than output rows");
    const float* bias = nullptr;
    if (bias_name) {
        const auto* b = find_weight(ir, bias_name);
        if (!b) return set_error(NFLOW_INVALID_ARG, std::string("ir_layer_create: no weight ") + bias_name);
        if (static_cast<int64_t>(b->data.size()) != n_out)
            return set_error(NFLOW_INVALID_ARG, "ir_layer_create: bias length differs from output rows");
        bias = b->data.data();
    }
    std::vector<int8_t> q(static_cast<size_t>(n_out * n_in));
    std::vector<int32_t> sum(static_cast<size_t>(n_out));
    int rc = nflow_host_quantise_weight_2d(w->data.data(), static_cast<int>(n_out), static_cast<int>(n_in),
                                           pc->second.scales.data(), pc->second.zps.data(), q.data(), sum.data());
    if (rc) return rc;
    return nflow_layer_create_int8(q.data(), pc->second.scales.data(), pc->second.zps.data(), bias, sum.data(),
                                   static_cast<int>(n_out), static_cast<int>(n_in), out);
}

int nflow_ir_fno_int8_dispatch(const nflow_ir* ir, int layer_index, int* use_int8, float* scale_A,
                               int32_t* zp_A) {
    clear_error();
    if (!ir || !use_int8) return set_error(NFLOW_INVALID_ARG, "ir_fno_int8_dispatch: null argument");
    if (layer_index < 0) return set_error(NFLOW_INVALID_ARG, "ir_fno_int8_dispatch: negative layer index");
    *use_int8 = 0;
    // Input key of locs.{i} (fno.cpp:529-531) and the cache key (:532).
    const std::string act_key =
        layer_index == 0 ? std::string("lift.output") : "locs." + std::to_string(layer_index - 1) + ".output";
    const std::string cache_key = "locs." + std::to_string(layer_index) + ".weight";
    // fno.cpp:131-136: no per-token or FP8 qparam for the input, a cached
    // blob (EnableInt8Gemm caches a 2-D weight with axis-0 channel qparams,
    // fno.cpp:329-331, 383-390), and a per-tensor activation qparam.
    if (ir->per_token.count(act_key) || ir->fp8.count(act_key)) return NFLOW_OK;
    const auto* w = find_weight(ir, cache_key.c_str());
    auto pc = ir->per_channel.find(cache_key);
    if (!w || pc == ir->per_channel.end() || w->dims.size() != 2 || pc->second.axis != 0) return NFLOW_OK;
    auto qa = ir->act_tensor.find(act_key);
    if (qa == ir->act_tensor.end()) return NFLOW_OK;
    *use_int8 = 1;
    if (scale_A) *scale_A = qa->second.scale;
    if (zp_A) *zp_A = qa->second.zp;
    return NFLOW_OK;
}

int nflow_ir_fno_x2_quant(const nflow_ir* ir, int layer_index, nflow_x2_quant* x2q) {
    clear_error();
    if (!ir || !x2q) return set_error(NFLOW_INVALID_ARG, "ir_fno_x2_quant: null argument");
    if (layer_index < 0) return set_error(NFLOW_INVALID_ARG, "ir_fno_x2_quant: negative layer index");
    *x2q = nflow_x2_quant{NFLOW_X2_NONE, 0.0f, 0, nullptr, nullptr, 0, 0, 0};
    // fno.cpp:571-648: only with a NIRQ block; FP8 first, then per-token,
    // then per-tensor, all keyed "locs.{i}.output".
    if (!ir->quant_enabled) return NFLOW_OK;
    const std::string key = "locs." + std::to_string(layer_index) + ".output";
    if (auto f = ir->fp8.find(key); f != ir->fp8.end()) {
        x2q->kind = NFLOW_X2_FP8_LOG2;
        x2q->scale = f->second;
        return NFLOW_OK;
    }
    if (auto t = ir->per_token.find(key); t != ir->per_token.end()) {
        x2q->kind = NFLOW_X2_PER_POSITION;
        x2q->scales = t->second.scales.data();
        x2q->zero_points = t->second.zps.data();
        x2q->n_positions = static_cast<int64_t>(t->second.scales.size());
        x2q->width = t->second.width;
        return NFLOW_OK;
    }
    if (auto q = ir->act_tensor.find(key); q != ir->act_tensor.end()) {
        x2q->kind = NFLOW_X2_PER_TENSOR;
        x2q->scale = q->second.scale;
        x2q->zero_point = q->second.zp;
    }
    return NFLOW_OK;
}

}  // extern "C"
