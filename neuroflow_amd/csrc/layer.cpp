// layer.cpp -- device-resident layer handles: the weight blob of one linear
// layer is built on the host once (per-channel scales, codes, weight sums),
// uploaded once, and every forward call runs the fused per-token kernels on
// it.  This is what fno::FNO1d::EnableInt8Gemm does with its Int8GemmLayer
// cache (cpp/src/fno.cpp:325-406, cpp/include/neuroflow/fno.h:66-87), with
// the blobs living in HBM instead of host vectors.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <climits>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "nflow_quant.h"
#include "fno_rt.h"
#include "status.h"

struct nflow_layer {
    int format = NFLOW_FORMAT_INT8;
    int out_features = 0;
    int in_features = 0;
    int device = 0;
    void* W = nullptr;            // int8 codes or E4M3 bytes, (out, in)
    float* scale_W = nullptr;     // (out)
    int32_t* zp_W = nullptr;      // (out), INT8 only
    int32_t* sum_W = nullptr;     // (out), INT8 only
    float* bias = nullptr;        // (out) or null
    // Symmetric INT8 blob: every zero point 0 and sum_W absent or equal to
    // each row's code sum.  The per-token forwards then pass neither zero
    // points nor sum_W: the zero-point terms vanish and the row-VNNI
    // formula's sum_W term equals the one formed from the codes, so the
    // outputs are the same bit for bit, and the kernels skip the integer
    // epilogue (the persistent GEMM's integer form costs ~7% at 65536 x 1024
    // x 1024).
    bool symmetric = false;
};

namespace nfq {

static void free_layer(nflow_layer* l) {
    if (!l) return;
    int cur = 0;
    const bool switch_dev = hipGetDevice(&cur) == hipSuccess && cur != l->device;
    if (switch_dev) (void)hipSetDevice(l->device);
    for (void* p : {l->W, static_cast<void*>(l->scale_W), static_cast<void*>(l->zp_W),
                    static_cast<void*>(l->sum_W), static_cast<void*>(l->bias)})
        if (p) (void)hipFree(p);
    if (switch_dev) (void)hipSetDevice(cur);
    delete l;
}

// Allocate and copy `bytes` from host memory; false (with the error set) on failure.
static bool upload(void** dst, const void* src, size_t bytes, const char* what) {
    if (hipMalloc(dst, bytes) != hipSuccess) {
        *dst = nullptr;
        set_error(NFLOW_INTERNAL, std::string("layer: device allocation failed for ") + what);
        return false;
    }
    if (hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        set_error(NFLOW_INTERNAL, std::string("layer: upload failed for ") + what);
        return false;
    }
    return true;
}

// The parameter block of an INT8 layer's per-token forwards (zp_A = 0).
static nflow_int8_linear_params token_params(const nflow_layer* l) {
    return nflow_int8_linear_params{static_cast<const int8_t*>(l->W), l->scale_W, l->symmetric ? nullptr : l->zp_W,
                                    l->bias, l->in_features, l->out_features, 1.0f, 0,
                                    l->symmetric ? nullptr : l->sum_W};
}

static int finish(nflow_layer* l, bool ok, nflow_layer** out) {
    if (!ok) {
        free_layer(l);
        return NFLOW_INTERNAL;
    }
    *out = l;
    return NFLOW_OK;
}

}  // namespace nfq

using namespace nfq;

extern "C" {

int nflow_layer_create(const float* W, const float* bias, int out_features, int in_features,
                       int format, nflow_layer** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "layer_create: null handle pointer");
    *out = nullptr;
    if (!W) return set_error(NFLOW_INVALID_ARG, "layer_create: null W");
    if (out_features <= 0 || in_features <= 0) return set_error(NFLOW_INVALID_ARG, "layer_create: bad dims");
    if (format != NFLOW_FORMAT_INT8 && format != NFLOW_FORMAT_FP8_E4M3)
        return set_error(NFLOW_INVALID_ARG, "layer_create: unknown format");
    const size_t n = static_cast<size_t>(out_features), nk = n * static_cast<size_t>(in_features);
    std::vector<float> scales(n);
    if (format == NFLOW_FORMAT_INT8) {
        std::vector<int8_t> q(nk);
        std::vector<int32_t> zp(n, 0), sum(n);
        int rc = nflow_host_per_channel_scales(W, out_features, in_features, 127.0f, scales.data());
        if (!rc) rc = nflow_host_quantise_weight_2d(W, out_features, in_features, scales.data(), zp.data(),
                                                    q.data(), sum.data());
        if (rc) return rc;
        return nflow_layer_create_int8(q.data(), scales.data(), zp.data(), bias, sum.data(), out_features,
                                       in_features, out);
    }
    std::vector<uint8_t> q(nk);
    int rc = nflow_host_fp8_quantise_weight(W, out_features, in_features, q.data(), scales.data());
    if (rc) return rc;
    nflow_layer* l = new (std::nothrow) nflow_layer;
    if (!l) return set_error(NFLOW_INTERNAL, "layer_create: out of host memory");
    l->format = NFLOW_FORMAT_FP8_E4M3;
    l->out_features = out_features;
    l->in_features = in_features;
    (void)hipGetDevice(&l->device);
    bool ok = upload(&l->W, q.data(), nk, "W") &&
              upload(reinterpret_cast<void**>(&l->scale_W), scales.data(), n * sizeof(float), "scale_W");
    if (ok && bias) ok = upload(reinterpret_cast<void**>(&l->bias), bias, n * sizeof(float), "bias");
    return finish(l, ok, out);
}

int nflow_layer_create_int8(const int8_t* W_q, const float* scale_W, const int32_t* zp_W,
                            const float* bias, const int32_t* sum_W_per_row, int out_features,
                            int in_features, nflow_layer** out) {
    clear_error();
    if (!out) return set_error(NFLOW_INVALID_ARG, "layer_create_int8: null handle pointer");
    *out = nullptr;
    if (!W_q || !scale_W || !zp_W) return set_error(NFLOW_INVALID_ARG, "layer_create_int8: null blob");
    if (out_features <= 0 || in_features <= 0)
        return set_error(NFLOW_INVALID_ARG, "layer_create_int8: bad dims");
    const size_t n = static_cast<size_t>(out_features), nk = n * static_cast<size_t>(in_features);
    nflow_layer* l = new (std::nothrow) nflow_layer;
    if (!l) return set_error(NFLOW_INTERNAL, "layer_create_int8: out of host memory");
    l->format = NFLOW_FORMAT_INT8;
    l->out_features = out_features;
    l->in_features = in_features;
    (void)hipGetDevice(&l->device);
    bool ok = upload(&l->W, W_q, nk, "W") &&
              upload(reinterpret_cast<void**>(&l->scale_W), scale_W, n * sizeof(float), "scale_W") &&
              upload(reinterpret_cast<void**>(&l->zp_W), zp_W, n * sizeof(int32_t), "zp_W");
    if (ok && bias) ok = upload(reinterpret_cast<void**>(&l->bias), bias, n * sizeof(float), "bias");
    if (ok && sum_W_per_row)
        ok = upload(reinterpret_cast<void**>(&l->sum_W), sum_W_per_row, n * sizeof(int32_t), "sum_W_per_row");
    bool sym = true;
    for (size_t r = 0; r < n && sym; ++r) {
        if (zp_W[r] != 0) sym = false;
        if (sym && sum_W_per_row) {
            int64_t t = 0;
            for (size_t k = 0; k < static_cast<size_t>(in_features); ++k) t += W_q[r * in_features + k];
            sym = t == sum_W_per_row[r];
        }
    }
    l->symmetric = sym;
    return finish(l, ok, out);
}

int nflow_layer_forward(const nflow_layer* layer, int64_t M, const float* x, float* y,
                        float* scale_A_out, int activation, void* stream) {
    clear_error();
    if (!layer) return set_error(NFLOW_INVALID_ARG, "layer_forward: null layer");
    if (layer->format == NFLOW_FORMAT_INT8) {
        const nflow_int8_linear_params p = token_params(layer);
        return nflow_int8_linear_forward_per_token(&p, M, x, y, scale_A_out, activation, stream);
    }
    const nflow_fp8_linear_params p{static_cast<const uint8_t*>(layer->W), layer->scale_W, layer->bias,
                                    layer->in_features, layer->out_features};
    return nflow_fp8_linear_forward_per_token(&p, M, x, y, scale_A_out, activation, stream);
}

int nflow_layer_forward_residual(const nflow_layer* layer, int64_t M, const float* x, const float* x1,
                                 float* y, float* scale_A_out, int activation, void* stream) {
    clear_error();
    if (!layer) return set_error(NFLOW_INVALID_ARG, "layer_forward_residual: null layer");
    if (layer->format == NFLOW_FORMAT_INT8) {
        const nflow_int8_linear_params p = token_params(layer);
        return nflow_int8_fno_layer_per_token(&p, M, x, x1, y, scale_A_out, activation, stream);
    }
    const nflow_fp8_linear_params p{static_cast<const uint8_t*>(layer->W), layer->scale_W, layer->bias,
                                    layer->in_features, layer->out_features};
    return nflow_fp8_fno_layer_per_token(&p, M, x, x1, y, scale_A_out, activation, stream);
}

int nflow_layer_forward_fno(const nflow_layer* layer, int64_t M, const float* x, const float* x1, float* y,
                            float* scale_A_out, int activation, const nflow_x2_quant* x2q, void* stream) {
    clear_error();
    if (!layer) return set_error(NFLOW_INVALID_ARG, "layer_forward_fno: null layer");
    if (layer->format == NFLOW_FORMAT_INT8) {
        const nflow_int8_linear_params p = token_params(layer);
        return nflow_int8_fno_layer_per_token_x2q(&p, M, x, x1, y, scale_A_out, activation, x2q, stream);
    }
    const nflow_fp8_linear_params p{static_cast<const uint8_t*>(layer->W), layer->scale_W, layer->bias,
                                    layer->in_features, layer->out_features};
    return nflow_fp8_fno_layer_per_token_x2q(&p, M, x, x1, y, scale_A_out, activation, x2q, stream);
}

int nflow_layer_forward_per_tensor(const nflow_layer* layer, int64_t M, const float* x, float* y, float scale_A,
                                   int32_t zp_A, void* stream) {
    clear_error();
    if (!layer) return set_error(NFLOW_INVALID_ARG, "layer_forward_per_tensor: null layer");
    if (layer->format != NFLOW_FORMAT_INT8)
        return set_error(NFLOW_UNSUPPORTED_OP, "layer_forward_per_tensor: INT8 layers only");
    if (M > INT32_MAX) return set_error(NFLOW_INVALID_ARG, "layer_forward_per_tensor: M exceeds the batched API's int");
    const nflow_int8_linear_params p{static_cast<const int8_t*>(layer->W), layer->scale_W, layer->zp_W,
                                     layer->bias, layer->in_features, layer->out_features, scale_A, zp_A,
                                     layer->sum_W};
    return nflow_int8_linear_forward_batched(&p, static_cast<int>(M), x, y, stream);
}

int nflow_layer_shape(const nflow_layer* layer, int* out_features, int* in_features, int* format) {
    clear_error();
    if (!layer) return set_error(NFLOW_INVALID_ARG, "layer_shape: null layer");
    if (out_features) *out_features = layer->out_features;
    if (in_features) *in_features = layer->in_features;
    if (format) *format = layer->format;
    return NFLOW_OK;
}

int nflow_layer_destroy(nflow_layer* layer) {
    clear_error();
    free_layer(layer);
    return NFLOW_OK;
}

}  // extern "C"

namespace nfq {

bool layer_int8_arrays(const nflow_layer* layer, LayerTailArgs* a, int* in_features, int* out_features) {
    if (!layer || layer->format != NFLOW_FORMAT_INT8) return false;
    a->W = static_cast<const int8_t*>(layer->W);
    a->sW = layer->scale_W;
    a->bias = layer->bias;
    // A symmetric blob's zero points are all 0: none passed, so that with
    // zp_A = 0 every integer term of the batched formula is known to vanish.
    a->zpW = layer->symmetric ? nullptr : layer->zp_W;
    a->sumW = layer->sum_W;
    *in_features = layer->in_features;
    *out_features = layer->out_features;
    return true;
}

}  // namespace nfq
