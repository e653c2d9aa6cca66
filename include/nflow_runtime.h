/*
 * nflow_runtime.h -- the FNO1d inference runtime on the MI355X.
 *
 * Replaces nflow::InferenceRuntime (cpp/include/neuroflow/runtime.h:64-121,
 * cpp/src/runtime.cpp:15-173) for FNO1d models, the op whose local-linear
 * layers the reference routes through its INT8 GEMM (EnableInt8Gemm,
 * runtime.cpp:150-166).  The whole forward (lift, spectral convolutions,
 * local-linear layers, projection) runs on the GPU; each element is
 * computed by the same float operations as the reference's x86 build, so the
 * output equals the reference runtime's bit for bit.
 *
 * C-ABI: plain pointers, status codes of nflow::StatusCode (nflow_quant.h),
 * the message of a failure from nflow_last_error().  Below it, for C++
 * callers, a header-only nflow::InferenceRuntime with the reference's
 * signatures over this C-ABI.
 *
 * Creation uploads the weights to the current device; runs use that device.
 * Runs, EnableInt8Gemm and the queries may be called from several threads:
 * a per-handle lock serialises them on the host, and a run enqueued on a
 * different stream than the handle's previous run first waits (an event)
 * for that run, because the runs of one handle share its device workspace.
 * Destroying a handle while another thread uses it is the caller's error.
 */
#ifndef NFLOW_RUNTIME_H
#define NFLOW_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#include "nflow_quant.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nflow_runtime nflow_runtime;

/* InferenceRuntime::Create (runtime.h:72-73, runtime.cpp:73-77) over
 * LoadNeuroIr + Init (runtime.cpp:15-48): reads the NeuroIR binary, applies
 * the NIRQ weight fake-quant (fno.cpp:209-300, 997-1020), uploads the
 * weights.  FileNotFound / ParseError / UnsupportedOp as the reference's
 * loader; an IR of another op than FNO1d or FNO2d is UnsupportedOp. */
int nflow_runtime_create(const char* ir_path, nflow_runtime** rt);
/* The same from an in-memory copy of the file. */
int nflow_runtime_create_memory(const void* data, size_t bytes, nflow_runtime** rt);
int nflow_runtime_destroy(nflow_runtime* rt);

/* InferenceRuntime::op() (runtime.h:112): "FNO1d" or "FNO2d". */
const char* nflow_runtime_op(const nflow_runtime* rt);
/* The IR's 7-entry configuration block as LoadBinary reads it
 * (ir_loader.h:131-160): FNO1d [in_ch, out_ch, width, modes, n_layers,
 * pad_factor, 0], FNO2d [in_ch, out_ch, width, modes_h, modes_w, n_layers,
 * pad_factor]; the activation (NFLOW_ACT_RELU / NFLOW_ACT_GELU_TANH) and
 * whether the IR carried a NIRQ block.  Any output may be NULL. */
int nflow_runtime_config(const nflow_runtime* rt, int32_t* config7, int* activation, int* quant_enabled);

/* InferenceRuntime::EnableInt8Gemm (runtime.h:99, runtime.cpp:155-166,
 * fno.cpp:360-406): builds and uploads the INT8 blob of every locs.{i}
 * weight with per-channel qparams; those layers then run as the INT8
 * LinearForwardBatched when LinearDispatchTryInt8 would take it
 * (fno.cpp:125-159).  A no-op for FNO2d, as in the reference. */
int nflow_runtime_enable_int8_gemm(nflow_runtime* rt);
/* No counterpart in the reference, whose FNO2d has no EnableInt8Gemm: for
 * FNO2d models, the same cache and dispatch as EnableInt8Gemm does for FNO1d
 * (fno.cpp:125-159, 360-406).  Each locs.{i} whose weight has axis-0
 * per-channel qparams, and whose input key (lift.output / locs.{i-1}.output)
 * has a per-tensor qparam and no FP8 or per-token one, then runs as the INT8
 * LinearForwardBatched + bias instead of the fp32 Linear.  For callers that
 * want C3's model on the INT8 GEMM; nflow_runtime_enable_int8_gemm stays the
 * reference's no-op for FNO2d.  UnsupportedOp for other models. */
int nflow_runtime_enable_int8_gemm_fno2d(nflow_runtime* rt);
/* InferenceRuntime::IsInt8GemmEnabled (runtime.h:103, runtime.cpp:168-171). */
int nflow_runtime_is_int8_gemm_enabled(const nflow_runtime* rt, int* enabled);
/* Whether locs.{layer_index} runs on the INT8 GEMM. */
int nflow_runtime_layer_dispatch(const nflow_runtime* rt, int layer_index, int* uses_int8);

/* InferenceRuntime::Run (runtime.h:77-78, runtime.cpp:79-94) on HOST buffers:
 * x (batch, n, in_ch), y (batch, n, out_ch) for FNO1d, x (batch, H, W,
 * in_ch), y (batch, H, W, out_ch) for FNO2d; float32, C-contiguous; copies
 * in, runs, copies out, synchronises.  Shape checks and their codes as
 * FNO1d::Forward (fno.cpp:409-425) / FNO2d::Forward (fno.cpp:778-795). */
int nflow_runtime_run(nflow_runtime* rt, const float* x, const int64_t* x_shape, int x_ndim, float* y,
                      const int64_t* y_shape, int y_ndim);
/* The same on DEVICE buffers, enqueued on `stream` without synchronising. */
int nflow_runtime_run_device(nflow_runtime* rt, const float* x, const int64_t* x_shape, int x_ndim, float* y,
                             const int64_t* y_shape, int y_ndim, void* stream);

#ifdef __cplusplus
}  /* extern "C" */

#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace nflow {

/* nflow::StatusCode / nflow::Status (cpp/include/neuroflow/tensor.h:29-60). */
enum class StatusCode {
    Ok = 0,
    InvalidArg = 1,
    FileNotFound = 2,
    ParseError = 3,
    ShapeMismatch = 4,
    UnsupportedOp = 5,
    Internal = 99,
};

class Status {
public:
    Status() = default;
    explicit Status(StatusCode code, std::string msg = "") : code_(code), msg_(std::move(msg)) {}
    bool ok() const { return code_ == StatusCode::Ok; }
    StatusCode code() const { return code_; }
    const std::string& message() const { return msg_; }
    static Status Ok() { return Status(StatusCode::Ok); }

private:
    StatusCode code_ = StatusCode::Ok;
    std::string msg_;
};

inline Status status_from(int rc) {
    if (rc == NFLOW_OK) return Status::Ok();
    const char* m = nflow_last_error();
    return Status(static_cast<StatusCode>(rc), m ? m : "");
}

/* nflow::InferenceRuntime (runtime.h:64-121) for FNO1d, on the device. */
class InferenceRuntime {
public:
    static Status Create(const std::string& ir_path, std::unique_ptr<InferenceRuntime>& out) {
        nflow_runtime* h = nullptr;
        const Status s = status_from(nflow_runtime_create(ir_path.c_str(), &h));
        if (!s.ok()) return s;
        out.reset(new InferenceRuntime(h));
        return s;
    }
    ~InferenceRuntime() { nflow_runtime_destroy(h_); }
    InferenceRuntime(const InferenceRuntime&) = delete;
    InferenceRuntime& operator=(const InferenceRuntime&) = delete;

    /* Host buffers, as the reference. */
    Status Run(const float* x, const std::vector<int64_t>& x_shape, float* y, const std::vector<int64_t>& y_shape) {
        return status_from(nflow_runtime_run(h_, x, x_shape.data(), static_cast<int>(x_shape.size()), y,
                                             y_shape.data(), static_cast<int>(y_shape.size())));
    }
    /* Device buffers on a HIP stream (no reference counterpart). */
    Status RunDevice(const float* x, const std::vector<int64_t>& x_shape, float* y,
                     const std::vector<int64_t>& y_shape, void* stream = nullptr) {
        return status_from(nflow_runtime_run_device(h_, x, x_shape.data(), static_cast<int>(x_shape.size()), y,
                                                    y_shape.data(), static_cast<int>(y_shape.size()), stream));
    }
    const std::string& op() const { return op_; }
    void EnableInt8Gemm() { (void)nflow_runtime_enable_int8_gemm(h_); }
    // No reference counterpart: the FNO2d INT8 opt-in above.
    Status EnableInt8GemmFno2d() { return status_from(nflow_runtime_enable_int8_gemm_fno2d(h_)); }
    bool IsInt8GemmEnabled() const {
        int e = 0;
        return nflow_runtime_is_int8_gemm_enabled(h_, &e) == NFLOW_OK && e != 0;
    }
    nflow_runtime* handle() const { return h_; }

private:
    explicit InferenceRuntime(nflow_runtime* h) : h_(h), op_(nflow_runtime_op(h)) {}
    nflow_runtime* h_;
    std::string op_;
};

}  // namespace nflow
#endif /* __cplusplus */

#endif /* NFLOW_RUNTIME_H */
