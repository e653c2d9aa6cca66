// neuroflow_cpp.cpp -- the pybind11 module `neuroflow_cpp` of the reference
// (cpp/bindings/pybind_module.cpp:58-238, fp8_e4m3_pybind.h:24-66), served
// by libnflow_quant: the same functions, classes, argument names, array
// conversions (float32 / uint8, C-contiguous, forcecast) and RuntimeError
// messages, with the model on the GPU.
//
//   infer(model_path, input_path, output_path)   .npy in, .npy out
//   infer_arrays(model_path, x) -> y
//   infer_deeponet_arrays(model_path, u, y)        (DeepONet: not served)
//   InferenceRuntime(path): op(), enable_int8_gemm(), is_int8_gemm_enabled(),
//                           run(x, y), and run_device(x_ptr, x_shape,
//                           y_ptr, y_shape, stream=0) on device pointers;
//                           enable_int8_gemm_fno2d() (FNO2d only, no reference
//                           counterpart)
//   fp8_e4m3_fake_quant(in, scale), fp8_e4m3_to_bits(in), fp8_e4m3_from_bits(in)
//
// The runtime serves FNO1d and FNO2d (include/nflow_runtime.h); creating it
// from an IR of another op fails with the runtime's UnsupportedOp message.
#include <hip/hip_runtime_api.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "nflow_quant.h"
#include "nflow_runtime.h"

namespace py = pybind11;

namespace {

using F32Array = py::array_t<float, py::array::c_style | py::array::forcecast>;
using U8Array = py::array_t<uint8_t, py::array::c_style | py::array::forcecast>;

std::string last_error() {
    const char* m = nflow_last_error();
    return m ? m : "";
}

std::vector<int64_t> shape_of(const py::buffer_info& b) { return std::vector<int64_t>(b.shape.begin(), b.shape.end()); }

// The op name of an IR file (the reference's LoadNeuroIr, runtime.cpp:15-19).
std::string ir_op(const std::string& path) {
    nflow_ir* ir = nullptr;
    if (nflow_ir_open(path.c_str(), &ir) != NFLOW_OK) throw std::runtime_error("load IR failed: " + last_error());
    int op = 0;
    (void)nflow_ir_header(ir, nullptr, &op, nullptr, nullptr, nullptr);
    nflow_ir_close(ir);
    static const char* kOps[] = {"", "FNO1d", "FNO2d", "FNO3d", "DeepONet", "TokenMixer", "GraphOp",
                                 "TokenMixer2D", "GraphOp2D"};
    return (op >= 1 && op <= 8) ? kOps[op] : "";
}

// The input rank of each op (pybind_module.cpp:76-83).
size_t expected_rank(const std::string& op) {
    if (op == "FNO1d" || op == "TokenMixer" || op == "GraphOp") return 3;
    if (op == "FNO2d" || op == "TokenMixer2D" || op == "GraphOp2D") return 4;
    if (op == "FNO3d") return 5;
    return 0;
}

std::unique_ptr<nflow::InferenceRuntime> create(const std::string& path) {
    std::unique_ptr<nflow::InferenceRuntime> rt;
    const nflow::Status s = nflow::InferenceRuntime::Create(path, rt);
    if (!s.ok()) throw std::runtime_error("create runtime failed: " + s.message());
    return rt;
}

// infer_arrays / infer: y shape = x shape with the last dim out_channels.
py::array_t<float> run_arrays(nflow::InferenceRuntime& rt, const F32Array& x) {
    py::buffer_info xb = x.request();
    if (static_cast<size_t>(xb.ndim) != expected_rank(rt.op()))
        throw std::runtime_error("input rank mismatch for op " + rt.op());
    int32_t cfg[7] = {};
    (void)nflow_runtime_config(rt.handle(), cfg, nullptr, nullptr);
    std::vector<int64_t> ys = shape_of(xb);
    ys.back() = cfg[1];
    py::array_t<float> y(std::vector<py::ssize_t>(ys.begin(), ys.end()));
    py::buffer_info yb = y.request();
    const nflow::Status s = rt.Run(static_cast<const float*>(xb.ptr), shape_of(xb), static_cast<float*>(yb.ptr), ys);
    if (!s.ok()) throw std::runtime_error("infer failed: " + s.message());
    return y;
}

// Elementwise device call on a host array (the FP8 codec entry points).
template <typename In, typename Out, typename Fn>
py::array_t<Out> on_device(const py::array_t<In, py::array::c_style | py::array::forcecast>& in, Fn fn) {
    auto u = in.template unchecked<1>();
    const py::ssize_t n = u.shape(0);
    py::array_t<Out> out(n);
    if (n == 0) return out;
    void* din = nullptr;
    void* dout = nullptr;
    if (hipMalloc(&din, n * sizeof(In)) != hipSuccess || hipMalloc(&dout, n * sizeof(Out)) != hipSuccess) {
        if (din) (void)hipFree(din);
        throw std::runtime_error("device allocation failed");
    }
    int rc = hipMemcpy(din, u.data(0), n * sizeof(In), hipMemcpyHostToDevice) == hipSuccess ? NFLOW_OK : NFLOW_INTERNAL;
    if (rc == NFLOW_OK) rc = fn(static_cast<const In*>(din), static_cast<Out*>(dout), static_cast<int64_t>(n));
    if (rc == NFLOW_OK && hipMemcpy(out.mutable_data(), dout, n * sizeof(Out), hipMemcpyDeviceToHost) != hipSuccess)
        rc = NFLOW_INTERNAL;
    (void)hipFree(din);
    (void)hipFree(dout);
    if (rc != NFLOW_OK) throw std::runtime_error("fp8 e4m3 failed: " + last_error());
    return out;
}

}  // namespace

PYBIND11_MODULE(neuroflow_cpp, m) {
    m.doc() = "NeuroFlow runtime on the MI355X - FNO1d / FNO2d inference on the GPU";

    m.def(
        "infer",
        [](const std::string& model_path, const std::string& input_path, const std::string& output_path) {
            const std::string op = ir_op(model_path);
            py::module_ np = py::module_::import("numpy");
            py::object xo;
            try {
                xo = np.attr("load")(input_path, py::arg("allow_pickle") = false);
            } catch (const py::error_already_set& e) {
                throw std::runtime_error(std::string("read input failed: ") + e.what());
            }
            F32Array x = F32Array::ensure(xo);
            const size_t rank = expected_rank(op);
            if (!x || rank == 0 || static_cast<size_t>(x.ndim()) != rank)
                throw std::runtime_error("input rank mismatch for op " + op);
            auto rt = create(model_path);
            py::array_t<float> y = run_arrays(*rt, x);
            try {
                np.attr("save")(output_path, y);
            } catch (const py::error_already_set& e) {
                throw std::runtime_error(std::string("write output failed: ") + e.what());
            }
            return std::string("ok");
        },
        py::arg("model_path"), py::arg("input_path"), py::arg("output_path"),
        "Run inference: load .nneuroir, read .npy, write .npy");

    m.def(
        "infer_arrays",
        [](const std::string& model_path, F32Array x) -> py::array_t<float> {
            const std::string op = ir_op(model_path);
            const size_t rank = expected_rank(op);
            if (rank == 0 || static_cast<size_t>(x.ndim()) != rank)
                throw std::runtime_error("input rank mismatch for op " + op);
            auto rt = create(model_path);
            return run_arrays(*rt, x);
        },
        py::arg("model_path"), py::arg("x"),
        "Run inference in-memory: load .nneuroir, take numpy array, return numpy array");

    py::class_<nflow::InferenceRuntime, std::unique_ptr<nflow::InferenceRuntime>>(
        m, "InferenceRuntime", "Persistent runtime (load once, run many)")
        .def(py::init([](const std::string& ir_path) { return create(ir_path); }))
        .def("op", &nflow::InferenceRuntime::op)
        .def("enable_int8_gemm", &nflow::InferenceRuntime::EnableInt8Gemm,
             "Route FNO1d's per-layer local Linear through the INT8 GEMM on the GPU. "
             "No-op for non-FNO1d models.")
        .def(
            "enable_int8_gemm_fno2d",
            [](nflow::InferenceRuntime& self) {
                const nflow::Status s = self.EnableInt8GemmFno2d();
                if (!s.ok()) throw std::runtime_error("enable_int8_gemm_fno2d failed: " + s.message());
            },
            "FNO2d only (no counterpart in the reference): run the local linear layers on the INT8 GEMM "
            "with FNO1d's dispatch conditions.")
        .def("is_int8_gemm_enabled", &nflow::InferenceRuntime::IsInt8GemmEnabled,
             "True iff enable_int8_gemm was effective.")
        .def(
            "run",
            [](nflow::InferenceRuntime& self, F32Array x, F32Array y) {
                py::buffer_info xb = x.request();
                py::buffer_info yb = y.request();
                nflow::Status s;
                {
                    py::gil_scoped_release nogil;
                    s = self.Run(static_cast<const float*>(xb.ptr), shape_of(xb), static_cast<float*>(yb.ptr),
                                 shape_of(yb));
                }
                if (!s.ok()) throw std::runtime_error("Run failed: " + s.message());
            },
            py::arg("x"), py::arg("y"),
            "Run FNO1d / FNO2d inference.  x and y are pre-allocated float32 numpy arrays with the "
            "expected input/output shapes.")
        .def(
            "run_device",
            [](nflow::InferenceRuntime& self, std::uintptr_t x, std::vector<int64_t> x_shape, std::uintptr_t y,
               std::vector<int64_t> y_shape, std::uintptr_t stream) {
                const nflow::Status s = self.RunDevice(reinterpret_cast<const float*>(x), x_shape,
                                                       reinterpret_cast<float*>(y), y_shape,
                                                       reinterpret_cast<void*>(stream));
                if (!s.ok()) throw std::runtime_error("Run failed: " + s.message());
            },
            py::arg("x_ptr"), py::arg("x_shape"), py::arg("y_ptr"), py::arg("y_shape"), py::arg("stream") = 0,
            "Run on device buffers (e.g. torch CUDA tensors' data_ptr()) on a HIP stream; "
            "returns without synchronising.");

    m.def(
        "infer_deeponet_arrays",
        [](const std::string& model_path, F32Array u, F32Array y) -> py::array_t<float> {
            (void)u;
            (void)y;
            const std::string op = ir_op(model_path);
            if (op != "DeepONet")
                throw std::runtime_error("infer_deeponet_arrays: model op is " + op + ", not DeepONet");
            create(model_path);  // throws: the device runtime serves FNO1d and FNO2d
            return py::array_t<float>();
        },
        py::arg("model_path"), py::arg("u"), py::arg("y"),
        "DeepONet inference (not served by the device runtime; raises)");

    m.def(
        "fp8_e4m3_fake_quant",
        [](F32Array in, float scale) {
            return on_device<float, float>(in, [scale](const float* a, float* b, int64_t n) {
                int rc = nflow_fp8_e4m3_fake_quant(a, scale, b, n, nullptr);
                return rc == NFLOW_OK && hipDeviceSynchronize() != hipSuccess ? NFLOW_INTERNAL : rc;
            });
        },
        py::arg("in"), py::arg("scale"), "Per-tensor FP8 E4M3 fake-quant (in: float32, out: float32).");
    m.def(
        "fp8_e4m3_to_bits",
        [](F32Array in) {
            return on_device<float, uint8_t>(in, [](const float* a, uint8_t* b, int64_t n) {
                int rc = nflow_fp8_e4m3_to_bits(a, b, n, nullptr);
                return rc == NFLOW_OK && hipDeviceSynchronize() != hipSuccess ? NFLOW_INTERNAL : rc;
            });
        },
        py::arg("in"), "Convert FP32 -> FP8 E4M3 byte.");
    m.def(
        "fp8_e4m3_from_bits",
        [](U8Array in) {
            return on_device<uint8_t, float>(in, [](const uint8_t* a, float* b, int64_t n) {
                int rc = nflow_fp8_e4m3_from_bits(a, b, n, nullptr);
                return rc == NFLOW_OK && hipDeviceSynchronize() != hipSuccess ? NFLOW_INTERNAL : rc;
            });
        },
        py::arg("in"), "Convert FP8 E4M3 byte -> FP32.");
}
