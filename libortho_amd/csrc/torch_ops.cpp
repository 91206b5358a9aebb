// Compiled torch binding of the C ABI (include/orth_hip.h) for the eager
// calls of the operator boundary: the reference's binding
// (/root/reference/torch_bind/bindings.cpp:9-48) rebuilt over this build's
// library.  It checks the tensors as libortho_amd/_C_ops.py does (same
// messages, RuntimeError), describes them as an orth_hip_layer_t on the
// stack and launches on torch's current HIP stream of the input's device,
// in one C++ call: no per-call ctypes argument conversion and no Python
// attribute reads.  Host code only (g++): the kernels stay in
// libortho_amd.so, which this module links.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <string>

#include "orth_hip.h"

namespace {

// A failed C-ABI call raises libortho_amd._lib.OrthoError(status, message),
// as the ctypes path does.
void check_rc(int rc) {
    if (rc == ORTH_OK) return;
    static py::object cls = py::module_::import("libortho_amd._lib").attr("OrthoError");
    PyErr_SetObject(cls.ptr(), py::make_tuple(rc, std::string(orth_hip_last_error())).ptr());
    throw py::error_already_set();
}

void req(bool cond, const std::string &msg) {
    if (!cond) throw std::runtime_error(msg);
}

int32_t io_dtype(const at::Tensor &t) {
    switch (t.scalar_type()) {
        case at::kHalf: return ORTH_DT_F16;
        case at::kBFloat16: return ORTH_DT_BF16;
        case at::kFloat: return ORTH_DT_F32;
        default: return -1;
    }
}

std::string shape_str(const at::Tensor &t) {
    std::string s = "(";
    for (int64_t i = 0; i < t.dim(); i++) s += (i ? ", " : "") + std::to_string(t.size(i));
    return s + (t.dim() == 1 ? ",)" : ")");
}

void check_io(const at::Tensor &x, const at::Tensor &y) {
    req(x.is_cuda(), "input must be on a ROCm GPU (libortho_amd has no CPU path)");
    req(y.device() == x.device(), "output must be on the same device as input");
    req(x.dim() == 2 && y.dim() == 2, "input and output must be 2-D [M, K] / [M, N]");
    req(io_dtype(x) >= 0, "input dtype is not float16, bfloat16 or float32");
    req(y.scalar_type() == x.scalar_type(), "output dtype must equal input dtype");
    req(x.is_contiguous() && y.is_contiguous(), "input and output must be contiguous");
    req(y.size(0) == x.size(0), "output has " + std::to_string(y.size(0)) + " rows, input " +
                                    std::to_string(x.size(0)));
}

void *ptr(const at::Tensor &t) { return t.numel() > 0 ? t.data_ptr() : nullptr; }

// The weight tensors as an orth_hip_layer_t (the checks of _C_ops.make_layer).
orth_hip_layer_t describe(const at::Tensor &q, const at::Tensor &s, const at::Tensor &v, const at::Tensor &c,
                          const at::Tensor &rp, int64_t K, int64_t N, double alpha, const at::Device &dev) {
    const char *names[5] = {"q_weight", "q_scales", "ortho_values", "ortho_col_indices", "ortho_row_ptr"};
    const at::Tensor *ts[5] = {&q, &s, &v, &c, &rp};
    for (int i = 0; i < 5; i++) {
        req(ts[i]->numel() == 0 || ts[i]->device() == dev,
            std::string(names[i]) + " is not on the input's device");
        req(ts[i]->is_contiguous(), std::string(names[i]) + " must be contiguous");
    }
    req(K > 0 && K % 2 == 0, "in_features must be positive and even (got " + std::to_string(K) + ")");
    req(q.scalar_type() == at::kByte, "q_weight must be uint8");
    req(q.dim() == 2 && q.size(0) == N && q.size(1) == K / 2,
        "q_weight must have shape (" + std::to_string(N) + ", " + std::to_string(K / 2) + ") (got " + shape_str(q) + ")");
    req(s.scalar_type() == at::kHalf || s.scalar_type() == at::kFloat, "q_scales must be float16 or float32");
    int64_t groups = 1;
    if (s.dim() == 1) {
        req(s.size(0) == N, "q_scales must have " + std::to_string(N) + " rows (got " + shape_str(s) + ")");
    } else {
        req(s.dim() == 2 && s.size(0) == N,
            "q_scales must be [" + std::to_string(N) + "] or [" + std::to_string(N) + ", K/G] (got " + shape_str(s) + ")");
        groups = s.size(1);
        req(groups >= 1 && K % groups == 0, "q_scales has " + std::to_string(groups) +
                                                " groups, which does not divide in_features " + std::to_string(K));
    }
    const int64_t nnz = v.numel();
    req(c.numel() == nnz, "ortho_col_indices has " + std::to_string(c.numel()) + " entries, ortho_values " +
                              std::to_string(nnz));
    if (nnz > 0) {
        req(v.scalar_type() == at::kHalf || v.scalar_type() == at::kFloat, "ortho_values must be float16 or float32");
        req(c.scalar_type() == at::kInt, "ortho_col_indices must be int32");
        req(rp.scalar_type() == at::kInt, "ortho_row_ptr must be int32");
        req(rp.numel() == N + 1, "ortho_row_ptr must have " + std::to_string(N + 1) + " entries (got " +
                                     std::to_string(rp.numel()) + ")");
    }
    orth_hip_layer_t L{};
    L.base.q_weight = ptr(q);
    L.base.q_scales = ptr(s);
    L.base.q_bits = 4;
    L.base.scale_dtype = s.scalar_type() == at::kHalf ? ORTH_DT_F16 : ORTH_DT_F32;
    L.base.scale_groups = groups;
    L.base.in_features = K;
    L.base.out_features = N;
    L.ortho.count = nnz;
    if (nnz > 0) {
        L.ortho.row_ptr = static_cast<const int32_t *>(ptr(rp));
        L.ortho.col_indices = static_cast<const int32_t *>(ptr(c));
        L.ortho.values = ptr(v);
        L.ortho.value_dtype = v.scalar_type() == at::kHalf ? ORTH_DT_F16 : ORTH_DT_F32;
    }
    L.alpha = (float)alpha;
    return L;
}

void launch(const orth_hip_layer_t &L, const c10::optional<at::Tensor> &plan, const c10::optional<at::Tensor> &bias,
            const at::Tensor &x, at::Tensor &y) {
    const at::Device dev = x.device();
    const bool has_plan = plan.has_value() && plan->defined() && plan->numel() > 0;
    if (has_plan)
        req(plan->device() == dev && plan->scalar_type() == at::kByte, "plan must be a uint8 tensor on input's device");
    const void *bp = nullptr;
    int32_t bdt = 0;
    if (bias.has_value() && bias->defined()) {
        req(bias->device() == dev && io_dtype(*bias) >= 0 && bias->numel() == y.size(1) && bias->is_contiguous(),
            "bias must be a contiguous float tensor of " + std::to_string(y.size(1)) +
                " elements on input's device");
        bp = ptr(*bias);
        bdt = io_dtype(*bias);
    }
    c10::DeviceGuard guard(dev);
    hipStream_t st = c10::hip::getCurrentHIPStream(dev.index()).stream();
    check_rc(orth_layer_forward_hip_ex(&L, has_plan ? ptr(*plan) : nullptr, has_plan ? plan->numel() : 0, bp, bdt,
                                       ptr(x), ptr(y), x.size(0), io_dtype(x), st));
}

// forward_planned(q, s, v, c, rp, input, output, alpha, plan=None, bias=None)
void forward_planned(const at::Tensor &q, const at::Tensor &s, const at::Tensor &v, const at::Tensor &c,
                     const at::Tensor &rp, const at::Tensor &x, at::Tensor y, double alpha,
                     const c10::optional<at::Tensor> &plan, const c10::optional<at::Tensor> &bias) {
    check_io(x, y);
    const orth_hip_layer_t L = describe(q, s, v, c, rp, x.size(1), y.size(1), alpha, x.device());
    launch(L, plan, bias, x, y);
}

// linear(x2d, q, s, v, c, rp, out_features, alpha, plan=None, bias=None) -> y [M, out_features]
at::Tensor linear(const at::Tensor &x, const at::Tensor &q, const at::Tensor &s, const at::Tensor &v,
                  const at::Tensor &c, const at::Tensor &rp, int64_t N, double alpha,
                  const c10::optional<at::Tensor> &plan, const c10::optional<at::Tensor> &bias) {
    req(x.is_cuda(), "OrthoLinear runs on a ROCm GPU only; move the module and the input to a cuda device "
                     "(the reference's CPU branch returns uninitialised memory)");
    req(x.dim() == 2, "input must be 2-D [M, K]");
    at::Tensor xc = x.contiguous();
    at::Tensor y = at::empty({xc.size(0), N}, xc.options());
    check_io(xc, y);
    const orth_hip_layer_t L = describe(q, s, v, c, rp, xc.size(1), N, alpha, xc.device());
    c10::optional<at::Tensor> bc;
    if (bias.has_value() && bias->defined()) bc = bias->contiguous();
    launch(L, plan, bc, xc, y);
    return y;
}

}  // namespace

PYBIND11_MODULE(_torch_ops, m) {
    m.doc() = "libortho_amd's compiled torch binding of the C ABI (eager calls)";
    m.def("forward_planned", &forward_planned, "the 8-argument forward plus a plan and a fused bias",
          py::arg("q_weight"), py::arg("q_scales"), py::arg("ortho_values"), py::arg("ortho_col_indices"),
          py::arg("ortho_row_ptr"), py::arg("input"), py::arg("output"), py::arg("alpha"),
          py::arg("plan") = py::none(), py::arg("bias") = py::none());
    m.def("linear", &linear, "OrthoLinear's forward on a 2-D input: the output allocated and written",
          py::arg("input"), py::arg("q_weight"), py::arg("q_scales"), py::arg("ortho_values"),
          py::arg("ortho_col_indices"), py::arg("ortho_row_ptr"), py::arg("out_features"), py::arg("alpha"),
          py::arg("plan") = py::none(), py::arg("bias") = py::none());
    m.def("abi_version", &orth_hip_abi_version);
}
