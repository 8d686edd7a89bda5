// The binary products' autograd node in C++ (built with
// torch.utils.cpp_extension by __graft_entry__.build(), linked against
// libclifford_hip.so). The forward and the backward call the library's C ABI
// (clf_product_fwd, clf_product_bwd_ld) on torch's current HIP stream, with
// the same semantics as the Python autograd.Function in products.py, which
// stays as the path when this module is not built. The autograd engine runs
// a Python backward on its device thread under the GIL; this node keeps
// Python off the backward path, which is most of a product's latency at the
// reference's published batch sizes (1 to 64 rows).
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include "../../include/clifford_hip.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

void check(int rc, const char* what) {
    if (rc == CLF_OK) return;
    const char* msg = clf_last_error();
    const std::string text = (msg && *msg) ? std::string(msg) : std::string(what) + " failed";
    // CLF_ERR_ARG / CLF_ERR_UNSUPPORTED surface as ValueError, HIP failures as RuntimeError
    TORCH_CHECK_VALUE(rc != CLF_ERR_ARG && rc != CLF_ERR_UNSUPPORTED, text);
    TORCH_CHECK(false, what, ": ", text);
}

// torch's ROCm build keeps GPU tensors on device type "cuda": its guard and
// stream helpers for that type are the ones masquerading as CUDA
void* stream_of(const at::Tensor& t) {
    return (void*)c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

at::Tensor product_fwd(const at::Tensor& a, const at::Tensor& b, int64_t op, int64_t n, int64_t neg, int64_t nul) {
    at::Tensor c = at::empty_like(a);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
    check(clf_product_fwd((int)op, (int)n, (uint32_t)neg, (uint32_t)nul, a.data_ptr<float>(), b.data_ptr<float>(),
                          c.data_ptr<float>(), a.size(0), stream_of(a)),
          "clf_product_fwd");
    return c;
}

struct ProductFn : public torch::autograd::Function<ProductFn> {
    static at::Tensor forward(AutogradContext* ctx, const at::Tensor& a, const at::Tensor& b, int64_t op, int64_t n,
                              int64_t neg, int64_t nul) {
        ctx->save_for_backward({a, b});
        ctx->saved_data["op"] = op;
        ctx->saved_data["n"] = n;
        ctx->saved_data["neg"] = neg;
        ctx->saved_data["nul"] = nul;
        return product_fwd(a, b, op, n, neg, nul);
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        const auto saved = ctx->get_saved_variables();
        const at::Tensor& a = saved[0];
        const at::Tensor& b = saved[1];
        const bool need_a = ctx->needs_input_grad(0), need_b = ctx->needs_input_grad(1);
        at::Tensor ga, gb;
        if (!need_a && !need_b) return {ga, gb, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
        if (need_a) ga = at::empty_like(a);
        if (need_b) gb = at::empty_like(b);
        at::Tensor gc = grads[0];
        const int64_t dim = a.size(1);
        int64_t ldg = dim;
        // the gradient of a sum arrives as a batch-stride-0 expansion: handed over as its one row
        if (gc.dim() == 2 && gc.size(0) > 1 && gc.stride(0) == 0) {
            at::Tensor row = gc.select(0, 0);
            if (row.stride(0) != 1 || (reinterpret_cast<uintptr_t>(row.data_ptr()) % 16) != 0)
                row = row.clone(at::MemoryFormat::Contiguous);
            gc = row;
            ldg = 0;
        } else {
            gc = gc.contiguous();
        }
        const c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
        check(clf_product_bwd_ld((int)ctx->saved_data["op"].toInt(), (int)ctx->saved_data["n"].toInt(),
                                 (uint32_t)ctx->saved_data["neg"].toInt(), (uint32_t)ctx->saved_data["nul"].toInt(),
                                 a.data_ptr<float>(), b.data_ptr<float>(), gc.data_ptr<float>(), ldg,
                                 need_a ? ga.data_ptr<float>() : nullptr, need_b ? gb.data_ptr<float>() : nullptr,
                                 a.size(0), stream_of(a)),
              "clf_product_bwd_ld");
        return {ga, gb, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
    }
};

at::Tensor product(const at::Tensor& a, const at::Tensor& b, int64_t op, int64_t n, int64_t neg, int64_t nul) {
    return ProductFn::apply(a, b, op, n, neg, nul);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("product", &product, "binary product with its backward node (2-D contiguous fp32 GPU rows)");
    m.def("product_fwd", &product_fwd, "binary product forward, no autograd node");
}
