// PyTorch autograd node of the fused 16 kHz pipeline, in C++.
//
// The same two calls as the Python autograd Function of the reference
// (torch_pesq/triton_ops/loss.py:104-147 with the backward chain of
// chain.py:780-1021, spectral.py:535-581, elementwise.py:233-269,607-652,
// iir.py:1248-1258), made through the C ABI of libpesq_hip.so.  Written in C++
// because autograd runs a Python backward on its worker thread under the
// interpreter lock, where every Python statement of the backward and the
// engine's Python node handling cost about 2.5 times what they cost on the
// main thread; a C++ node runs there without Python.
//
// The entry point checks the tensors' device, dtype, shape and layout (the
// library checks the lengths; the Python caller raises the reference's
// exception types first), allocates the outputs and workspaces on the
// caller's device and enqueues the library calls on PyTorch's current stream.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <array>
#include <stdexcept>
#include <string>

#include "pesq_hip.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

void check(int status, const char *what) {
    if (status != PESQ_OK) {
        throw std::runtime_error(std::string(what) + ": " + pesq_last_error() + " (status " +
                                 std::to_string(status) + ")");
    }
}

hipStream_t current_stream(const at::Tensor &t) {
    return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

template <class T>
T *data_or_null(const at::Tensor &t) {
    return t.defined() ? static_cast<T *>(t.data_ptr()) : nullptr;
}

// Identity whose derivative raises: attached to the gradients when a double
// backward would need the derivative of the pipeline's backward, as Python's
// @once_differentiable does.
struct OnceDifferentiable : public torch::autograd::Function<OnceDifferentiable> {
    static at::Tensor forward(AutogradContext *, const at::Tensor &x) { return x.clone(); }
    static variable_list backward(AutogradContext *, variable_list) {
        throw std::runtime_error(
            "trying to differentiate twice a function that was marked with @once_differentiable");
    }
};

struct Pipeline : public torch::autograd::Function<Pipeline> {
    // (ref, deg) [batch, len] float32 at 16 kHz -> (d_symm, d_asymm, mos, loss) [batch]
    // grad_mask (PESQ_GRAD_*) names the inputs the backward will differentiate
    static variable_list forward(AutogradContext *ctx, const at::Tensor &ref, const at::Tensor &deg,
                                 const at::Tensor &table, double factor, int64_t grad_mask) {
        const int mask = static_cast<int>(grad_mask);
        const c10::DeviceGuard guard(ref.device());
        const int64_t batch = ref.size(0), len = ref.size(1);
        size_t ws_bytes = 0;
        check(pesq_pipeline_forward_workspace(batch, len, mask, &ws_bytes),
              "pesq_pipeline_forward_workspace");
        at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, ref.options().dtype(at::kByte));
        std::array<at::Tensor, 4> out;
        for (at::Tensor &o : out) o = at::empty({batch}, ref.options());
        check(pesq_pipeline_forward(ref.data_ptr<float>(), deg.data_ptr<float>(), batch, len,
                                    table.data_ptr(), factor, mask, out[0].data_ptr<float>(),
                                    out[1].data_ptr<float>(), out[2].data_ptr<float>(),
                                    out[3].data_ptr<float>(), ws.data_ptr(), current_stream(ref)),
              "pesq_pipeline_forward");
        ctx->set_materialize_grads(false);
        ctx->save_for_backward({ws, table});
        ctx->saved_data["batch"] = batch;
        ctx->saved_data["len"] = len;
        ctx->saved_data["mask"] = mask;
        ctx->saved_data["factor"] = factor;
        return {out[0], out[1], out[2], out[3]};
    }

    static variable_list backward(AutogradContext *ctx, variable_list grads) {
        const int64_t batch = ctx->saved_data["batch"].toInt();
        const int64_t len = ctx->saved_data["len"].toInt();
        const int mask = static_cast<int>(ctx->saved_data["mask"].toInt());
        const double factor = ctx->saved_data["factor"].toDouble();
        variable_list result(5);  // one per argument of forward: ref, deg, table, factor, mask
        bool any = false, upstream_requires_grad = false;
        for (const at::Tensor &g : grads) {
            any = any || g.defined();
            upstream_requires_grad = upstream_requires_grad || (g.defined() && g.requires_grad());
        }
        if (mask == 0 || !any) return result;

        const variable_list saved = ctx->get_saved_variables();
        const at::Tensor &ws = saved[0];
        const at::Tensor &table = saved[1];
        const c10::DeviceGuard guard(ws.device());
        std::array<at::Tensor, 4> g;
        {
            const at::NoGradGuard no_grad;
            for (size_t i = 0; i < 4; ++i)
                if (grads[i].defined()) g[i] = grads[i].to(at::kFloat).contiguous();
        }
        size_t bw_bytes = 0;
        check(pesq_pipeline_backward_workspace(batch, len, mask, &bw_bytes),
              "pesq_pipeline_backward_workspace");
        at::Tensor scratch = at::empty({static_cast<int64_t>(bw_bytes)}, ws.options());
        const auto f32 = ws.options().dtype(at::kFloat);
        at::Tensor g_ref, g_deg;
        if (mask & PESQ_GRAD_REF) g_ref = at::empty({batch, len}, f32);
        if (mask & PESQ_GRAD_DEG) g_deg = at::empty({batch, len}, f32);
        check(pesq_pipeline_backward(data_or_null<float>(g[0]), data_or_null<float>(g[1]),
                                     data_or_null<float>(g[2]), data_or_null<float>(g[3]), batch,
                                     len, table.data_ptr(), factor, mask,
                                     data_or_null<float>(g_ref), data_or_null<float>(g_deg),
                                     ws.data_ptr(), scratch.data_ptr(), current_stream(ws)),
              "pesq_pipeline_backward");
        result[0] = g_ref;
        result[1] = g_deg;
        if (torch::autograd::GradMode::is_enabled() && upstream_requires_grad) {
            for (size_t i = 0; i < 2; ++i)
                if (result[i].defined())
                    result[i] = OnceDifferentiable::apply(result[i].detach().requires_grad_(true));
        }
        return result;
    }
};

// ---------------------------------------------------------------------------
// resampler (torch_pesq/triton_ops/resample.py:381-410,442-574): forward,
// adjoint, and the adjoint's own derivative (the forward) for double backward
// ---------------------------------------------------------------------------

// The filter bank of one rate pair: the per phase tap ranges for the untiled
// kernels, the compact tables of the tiled ones and their geometry (`info`, a
// host copy of pesq_resample_plan_info).
struct ResampleBank {
    at::Tensor kernel, tap_lo, tap_hi, phase_lo, phase_hi, plan, info;
    int64_t orig_step = 0, new_step = 0, width = 0;

    const pesq_resample_plan_info &plan_info() const {
        return *static_cast<const pesq_resample_plan_info *>(info.data_ptr());
    }
    void save(AutogradContext *ctx) const {
        auto &d = ctx->saved_data;
        d["kernel"] = kernel;
        d["tap_lo"] = tap_lo;
        d["tap_hi"] = tap_hi;
        d["phase_lo"] = phase_lo;
        d["phase_hi"] = phase_hi;
        d["plan"] = plan;
        d["info"] = info;
        d["orig_step"] = orig_step;
        d["new_step"] = new_step;
        d["width"] = width;
    }
    static ResampleBank load(AutogradContext *ctx) {
        auto &d = ctx->saved_data;
        ResampleBank b;
        b.kernel = d["kernel"].toTensor();
        b.tap_lo = d["tap_lo"].toTensor();
        b.tap_hi = d["tap_hi"].toTensor();
        b.phase_lo = d["phase_lo"].toTensor();
        b.phase_hi = d["phase_hi"].toTensor();
        b.plan = d["plan"].toTensor();
        b.info = d["info"].toTensor();
        b.orig_step = d["orig_step"].toInt();
        b.new_step = d["new_step"].toInt();
        b.width = d["width"].toInt();
        return b;
    }
};

// forward: src [rows, n_in] -> [rows, n_other]; adjoint: src [rows, n_out] -> [rows, n_other]
at::Tensor resample_launch(const at::Tensor &src, int64_t n_other, const ResampleBank &b,
                           bool forward) {
    const c10::DeviceGuard guard(src.device());
    const int64_t rows = src.size(0);
    const int64_t n_in = forward ? src.size(1) : n_other;
    const int64_t n_out = forward ? n_other : src.size(1);
    at::Tensor out = at::empty({rows, n_other}, src.options());
    const pesq_resample_plan_info &info = b.plan_info();
    const hipStream_t stream = current_stream(src);
    const float *x = src.data_ptr<float>();
    float *y = out.data_ptr<float>();
    const int64_t ntaps = b.kernel.size(1);
    if (forward && info.fwd_span > 0) {
        check(pesq_resample_plan_forward(x, y, rows, n_in, n_out, &info, b.plan.data_ptr(), stream),
              "pesq_resample_plan_forward");
    } else if (!forward && info.bwd_span > 0) {
        check(pesq_resample_plan_backward(x, y, rows, n_in, n_out, &info, b.plan.data_ptr(), stream),
              "pesq_resample_plan_backward");
    } else if (forward) {
        check(pesq_resample_forward(x, y, rows, n_in, n_out, b.kernel.data_ptr<float>(),
                                    b.tap_lo.data_ptr<int32_t>(), b.tap_hi.data_ptr<int32_t>(),
                                    b.orig_step, b.new_step, b.width, ntaps, stream),
              "pesq_resample_forward");
    } else {
        check(pesq_resample_backward(x, y, rows, n_in, n_out, b.kernel.data_ptr<float>(),
                                     b.phase_lo.data_ptr<int32_t>(), b.phase_hi.data_ptr<int32_t>(),
                                     b.orig_step, b.new_step, b.width, ntaps, stream),
              "pesq_resample_backward");
    }
    return out;
}

struct ResampleAdjoint;

struct Resample : public torch::autograd::Function<Resample> {
    static at::Tensor forward(AutogradContext *ctx, const at::Tensor &x, int64_t n_out,
                              const ResampleBank &b) {
        b.save(ctx);
        ctx->saved_data["n_in"] = x.size(1);
        return resample_launch(x, n_out, b, true);
    }
    static variable_list backward(AutogradContext *ctx, variable_list grads);
};

struct ResampleAdjoint : public torch::autograd::Function<ResampleAdjoint> {
    static at::Tensor forward(AutogradContext *ctx, const at::Tensor &grad_y, int64_t n_in,
                              const ResampleBank &b) {
        b.save(ctx);
        ctx->saved_data["n_out"] = grad_y.size(1);
        return resample_launch(grad_y.contiguous(), n_in, b, false);
    }
    static variable_list backward(AutogradContext *ctx, variable_list grads) {
        if (!grads[0].defined() || !ctx->needs_input_grad(0)) return {at::Tensor(), at::Tensor(), at::Tensor()};
        const ResampleBank b = ResampleBank::load(ctx);
        const int64_t n_out = ctx->saved_data["n_out"].toInt();
        return {Resample::apply(grads[0].to(at::kFloat).contiguous(), n_out, b), at::Tensor(),
                at::Tensor()};
    }
};

variable_list Resample::backward(AutogradContext *ctx, variable_list grads) {
    if (!grads[0].defined() || !ctx->needs_input_grad(0)) return {at::Tensor(), at::Tensor(), at::Tensor()};
    const ResampleBank b = ResampleBank::load(ctx);
    const int64_t n_in = ctx->saved_data["n_in"].toInt();
    return {ResampleAdjoint::apply(grads[0].to(at::kFloat), n_in, b), at::Tensor(), at::Tensor()};
}

at::Tensor resample(const at::Tensor &x, int64_t n_out, const at::Tensor &kernel,
                    const at::Tensor &tap_lo, const at::Tensor &tap_hi, const at::Tensor &phase_lo,
                    const at::Tensor &phase_hi, const at::Tensor &plan, const at::Tensor &info,
                    int64_t orig_step, int64_t new_step, int64_t width) {
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() == 2 && x.is_contiguous(),
                "resample: x must be a contiguous [rows, samples] float32 GPU tensor");
    for (const at::Tensor *t : {&kernel, &tap_lo, &tap_hi, &phase_lo, &phase_hi, &plan})
        TORCH_CHECK(t->is_cuda() && t->get_device() == x.get_device() && t->is_contiguous(),
                    "resample: the filter tables must be contiguous and on the signal's device");
    TORCH_CHECK(kernel.scalar_type() == at::kFloat && kernel.dim() == 2 &&
                    kernel.size(0) == new_step,
                "resample: kernel must be [new_step, width_total] float32");
    TORCH_CHECK(tap_lo.scalar_type() == at::kInt && tap_hi.scalar_type() == at::kInt &&
                    phase_lo.scalar_type() == at::kInt && phase_hi.scalar_type() == at::kInt &&
                    tap_lo.numel() == new_step && tap_hi.numel() == new_step &&
                    phase_lo.numel() == kernel.size(1) && phase_hi.numel() == kernel.size(1),
                "resample: tap and phase ranges must be int32 of the bank's shape");
    TORCH_CHECK(!info.is_cuda() && info.scalar_type() == at::kByte && info.is_contiguous() &&
                    info.numel() == static_cast<int64_t>(sizeof(pesq_resample_plan_info)),
                "resample: info must be the host bytes of pesq_resample_plan_info");
    TORCH_CHECK(n_out >= 0, "resample: negative output length");
    ResampleBank b;
    b.kernel = kernel;
    b.tap_lo = tap_lo;
    b.tap_hi = tap_hi;
    b.phase_lo = phase_lo;
    b.phase_hi = phase_hi;
    b.plan = plan;
    b.info = info;
    b.orig_step = orig_step;
    b.new_step = new_step;
    b.width = width;
    const pesq_resample_plan_info &pi = b.plan_info();
    TORCH_CHECK(pi.orig_step == orig_step && pi.new_step == new_step && pi.width == width &&
                    pi.width_total == kernel.size(1) && plan.numel() >= pi.bytes,
                "resample: info does not describe this filter bank");
    return Resample::apply(x, n_out, b);
}

std::vector<at::Tensor> pipeline(const at::Tensor &ref, const at::Tensor &deg,
                                 const at::Tensor &table, double factor) {
    TORCH_CHECK(ref.is_cuda() && deg.is_cuda() && table.is_cuda(),
                "pipeline: ref, deg and table must be GPU tensors");
    TORCH_CHECK(ref.get_device() == deg.get_device() && ref.get_device() == table.get_device(),
                "pipeline: ref, deg and table must be on the same device");
    TORCH_CHECK(ref.scalar_type() == at::kFloat && deg.scalar_type() == at::kFloat,
                "pipeline: ref and deg must be float32");
    TORCH_CHECK(ref.dim() == 2 && ref.sizes() == deg.sizes(),
                "pipeline: ref and deg must be [batch, samples] of the same shape");
    TORCH_CHECK(ref.is_contiguous() && deg.is_contiguous() && table.is_contiguous(),
                "pipeline: ref, deg and table must be contiguous");
    TORCH_CHECK(table.scalar_type() == at::kByte &&
                    table.numel() == static_cast<int64_t>(pesq_model_table_bytes()),
                "pipeline: table must be the packed model table (uint8, ",
                pesq_model_table_bytes(), " bytes)");
    // what Python's ctx.needs_input_grad gives: the inputs autograd will ask for
    const bool grad = torch::autograd::GradMode::is_enabled();
    const int64_t mask = (grad && ref.requires_grad() ? PESQ_GRAD_REF : 0) |
                         (grad && deg.requires_grad() ? PESQ_GRAD_DEG : 0);
    return Pipeline::apply(ref, deg, table, factor, mask);
}

}  // namespace

PYBIND11_MODULE(_pesq_torch, m) {
    m.doc() = "PyTorch autograd nodes of the PESQ HIP library";
    m.def("pipeline", &pipeline, "(ref, deg, table, factor) -> [d_symm, d_asymm, mos, loss]",
          pybind11::arg("ref"), pybind11::arg("deg"), pybind11::arg("table"),
          pybind11::arg("factor"));
    m.def("resample", &resample,
          "(x, n_out, kernel, tap_lo, tap_hi, phase_lo, phase_hi, plan, info, orig_step, "
          "new_step, width) -> y, differentiable twice");
}
