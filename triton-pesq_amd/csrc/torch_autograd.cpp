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
#include <vector>
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

// forward: x [rows, n_in] -> y [rows, n_out]; adjoint: x [rows, n_out] -> y [rows, n_in]
void resample_enqueue(const float *x, float *y, int64_t rows, int64_t n_in, int64_t n_out,
                      const ResampleBank &b, bool forward, hipStream_t stream) {
    const pesq_resample_plan_info &info = b.plan_info();
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
}

// resample_enqueue of two signals of one shape (x0 -> y0, x1 -> y1), in one
// launch where the bank has the tiled kernels
void resample_enqueue_pair(const float *x0, float *y0, const float *x1, float *y1, int64_t rows,
                           int64_t n_in, int64_t n_out, const ResampleBank &b, bool forward,
                           hipStream_t stream) {
    const pesq_resample_plan_info &info = b.plan_info();
    if (forward && info.fwd_span > 0) {
        check(pesq_resample_plan_forward_pair(x0, y0, x1, y1, rows, n_in, n_out, &info,
                                              b.plan.data_ptr(), stream),
              "pesq_resample_plan_forward_pair");
    } else if (!forward && info.bwd_span > 0) {
        check(pesq_resample_plan_backward_pair(x0, y0, x1, y1, rows, n_in, n_out, &info,
                                               b.plan.data_ptr(), stream),
              "pesq_resample_plan_backward_pair");
    } else {
        resample_enqueue(x0, y0, rows, n_in, n_out, b, forward, stream);
        resample_enqueue(x1, y1, rows, n_in, n_out, b, forward, stream);
    }
}

// forward: src [rows, n_in] -> [rows, n_other]; adjoint: src [rows, n_out] -> [rows, n_other]
at::Tensor resample_launch(const at::Tensor &src, int64_t n_other, const ResampleBank &b,
                           bool forward) {
    const c10::DeviceGuard guard(src.device());
    const int64_t rows = src.size(0);
    const int64_t n_in = forward ? src.size(1) : n_other;
    const int64_t n_out = forward ? n_other : src.size(1);
    at::Tensor out = at::empty({rows, n_other}, src.options());
    resample_enqueue(src.data_ptr<float>(), out.data_ptr<float>(), rows, n_in, n_out, b, forward,
                     current_stream(src));
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

// Resample of the reference and the degraded signal (two [batch, n_in]
// tensors of one shape) as one node: one launch forward, and one for the
// adjoints when both signals take a gradient.  An output whose input takes
// no gradient is marked non-differentiable, so the pipeline after it forms
// only the gradients the caller asks for.  Under a double backward (grad
// mode on in the backward) the adjoints are the differentiable
// ResampleAdjoint nodes of the single signal path.
struct ResamplePair : public torch::autograd::Function<ResamplePair> {
    static variable_list forward(AutogradContext *ctx, const at::Tensor &x0, const at::Tensor &x1,
                                 int64_t n_out, const ResampleBank &b) {
        b.save(ctx);
        // an output nothing differentiates gets no zero filled gradient
        ctx->set_materialize_grads(false);
        const int64_t rows = x0.size(0), n_in = x0.size(1);
        ctx->saved_data["n_in"] = n_in;
        const c10::DeviceGuard guard(x0.device());
        at::Tensor y0 = at::empty({rows, n_out}, x0.options());
        at::Tensor y1 = at::empty({rows, n_out}, x0.options());
        resample_enqueue_pair(x0.data_ptr<float>(), y0.data_ptr<float>(), x1.data_ptr<float>(),
                              y1.data_ptr<float>(), rows, n_in, n_out, b, true,
                              current_stream(x0));
        if (!x0.requires_grad()) ctx->mark_non_differentiable({y0});
        if (!x1.requires_grad()) ctx->mark_non_differentiable({y1});
        return {y0, y1};
    }
    static variable_list backward(AutogradContext *ctx, variable_list grads) {
        const bool want0 = grads[0].defined() && ctx->needs_input_grad(0);
        const bool want1 = grads[1].defined() && ctx->needs_input_grad(1);
        variable_list out(4);
        if (!want0 && !want1) return out;
        const ResampleBank b = ResampleBank::load(ctx);
        const int64_t n_in = ctx->saved_data["n_in"].toInt();
        if (torch::autograd::GradMode::is_enabled() || !(want0 && want1)) {
            if (want0) out[0] = ResampleAdjoint::apply(grads[0].to(at::kFloat), n_in, b);
            if (want1) out[1] = ResampleAdjoint::apply(grads[1].to(at::kFloat), n_in, b);
            return out;
        }
        const at::Tensor g0 = grads[0].to(at::kFloat).contiguous();
        const at::Tensor g1 = grads[1].to(at::kFloat).contiguous();
        const c10::DeviceGuard guard(g0.device());
        const int64_t rows = g0.size(0), n_out = g0.size(1);
        out[0] = at::empty({rows, n_in}, g0.options());
        out[1] = at::empty({rows, n_in}, g0.options());
        resample_enqueue_pair(g0.data_ptr<float>(), out[0].data_ptr<float>(), g1.data_ptr<float>(),
                              out[1].data_ptr<float>(), rows, n_in, n_out, b, false,
                              current_stream(g0));
        return out;
    }
};

// checks the bank's tensors against a signal on `device` and bundles them
ResampleBank make_bank(int device, const at::Tensor &kernel, const at::Tensor &tap_lo,
                       const at::Tensor &tap_hi, const at::Tensor &phase_lo,
                       const at::Tensor &phase_hi, const at::Tensor &plan, const at::Tensor &info,
                       int64_t orig_step, int64_t new_step, int64_t width) {
    for (const at::Tensor *t : {&kernel, &tap_lo, &tap_hi, &phase_lo, &phase_hi, &plan})
        TORCH_CHECK(t->is_cuda() && t->get_device() == device && t->is_contiguous(),
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
    return b;
}

at::Tensor resample(const at::Tensor &x, int64_t n_out, const at::Tensor &kernel,
                    const at::Tensor &tap_lo, const at::Tensor &tap_hi, const at::Tensor &phase_lo,
                    const at::Tensor &phase_hi, const at::Tensor &plan, const at::Tensor &info,
                    int64_t orig_step, int64_t new_step, int64_t width) {
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() == 2 && x.is_contiguous(),
                "resample: x must be a contiguous [rows, samples] float32 GPU tensor");
    TORCH_CHECK(n_out >= 0, "resample: negative output length");
    const ResampleBank b = make_bank(x.get_device(), kernel, tap_lo, tap_hi, phase_lo, phase_hi,
                                     plan, info, orig_step, new_step, width);
    return Resample::apply(x, n_out, b);
}

void check_pipeline_inputs(const at::Tensor &ref, const at::Tensor &deg, const at::Tensor &table) {
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
}

std::vector<at::Tensor> pipeline(const at::Tensor &ref, const at::Tensor &deg,
                                 const at::Tensor &table, double factor) {
    check_pipeline_inputs(ref, deg, table);
    // what Python's ctx.needs_input_grad gives: the inputs autograd will ask for
    const bool grad = torch::autograd::GradMode::is_enabled();
    const int64_t mask = (grad && ref.requires_grad() ? PESQ_GRAD_REF : 0) |
                         (grad && deg.requires_grad() ? PESQ_GRAD_DEG : 0);
    return Pipeline::apply(ref, deg, table, factor, mask);
}

// pipeline() of the two signals resampled to 16 kHz (n_out samples per row):
// the computation the Python calls make one at a time (each signal resampled,
// then the pipeline node), with both resamplings in one node and one launch
// and no Python in between.  bank:
// the resampler's (kernel, tap_lo, tap_hi, phase_lo, phase_hi, plan, info),
// steps its (orig_step, new_step, width).
std::vector<at::Tensor> pipeline_resampled(const at::Tensor &ref, const at::Tensor &deg,
                                           const at::Tensor &table, double factor,
                                           const std::vector<at::Tensor> &bank,
                                           const std::vector<int64_t> &steps, int64_t n_out) {
    TORCH_CHECK(bank.size() == 7 && steps.size() == 3,
                "pipeline_resampled: the resampler bank is 7 tensors and 3 steps");
    TORCH_CHECK(ref.is_cuda() && deg.is_cuda() && ref.scalar_type() == at::kFloat &&
                    deg.scalar_type() == at::kFloat && ref.dim() == 2 &&
                    ref.sizes() == deg.sizes() && ref.is_contiguous() && deg.is_contiguous(),
                "pipeline_resampled: ref and deg must be contiguous [batch, samples] float32 GPU "
                "tensors of one shape");
    TORCH_CHECK(n_out >= 0, "pipeline_resampled: negative output length");
    const ResampleBank b = make_bank(ref.get_device(), bank[0], bank[1], bank[2], bank[3],
                                     bank[4], bank[5], bank[6], steps[0], steps[1], steps[2]);
    const variable_list r16 = ResamplePair::apply(ref, deg, n_out, b);
    return pipeline(r16[0], r16[1], table, factor);
}

// ---------------------------------------------------------------------------
// graphed loss (torch_pesq/triton_ops/loss.py:149-201): the loss of one input
// shape and one set of requires_grad flags, captured as two HIP graphs over
// static buffers: the forward (resampling to 16 kHz, pipeline forward) and the
// backward (pipeline backward, resampler adjoint).  A call copies its inputs
// into the static ones (unless they are those), replays the forward graph and
// returns the static loss; the autograd node copies the upstream gradient in,
// replays the backward graph and returns the static gradients.  As with
// torch.cuda.make_graphed_callables, which the reference uses, the results
// alias the static buffers (the next replay overwrites them) and the backward
// is differentiable once.  The graphs hold the same library calls the eager
// nodes make, so both give the same bits.
// ---------------------------------------------------------------------------

void check_hip(hipError_t status, const char *what) {
    if (status != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

struct GraphedLoss : torch::CustomClassHolder {
    at::Tensor table;
    double factor = 0.0;
    int mask = 0;
    bool resampled = false;
    ResampleBank bank;
    std::vector<int64_t> shape;  // of the example inputs, [batch, samples] or [samples]
    int64_t batch = 0, n_src = 0, n16 = 0;
    at::Tensor ref_s, deg_s;        // static inputs [batch, n_src]
    at::Tensor ref16, deg16;        // their 16 kHz rows (the static inputs themselves at 16 kHz)
    std::array<at::Tensor, 4> out;  // d_symm, d_asymm, mos, loss [batch]
    at::Tensor ws, scratch;         // forward workspace, backward scratch
    at::Tensor g_loss;              // upstream gradient of the loss [batch]
    at::Tensor g_ref16, g_deg16, g_ref, g_deg;

    // An executable graph and an event recorded after each of its launches,
    // on the stream of that launch: the graph, and the static buffers its
    // replays use, are released only after the event of its last launch has
    // completed, whichever stream (of several the caller may use) ran it.
    struct Exec {
        hipGraphExec_t exec = nullptr;
        hipEvent_t done = nullptr;
    };
    Exec fwd, bwd;  // forward from the static inputs, backward

    // Forward graphs that read a caller's own input buffers, by address: a
    // caller passing the same (ref, deg) buffers on two calls in a row (a
    // resident batch, an allocation the caching allocator hands out again)
    // gets one captured for them and from then on skips the two input copies.
    struct Direct {
        const void *ref, *deg;
        Exec graph;
    };
    static constexpr size_t kDirectGraphs = 4;
    std::vector<Direct> direct;  // the most recent capture last
    const void *last_ref = nullptr, *last_deg = nullptr;

    GraphedLoss() = default;
    GraphedLoss(const GraphedLoss &) = delete;
    GraphedLoss &operator=(const GraphedLoss &) = delete;
    ~GraphedLoss() override {
        // every graph's last replay has finished before the graphs and the
        // static buffers (freed after this body) go
        release(fwd);
        release(bwd);
        for (Direct &d : direct) release(d.graph);
    }

    static void launch(const Exec &e, hipStream_t stream) {
        check_hip(hipGraphLaunch(e.exec, stream), "hipGraphLaunch");
        check_hip(hipEventRecord(e.done, stream), "hipEventRecord");
    }

    // waits for the graph's last replay, then destroys it
    static void release(Exec &e) {
        if (e.done) (void)hipEventSynchronize(e.done);
        if (e.exec) (void)hipGraphExecDestroy(e.exec);
        if (e.done) (void)hipEventDestroy(e.done);
        e = Exec{};
    }

    void enqueue_forward(const float *ref_in, const float *deg_in, hipStream_t stream) const {
        if (resampled) {
            resample_enqueue_pair(ref_in, ref16.data_ptr<float>(), deg_in, deg16.data_ptr<float>(),
                                  batch, n_src, n16, bank, true, stream);
            ref_in = ref16.data_ptr<float>();
            deg_in = deg16.data_ptr<float>();
        }
        check(pesq_pipeline_forward(ref_in, deg_in, batch, n16, table.data_ptr(), factor, mask,
                                    out[0].data_ptr<float>(), out[1].data_ptr<float>(),
                                    out[2].data_ptr<float>(), out[3].data_ptr<float>(),
                                    ws.data_ptr(), stream),
              "pesq_pipeline_forward");
    }

    // the forward graph for a call's inputs (copying them into the static
    // inputs when it is the static one)
    const Exec &forward_graph(const at::Tensor &ref, const at::Tensor &deg, hipStream_t stream) {
        const void *rp = ref.data_ptr(), *dp = deg.data_ptr();
        const bool plain = ref.scalar_type() == at::kFloat && deg.scalar_type() == at::kFloat &&
                           ref.is_contiguous() && deg.is_contiguous() &&
                           rp != ref_s.data_ptr() && dp != deg_s.data_ptr();
        const bool repeated = rp == last_ref && dp == last_deg;
        last_ref = rp;
        last_deg = dp;
        if (plain) {
            for (const Direct &d : direct)
                if (d.ref == rp && d.deg == dp) return d.graph;
            if (repeated) {
                if (direct.size() == kDirectGraphs) {
                    release(direct.front().graph);
                    direct.erase(direct.begin());
                }
                const auto *r = static_cast<const float *>(rp);
                const auto *d = static_cast<const float *>(dp);
                direct.push_back({rp, dp, capture([&](hipStream_t s) { enqueue_forward(r, d, s); })});
                return direct.back().graph;
            }
        }
        stage(ref, ref_s, stream);
        stage(deg, deg_s, stream);
        return fwd;
    }

    void enqueue_backward(hipStream_t stream) const {
        check(pesq_pipeline_backward(nullptr, nullptr, nullptr, g_loss.data_ptr<float>(), batch,
                                     n16, table.data_ptr(), factor, mask,
                                     data_or_null<float>(g_ref16), data_or_null<float>(g_deg16),
                                     ws.data_ptr(), scratch.data_ptr(), stream),
              "pesq_pipeline_backward");
        if (resampled && g_ref.defined() && g_deg.defined()) {
            resample_enqueue_pair(g_ref16.data_ptr<float>(), g_ref.data_ptr<float>(),
                                  g_deg16.data_ptr<float>(), g_deg.data_ptr<float>(), batch, n_src,
                                  n16, bank, false, stream);
        } else if (resampled) {
            if (g_ref.defined())
                resample_enqueue(g_ref16.data_ptr<float>(), g_ref.data_ptr<float>(), batch, n_src,
                                 n16, bank, false, stream);
            if (g_deg.defined())
                resample_enqueue(g_deg16.data_ptr<float>(), g_deg.data_ptr<float>(), batch, n_src,
                                 n16, bank, false, stream);
        }
    }

    // the calls of enqueue(stream) as an executable graph, captured on a
    // stream of its own (capture records, it does not run anything)
    template <class F>
    Exec capture(F &&enqueue) {
        hipStream_t stream = nullptr;
        check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipError_t status = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
        if (status == hipSuccess) {
            try {
                enqueue(stream);
            } catch (...) {
                (void)hipStreamEndCapture(stream, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                (void)hipStreamDestroy(stream);
                throw;
            }
            status = hipStreamEndCapture(stream, &graph);
        }
        if (status == hipSuccess) status = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipStreamDestroy(stream);
        check_hip(status, "capturing the graphed loss");
        Exec out{exec, nullptr};
        status = hipEventCreateWithFlags(&out.done, hipEventDisableTiming);
        if (status != hipSuccess) {
            (void)hipGraphExecDestroy(exec);
            check_hip(status, "hipEventCreateWithFlags");
        }
        return out;
    }

    // copies a call's input into its static buffer
    void stage(const at::Tensor &src, const at::Tensor &dst, hipStream_t stream) const {
        if (src.data_ptr() == dst.data_ptr()) return;
        if (src.scalar_type() == at::kFloat && src.is_contiguous()) {
            check_hip(hipMemcpyAsync(dst.data_ptr(), src.data_ptr(), dst.nbytes(),
                                     hipMemcpyDeviceToDevice, stream),
                      "hipMemcpyAsync");
        } else {
            const at::NoGradGuard no_grad;
            dst.view(src.sizes()).copy_(src);
        }
    }
};

struct GraphedCall : public torch::autograd::Function<GraphedCall> {
    static at::Tensor forward(AutogradContext *ctx, const at::Tensor &ref, const at::Tensor &deg,
                              const c10::intrusive_ptr<GraphedLoss> &g) {
        TORCH_CHECK(ref.defined() && deg.defined() && ref.sizes() == g->shape &&
                        deg.sizes() == g->shape,
                    "graphed loss: the inputs must have the shape it was captured for, ",
                    c10::IntArrayRef(g->shape));
        TORCH_CHECK(ref.device() == g->ref_s.device() && deg.device() == g->ref_s.device(),
                    "graphed loss: the inputs must be on ", g->ref_s.device());
        const c10::DeviceGuard guard(g->ref_s.device());
        const hipStream_t stream = current_stream(g->ref_s);
        GraphedLoss::launch(g->forward_graph(ref, deg, stream), stream);
        ctx->saved_data["graphed"] = c10::IValue::make_capsule(g);
        ctx->set_materialize_grads(false);
        return g->out[3].detach();
    }

    static variable_list backward(AutogradContext *ctx, variable_list grads) {
        const auto g =
            c10::static_intrusive_pointer_cast<GraphedLoss>(ctx->saved_data["graphed"].toCapsule());
        variable_list result(3);  // ref, deg, the graphs
        if (!grads[0].defined() || g->bwd.exec == nullptr) return result;
        const c10::DeviceGuard guard(g->g_loss.device());
        const hipStream_t stream = current_stream(g->g_loss);
        if (grads[0].data_ptr() != g->g_loss.data_ptr()) {
            const at::NoGradGuard no_grad;
            g->g_loss.copy_(grads[0]);
        }
        GraphedLoss::launch(g->bwd, stream);
        if (g->g_ref.defined()) result[0] = g->g_ref.view(g->shape).detach();
        if (g->g_deg.defined()) result[1] = g->g_deg.view(g->shape).detach();
        if (torch::autograd::GradMode::is_enabled() && grads[0].requires_grad()) {
            for (size_t i = 0; i < 2; ++i)
                if (result[i].defined())
                    result[i] = OnceDifferentiable::apply(result[i].requires_grad_(true));
        }
        return result;
    }
};

// the Python object PesqLossTriton.graphed returns
// The static buffers of a graphed loss for examples ref, deg (their shape and
// requires_grad flags).  bank: the resampler's (kernel, tap_lo, tap_hi,
// phase_lo, phase_hi, plan, info) and steps its (orig_step, new_step, width,
// output length), both empty at 16 kHz.
c10::intrusive_ptr<GraphedLoss> graphed_buffers(const at::Tensor &ref, const at::Tensor &deg,
                                                const at::Tensor &table, double factor,
                                                const std::vector<at::Tensor> &bank,
                                                const std::vector<int64_t> &steps) {
    TORCH_CHECK(ref.dim() >= 1 && ref.dim() <= 2 && ref.sizes() == deg.sizes(),
                "graphed loss: ref and deg must be [batch, samples] or [samples] of one shape");
    TORCH_CHECK(bank.empty() ? steps.empty() : bank.size() == 7 && steps.size() == 4,
                "graphed loss: the resampler bank is 7 tensors and 4 sizes");
    auto g = c10::make_intrusive<GraphedLoss>();
    g->shape = ref.sizes().vec();
    g->table = table;
    g->factor = factor;
    g->mask = (ref.requires_grad() ? PESQ_GRAD_REF : 0) | (deg.requires_grad() ? PESQ_GRAD_DEG : 0);
    g->batch = ref.dim() == 2 ? ref.size(0) : 1;
    g->n_src = ref.size(-1);
    const c10::DeviceGuard guard(ref.device());
    const auto f32 = ref.options().dtype(at::kFloat).requires_grad(false);
    g->ref_s = at::empty({g->batch, g->n_src}, f32);
    g->deg_s = at::empty({g->batch, g->n_src}, f32);
    g->resampled = !bank.empty();
    if (g->resampled) {
        g->bank = make_bank(ref.get_device(), bank[0], bank[1], bank[2], bank[3], bank[4], bank[5],
                            bank[6], steps[0], steps[1], steps[2]);
        g->n16 = steps[3];
        TORCH_CHECK(g->n16 > 0, "graphed loss: empty signals");
        g->ref16 = at::empty({g->batch, g->n16}, f32);
        g->deg16 = at::empty({g->batch, g->n16}, f32);
    } else {
        g->n16 = g->n_src;
        g->ref16 = g->ref_s;
        g->deg16 = g->deg_s;
    }
    check_pipeline_inputs(g->ref16, g->deg16, table);
    size_t bytes = 0;
    check(pesq_pipeline_forward_workspace(g->batch, g->n16, g->mask, &bytes),
          "pesq_pipeline_forward_workspace");
    g->ws = at::empty({static_cast<int64_t>(bytes)}, f32.dtype(at::kByte));
    for (at::Tensor &o : g->out) o = at::empty({g->batch}, f32);
    if (g->mask != 0) {
        check(pesq_pipeline_backward_workspace(g->batch, g->n16, g->mask, &bytes),
              "pesq_pipeline_backward_workspace");
        g->scratch = at::empty({static_cast<int64_t>(bytes)}, f32.dtype(at::kByte));
        g->g_loss = at::empty({g->batch}, f32);
        if (g->mask & PESQ_GRAD_REF) g->g_ref16 = at::empty({g->batch, g->n16}, f32);
        if (g->mask & PESQ_GRAD_DEG) g->g_deg16 = at::empty({g->batch, g->n16}, f32);
        if (g->resampled) {
            if (g->g_ref16.defined()) g->g_ref = at::empty({g->batch, g->n_src}, f32);
            if (g->g_deg16.defined()) g->g_deg = at::empty({g->batch, g->n_src}, f32);
        } else {
            g->g_ref = g->g_ref16;
            g->g_deg = g->g_deg16;
        }
    }
    return g;
}

// the Python object PesqLossTriton.graphed returns
class GraphedLossCallable {
  public:
    GraphedLossCallable(const at::Tensor &ref, const at::Tensor &deg, const at::Tensor &table,
                        double factor, const std::vector<at::Tensor> &bank,
                        const std::vector<int64_t> &steps)
        : graphed_(graphed_buffers(ref, deg, table, factor, bank, steps)) {
        // the static buffers are allocated on the current stream; the capture
        // stream only records
        GraphedLoss &s = *graphed_;
        const c10::DeviceGuard guard(s.ref_s.device());
        s.fwd = s.capture([&s](hipStream_t stream) {
            s.enqueue_forward(s.ref_s.data_ptr<float>(), s.deg_s.data_ptr<float>(), stream);
        });
        if (s.mask != 0) s.bwd = s.capture([&s](hipStream_t stream) { s.enqueue_backward(stream); });
    }

    at::Tensor call(const at::Tensor &ref, const at::Tensor &deg) const {
        return GraphedCall::apply(ref, deg, graphed_);
    }

  private:
    c10::intrusive_ptr<GraphedLoss> graphed_;
};

// A whole training step of the loss, grad(loss.sum(), inputs), as one HIP
// graph: the forward, then the backward with upstream gradients of one (the
// derivative of the sum), on static inputs the caller writes into.  No
// counterpart in the reference, whose graphs stop at the autograd boundary;
// it is the step the library's calls make capturable as a whole.
class GraphedStep {
  public:
    GraphedStep(const at::Tensor &ref, const at::Tensor &deg, const at::Tensor &table,
                double factor, const std::vector<at::Tensor> &bank,
                const std::vector<int64_t> &steps)
        : graphed_(graphed_buffers(ref, deg, table, factor, bank, steps)) {
        GraphedLoss &s = *graphed_;
        TORCH_CHECK(s.mask != 0, "graphed step: ref or deg must require a gradient");
        const c10::DeviceGuard guard(s.ref_s.device());
        s.g_loss.fill_(1.0);  // d sum / d loss, written once, before any replay
        s.fwd = s.capture([&s](hipStream_t stream) {
            s.enqueue_forward(s.ref_s.data_ptr<float>(), s.deg_s.data_ptr<float>(), stream);
            s.enqueue_backward(stream);
        });
    }

    void replay() const {
        GraphedLoss &s = *graphed_;
        const c10::DeviceGuard guard(s.ref_s.device());
        GraphedLoss::launch(s.fwd, current_stream(s.ref_s));
    }

    // the static inputs (ref, deg), shaped like the examples
    std::vector<at::Tensor> inputs() const {
        return {graphed_->ref_s.view(graphed_->shape), graphed_->deg_s.view(graphed_->shape)};
    }

    // loss [batch] and the gradients of ref and deg (undefined, i.e. None,
    // for an input whose example did not require one)
    std::vector<at::Tensor> outputs() const {
        const GraphedLoss &s = *graphed_;
        return {s.out[3], s.g_ref.defined() ? s.g_ref.view(s.shape) : at::Tensor(),
                s.g_deg.defined() ? s.g_deg.view(s.shape) : at::Tensor()};
    }

  private:
    c10::intrusive_ptr<GraphedLoss> graphed_;
};

}  // namespace

PYBIND11_MODULE(_pesq_torch, m) {
    m.doc() = "PyTorch autograd nodes of the PESQ HIP library";
    m.def("pipeline", &pipeline, "(ref, deg, table, factor) -> [d_symm, d_asymm, mos, loss]",
          pybind11::arg("ref"), pybind11::arg("deg"), pybind11::arg("table"),
          pybind11::arg("factor"));
    m.def("pipeline_resampled", &pipeline_resampled,
          "(ref, deg, table, factor, bank, steps, n_out) -> [d_symm, d_asymm, mos, loss] of the "
          "signals resampled to 16 kHz",
          pybind11::arg("ref"), pybind11::arg("deg"), pybind11::arg("table"),
          pybind11::arg("factor"), pybind11::arg("bank"), pybind11::arg("steps"),
          pybind11::arg("n_out"));
    m.def("resample", &resample,
          "(x, n_out, kernel, tap_lo, tap_hi, phase_lo, phase_hi, plan, info, orig_step, "
          "new_step, width) -> y, differentiable twice");
    pybind11::class_<GraphedLossCallable>(m, "GraphedLoss",
                                          "loss(ref, deg) of one input shape replayed from HIP graphs")
        .def(pybind11::init<const at::Tensor &, const at::Tensor &, const at::Tensor &, double,
                            const std::vector<at::Tensor> &, const std::vector<int64_t> &>(),
             pybind11::arg("ref"), pybind11::arg("deg"), pybind11::arg("table"),
             pybind11::arg("factor"), pybind11::arg("bank"), pybind11::arg("steps"))
        .def("__call__", &GraphedLossCallable::call, pybind11::arg("ref"), pybind11::arg("deg"));
    pybind11::class_<GraphedStep>(m, "GraphedStep",
                                  "grad(loss(ref, deg).sum(), inputs) of one input shape as one "
                                  "HIP graph on static inputs")
        .def(pybind11::init<const at::Tensor &, const at::Tensor &, const at::Tensor &, double,
                            const std::vector<at::Tensor> &, const std::vector<int64_t> &>(),
             pybind11::arg("ref"), pybind11::arg("deg"), pybind11::arg("table"),
             pybind11::arg("factor"), pybind11::arg("bank"), pybind11::arg("steps"))
        .def("replay", &GraphedStep::replay)
        .def("inputs", &GraphedStep::inputs)
        .def("outputs", &GraphedStep::outputs);
}
