// klp_torch.cpp — kernel_opt's compiled binding over the C ABI of
// libkernel_opt_hip.so (include/kernel_opt_hip.h).
//
// It restates, in C++, the two Python layers of the reference that sit on
// the hot path of every call:
//  - the pybind11 module kernel_opt._C (reference csrc/bindings.cpp:17-27):
//    fused_logprob_entropy_naive / _v1 / _v1_backward with caller-allocated
//    outputs, the reference's TORCH_CHECK messages as RuntimeError
//    (csrc/fused_logprob.cu:294-311,362-374,412-424), work queued on the
//    current stream of the logits' device;
//  - the autograd op of python/kernel_opt/ops.py:49-111: input assertions
//    (AssertionError, ops.py:16-21), three float32 outputs shaped like the
//    targets (ops.py:24-30), (logits, targets, lse, entropy) saved for a
//    backward that allocates only d_logits (ops.py:62,83) and returns no
//    gradient for the targets (ops.py:89).
// Upstream gradients the loss does not use arrive undefined and reach the
// kernel as null pointers (the reference allocates zeros, ops.py:71-76).
//
// Relaxations, as in kernel_opt/_C.py: logits whose rows have unit stride
// and are reachable through at most two leading strides are accepted without
// a copy (the shifted slice logits[:, :-1, :]); a temperature T other than 1
// scales each logit by fp32(1/T) inside the kernels.
//
// Why compiled: through ctypes the forward cost ~15 us of host time per call
// and the autograd forward + backward ~100 us (Python checks, three
// allocations, the autograd.Function machinery), more than an eager
// log_softmax forward + backward; small batches are paced by the host.
#include <ATen/ATen.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/python.h>

#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <array>
#include <cmath>
#include <list>
#include <mutex>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "kernel_opt_hip.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// An input-contract violation of the Python-level entry points (the
// reference's ops.py asserts); surfaces in Python as AssertionError.
struct AssertFailure : std::exception {
    explicit AssertFailure(std::string m) : msg(std::move(m)) {}
    const char* what() const noexcept override { return msg.c_str(); }
    std::string msg;
};

// Raised, before anything is allocated or launched, when the current stream
// is being captured into a graph: captured calls take kernel_opt's Python
// path (ctypes over the same C ABI), which catches this.  The binding is not
// used under capture: the one capture run through it (a split-row forward and
// its autograd backward) ended in a host segmentation fault inside
// capture_end whose cause is not known.
struct CaptureDeclined : std::exception {
    const char* what() const noexcept override {
        return "kernel_opt: the compiled binding does not run under graph capture";
    }
};

void decline_under_capture(int device) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hipStream_t stream =
        c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream();
    if (hipStreamIsCapturing(stream, &status) != hipSuccess)
        throw std::runtime_error("kernel_opt: hipStreamIsCapturing failed");
    if (status != hipStreamCaptureStatusNone) throw CaptureDeclined();
}

void require(bool cond, const char* msg) {
    if (!cond) throw std::runtime_error(msg);
}

void check_status(int rc) {
    if (rc == KLP_OK) return;
    char buf[1024];
    buf[0] = '\0';
    klp_last_error(buf, sizeof buf);
    if (buf[0] == '\0')
        throw std::runtime_error("kernel_opt: native call failed with status " +
                                 std::to_string(rc));
    throw std::runtime_error(buf);
}

int dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kBFloat16: return KLP_BF16;
        case at::kHalf: return KLP_FP16;
        case at::kFloat: return KLP_FP32;
        default: return -1;
    }
}

const float* fptr(const at::Tensor& t) {
    return t.defined() ? static_cast<const float*>(t.data_ptr()) : nullptr;
}
float* out_ptr(at::Tensor& t) { return static_cast<float*>(t.data_ptr()); }

// (rows_inner, stride_outer, stride_inner) of the rows of t (row r starts at
// (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner
// elements), or nothing when the rows need more than two leading strides or
// do not have unit stride.  Same walk as kernel_opt._C.row_layout.
std::optional<std::array<int64_t, 3>> row_layout(const at::Tensor& t) {
    const int64_t nd = t.dim();
    if (nd == 0) return std::nullopt;
    const int64_t V = t.size(-1);
    if (t.is_contiguous()) {
        const int64_t n = V ? t.numel() / V : 0;
        if (n >= 2) return std::array<int64_t, 3>{n, 0, V};
    }
    if (V > 1 && t.stride(-1) != 1) return std::nullopt;
    std::vector<std::pair<int64_t, int64_t>> merged;  // (size, stride)
    int64_t n_rows = 1;
    for (int64_t d = 0; d + 1 < nd; ++d) {
        const int64_t size = t.size(d), stride = t.stride(d);
        n_rows *= size;
        if (size == 1) continue;
        if (!merged.empty() && merged.back().second == stride * size) {
            merged.back().first *= size;
            merged.back().second = stride;
        } else {
            merged.emplace_back(size, stride);
        }
    }
    if (merged.empty()) return std::array<int64_t, 3>{std::max<int64_t>(n_rows, 1), 0, 0};
    if (merged.size() == 1) return std::array<int64_t, 3>{merged[0].first, 0, merged[0].second};
    if (merged.size() == 2)
        return std::array<int64_t, 3>{merged[1].first, merged[0].second, merged[1].second};
    return std::nullopt;
}

// The kernels' temperature argument: nothing when T is absent or 1.
std::optional<float> temperature_arg(std::optional<double> temperature) {
    if (!temperature.has_value() || *temperature == 1.0) return std::nullopt;
    const double t = *temperature;
    if (!(t > 0.0) || std::isinf(t))
        throw std::runtime_error("temperature must be finite and > 0, got " + std::to_string(t));
    return static_cast<float>(t);
}

// ---------------------------------------------------------------------------
// Split-row workspaces, one per (device, stream): launches that share one are
// ordered by their stream.  Allocated zero-filled (a fill kernel on that
// stream) and left zero by the forward.  The 16 most recently used are kept;
// a dropped one returns to the caching allocator on its own stream.  (Calls
// under graph capture never get here: see CaptureDeclined.)
// ---------------------------------------------------------------------------
struct Workspace {
    int device;
    hipStream_t stream;
    at::Tensor buf;
};
// Never destroyed: freeing device tensors from static destructors at exit
// would run after the caching allocator is gone.
std::mutex g_ws_mutex;
std::list<Workspace>& g_ws = *new std::list<Workspace>();  // most recently used first
constexpr size_t kWorkspacesKept = 16;

at::Tensor workspace(int device, hipStream_t stream, size_t nbytes) {
    if (nbytes == 0) return at::Tensor();
    const auto opts = at::TensorOptions().dtype(at::kByte).device(at::kCUDA, device);
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    for (auto it = g_ws.begin(); it != g_ws.end(); ++it) {
        if (it->device != device || it->stream != stream) continue;
        if (static_cast<size_t>(it->buf.numel()) < nbytes)
            it->buf = at::zeros({static_cast<int64_t>(nbytes)}, opts);
        g_ws.splice(g_ws.begin(), g_ws, it);
        return g_ws.front().buf;
    }
    g_ws.push_front(Workspace{device, stream, at::zeros({static_cast<int64_t>(nbytes)}, opts)});
    while (g_ws.size() > kWorkspacesKept) g_ws.pop_back();
    return g_ws.front().buf;
}

// ---------------------------------------------------------------------------
// Launchers into caller-allocated tensors (kernel_opt._C's fwd_launch /
// bwd_launch without a pinned launch shape).
// ---------------------------------------------------------------------------
struct Rows {
    std::array<int64_t, 3> layout;
    int64_t n, v;
};

Rows forward_checks(const at::Tensor& logits, const at::Tensor& targets, const at::Tensor& logprob,
                    const at::Tensor& entropy, const at::Tensor& lse, bool per_output) {
    require(logits.is_cuda(), "logits must be CUDA");
    require(targets.is_cuda(), "targets must be CUDA");
    const auto rows = row_layout(logits);
    require(rows.has_value(), "logits must be contiguous");
    require(targets.scalar_type() == at::kLong, "targets must be int64");
    if (per_output) {
        require(logprob.scalar_type() == at::kFloat, "logprob must be float32");
        require(entropy.scalar_type() == at::kFloat, "entropy must be float32");
        require(lse.scalar_type() == at::kFloat, "lse must be float32");
    } else {
        require(logprob.scalar_type() == at::kFloat && entropy.scalar_type() == at::kFloat &&
                    lse.scalar_type() == at::kFloat,
                "outputs must be float32");
    }
    require(dtype_code(logits.scalar_type()) >= 0, "logits dtype must be bf16, fp16, or fp32");
    const int64_t V = logits.size(-1);
    require(V > 0, "logits last dim (vocab) must be >= 1");
    const int64_t N = logits.numel() / V;
    require(targets.numel() == N, "targets numel must match leading dims of logits");
    require(logprob.numel() == N && entropy.numel() == N && lse.numel() == N,
            "output tensor numels must equal leading-dim count");
    require(targets.is_contiguous(), "targets must be contiguous");
    require(logprob.is_contiguous() && entropy.is_contiguous() && lse.is_contiguous(),
            "outputs must be contiguous");
    const auto d = logits.get_device();
    require(targets.get_device() == d && logprob.get_device() == d && entropy.get_device() == d &&
                lse.get_device() == d,
            "all tensors must be on the device of logits");
    return Rows{*rows, N, V};
}

void forward_into(const at::Tensor& logits, const at::Tensor& targets, at::Tensor& logprob,
                  at::Tensor& entropy, at::Tensor& lse, std::optional<double> temperature) {
    const Rows r = forward_checks(logits, targets, logprob, entropy, lse, false);
    const auto temp = temperature_arg(temperature);
    const int dev = logits.get_device();
    decline_under_capture(dev);
    if (r.n == 0) return;
    const int code = dtype_code(logits.scalar_type());
    const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev));
    hipStream_t stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
    at::Tensor ws = workspace(dev, stream, klp_fwd_workspace_bytes(code, r.n, r.v));
    const auto& L = r.layout;
    int rc;
    if (temp.has_value())
        rc = klp_fwd_temp(logits.data_ptr(), code, r.n, r.v, L[0], L[1], L[2],
                          targets.data_ptr<int64_t>(), *temp, out_ptr(logprob), out_ptr(entropy),
                          out_ptr(lse), ws.defined() ? ws.data_ptr() : nullptr,
                          ws.defined() ? static_cast<size_t>(ws.numel()) : 0, stream);
    else
        rc = klp_fwd(logits.data_ptr(), code, r.n, r.v, L[0], L[1], L[2],
                     targets.data_ptr<int64_t>(), out_ptr(logprob), out_ptr(entropy), out_ptr(lse),
                     ws.defined() ? ws.data_ptr() : nullptr,
                     ws.defined() ? static_cast<size_t>(ws.numel()) : 0, stream);
    check_status(rc);
}

void naive_into(const at::Tensor& logits, const at::Tensor& targets, at::Tensor& logprob,
                at::Tensor& entropy, at::Tensor& lse) {
    const Rows r = forward_checks(logits, targets, logprob, entropy, lse, true);
    const int dev = logits.get_device();
    decline_under_capture(dev);
    if (r.n == 0) return;
    const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev));
    hipStream_t stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
    const auto& L = r.layout;
    check_status(klp_fwd_naive(logits.data_ptr(), dtype_code(logits.scalar_type()), r.n, r.v, L[0],
                               L[1], L[2], targets.data_ptr<int64_t>(), out_ptr(logprob),
                               out_ptr(entropy), out_ptr(lse), stream));
}

void backward_into(const at::Tensor& logits, const at::Tensor& targets, const at::Tensor& lse,
                   const at::Tensor& entropy, const at::Tensor& g_logp, const at::Tensor& g_ent,
                   const at::Tensor& g_lse, at::Tensor& d_logits,
                   std::optional<double> temperature) {
    require(logits.is_cuda(), "logits must be contiguous CUDA");
    const auto rows = row_layout(logits);
    require(rows.has_value(), "logits must be contiguous CUDA");
    require(targets.scalar_type() == at::kLong, "targets must be int64");
    require(lse.scalar_type() == at::kFloat && entropy.scalar_type() == at::kFloat,
            "saved lse / entropy must be fp32");
    std::vector<const at::Tensor*> grads;
    for (const at::Tensor* g : {&g_logp, &g_ent, &g_lse})
        if (g->defined()) grads.push_back(g);
    for (const at::Tensor* g : grads)
        require(g->scalar_type() == at::kFloat, "upstream gradients must be fp32");
    for (const at::Tensor* g : grads)
        require(g->is_contiguous(), "upstream gradients must be contiguous");
    require(d_logits.scalar_type() == logits.scalar_type() && d_logits.is_contiguous() &&
                d_logits.sizes() == logits.sizes(),
            "d_logits must match logits dtype/shape and be contiguous");
    require(dtype_code(logits.scalar_type()) >= 0, "logits dtype must be bf16, fp16, or fp32");
    const int64_t V = logits.size(-1);
    require(V > 0, "logits last dim (vocab) must be >= 1");
    const int64_t N = logits.numel() / V;
    bool counts = targets.numel() == N && lse.numel() == N && entropy.numel() == N;
    for (const at::Tensor* g : grads) counts = counts && g->numel() == N;
    require(counts, "leading-dim count mismatch");
    require(targets.is_contiguous() && lse.is_contiguous() && entropy.is_contiguous(),
            "targets / saved lse / entropy must be contiguous");
    const auto d = logits.get_device();
    bool same = targets.get_device() == d && lse.get_device() == d && entropy.get_device() == d &&
                d_logits.get_device() == d;
    for (const at::Tensor* g : grads) same = same && g->get_device() == d;
    require(same, "all tensors must be on the device of logits");
    const auto temp = temperature_arg(temperature);
    decline_under_capture(d);
    if (N == 0) return;
    const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(d));
    hipStream_t stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(d)).stream();
    const auto& L = *rows;
    const int code = dtype_code(logits.scalar_type());
    int rc;
    if (temp.has_value())
        rc = klp_bwd_temp(logits.data_ptr(), code, N, V, L[0], L[1], L[2],
                          targets.data_ptr<int64_t>(), *temp, fptr(lse), fptr(entropy),
                          fptr(g_logp), fptr(g_ent), fptr(g_lse), d_logits.data_ptr(), stream);
    else
        rc = klp_bwd(logits.data_ptr(), code, N, V, L[0], L[1], L[2], targets.data_ptr<int64_t>(),
                     fptr(lse), fptr(entropy), fptr(g_logp), fptr(g_ent), fptr(g_lse),
                     d_logits.data_ptr(), stream);
    check_status(rc);
}

// ---------------------------------------------------------------------------
// ops.py's entry points.
// ---------------------------------------------------------------------------
std::string shape_str(at::IntArrayRef s) {
    std::string r = "torch.Size([";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "])";
}

// reference ops.py:16-21
void check_inputs(const at::Tensor& logits, const at::Tensor& targets) {
    if (!(logits.is_cuda() && targets.is_cuda())) throw AssertFailure("");
    if (!(row_layout(logits).has_value() && targets.is_contiguous())) throw AssertFailure("");
    if (targets.scalar_type() != at::kLong) throw AssertFailure("");
    if (logits.dim() == 0 || logits.sizes().slice(0, logits.dim() - 1) != targets.sizes())
        throw AssertFailure("logits[...,V]=" + shape_str(logits.sizes()) + " vs targets[...]=" +
                            shape_str(targets.sizes()));
}

// reference ops.py:24-30
std::array<at::Tensor, 3> alloc_outputs(const at::Tensor& targets) {
    const auto opts = at::TensorOptions().dtype(at::kFloat).device(targets.device());
    return {at::empty(targets.sizes(), opts), at::empty(targets.sizes(), opts),
            at::empty(targets.sizes(), opts)};
}

std::optional<double> saved_temperature(AutogradContext* ctx) {
    const auto& v = ctx->saved_data["temperature"];
    if (v.isNone()) return std::nullopt;
    return v.toDouble();
}

class FusedLogprobEntropy : public torch::autograd::Function<FusedLogprobEntropy> {
   public:
    static variable_list forward(AutogradContext* ctx, const at::Tensor& logits,
                                 const at::Tensor& targets, std::optional<double> temperature) {
        auto out = alloc_outputs(targets);
        forward_into(logits, targets, out[0], out[1], out[2], temperature);
        ctx->save_for_backward({logits, targets, out[2], out[1]});
        ctx->saved_data["temperature"] =
            temperature.has_value() ? c10::IValue(*temperature) : c10::IValue();
        ctx->set_materialize_grads(false);
        return {out[0], out[1], out[2]};
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        const auto saved = ctx->get_saved_variables();
        if (!ctx->needs_input_grad(0)) return {at::Tensor(), at::Tensor(), at::Tensor()};
        const at::Tensor &logits = saved[0], &targets = saved[1], &lse = saved[2],
                         &entropy = saved[3];
        auto prep = [](const at::Tensor& g) {
            return g.defined() ? g.to(at::kFloat).contiguous() : at::Tensor();
        };
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(c10::hip::getCurrentHIPStream(logits.device().index()).stream(),
                                 &status) != hipSuccess ||
            status != hipStreamCaptureStatusNone)
            throw std::runtime_error(
                "kernel_opt: this backward belongs to a forward run outside graph capture and "
                "cannot itself be captured; capture the forward with it");
        at::Tensor d_logits = at::empty(logits.sizes(), logits.options());
        backward_into(logits, targets, lse, entropy, prep(grads[0]), prep(grads[1]),
                      prep(grads[2]), d_logits, saved_temperature(ctx));
        return {d_logits, at::Tensor(), at::Tensor()};
    }
};

// reference ops.py:92-111 (eager path)
std::vector<at::Tensor> fused_logprob_entropy(const at::Tensor& logits, const at::Tensor& targets,
                                              std::optional<double> temperature) {
    check_inputs(logits, targets);
    decline_under_capture(logits.get_device());
    return FusedLogprobEntropy::apply(logits, targets, temperature);
}

// reference ops.py:41-46
std::vector<at::Tensor> fused_logprob_entropy_forward(const at::Tensor& logits,
                                                      const at::Tensor& targets,
                                                      std::optional<double> temperature) {
    check_inputs(logits, targets);
    decline_under_capture(logits.get_device());
    auto out = alloc_outputs(targets);
    forward_into(logits, targets, out[0], out[1], out[2], temperature);
    return {out[0], out[1], out[2]};
}

// reference ops.py:33-38
std::vector<at::Tensor> fused_logprob_entropy_naive(const at::Tensor& logits,
                                                    const at::Tensor& targets) {
    check_inputs(logits, targets);
    decline_under_capture(logits.get_device());
    auto out = alloc_outputs(targets);
    naive_into(logits, targets, out[0], out[1], out[2]);
    return {out[0], out[1], out[2]};
}

// ---------------------------------------------------------------------------
// GRPO loss over per-token log-probabilities: kernel_opt.grpo's autograd op
// (the loss the reference writes in eager PyTorch at
// examples/compare_one_step.py:232-236; klp_grpo_fwd / klp_grpo_bwd).  The
// argument handling restates grpo._f32 and grpo.fused_grpo_loss with the same
// messages; loss-type strings are resolved in Python.
// ---------------------------------------------------------------------------
std::string tuple_str(at::IntArrayRef s) {
    std::string r = "(";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + (s.size() == 1 ? ",)" : ")");
}

// A constant operand: on logp's device, float32, of the given shape,
// contiguous; undefined when absent.
at::Tensor grpo_operand(const std::optional<at::Tensor>& t, const char* name,
                        at::IntArrayRef shape, const at::Device& dev) {
    if (!t.has_value() || !t->defined()) return at::Tensor();
    if (t->device() != dev) throw std::runtime_error(std::string(name) + " must be on " + dev.str());
    at::Tensor f = t->detach().to(at::kFloat);
    if (f.sizes() != shape)
        throw std::runtime_error(std::string(name) + " has shape " + tuple_str(f.sizes()) +
                                 ", expected " + tuple_str(shape));
    return f.contiguous();
}

struct GrpoArgs {
    double eps_low, eps_high, beta, norm;
    int64_t kind, level, per_token;
};

class FusedGrpoLoss : public torch::autograd::Function<FusedGrpoLoss> {
   public:
    static variable_list forward(AutogradContext* ctx, const at::Tensor& logp, const at::Tensor& old,
                                 const std::optional<at::Tensor>& ref, const at::Tensor& adv,
                                 const std::optional<at::Tensor>& mask, double eps_low,
                                 double eps_high, double beta, double norm, int64_t kind,
                                 int64_t level, int64_t per_token) {
        const int64_t B = logp.size(0), S = logp.size(1);
        const at::Tensor lp = logp.contiguous();
        const at::Tensor r = ref.value_or(at::Tensor()), m = mask.value_or(at::Tensor());
        const auto f32 = at::TensorOptions().dtype(at::kFloat).device(logp.device());
        at::Tensor ws = at::empty({static_cast<int64_t>(klp_grpo_workspace_bytes(B))},
                                  f32.dtype(at::kByte));
        at::Tensor loss = at::empty({}, f32);
        at::Tensor stats = at::empty({4}, f32);
        const int dev = logp.get_device();
        const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev));
        hipStream_t stream =
            c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
        check_status(klp_grpo_fwd(fptr(lp), fptr(old), fptr(r), fptr(adv), fptr(m), B, S,
                                  static_cast<float>(eps_low), static_cast<float>(eps_high),
                                  static_cast<float>(beta), static_cast<float>(norm),
                                  static_cast<int>(kind), static_cast<int>(level),
                                  static_cast<int>(per_token), out_ptr(loss), out_ptr(stats),
                                  ws.data_ptr(), static_cast<size_t>(ws.numel()), stream));
        ctx->save_for_backward({lp, old, r, adv, m, ws});
        ctx->saved_data["args"] = c10::List<double>({eps_low, eps_high, beta, norm,
                                                     static_cast<double>(kind),
                                                     static_cast<double>(level),
                                                     static_cast<double>(per_token)});
        ctx->mark_non_differentiable({stats});
        ctx->set_materialize_grads(false);
        return {loss, stats};
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        variable_list none(12);
        if (!grads[0].defined() || !ctx->needs_input_grad(0)) return none;
        const auto saved = ctx->get_saved_variables();
        const at::Tensor &lp = saved[0], &old = saved[1], &ref = saved[2], &adv = saved[3],
                         &mask = saved[4], &ws = saved[5];
        const auto a = ctx->saved_data["args"].toDoubleList();
        const int dev = lp.get_device();
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(
                c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream(),
                &status) != hipSuccess ||
            status != hipStreamCaptureStatusNone)
            throw std::runtime_error(
                "kernel_opt: this backward belongs to a forward run outside graph capture and "
                "cannot itself be captured; capture the forward with it");
        const at::Tensor g = grads[0].detach().to(at::kFloat).reshape({1}).contiguous();
        at::Tensor d = at::empty_like(lp);
        const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev));
        hipStream_t stream =
            c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
        check_status(klp_grpo_bwd(fptr(lp), fptr(old), fptr(ref), fptr(adv), fptr(mask),
                                  lp.size(0), lp.size(1), static_cast<float>(a[0]),
                                  static_cast<float>(a[1]), static_cast<float>(a[2]),
                                  static_cast<float>(a[3]), static_cast<int>(a[4]),
                                  static_cast<int>(a[5]), static_cast<int>(a[6]), fptr(g),
                                  out_ptr(d), ws.data_ptr(), static_cast<size_t>(ws.numel()),
                                  stream));
        none[0] = d;
        return none;
    }
};

// grpo.fused_grpo_loss after its loss-type resolution (grpo._config).
std::vector<at::Tensor> fused_grpo_loss(const at::Tensor& logp, const std::optional<at::Tensor>& old,
                                        const at::Tensor& advantages,
                                        const std::optional<at::Tensor>& mask,
                                        const std::optional<at::Tensor>& ref, double eps_low,
                                        double eps_high, double beta, double norm, int64_t kind,
                                        int64_t level) {
    if (logp.dim() != 2)
        throw std::runtime_error("logp must be [B, S], got shape " + tuple_str(logp.sizes()));
    if (!logp.is_cuda()) throw std::runtime_error("logp must be a GPU tensor");
    if (logp.scalar_type() != at::kFloat) throw std::runtime_error("logp must be float32");
    decline_under_capture(logp.get_device());
    const int64_t B = logp.size(0), S = logp.size(1);
    const at::Device dev = logp.device();
    const at::Tensor o = grpo_operand(old, "old_logp", {B, S}, dev);
    const bool per_token = advantages.dim() != 1;
    const at::Tensor adv = per_token ? grpo_operand(advantages, "advantages", {B, S}, dev)
                                     : grpo_operand(advantages, "advantages", {B}, dev);
    const at::Tensor m = grpo_operand(mask, "mask", {B, S}, dev);
    const at::Tensor r = beta != 0.0 ? grpo_operand(ref, "ref_logp", {B, S}, dev) : at::Tensor();
    if (B == 0 || S == 0)  // no tokens: every normaliser sees an empty (zero) masked sum
        return {logp.sum() * 0.0, at::zeros({4}, logp.options())};
    auto out = FusedGrpoLoss::apply(logp, o, r.defined() ? std::optional<at::Tensor>(r) : std::nullopt,
                                    adv, m.defined() ? std::optional<at::Tensor>(m) : std::nullopt,
                                    eps_low, eps_high, beta, norm, kind, level,
                                    static_cast<int64_t>(per_token));
    return {out[0], out[1]};
}

// ---------------------------------------------------------------------------
// Fused GRPO step: kernel_opt.grpo_step's autograd op over klp_grpo_step
// (logprob, entropy, the token's GRPO loss and d_logits in one read of the
// logits).  Restates grpo_step.grpo_token_weights, grpo_step_launch and
// _FusedGrpoStep; the Python wrapper keeps the argument checks, the choice
// between this and the unfused composition, and the stats.
// ---------------------------------------------------------------------------
// klp_grpo_step's row counters, one per (device, stream): zeroed when
// allocated (a fill kernel on that stream) and left zero by every launch, so
// launches on one stream share one; the 16 most recently used are kept.
struct Sched {
    int device;
    hipStream_t stream;
    at::Tensor buf;
};
std::mutex g_sched_mutex;
std::list<Sched>& g_sched = *new std::list<Sched>();  // never destroyed, as g_ws

at::Tensor sched_counter(int device, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_sched_mutex);
    for (auto it = g_sched.begin(); it != g_sched.end(); ++it) {
        if (it->device != device || it->stream != stream) continue;
        g_sched.splice(g_sched.begin(), g_sched, it);
        return g_sched.front().buf;
    }
    const auto opts = at::TensorOptions().dtype(at::kLong).device(at::kCUDA, device);
    g_sched.push_front(Sched{device, stream, at::zeros({KLP_GRPO_STEP_SCHED_BYTES / 8}, opts)});
    while (g_sched.size() > kWorkspacesKept) g_sched.pop_back();
    return g_sched.front().buf;
}

// grpo_step.grpo_token_weights: kind 0 "grpo" (B * max(row sum, 1)), 1 "bnpo"
// (max(mask sum, 1)), 2 a fixed normaliser whose float32 reciprocal the
// caller passes as `scale` ("dr_grpo", "dapo").  The same values bit for bit
// in fewer launches: a bool or integer mask is summed in float32 and
// multiplied with float32 promotion instead of being converted first (its
// 0 / 1 sums are exact either way), and the Python statement's `* 1.0` after
// the reciprocal changes no value.
at::Tensor token_weights(const at::Tensor& m, int64_t kind, double scale) {
    if (kind == 0) {
        const at::Tensor den =
            m.sum({1}, true, at::kFloat).clamp_min(1.0) * static_cast<double>(m.size(0));
        return m * den.reciprocal();
    }
    if (kind == 1) return m * m.sum(at::kFloat).clamp_min(1.0).reciprocal();
    return m * scale;
}

// True when klp_grpo_step takes these rows (grpo_step._fused_supported).
bool grpo_step_supported(const at::Tensor& logits, const std::optional<std::array<int64_t, 3>>& rows) {
    const int code = dtype_code(logits.scalar_type());
    if (!rows.has_value() || code < 0) return false;
    const int64_t V = logits.size(-1), esz = logits.element_size();
    if (V > klp_grpo_step_max_vocab(code)) return false;
    const auto& L = *rows;
    return (V * esz) % 16 == 0 && reinterpret_cast<uintptr_t>(logits.data_ptr()) % 16 == 0 &&
           (L[2] * esz) % 16 == 0 && (L[1] * esz) % 16 == 0;
}

class FusedGrpoStep : public torch::autograd::Function<FusedGrpoStep> {
   public:
    static variable_list forward(AutogradContext* ctx, const at::Tensor& logits,
                                 const at::Tensor& targets, const at::Tensor& old,
                                 const std::optional<at::Tensor>& ref, const at::Tensor& adv,
                                 const at::Tensor& weight, double temperature, double eps_low,
                                 double eps_high, double beta, int64_t per_token,
                                 double grad_scale) {
        const int64_t B = logits.size(0), S = logits.size(1), V = logits.size(2);
        const auto rows = row_layout(logits);
        require(rows.has_value(), "logits must be contiguous");
        const auto f32 = at::TensorOptions().dtype(at::kFloat).device(logits.device());
        at::Tensor logp = at::empty({B, S}, f32), ent = at::empty({B, S}, f32),
                   lse = at::empty({B, S}, f32), loss_tok = at::empty({B, S}, f32);
        at::Tensor d_logits = at::empty({B, S, V}, logits.options());
        const int dev = logits.get_device();
        const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev));
        hipStream_t stream =
            c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
        const at::Tensor sched = sched_counter(dev, stream);
        const at::Tensor r = ref.value_or(at::Tensor());
        const auto& L = *rows;
        check_status(klp_grpo_step(
            logits.data_ptr(), dtype_code(logits.scalar_type()), B * S, V, L[0], L[1], L[2],
            targets.data_ptr<int64_t>(), static_cast<float>(temperature), fptr(old), fptr(r),
            fptr(adv), fptr(weight), S, static_cast<float>(eps_low), static_cast<float>(eps_high),
            static_cast<float>(beta), static_cast<int>(per_token), static_cast<float>(grad_scale),
            out_ptr(logp), out_ptr(ent), out_ptr(lse), out_ptr(loss_tok), d_logits.data_ptr(),
            sched.data_ptr(), stream));
        ctx->saved_data["d_logits"] = d_logits;
        ctx->saved_data["grad_scale"] = grad_scale;
        ctx->mark_non_differentiable({logp, ent});
        return {loss_tok.sum(), logp, ent};
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        variable_list none(12);
        c10::IValue& held = ctx->saved_data["d_logits"];
        if (!held.isTensor())
            throw std::runtime_error(
                "fused_grpo_step: the backward can run only once per forward (retain_graph "
                "replays are not supported)");
        at::Tensor d = held.toTensor();
        held = c10::IValue();
        if (!grads[0].defined() || !ctx->needs_input_grad(0)) return none;
        const int dev = d.get_device();
        hipStream_t stream =
            c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &status) != hipSuccess ||
            status != hipStreamCaptureStatusNone)
            throw std::runtime_error(
                "kernel_opt: this backward belongs to a forward run outside graph capture and "
                "cannot itself be captured; capture the forward with it");
        // d *= g / grad_scale on the device (grpo_step.scale_by_upstream):
        // nothing is written when g equals the declared grad_scale.
        const float applied = static_cast<float>(ctx->saved_data["grad_scale"].toDouble());
        const at::Tensor g = grads[0].detach().to(d.device(), at::kFloat).reshape({1}).contiguous();
        const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev));
        check_status(klp_rescale_inplace(d.data_ptr(), dtype_code(d.scalar_type()), d.numel(),
                                         fptr(g), applied, stream));
        none[0] = d;
        return none;
    }
};

// The fused path of grpo_step.fused_grpo_step after its argument checks:
// (loss, logp, entropy), or nothing when klp_grpo_step does not take these
// logits (the caller then runs the unfused composition).
std::optional<std::vector<at::Tensor>> fused_grpo_step(
    const at::Tensor& logits, const at::Tensor& targets, const at::Tensor& old_logp,
    const at::Tensor& advantages, const std::optional<at::Tensor>& mask,
    const std::optional<at::Tensor>& ref_logp, double temperature, double eps_low,
    double eps_high, double beta, int64_t weight_kind, double weight_scale, double grad_scale) {
    require(logits.is_cuda() && logits.dim() == 3, "logits must be a [B, S, V] GPU tensor");
    decline_under_capture(logits.get_device());
    if (!grpo_step_supported(logits, row_layout(logits))) return std::nullopt;
    const int64_t B = logits.size(0), S = logits.size(1);
    const at::Device dev = logits.device();
    const at::Tensor old = grpo_operand(old_logp, "old_logp", {B, S}, dev);
    const bool per_token = advantages.dim() != 1;
    const at::Tensor adv = per_token ? grpo_operand(advantages, "advantages", {B, S}, dev)
                                     : grpo_operand(advantages, "advantages", {B}, dev);
    if (targets.device() != dev)
        throw std::runtime_error("targets must be on " + dev.str() + ", got " +
                                 targets.device().str());
    require(targets.scalar_type() == at::kLong, "targets must be int64");
    require(targets.is_contiguous(), "targets must be contiguous");
    if (targets.sizes() != at::IntArrayRef({B, S}))
        throw std::runtime_error("targets has shape " + tuple_str(targets.sizes()) +
                                 ", expected " + tuple_str({B, S}));
    // The mask is checked as grpo_operand checks it.  A floating mask is
    // taken in float32, as the Python statement takes every mask; a bool or
    // integer mask stays as it is (token_weights promotes it to float32, and
    // its 0 / 1 sums are exact either way, so the weights are the same bits).
    at::Tensor m;
    const bool has_mask = mask.has_value() && mask->defined();
    if (has_mask) {
        if (mask->device() != dev) throw std::runtime_error("mask must be on " + dev.str());
        if (mask->sizes() != at::IntArrayRef({B, S}))
            throw std::runtime_error("mask has shape " + tuple_str(mask->sizes()) +
                                     ", expected " + tuple_str({B, S}));
        m = mask->detach();
        if (at::isFloatingType(m.scalar_type()) && m.scalar_type() != at::kFloat)
            m = m.to(at::kFloat);
    }
    const at::Tensor ref = (beta != 0.0 && ref_logp.has_value() && ref_logp->defined())
                               ? grpo_operand(ref_logp, "ref_logp", {B, S}, dev)
                               : at::Tensor();
    // No mask, or a bool / uint8 / int32 / int64 one: klp_grpo_token_weights
    // computes the weights in one launch, the same bits as token_weights
    // (its integer sums are exact, as the eager float32 sums of a 0 / 1 mask
    // are).  A floating mask takes token_weights, and so does a fixed
    // normaliser whose float32 reciprocal is not finite and > 0 (a zero or
    // negative normaliser: the entry point rejects such a scale, the eager
    // statement gives inf / negative weights).
    int mask_code = -1;
    if (has_mask) {
        const auto st = m.scalar_type();
        mask_code = (st == at::kBool || st == at::kByte) ? KLP_MASK_U8
                    : st == at::kInt                     ? KLP_MASK_I32
                    : st == at::kLong                    ? KLP_MASK_I64
                                                         : -1;
    }
    const float fixed_scale = static_cast<float>(weight_scale);
    const bool scale_ok = weight_kind != KLP_GRPO_LOSS_FIXED ||
                          (fixed_scale > 0.0f && fixed_scale < INFINITY);
    at::Tensor weight;
    if ((!has_mask || mask_code >= 0) && scale_ok) {
        const at::Tensor mc = has_mask ? m.contiguous() : at::Tensor();
        weight = at::empty({B, S}, at::TensorOptions().dtype(at::kFloat).device(dev));
        // "bnpo" keeps per-workgroup partial sums between its two launches;
        // the caching allocator hands back the block in stream order.
        const at::Tensor ws =
            weight_kind == KLP_GRPO_LOSS_BNPO
                ? at::empty({KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES},
                            at::TensorOptions().dtype(at::kByte).device(dev))
                : at::Tensor();
        const c10::hip::HIPGuard guard(static_cast<c10::DeviceIndex>(dev.index()));
        hipStream_t stream =
            c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev.index())).stream();
        check_status(klp_grpo_token_weights(has_mask ? mc.data_ptr() : nullptr,
                                            has_mask ? mask_code : KLP_MASK_U8, B, S,
                                            static_cast<int>(weight_kind), fixed_scale,
                                            weight.data_ptr<float>(),
                                            ws.defined() ? ws.data_ptr() : nullptr, stream));
    } else {
        const at::Tensor mf =
            has_mask ? m : at::ones({B, S}, at::TensorOptions().dtype(at::kFloat).device(dev));
        weight = token_weights(mf, weight_kind, weight_scale).contiguous();
    }
    // klp_grpo_step reads the weights as float32 [B, S].
    require(weight.scalar_type() == at::kFloat,
            "mask must be bool, integer or floating point (token weights are float32)");
    auto out = FusedGrpoStep::apply(logits, targets, old,
                                    ref.defined() ? std::optional<at::Tensor>(ref) : std::nullopt,
                                    adv, weight, temperature, eps_low, eps_high, beta,
                                    static_cast<int64_t>(per_token), grad_scale);
    return std::vector<at::Tensor>{out[0], out[1], out[2]};
}

}  // namespace

PYBIND11_MODULE(klp_torch, m) {
    m.doc() = "kernel_opt's compiled binding over libkernel_opt_hip.so";
    pybind11::register_exception<AssertFailure>(m, "InputAssertionError", PyExc_AssertionError);
    pybind11::register_exception<CaptureDeclined>(m, "CaptureDeclined");
    // kernel_opt._C (reference csrc/bindings.cpp:17-27)
    m.def(
        "fused_logprob_entropy_v1",
        [](const at::Tensor& logits, const at::Tensor& targets, at::Tensor logprob,
           at::Tensor entropy, at::Tensor lse_out) {
            forward_into(logits, targets, logprob, entropy, lse_out, std::nullopt);
        },
        "production forward into caller-allocated outputs");
    m.def(
        "fused_logprob_entropy_naive",
        [](const at::Tensor& logits, const at::Tensor& targets, at::Tensor logprob,
           at::Tensor entropy, at::Tensor lse_out) {
            naive_into(logits, targets, logprob, entropy, lse_out);
        },
        "naive forward (one thread per row) into caller-allocated outputs");
    m.def(
        "fused_logprob_entropy_v1_backward",
        [](const at::Tensor& logits, const at::Tensor& targets, const at::Tensor& lse,
           const at::Tensor& entropy, std::optional<at::Tensor> g_logp,
           std::optional<at::Tensor> g_ent, std::optional<at::Tensor> g_lse, at::Tensor d_logits) {
            backward_into(logits, targets, lse, entropy, g_logp.value_or(at::Tensor()),
                          g_ent.value_or(at::Tensor()), g_lse.value_or(at::Tensor()), d_logits,
                          std::nullopt);
        },
        "backward into a caller-allocated d_logits (None gradients act as zeros)");
    // launchers with a temperature (kernel_opt._C.fwd_launch / bwd_launch)
    m.def(
        "fwd_launch",
        [](const at::Tensor& logits, const at::Tensor& targets, at::Tensor logprob,
           at::Tensor entropy, at::Tensor lse_out, std::optional<double> temperature) {
            forward_into(logits, targets, logprob, entropy, lse_out, temperature);
        },
        pybind11::arg("logits"), pybind11::arg("targets"), pybind11::arg("logprob"),
        pybind11::arg("entropy"), pybind11::arg("lse_out"),
        pybind11::arg("temperature") = pybind11::none());
    m.def(
        "bwd_launch",
        [](const at::Tensor& logits, const at::Tensor& targets, const at::Tensor& lse,
           const at::Tensor& entropy, std::optional<at::Tensor> g_logp,
           std::optional<at::Tensor> g_ent, std::optional<at::Tensor> g_lse, at::Tensor d_logits,
           std::optional<double> temperature) {
            backward_into(logits, targets, lse, entropy, g_logp.value_or(at::Tensor()),
                          g_ent.value_or(at::Tensor()), g_lse.value_or(at::Tensor()), d_logits,
                          temperature);
        },
        pybind11::arg("logits"), pybind11::arg("targets"), pybind11::arg("lse"),
        pybind11::arg("entropy"), pybind11::arg("g_logp"), pybind11::arg("g_ent"),
        pybind11::arg("g_lse"), pybind11::arg("d_logits"),
        pybind11::arg("temperature") = pybind11::none());
    // kernel_opt.ops (reference python/kernel_opt/ops.py)
    m.def("fused_logprob_entropy", &fused_logprob_entropy, pybind11::arg("logits"),
          pybind11::arg("targets"), pybind11::arg("temperature") = pybind11::none());
    m.def("fused_logprob_entropy_forward", &fused_logprob_entropy_forward,
          pybind11::arg("logits"), pybind11::arg("targets"),
          pybind11::arg("temperature") = pybind11::none());
    m.def("fused_logprob_entropy_naive_op", &fused_logprob_entropy_naive, pybind11::arg("logits"),
          pybind11::arg("targets"));
    // kernel_opt.grpo (the GRPO loss of per-token log-probabilities)
    m.def("fused_grpo_loss", &fused_grpo_loss, pybind11::arg("logp"), pybind11::arg("old_logp"),
          pybind11::arg("advantages"), pybind11::arg("mask"), pybind11::arg("ref_logp"),
          pybind11::arg("eps_low"), pybind11::arg("eps_high"), pybind11::arg("beta"),
          pybind11::arg("norm"), pybind11::arg("kind"), pybind11::arg("level"));
    // kernel_opt.grpo_step (the fused GRPO step)
    m.def("fused_grpo_step", &fused_grpo_step, pybind11::arg("logits"), pybind11::arg("targets"),
          pybind11::arg("old_logp"), pybind11::arg("advantages"), pybind11::arg("mask"),
          pybind11::arg("ref_logp"), pybind11::arg("temperature"), pybind11::arg("eps_low"),
          pybind11::arg("eps_high"), pybind11::arg("beta"), pybind11::arg("weight_kind"),
          pybind11::arg("weight_scale"), pybind11::arg("grad_scale") = 1.0);
    m.def(
        "workspaces_cached",
        []() {
            std::lock_guard<std::mutex> lock(g_ws_mutex);
            return g_ws.size();
        },
        "split-row workspaces held for (device, stream) pairs (at most 16)");
    m.def(
        "row_layout",
        [](const at::Tensor& t) -> pybind11::object {
            const auto r = row_layout(t);
            if (!r.has_value()) return pybind11::none();
            return pybind11::make_tuple((*r)[0], (*r)[1], (*r)[2]);
        },
        "row addressing of a tensor's rows, as kernel_opt._C.row_layout");
}
