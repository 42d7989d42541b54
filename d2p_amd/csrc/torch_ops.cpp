// torch_ops.cpp -- PyTorch dispatcher registration of the d2p operators on ROCm.
//
// Schemas are byte-identical to the reference's TORCH_LIBRARY_FRAGMENT(d2p, m):
//   /root/reference/src/sw/registry.cpp:30-44
//   /root/reference/src/sw_affine/registry.cpp:74-89
//   /root/reference/src/dtw/registry.cpp:127-132
// On PyTorch-ROCm a HIP tensor carries the CUDA dispatch key, so the HIP
// implementations register under CUDA / AutogradCUDA.  Every implementation
// validates on the host (same messages as the reference), allocates outputs and
// workspaces through the torch caching allocator, and calls the C ABI of
// libd2p_amd.so on the current HIP stream.  There is no CPU implementation: CPU
// tensors raise.

#include <torch/torch.h>
#include <torch/library.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cstdlib>
#include <cstring>
#include <limits>
#include <tuple>
#include <vector>

#include "../../include/d2p_amd.h"

namespace {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

#define D2P_CALL(expr)                                                          \
    do {                                                                        \
        int rc_ = (expr);                                                       \
        TORCH_CHECK(rc_ == 0, "d2p_amd kernel call failed: ", d2p_last_error()); \
    } while (0)

// same wording as /root/reference/src/common/torch_utils.h:31-66
#define CHECK_INPUT_DEV(x)                                                      \
    TORCH_CHECK((x).is_cuda(), #x " must be a CUDA tensor");                   \
    TORCH_CHECK((x).is_contiguous(), #x " must be contiguous");                \
    TORCH_CHECK((x).scalar_type() == torch::kFloat32, #x " must be float32, got ", \
                (x).scalar_type())

inline void* current_stream() {
    return (void*)c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
}

struct Dims {
    int B, L1, L2;
};

int checked_dim(int64_t v, const char* name) {
    TORCH_CHECK(v >= 0 && v <= std::numeric_limits<int>::max(), name,
                " must fit int32 CUDA kernel indexing, got ", v);
    return static_cast<int>(v);
}

// /root/reference/src/sw/torch_cuda.cpp:41-65 (message prefix per family)
Dims checked_dims(const Tensor& x, const char* family) {
    TORCH_CHECK(x.dim() == 3, "scores must be 3D (B, L1, L2)");
    Dims d{checked_dim(x.size(0), "scores batch dimension"),
           checked_dim(x.size(1), "scores L1 dimension"),
           checked_dim(x.size(2), "scores L2 dimension")};
    const int64_t cells = (int64_t(d.L1) + 1) * (int64_t(d.L2) + 1);
    TORCH_CHECK(cells <= std::numeric_limits<int>::max(), family,
                " CUDA DP table is too large for 32-bit kernel indexing: ",
                "(L1 + 1) * (L2 + 1) = ", cells, " exceeds ", std::numeric_limits<int>::max());
    return d;
}

// /root/reference/src/sw/torch_cuda.cpp:67-111
Tensor resolve_lengths(const c10::optional<Tensor>& lengths_opt, const Dims& d,
                       const torch::Device& device, const char* input = "scores") {
    if (!lengths_opt.has_value() || !lengths_opt->defined()) {
        // full lengths: the kernels take a null lengths pointer as (L1, L2) for every
        // element, so nothing is built, copied or validated
        return Tensor();
    }
    const Tensor& lengths = *lengths_opt;
    TORCH_CHECK(lengths.is_cuda(), "lengths must be a CUDA tensor");
    TORCH_CHECK(lengths.is_contiguous(), "lengths must be contiguous");
    TORCH_CHECK(lengths.dim() == 2 && lengths.size(0) == d.B && lengths.size(1) == 2,
                "lengths must be [B, 2] with B = ", d.B, ", got ", lengths.sizes());
    TORCH_CHECK(lengths.scalar_type() == torch::kInt32, "lengths must be int32");
    TORCH_CHECK(lengths.device() == device, "lengths must be on same device as ", input,
                ", got ", lengths.device(), " vs ", device);
    // The values are checked on the host, as the reference does
    // (/root/reference/src/sw_affine/torch_cuda.cpp:85-96): a copy that waits for the
    // stream.  A tensor checked by this thread's previous call against the same (L1, L2),
    // still alive, on the same memory and not modified since (same version counter,
    // which every in-place change and every view's change bumps), is not copied again,
    // so a training loop
    // that passes the same lengths every step does not synchronise each call.
    // (Inference tensors carry no version counter: always checked.)
    struct Checked {
        c10::weak_intrusive_ptr<c10::TensorImpl, c10::UndefinedTensorImpl> impl{
            c10::intrusive_ptr<c10::TensorImpl, c10::UndefinedTensorImpl>()};
        int64_t version = 0;
        const void* data = nullptr;
        int L1 = -1, L2 = -1;
    };
    static thread_local Checked last;
    const bool versioned = !lengths.is_inference();
    if (versioned && last.L1 == d.L1 && last.L2 == d.L2 && last.data == lengths.data_ptr() &&
        last.version == lengths._version()) {
        auto alive = last.impl.lock();
        if (alive.get() == lengths.unsafeGetTensorImpl()) return lengths;
    }
    auto host = lengths.to(torch::kCPU);
    auto acc = host.accessor<int32_t, 2>();
    for (int b = 0; b < d.B; ++b) {
        TORCH_CHECK(acc[b][0] >= 0 && acc[b][0] <= d.L1, "lengths[", b,
                    ",0] must be between 0 and ", d.L1, ", got ", acc[b][0]);
        TORCH_CHECK(acc[b][1] >= 0 && acc[b][1] <= d.L2, "lengths[", b,
                    ",1] must be between 0 and ", d.L2, ", got ", acc[b][1]);
    }
    if (versioned) {
        last.impl = c10::weak_intrusive_ptr<c10::TensorImpl, c10::UndefinedTensorImpl>(
            lengths.getIntrusivePtr());
        last.version = lengths._version();
        last.data = lengths.data_ptr();
        last.L1 = d.L1;
        last.L2 = d.L2;
    }
    return lengths;
}

// D2P_AMD_CHECK_STATUS=1 (opt-in; it synchronises the stream after every call):
// raise when a pipeline wait of some batch element gave up.  Without it such an
// element's outputs come back NaN (the kernel library overwrites them), and nothing
// waits for the device.
bool status_check_enabled() {
    const char* e = std::getenv("D2P_AMD_CHECK_STATUS");
    return e != nullptr && e[0] != '\0' && std::strcmp(e, "0") != 0;
}

void check_status(const Tensor& ws, int B) {
    if (B <= 0 || !status_check_enabled()) return;
    int st = 0;
    D2P_CALL(d2p_sw_status(ws.data_ptr(), B, &st, current_stream()));
    TORCH_CHECK(st == 0, "d2p_amd: a pipeline wait of the DP sweeps gave up (status ", st,
                "); the affected batch elements' outputs are NaN");
}

// The lengths argument of the C ABI: null for full lengths.
const int* lengths_ptr(const Tensor& lengths) {
    return lengths.defined() ? lengths.data_ptr<int>() : nullptr;
}

// Lengths as an autograd Function input: absent (full lengths) is passed as an empty
// optional, which the Function treats as a non-differentiable, non-tensor input
// (an undefined Tensor input has no device for the autograd node to record).
c10::optional<Tensor> lengths_arg(const Tensor& lengths) {
    return lengths.defined() ? c10::optional<Tensor>(lengths) : c10::nullopt;
}

Tensor workspace(size_t bytes, const Tensor& like) {
    return torch::empty({(int64_t)std::max<size_t>(bytes, 1)},
                        like.options().dtype(torch::kUInt8));
}

float scalar_value(const Tensor& t, const char* name) {
    TORCH_CHECK(t.numel() == 1, name, " must be a scalar tensor");
    return t.to(torch::kCPU, torch::kFloat32).item<float>();
}

Tensor grad_param_sum(const Tensor& grad_value, const Tensor& per_batch) {
    return (grad_value.to(torch::kFloat32) * per_batch).sum().reshape({1});
}

// g[b] * src, through the C ABI (autograd backward of value -> scores).  The factors
// are read in place by stride: the gradient of `value.sum()` arrives as one value
// expanded over the batch (stride 0), which needs no copy.  With lengths (the checked
// int32 [B, 2] tensor of the forward) src is a [B, L1, L2] table that is zero outside
// them: only the cells inside are read.
Tensor scale_by_batch(const Tensor& src, const Tensor& g, const Tensor& lengths = Tensor()) {
    Tensor gg = g.to(src.device(), torch::kFloat32);
    TORCH_CHECK(gg.numel() == src.size(0), "grad_value must have one entry per batch element");
    if (gg.dim() != 1) gg = gg.reshape({-1});
    if (gg.numel() > 0 && gg.stride(0) < 0) gg = gg.contiguous();
    Tensor out = torch::empty_like(src);
    if (lengths.defined() && src.dim() == 3) {
        D2P_CALL(d2p_scale_by_batch_lengths(src.data_ptr<float>(), gg.data_ptr<float>(),
                                            (long long)gg.stride(0), lengths.data_ptr<int>(),
                                            out.data_ptr<float>(), (int)src.size(0),
                                            (int)src.size(1), (int)src.size(2),
                                            current_stream()));
        return out;
    }
    D2P_CALL(d2p_scale_by_batch_strided(src.data_ptr<float>(), gg.data_ptr<float>(),
                                        (long long)gg.stride(0), out.data_ptr<float>(),
                                        (int)src.size(0),
                                        (long long)(src.numel() /
                                                    std::max<int64_t>(src.size(0), 1)),
                                        current_stream()));
    return out;
}

// ---------------------------------------------------------------------------
// linear-gap soft Smith-Waterman
// ---------------------------------------------------------------------------

struct SwOut {
    Tensor partition, marginals, grad_gap, grad_T;
};

SwOut sw_run(const Tensor& scores, const Tensor& lengths, const Dims& d, float gap, float T) {
    auto opt = scores.options();
    SwOut o{torch::empty({d.B}, opt), torch::empty({d.B, d.L1, d.L2}, opt),
            torch::empty({d.B}, opt), torch::empty({d.B}, opt)};
    const size_t ws_bytes = d2p_sw_workspace_bytes(d.B, d.L1, d.L2);
    Tensor ws = workspace(ws_bytes, scores);
    D2P_CALL(d2p_sw_forward_marginals(
        scores.data_ptr<float>(), lengths_ptr(lengths), d.B, d.L1, d.L2, gap, T,
        o.partition.data_ptr<float>(), o.marginals.data_ptr<float>(),
        o.grad_gap.data_ptr<float>(), o.grad_T.data_ptr<float>(), ws.data_ptr(), ws_bytes,
        current_stream()));
    check_status(ws, d.B);
    return o;
}

// Second-order entry points (HVP, Jacobians, marginal-path backward) through the C ABI.
Tensor second_workspace(const Dims& d, const Tensor& like) {
    return workspace(d2p_sw_second_workspace_bytes(d.B, d.L1, d.L2), like);
}

// global: soft Needleman-Wunsch instead of Smith-Waterman (same workspace)
Tensor sw_hvp_run(const Tensor& scores, const Tensor& tangent, const Tensor& lengths,
                  const Dims& d, float gap, float T, bool global = false) {
    Tensor out = torch::empty({d.B, d.L1, d.L2}, scores.options());
    Tensor ws = second_workspace(d, scores);
    D2P_CALL((global ? d2p_nw_hvp : d2p_sw_hvp)(
        scores.data_ptr<float>(), tangent.data_ptr<float>(), lengths_ptr(lengths), d.B, d.L1,
        d.L2, gap, T, out.data_ptr<float>(), ws.data_ptr(), ws.numel(), current_stream()));
    check_status(ws, d.B);
    return out;
}

Tensor sw_param_jacobian_run(const Tensor& scores, int param_type, const Tensor& lengths,
                             const Dims& d, float gap, float T, bool global = false) {
    Tensor out = torch::empty({d.B, d.L1, d.L2}, scores.options());
    Tensor ws = second_workspace(d, scores);
    D2P_CALL((global ? d2p_nw_param_jacobian : d2p_sw_param_jacobian)(
        scores.data_ptr<float>(), param_type, lengths_ptr(lengths), d.B, d.L1, d.L2, gap, T,
        out.data_ptr<float>(), ws.data_ptr(), ws.numel(), current_stream()));
    check_status(ws, d.B);
    return out;
}

// returns (grad_scores [B,L1,L2], per-element <ga, dP/dgap> [B], <ga, dP/dT> [B])
std::tuple<Tensor, Tensor, Tensor> sw_backward_full_run(const Tensor& scores, const Tensor& ga,
                                                        const Tensor& lengths, const Dims& d,
                                                        float gap, float T, bool global = false) {
    auto opt = scores.options();
    Tensor gs = torch::empty({d.B, d.L1, d.L2}, opt);
    Tensor gg = torch::empty({d.B}, opt), gt = torch::empty({d.B}, opt);
    Tensor ws = second_workspace(d, scores);
    D2P_CALL((global ? d2p_nw_backward_full : d2p_sw_backward_full)(scores.data_ptr<float>(), ga.data_ptr<float>(),
                                  lengths_ptr(lengths), d.B, d.L1, d.L2, gap, T,
                                  gs.data_ptr<float>(), gg.data_ptr<float>(), gt.data_ptr<float>(),
                                  ws.data_ptr(), ws.numel(), current_stream()));
    check_status(ws, d.B);
    return {gs, gg, gt};
}

// The marginal cotangent as the reference prepares it
// (/root/reference/src/sw/torch_cuda.cpp:325-338): same shape, float32, contiguous.
Tensor prepare_cotangent(Tensor g, const Tensor& like, const char* name) {
    TORCH_CHECK(g.sizes() == like.sizes(), name, " shape mismatch: expected ", like.sizes(),
                " but got ", g.sizes());
    TORCH_CHECK(g.is_cuda(), name, " must be on CUDA, got ", g.device());
    if (g.scalar_type() != torch::kFloat32) g = g.to(torch::kFloat32);
    if (g.device() != like.device()) g = g.to(like.device());
    return g.contiguous();
}

// Autograd semantics of SoftSWRegularCUDAFunction
// (/root/reference/src/sw/torch_cuda.cpp:178-411): outputs {value, marginals};
// d value / d scores = marginals, so the value path scales the saved marginals; the
// marginal path adds the HVP against the marginal cotangent and its dot products
// with dP/dgap and dP/dT; parameter gradients are summed over the batch, shape [1].
// Two Function classes share this logic: float parameters (no parameter inputs)
// and tensor parameters (gap / temperature receive gradients).
tensor_list sw_autograd_forward(AutogradContext* ctx, const Tensor& scores,
                                const Tensor& lengths, double gap, double temperature) {
    ctx->set_materialize_grads(false);
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    SwOut o = sw_run(scores, lengths, d, (float)gap, (float)temperature);
    ctx->save_for_backward({scores, lengths, o.marginals, o.grad_gap, o.grad_T});
    ctx->saved_data["gap"] = gap;
    ctx->saved_data["temperature"] = temperature;
    return {o.partition, o.marginals};
}

// returns {grad_scores, grad_gap, grad_T}
tensor_list sw_autograd_backward(AutogradContext* ctx, const tensor_list& grads,
                                 bool want_gap, bool want_T) {
    auto saved = ctx->get_saved_variables();
    Tensor scores = saved[0], lengths = saved[1], marg = saved[2], ggap = saved[3], gT = saved[4];
    c10::hip::HIPGuardMasqueradingAsCUDA guard(marg.device());
    Tensor grad_value = grads[0], grad_marg = grads[1];
    Tensor grad_scores, grad_gap, grad_T;
    if (grad_value.defined() && grad_value.numel() > 0) {
        grad_scores = scale_by_batch(marg, grad_value, lengths);
        if (want_gap) grad_gap = grad_param_sum(grad_value, ggap);
        if (want_T) grad_T = grad_param_sum(grad_value, gT);
    }
    if (grad_marg.defined() && grad_marg.numel() > 0) {
        Tensor gm = prepare_cotangent(grad_marg, scores, "grad_posteriors");
        const float gap = (float)ctx->saved_data["gap"].toDouble();
        const float T = (float)ctx->saved_data["temperature"].toDouble();
        Dims d = checked_dims(scores, "SW");
        auto r = sw_backward_full_run(scores, gm, lengths, d, gap, T);
        grad_scores = grad_scores.defined() ? grad_scores + std::get<0>(r) : std::get<0>(r);
        Tensor tg = std::get<1>(r).sum().reshape({1}), tt = std::get<2>(r).sum().reshape({1});
        if (want_gap) grad_gap = grad_gap.defined() ? grad_gap + tg : tg;
        if (want_T) grad_T = grad_T.defined() ? grad_T + tt : tt;
    }
    return {grad_scores, grad_gap, grad_T};
}

class SoftSWFloatFunction : public torch::autograd::Function<SoftSWFloatFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor scores,
                               c10::optional<Tensor> lengths, double gap, double temperature) {
        return sw_autograd_forward(ctx, scores, lengths.value_or(Tensor()), gap, temperature);
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto g = sw_autograd_backward(ctx, grads, false, false);
        return {g[0], Tensor(), Tensor(), Tensor()};
    }
};

class SoftSWTensorFunction : public torch::autograd::Function<SoftSWTensorFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor scores, Tensor gap_t, Tensor temp_t,
                               Tensor lengths, double gap, double temperature) {
        return sw_autograd_forward(ctx, scores, lengths, gap, temperature);
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto g = sw_autograd_backward(ctx, grads, ctx->needs_input_grad(1),
                                      ctx->needs_input_grad(2));
        return {g[0], g[1], g[2], Tensor(), Tensor(), Tensor()};
    }
};

std::vector<Tensor> soft_sw_t(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    const float g = scalar_value(gap, "gap");
    const float T = scalar_value(temperature, "temperature");
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return SoftSWTensorFunction::apply(scores, gap, temperature, l, g, T);
}

std::vector<Tensor> soft_sw_float(Tensor scores, double gap, double temperature,
                                  c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return SoftSWFloatFunction::apply(scores, lengths_arg(l), gap, temperature);
}

std::tuple<Tensor, Tensor, Tensor, Tensor> soft_sw_with_grads(Tensor scores, double gap,
                                                              double temperature,
                                                              c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    SwOut o = sw_run(scores, l, d, (float)gap, (float)temperature);
    return {o.partition, o.marginals, o.grad_gap, o.grad_T};
}

Tensor soft_sw_hvp(Tensor scores, Tensor tangent, double gap, double temperature,
                   c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    CHECK_INPUT_DEV(tangent);
    TORCH_CHECK(scores.dim() == 3, "scores must be 3D");
    TORCH_CHECK(scores.sizes() == tangent.sizes(), "scores and tangent must have same shape");
    TORCH_CHECK(tangent.device() == scores.device(), "tangent must be on same device as scores, got ",
                tangent.device(), " vs ", scores.device());
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return sw_hvp_run(scores, tangent, l, d, (float)gap, (float)temperature);
}

Tensor soft_sw_param_jacobian(Tensor scores, int64_t param_type, double gap, double temperature,
                              c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    TORCH_CHECK(param_type >= 0 && param_type <= 1, "param_type must be 0 or 1");
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return sw_param_jacobian_run(scores, (int)param_type, l, d, (float)gap, (float)temperature);
}

std::tuple<Tensor, Tensor, Tensor> soft_sw_backward_full(Tensor scores, Tensor grad_alignment,
                                                         double gap, double temperature,
                                                         c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    TORCH_CHECK(grad_alignment.sizes() == scores.sizes(),
                "grad_alignment must have same shape as scores");
    TORCH_CHECK(grad_alignment.is_cuda(), "grad_alignment must be a CUDA tensor");
    TORCH_CHECK(grad_alignment.device() == scores.device(),
                "grad_alignment must be on same device as scores, got ", grad_alignment.device(),
                " vs ", scores.device());
    Dims d = checked_dims(scores, "SW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    Tensor ga = grad_alignment.contiguous();
    if (ga.scalar_type() != torch::kFloat32) ga = ga.to(torch::kFloat32);
    auto r = sw_backward_full_run(scores, ga, l, d, (float)gap, (float)temperature);
    return {std::get<0>(r), std::get<1>(r).sum().reshape({1}), std::get<2>(r).sum().reshape({1})};
}

std::vector<Tensor> sw_forward(Tensor s, double g, double t, c10::optional<Tensor> l) {
    return soft_sw_float(s, g, t, l);
}
std::vector<Tensor> sw_forward_t(Tensor s, Tensor g, Tensor t, Tensor l) { return soft_sw_t(s, g, t, l); }
std::tuple<Tensor, Tensor> sw_value_grad_params(Tensor s, double g, double t,
                                                c10::optional<Tensor> l) {
    auto r = soft_sw_with_grads(s, g, t, l);
    return {std::get<2>(r), std::get<3>(r)};
}
std::tuple<Tensor, Tensor, Tensor> sw_marginals_backward(Tensor s, Tensor gm, double g, double t,
                                                         c10::optional<Tensor> l) {
    return soft_sw_backward_full(s, gm, g, t, l);
}
Tensor sw_marginals_hvp(Tensor s, Tensor v, double g, double t, c10::optional<Tensor> l) {
    return soft_sw_hvp(s, v, g, t, l);
}
Tensor sw_marginals_grad_gap(Tensor s, double g, double t, c10::optional<Tensor> l) {
    return soft_sw_param_jacobian(s, 0, g, t, l);
}
Tensor sw_marginals_grad_temp(Tensor s, double g, double t, c10::optional<Tensor> l) {
    return soft_sw_param_jacobian(s, 1, g, t, l);
}

// ---------------------------------------------------------------------------
// linear-gap soft Needleman-Wunsch (global alignment)
// ---------------------------------------------------------------------------

SwOut nw_run(const Tensor& scores, const Tensor& lengths, const Dims& d, float gap, float T) {
    auto opt = scores.options();
    SwOut o{torch::empty({d.B}, opt), torch::empty({d.B, d.L1, d.L2}, opt),
            torch::empty({d.B}, opt), torch::empty({d.B}, opt)};
    const size_t ws_bytes = d2p_nw_workspace_bytes(d.B, d.L1, d.L2);
    Tensor ws = workspace(ws_bytes, scores);
    D2P_CALL(d2p_nw_forward_marginals(
        scores.data_ptr<float>(), lengths_ptr(lengths), d.B, d.L1, d.L2, gap, T,
        o.partition.data_ptr<float>(), o.marginals.data_ptr<float>(),
        o.grad_gap.data_ptr<float>(), o.grad_T.data_ptr<float>(), ws.data_ptr(), ws_bytes,
        current_stream()));
    check_status(ws, d.B);
    return o;
}

// Autograd semantics of SoftNWCUDAFunction (/root/reference/src/nw/torch_cuda.cpp:115-330):
// outputs {value, marginals}; d value / d scores = marginals, so the value path scales
// the saved marginals; the marginal path adds the HVP against the marginal cotangent
// and its dot products with dP/dgap and dP/dT; parameter gradients are summed over the
// batch, shape [1].
tensor_list nw_autograd_forward(AutogradContext* ctx, const Tensor& scores,
                                const Tensor& lengths, double gap, double temperature) {
    ctx->set_materialize_grads(false);
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    SwOut o = nw_run(scores, lengths, d, (float)gap, (float)temperature);
    ctx->save_for_backward({scores, lengths, o.marginals, o.grad_gap, o.grad_T});
    ctx->saved_data["gap"] = gap;
    ctx->saved_data["temperature"] = temperature;
    return {o.partition, o.marginals};
}

tensor_list nw_autograd_backward(AutogradContext* ctx, const tensor_list& grads, bool want_gap,
                                 bool want_T) {
    auto saved = ctx->get_saved_variables();
    Tensor scores = saved[0], lengths = saved[1], marg = saved[2], ggap = saved[3], gT = saved[4];
    c10::hip::HIPGuardMasqueradingAsCUDA guard(marg.device());
    Tensor grad_value = grads[0], grad_marg = grads[1];
    Tensor grad_scores, grad_gap, grad_T;
    if (grad_value.defined() && grad_value.numel() > 0) {
        grad_scores = scale_by_batch(marg, grad_value, lengths);
        if (want_gap) grad_gap = grad_param_sum(grad_value, ggap);
        if (want_T) grad_T = grad_param_sum(grad_value, gT);
    }
    if (grad_marg.defined() && grad_marg.numel() > 0) {
        Tensor gm = prepare_cotangent(grad_marg, scores, "grad_posteriors");
        const float gap = (float)ctx->saved_data["gap"].toDouble();
        const float T = (float)ctx->saved_data["temperature"].toDouble();
        Dims d = checked_dims(scores, "NW");
        auto r = sw_backward_full_run(scores, gm, lengths, d, gap, T, true);
        grad_scores = grad_scores.defined() ? grad_scores + std::get<0>(r) : std::get<0>(r);
        Tensor tg = std::get<1>(r).sum().reshape({1}), tt = std::get<2>(r).sum().reshape({1});
        if (want_gap) grad_gap = grad_gap.defined() ? grad_gap + tg : tg;
        if (want_T) grad_T = grad_T.defined() ? grad_T + tt : tt;
    }
    return {grad_scores, grad_gap, grad_T};
}

class SoftNWFloatFunction : public torch::autograd::Function<SoftNWFloatFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor scores,
                               c10::optional<Tensor> lengths, double gap, double temperature) {
        return nw_autograd_forward(ctx, scores, lengths.value_or(Tensor()), gap, temperature);
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto g = nw_autograd_backward(ctx, grads, false, false);
        return {g[0], Tensor(), Tensor(), Tensor()};
    }
};

class SoftNWTensorFunction : public torch::autograd::Function<SoftNWTensorFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor scores, Tensor gap_t, Tensor temp_t,
                               Tensor lengths, double gap, double temperature) {
        return nw_autograd_forward(ctx, scores, lengths, gap, temperature);
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto g = nw_autograd_backward(ctx, grads, ctx->needs_input_grad(1),
                                      ctx->needs_input_grad(2));
        return {g[0], g[1], g[2], Tensor(), Tensor(), Tensor()};
    }
};

std::vector<Tensor> soft_nw_t(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    const float g = scalar_value(gap, "gap");
    const float T = scalar_value(temperature, "temperature");
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return SoftNWTensorFunction::apply(scores, gap, temperature, l, g, T);
}

std::vector<Tensor> soft_nw_float(Tensor scores, double gap, double temperature,
                                  c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return SoftNWFloatFunction::apply(scores, lengths_arg(l), gap, temperature);
}

std::tuple<Tensor, Tensor, Tensor, Tensor> soft_nw_with_grads(Tensor scores, double gap,
                                                              double temperature,
                                                              c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    SwOut o = nw_run(scores, l, d, (float)gap, (float)temperature);
    return {o.partition, o.marginals, o.grad_gap, o.grad_T};
}

std::vector<Tensor> nw_forward(Tensor s, double g, double t, c10::optional<Tensor> l) {
    return soft_nw_float(s, g, t, l);
}
std::vector<Tensor> nw_forward_t(Tensor s, Tensor g, Tensor t, Tensor l) { return soft_nw_t(s, g, t, l); }
std::tuple<Tensor, Tensor> nw_value_grad_params(Tensor s, double g, double t,
                                                c10::optional<Tensor> l) {
    auto r = soft_nw_with_grads(s, g, t, l);
    return {std::get<2>(r), std::get<3>(r)};
}

// second order: soft_nw_{hvp,param_jacobian,backward_full}_cuda
// (/root/reference/src/nw/torch_cuda.cpp:442-709) and their nw_marginals_* aliases
Tensor soft_nw_hvp(Tensor scores, Tensor tangent, double gap, double temperature,
                   c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    CHECK_INPUT_DEV(tangent);
    TORCH_CHECK(scores.sizes() == tangent.sizes(), "scores and tangent must have same shape");
    TORCH_CHECK(tangent.device() == scores.device(), "tangent must be on same device as scores, got ",
                tangent.device(), " vs ", scores.device());
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return sw_hvp_run(scores, tangent, l, d, (float)gap, (float)temperature, true);
}

Tensor soft_nw_param_jacobian(Tensor scores, int64_t param_type, double gap, double temperature,
                              c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    TORCH_CHECK(param_type >= 0 && param_type <= 1, "param_type must be 0 or 1");
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return sw_param_jacobian_run(scores, (int)param_type, l, d, (float)gap, (float)temperature,
                                 true);
}

std::tuple<Tensor, Tensor, Tensor> soft_nw_backward_full(Tensor scores, Tensor grad_alignment,
                                                         double gap, double temperature,
                                                         c10::optional<Tensor> lengths) {
    CHECK_INPUT_DEV(scores);
    TORCH_CHECK(grad_alignment.sizes() == scores.sizes(),
                "grad_alignment must have same shape as scores");
    TORCH_CHECK(grad_alignment.is_cuda(), "grad_alignment must be a CUDA tensor");
    TORCH_CHECK(grad_alignment.device() == scores.device(),
                "grad_alignment must be on same device as scores, got ", grad_alignment.device(),
                " vs ", scores.device());
    Dims d = checked_dims(scores, "NW");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    Tensor ga = grad_alignment.contiguous();
    if (ga.scalar_type() != torch::kFloat32) ga = ga.to(torch::kFloat32);
    auto r = sw_backward_full_run(scores, ga, l, d, (float)gap, (float)temperature, true);
    return {std::get<0>(r), std::get<1>(r).sum().reshape({1}), std::get<2>(r).sum().reshape({1})};
}

std::tuple<Tensor, Tensor, Tensor> nw_marginals_backward(Tensor s, Tensor gm, double g, double t,
                                                         c10::optional<Tensor> l) {
    return soft_nw_backward_full(s, gm, g, t, l);
}
Tensor nw_marginals_hvp(Tensor s, Tensor v, double g, double t, c10::optional<Tensor> l) {
    return soft_nw_hvp(s, v, g, t, l);
}
Tensor nw_marginals_grad_gap(Tensor s, double g, double t, c10::optional<Tensor> l) {
    return soft_nw_param_jacobian(s, 0, g, t, l);
}
Tensor nw_marginals_grad_temp(Tensor s, double g, double t, c10::optional<Tensor> l) {
    return soft_nw_param_jacobian(s, 1, g, t, l);
}

// ---------------------------------------------------------------------------
// affine-gap soft Smith-Waterman
// ---------------------------------------------------------------------------

// /root/reference/src/sw_affine/torch_cuda.cpp:34-66
Dims checked_dims_affine(const Tensor& x) {
    TORCH_CHECK(x.dim() == 3, "scores must be 3D (B, L1, L2)");
    Dims d{checked_dim(x.size(0), "scores batch dimension"),
           checked_dim(x.size(1), "scores L1 dimension"),
           checked_dim(x.size(2), "scores L2 dimension")};
    const int64_t cells = 3 * (int64_t(d.L1) + 1) * (int64_t(d.L2) + 1);
    TORCH_CHECK(cells <= std::numeric_limits<int>::max(),
                "sw_affine DP table too large: 3 * (L1 + 1) * (L2 + 1) exceeds CUDA int index range");
    return d;
}

// /root/reference/src/nw_affine/torch_cuda.cpp:32-78 (global alignment)
Dims checked_dims_nwa(const Tensor& x) {
    TORCH_CHECK(x.dim() == 3, "scores must be 3D (B, L1, L2)");
    auto dim = [](int64_t v, const char* name) {
        TORCH_CHECK(v >= 0 && v <= std::numeric_limits<int>::max(), "scores dimension ", name,
                    " must fit in int32, got ", v);
        return (int)v;
    };
    Dims d{dim(x.size(0), "B"), dim(x.size(1), "L1"), dim(x.size(2), "L2")};
    TORCH_CHECK(d.L1 <= std::numeric_limits<int>::max() - d.L2,
                "scores dimensions L1 + L2 must fit in int32, got ", d.L1, " + ", d.L2);
    const int64_t cells = 3 * (int64_t(d.L1) + 1) * (int64_t(d.L2) + 1);
    TORCH_CHECK(cells <= std::numeric_limits<int>::max(),
                "nw_affine alpha workspace size must fit in int32, got ", cells);
    return d;
}

// the affine family: local (soft_sw_affine) or global (soft_nw_affine) alignment
Dims checked_dims_aff(const Tensor& x, bool global) {
    return global ? checked_dims_nwa(x) : checked_dims_affine(x);
}

struct SwaOut {
    Tensor partition, marginals, grad_open, grad_ext, grad_T;
};

SwaOut swa_run(const Tensor& scores, const Tensor& lengths, const Dims& d, float go, float ge,
               float T, bool global = false) {
    auto opt = scores.options();
    SwaOut o{torch::empty({d.B}, opt), torch::empty({d.B, d.L1, d.L2}, opt),
             torch::empty({d.B}, opt), torch::empty({d.B}, opt), torch::empty({d.B}, opt)};
    const size_t ws_bytes = global ? d2p_nwa_workspace_bytes(d.B, d.L1, d.L2)
                                   : d2p_swa_workspace_bytes(d.B, d.L1, d.L2);
    Tensor ws = workspace(ws_bytes, scores);
    auto fn = global ? d2p_nwa_forward_marginals : d2p_swa_forward_marginals;
    D2P_CALL(fn(scores.data_ptr<float>(), lengths_ptr(lengths), d.B, d.L1, d.L2, go, ge, T,
                o.partition.data_ptr<float>(), o.marginals.data_ptr<float>(),
                o.grad_open.data_ptr<float>(), o.grad_ext.data_ptr<float>(),
                o.grad_T.data_ptr<float>(), ws.data_ptr(), ws_bytes, current_stream()));
    check_status(ws, d.B);
    return o;
}

Tensor swa_second_workspace(const Dims& d, const Tensor& like, bool global = false) {
    return workspace(global ? d2p_nwa_second_workspace_bytes(d.B, d.L1, d.L2)
                            : d2p_swa_second_workspace_bytes(d.B, d.L1, d.L2),
                     like);
}

// returns (grad_scores [B,L1,L2], per-element <ga, dP/dopen>, <ga, dP/dext>, <ga, dP/dT> [B])
std::tuple<Tensor, Tensor, Tensor, Tensor> swa_backward_full_run(const Tensor& scores,
                                                                 const Tensor& ga,
                                                                 const Tensor& lengths,
                                                                 const Dims& d, float go, float ge,
                                                                 float T, bool global = false) {
    auto opt = scores.options();
    Tensor gs = torch::empty({d.B, d.L1, d.L2}, opt);
    Tensor g_o = torch::empty({d.B}, opt), g_e = torch::empty({d.B}, opt);
    Tensor g_t = torch::empty({d.B}, opt);
    Tensor ws = swa_second_workspace(d, scores, global);
    auto fn = global ? d2p_nwa_backward_full : d2p_swa_backward_full;
    D2P_CALL(fn(scores.data_ptr<float>(), ga.data_ptr<float>(), lengths_ptr(lengths), d.B, d.L1,
                d.L2, go, ge, T, gs.data_ptr<float>(), g_o.data_ptr<float>(),
                g_e.data_ptr<float>(), g_t.data_ptr<float>(), ws.data_ptr(), ws.numel(),
                current_stream()));
    check_status(ws, d.B);
    return {gs, g_o, g_e, g_t};
}

// Autograd semantics of SoftSWAffineCUDAFunction
// (/root/reference/src/sw_affine/torch_cuda.cpp:126-400) and of
// SoftNWAffineCUDAFunction (/root/reference/src/nw_affine/torch_cuda.cpp:164-345):
// outputs {value, marginals}; d value / d scores = marginals; parameter gradients
// sum_b grad_value[b] * dS_b/dtheta.
tensor_list swa_autograd_forward(AutogradContext* ctx, const Tensor& scores, const Tensor& lengths,
                                 double go, double ge, double T, bool global) {
    ctx->set_materialize_grads(false);
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    SwaOut o = swa_run(scores, lengths, d, (float)go, (float)ge, (float)T, global);
    ctx->save_for_backward({scores, lengths, o.marginals, o.grad_open, o.grad_ext, o.grad_T});
    ctx->saved_data["gap_open"] = go;
    ctx->saved_data["gap_ext"] = ge;
    ctx->saved_data["temperature"] = T;
    ctx->saved_data["global"] = global;
    return {o.partition, o.marginals};
}

// returns {grad_scores, grad_open, grad_ext, grad_T}
tensor_list swa_autograd_backward(AutogradContext* ctx, const tensor_list& grads, bool want_o,
                                  bool want_e, bool want_T) {
    auto saved = ctx->get_saved_variables();
    Tensor scores = saved[0], lengths = saved[1], marg = saved[2];
    c10::hip::HIPGuardMasqueradingAsCUDA guard(marg.device());
    Tensor grad_value = grads[0], grad_marg = grads[1];
    Tensor gs, go, ge, gT;
    if (grad_value.defined() && grad_value.numel() > 0) {
        gs = scale_by_batch(marg, grad_value, lengths);
        if (want_o) go = grad_param_sum(grad_value, saved[3]);
        if (want_e) ge = grad_param_sum(grad_value, saved[4]);
        if (want_T) gT = grad_param_sum(grad_value, saved[5]);
    }
    if (grad_marg.defined() && grad_marg.numel() > 0) {
        // marginal path: HVP against the cotangent plus its dot products with
        // dP/dopen, dP/dext and dP/dT (/root/reference/src/sw_affine/torch_cuda.cpp:284-393,
        // /root/reference/src/nw_affine/torch_cuda.cpp:277-342)
        Tensor gm = prepare_cotangent(grad_marg, scores, "grad_posteriors");
        const bool global = ctx->saved_data["global"].toBool();
        Dims d = checked_dims_aff(scores, global);
        auto r = swa_backward_full_run(scores, gm, lengths, d,
                                       (float)ctx->saved_data["gap_open"].toDouble(),
                                       (float)ctx->saved_data["gap_ext"].toDouble(),
                                       (float)ctx->saved_data["temperature"].toDouble(), global);
        gs = gs.defined() ? gs + std::get<0>(r) : std::get<0>(r);
        Tensor to = std::get<1>(r).sum().reshape({1}), te = std::get<2>(r).sum().reshape({1});
        Tensor tt = std::get<3>(r).sum().reshape({1});
        if (want_o) go = go.defined() ? go + to : to;
        if (want_e) ge = ge.defined() ? ge + te : te;
        if (want_T) gT = gT.defined() ? gT + tt : tt;
    }
    return {gs, go, ge, gT};
}

class SoftSWAffineFloatFunction : public torch::autograd::Function<SoftSWAffineFloatFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor scores,
                               c10::optional<Tensor> lengths, double go, double ge, double T,
                               bool global) {
        return swa_autograd_forward(ctx, scores, lengths.value_or(Tensor()), go, ge, T, global);
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto g = swa_autograd_backward(ctx, grads, false, false, false);
        return {g[0], Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

class SoftSWAffineTensorFunction : public torch::autograd::Function<SoftSWAffineTensorFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor scores, Tensor go_t, Tensor ge_t,
                               Tensor temp_t, Tensor lengths, double go, double ge, double T,
                               bool global) {
        return swa_autograd_forward(ctx, scores, lengths, go, ge, T, global);
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto g = swa_autograd_backward(ctx, grads, ctx->needs_input_grad(1),
                                       ctx->needs_input_grad(2), ctx->needs_input_grad(3));
        return {g[0], g[1], g[2], g[3], Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

std::vector<Tensor> aff_t(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temperature,
                          Tensor lengths, bool global) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    const float go = scalar_value(gap_open, "gap_open");
    const float ge = scalar_value(gap_ext, "gap_ext");
    const float T = scalar_value(temperature, "temperature");
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return SoftSWAffineTensorFunction::apply(scores, gap_open, gap_ext, temperature, l, go, ge, T,
                                             global);
}

std::vector<Tensor> aff_float(Tensor scores, double gap_open, double gap_ext, double temperature,
                              c10::optional<Tensor> lengths, bool global) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    return SoftSWAffineFloatFunction::apply(scores, lengths_arg(l), gap_open, gap_ext,
                                            temperature, global);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> aff_with_grads(Tensor scores, double gap_open,
                                                                  double gap_ext,
                                                                  double temperature,
                                                                  c10::optional<Tensor> lengths,
                                                                  bool global) {
    CHECK_INPUT_DEV(scores);
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    SwaOut o = swa_run(scores, l, d, (float)gap_open, (float)gap_ext, (float)temperature, global);
    return {o.partition, o.marginals, o.grad_open, o.grad_ext, o.grad_T};
}

// /root/reference/src/sw_affine/torch_cuda.cpp:508-578,
// /root/reference/src/nw_affine/torch_cuda.cpp:435-482
Tensor aff_hvp(Tensor scores, Tensor tangent, double gap_open, double gap_ext, double temperature,
               c10::optional<Tensor> lengths, bool global) {
    CHECK_INPUT_DEV(scores);
    CHECK_INPUT_DEV(tangent);
    TORCH_CHECK(scores.dim() == 3, global ? "scores must be 3D (B, L1, L2)" : "scores must be 3D");
    if (global) TORCH_CHECK(tangent.dim() == 3, "tangent must be 3D (B, L1, L2)");
    TORCH_CHECK(scores.sizes() == tangent.sizes(), "scores and tangent must have same shape");
    TORCH_CHECK(tangent.device() == scores.device(), "tangent must be on same device as scores, got ",
                tangent.device(), " vs ", scores.device());
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    Tensor out = torch::empty({d.B, d.L1, d.L2}, scores.options());
    Tensor ws = swa_second_workspace(d, scores, global);
    auto fn = global ? d2p_nwa_hvp : d2p_swa_hvp;
    D2P_CALL(fn(scores.data_ptr<float>(), tangent.data_ptr<float>(), lengths_ptr(l), d.B, d.L1,
                d.L2, (float)gap_open, (float)gap_ext, (float)temperature, out.data_ptr<float>(),
                ws.data_ptr(), ws.numel(), current_stream()));
    check_status(ws, d.B);
    return out;
}

// /root/reference/src/sw_affine/torch_cuda.cpp:580-679,
// /root/reference/src/nw_affine/torch_cuda.cpp:484-553
Tensor aff_param_jacobian(Tensor scores, int64_t param_type, double gap_open, double gap_ext,
                          double temperature, c10::optional<Tensor> lengths, bool global) {
    CHECK_INPUT_DEV(scores);
    TORCH_CHECK(scores.dim() == 3, global ? "scores must be 3D (B, L1, L2)" : "scores must be 3D");
    TORCH_CHECK(param_type >= 0 && param_type <= 2, "param_type must be 0, 1, or 2");
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    Tensor out = torch::empty({d.B, d.L1, d.L2}, scores.options());
    Tensor ws = swa_second_workspace(d, scores, global);
    auto fn = global ? d2p_nwa_param_jacobian : d2p_swa_param_jacobian;
    D2P_CALL(fn(scores.data_ptr<float>(), (int)param_type, lengths_ptr(l), d.B, d.L1, d.L2,
                (float)gap_open, (float)gap_ext, (float)temperature, out.data_ptr<float>(),
                ws.data_ptr(), ws.numel(), current_stream()));
    check_status(ws, d.B);
    return out;
}

// /root/reference/src/sw_affine/torch_cuda.cpp:681-817,
// /root/reference/src/nw_affine/torch_cuda.cpp:555-665
std::tuple<Tensor, Tensor, Tensor, Tensor> aff_backward_full(Tensor scores, Tensor grad_alignment,
                                                             double gap_open, double gap_ext,
                                                             double temperature,
                                                             c10::optional<Tensor> lengths,
                                                             bool global) {
    CHECK_INPUT_DEV(scores);
    TORCH_CHECK(scores.dim() == 3, "scores must be 3D (B, L1, L2)");
    if (global) TORCH_CHECK(grad_alignment.dim() == 3, "grad_alignment must be 3D (B, L1, L2)");
    TORCH_CHECK(grad_alignment.sizes() == scores.sizes(),
                "grad_alignment must have same shape as scores");
    TORCH_CHECK(grad_alignment.is_cuda(), "grad_alignment must be a CUDA tensor");
    TORCH_CHECK(grad_alignment.device() == scores.device(),
                "grad_alignment must be on same device as scores, got ", grad_alignment.device(),
                " vs ", scores.device());
    Dims d = checked_dims_aff(scores, global);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(scores.device());
    Tensor l = resolve_lengths(lengths, d, scores.device());
    Tensor ga = grad_alignment.contiguous();
    if (ga.scalar_type() != torch::kFloat32) ga = ga.to(torch::kFloat32);
    auto r = swa_backward_full_run(scores, ga, l, d, (float)gap_open, (float)gap_ext,
                                   (float)temperature, global);
    return {std::get<0>(r), std::get<1>(r).sum().reshape({1}), std::get<2>(r).sum().reshape({1}),
            std::get<3>(r).sum().reshape({1})};
}

// soft_sw_affine ops
std::vector<Tensor> swa_t(Tensor s, Tensor go, Tensor ge, Tensor t, Tensor l) {
    return aff_t(s, go, ge, t, l, false);
}
std::vector<Tensor> swa_float(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return aff_float(s, go, ge, t, l, false);
}
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> swa_with_grads(Tensor s, double go, double ge,
                                                                  double t,
                                                                  c10::optional<Tensor> l) {
    return aff_with_grads(s, go, ge, t, l, false);
}
std::tuple<Tensor, Tensor, Tensor> swa_value_grad_params(Tensor s, double go, double ge, double t,
                                                         c10::optional<Tensor> l) {
    auto r = swa_with_grads(s, go, ge, t, l);
    return {std::get<2>(r), std::get<3>(r), std::get<4>(r)};
}
Tensor swa_hvp(Tensor s, Tensor v, double go, double ge, double t, c10::optional<Tensor> l) {
    return aff_hvp(s, v, go, ge, t, l, false);
}
Tensor swa_param_jacobian(Tensor s, int64_t p, double go, double ge, double t,
                          c10::optional<Tensor> l) {
    return aff_param_jacobian(s, p, go, ge, t, l, false);
}
std::tuple<Tensor, Tensor, Tensor, Tensor> swa_backward_full(Tensor s, Tensor ga, double go,
                                                             double ge, double t,
                                                             c10::optional<Tensor> l) {
    return aff_backward_full(s, ga, go, ge, t, l, false);
}

// soft_nw_affine ops (/root/reference/src/nw_affine/registry.cpp:35-50): the same
// sweeps in global-alignment mode
std::vector<Tensor> nwa_t(Tensor s, Tensor go, Tensor ge, Tensor t, Tensor l) {
    return aff_t(s, go, ge, t, l, true);
}
std::vector<Tensor> nwa_float(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return aff_float(s, go, ge, t, l, true);
}
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> nwa_with_grads(Tensor s, double go, double ge,
                                                                  double t,
                                                                  c10::optional<Tensor> l) {
    return aff_with_grads(s, go, ge, t, l, true);
}
// (score, grad_gap_open, grad_gap_ext): /root/reference/src/nw_affine/torch_cuda.cpp:687-698
std::tuple<Tensor, Tensor, Tensor> nwa_value_grad_params(Tensor s, double go, double ge, double t,
                                                         c10::optional<Tensor> l) {
    auto r = nwa_with_grads(s, go, ge, t, l);
    return {std::get<0>(r), std::get<2>(r), std::get<3>(r)};
}
Tensor nwa_hvp(Tensor s, Tensor v, double go, double ge, double t, c10::optional<Tensor> l) {
    return aff_hvp(s, v, go, ge, t, l, true);
}
Tensor nwa_param_jacobian(Tensor s, int64_t p, double go, double ge, double t,
                          c10::optional<Tensor> l) {
    return aff_param_jacobian(s, p, go, ge, t, l, true);
}
std::tuple<Tensor, Tensor, Tensor, Tensor> nwa_backward_full(Tensor s, Tensor ga, double go,
                                                             double ge, double t,
                                                             c10::optional<Tensor> l) {
    return aff_backward_full(s, ga, go, ge, t, l, true);
}
Tensor nwa_marg_grad_open(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return nwa_param_jacobian(s, 0, go, ge, t, l);
}
Tensor nwa_marg_grad_ext(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return nwa_param_jacobian(s, 1, go, ge, t, l);
}
Tensor nwa_marg_grad_temp(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return nwa_param_jacobian(s, 2, go, ge, t, l);
}

// sw_affine_marginals_grad_{gap_open,gap_ext,temp}
// (/root/reference/src/sw_affine/torch_cuda.cpp:878-910)
Tensor swa_marg_grad_open(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return swa_param_jacobian(s, 0, go, ge, t, l);
}
Tensor swa_marg_grad_ext(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return swa_param_jacobian(s, 1, go, ge, t, l);
}
Tensor swa_marg_grad_temp(Tensor s, double go, double ge, double t, c10::optional<Tensor> l) {
    return swa_param_jacobian(s, 2, go, ge, t, l);
}

// ---------------------------------------------------------------------------
// soft DTW
// ---------------------------------------------------------------------------

// /root/reference/src/dtw/torch_cuda.cpp:33-83
Dims checked_dims_dtw(const Tensor& costs) {
    TORCH_CHECK(costs.dim() == 3, "costs must be 3D (B, L1, L2)");
    const int64_t B = costs.size(0), L1 = costs.size(1), L2 = costs.size(2);
    TORCH_CHECK(B >= 0 && B <= std::numeric_limits<int>::max(),
                "DTW batch size is too large for CUDA kernels: ", B);
    TORCH_CHECK(L1 >= 0 && L1 <= std::numeric_limits<int>::max() - 1,
                "DTW L1 dimension is too large for CUDA kernels: ", L1);
    TORCH_CHECK(L2 >= 0 && L2 <= std::numeric_limits<int>::max() - 1,
                "DTW L2 dimension is too large for CUDA kernels: ", L2);
    const int64_t cells = (L1 + 1) * (L2 + 1);
    TORCH_CHECK(cells <= std::numeric_limits<int>::max(),
                "DTW alpha table is too large for CUDA kernels: ", cells);
    return Dims{(int)B, (int)L1, (int)L2};
}

int checked_bandwidth(int64_t bw) {
    TORCH_CHECK(bw >= std::numeric_limits<int>::min() && bw <= std::numeric_limits<int>::max(),
                "DTW bandwidth is out of CUDA int range: ", bw);
    return (int)bw;
}

struct DtwOut {
    Tensor value, marginals, grad_T;
};

DtwOut dtw_run(const Tensor& costs, const Tensor& lengths, const Dims& d, float T, int bw) {
    auto opt = costs.options();
    DtwOut o{torch::empty({d.B}, opt), torch::empty({d.B, d.L1, d.L2}, opt),
             torch::empty({d.B}, opt)};
    const size_t ws_bytes = d2p_dtw_workspace_bytes_banded(d.B, d.L1, d.L2, bw);
    Tensor ws = workspace(ws_bytes, costs);
    D2P_CALL(d2p_dtw_forward_marginals(
        costs.data_ptr<float>(), lengths_ptr(lengths), d.B, d.L1, d.L2, T, bw,
        o.value.data_ptr<float>(), o.marginals.data_ptr<float>(), o.grad_T.data_ptr<float>(),
        ws.data_ptr(), ws_bytes, current_stream()));
    check_status(ws, d.B);
    return o;
}

Tensor dtw_second_workspace(const Dims& d, int bw, const Tensor& like) {
    return workspace(d2p_dtw_second_workspace_bytes_banded(d.B, d.L1, d.L2, bw), like);
}

// (grad_costs = H . ga, per-element <ga, dP/dT>)
std::tuple<Tensor, Tensor> dtw_backward_full_run(const Tensor& costs, const Tensor& ga,
                                                 const Tensor& lengths, const Dims& d, float T,
                                                 int bw) {
    Tensor gc = torch::empty({d.B, d.L1, d.L2}, costs.options());
    Tensor gt = torch::empty({d.B}, costs.options());
    Tensor ws = dtw_second_workspace(d, bw, costs);
    D2P_CALL(d2p_dtw_backward_full(costs.data_ptr<float>(), ga.data_ptr<float>(),
                                   lengths_ptr(lengths), d.B, d.L1, d.L2, T, bw,
                                   gc.data_ptr<float>(), gt.data_ptr<float>(), ws.data_ptr(),
                                   ws.numel(), current_stream()));
    check_status(ws, d.B);
    return {gc, gt};
}

// Autograd semantics of SoftDTWCUDAFunction (/root/reference/src/dtw/torch_cuda.cpp:139-325):
// inputs (costs, temperature, lengths, bandwidth), outputs {value, marginals}; the
// marginal path adds the HVP against the marginal cotangent and <cotangent, dP/dT>.
class SoftDTWFunction : public torch::autograd::Function<SoftDTWFunction> {
   public:
    static tensor_list forward(AutogradContext* ctx, Tensor costs, Tensor temperature,
                               c10::optional<Tensor> lengths, int64_t bandwidth) {
        ctx->set_materialize_grads(false);
        CHECK_INPUT_DEV(costs);
        Dims d = checked_dims_dtw(costs);
        TORCH_CHECK(temperature.numel() == 1, "temperature must be a scalar tensor");
        c10::hip::HIPGuardMasqueradingAsCUDA guard(costs.device());
        const int bw = checked_bandwidth(bandwidth);
        Tensor l = resolve_lengths(lengths, d, costs.device(), "costs");
        const float T = scalar_value(temperature, "temperature");
        DtwOut o = dtw_run(costs, l, d, T, bw);
        ctx->save_for_backward({costs, l, o.marginals, o.grad_T});
        ctx->saved_data["temperature"] = (double)T;
        ctx->saved_data["bandwidth"] = (int64_t)bw;
        return {o.value, o.marginals};
    }
    static tensor_list backward(AutogradContext* ctx, tensor_list grads) {
        auto saved = ctx->get_saved_variables();
        Tensor costs = saved[0], lengths = saved[1], marg = saved[2], gT = saved[3];
        c10::hip::HIPGuardMasqueradingAsCUDA guard(marg.device());
        Tensor grad_value = grads[0], grad_marg = grads[1];
        Tensor gc, gt;
        if (grad_value.defined() && grad_value.numel() > 0) {
            gc = scale_by_batch(marg, grad_value, lengths);
            if (ctx->needs_input_grad(1)) gt = grad_param_sum(grad_value, gT);
        }
        if (grad_marg.defined() && grad_marg.numel() > 0) {
            Tensor gm = prepare_cotangent(grad_marg, costs, "grad_posteriors");
            Dims d = checked_dims_dtw(costs);
            auto r = dtw_backward_full_run(costs, gm, lengths, d,
                                           (float)ctx->saved_data["temperature"].toDouble(),
                                           (int)ctx->saved_data["bandwidth"].toInt());
            gc = gc.defined() ? gc + std::get<0>(r) : std::get<0>(r);
            if (ctx->needs_input_grad(1)) {
                Tensor t = std::get<1>(r).sum().reshape({1});
                gt = gt.defined() ? gt + t : t;
            }
        }
        return {gc, gt, Tensor(), Tensor()};
    }
};

std::vector<Tensor> dtw_t(Tensor costs, Tensor temperature, Tensor lengths, int64_t bandwidth) {
    return SoftDTWFunction::apply(costs, temperature, lengths, bandwidth);
}

std::vector<Tensor> dtw_float(Tensor costs, double temperature, c10::optional<Tensor> lengths,
                              c10::optional<int64_t> bandwidth) {
    CHECK_INPUT_DEV(costs);
    Dims d = checked_dims_dtw(costs);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(costs.device());
    Tensor temp_t = torch::tensor({(float)temperature}, costs.options());
    Tensor l = resolve_lengths(lengths, d, costs.device(), "costs");
    return SoftDTWFunction::apply(costs, temp_t, lengths_arg(l),
                                  bandwidth.has_value() ? *bandwidth : -1);
}

std::tuple<Tensor, Tensor, Tensor> dtw_with_grads(Tensor costs, double temperature,
                                                  c10::optional<Tensor> lengths,
                                                  c10::optional<int64_t> bandwidth) {
    CHECK_INPUT_DEV(costs);
    Dims d = checked_dims_dtw(costs);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(costs.device());
    Tensor l = resolve_lengths(lengths, d, costs.device(), "costs");
    const int bw = checked_bandwidth(bandwidth.has_value() ? *bandwidth : -1);
    DtwOut o = dtw_run(costs, l, d, (float)temperature, bw);
    return {o.value, o.marginals, o.grad_T};
}

Tensor dtw_hvp(Tensor costs, Tensor tangent, double temperature, c10::optional<Tensor> lengths,
               c10::optional<int64_t> bandwidth) {
    CHECK_INPUT_DEV(costs);
    CHECK_INPUT_DEV(tangent);
    TORCH_CHECK(tangent.sizes() == costs.sizes(), "tangent must have same shape as costs");
    TORCH_CHECK(tangent.device() == costs.device(), "tangent must be on same device as costs, got ",
                tangent.device(), " vs ", costs.device());
    Dims d = checked_dims_dtw(costs);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(costs.device());
    Tensor l = resolve_lengths(lengths, d, costs.device(), "costs");
    const int bw = checked_bandwidth(bandwidth.has_value() ? *bandwidth : -1);
    Tensor out = torch::empty({d.B, d.L1, d.L2}, costs.options());
    Tensor ws = dtw_second_workspace(d, bw, costs);
    D2P_CALL(d2p_dtw_hvp(costs.data_ptr<float>(), tangent.data_ptr<float>(), lengths_ptr(l),
                         d.B, d.L1, d.L2, (float)temperature, bw, out.data_ptr<float>(),
                         ws.data_ptr(), ws.numel(), current_stream()));
    check_status(ws, d.B);
    return out;
}

Tensor dtw_param_jacobian(Tensor costs, double temperature, c10::optional<Tensor> lengths,
                          c10::optional<int64_t> bandwidth) {
    CHECK_INPUT_DEV(costs);
    Dims d = checked_dims_dtw(costs);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(costs.device());
    Tensor l = resolve_lengths(lengths, d, costs.device(), "costs");
    const int bw = checked_bandwidth(bandwidth.has_value() ? *bandwidth : -1);
    Tensor out = torch::empty({d.B, d.L1, d.L2}, costs.options());
    Tensor ws = dtw_second_workspace(d, bw, costs);
    D2P_CALL(d2p_dtw_param_jacobian(costs.data_ptr<float>(), lengths_ptr(l), d.B, d.L1, d.L2,
                                    (float)temperature, bw, out.data_ptr<float>(), ws.data_ptr(),
                                    ws.numel(), current_stream()));
    check_status(ws, d.B);
    return out;
}

std::tuple<Tensor, Tensor> dtw_backward_full(Tensor costs, Tensor grad_alignment,
                                             double temperature, c10::optional<Tensor> lengths,
                                             c10::optional<int64_t> bandwidth) {
    CHECK_INPUT_DEV(costs);
    TORCH_CHECK(grad_alignment.sizes() == costs.sizes(),
                "grad_alignment must have same shape as costs");
    TORCH_CHECK(grad_alignment.is_cuda(), "grad_alignment must be a CUDA tensor");
    TORCH_CHECK(grad_alignment.device() == costs.device(),
                "grad_alignment must be on same device as costs, got ", grad_alignment.device(),
                " vs ", costs.device());
    Dims d = checked_dims_dtw(costs);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(costs.device());
    Tensor l = resolve_lengths(lengths, d, costs.device(), "costs");
    const int bw = checked_bandwidth(bandwidth.has_value() ? *bandwidth : -1);
    Tensor ga = grad_alignment.contiguous();
    if (ga.scalar_type() != torch::kFloat32) ga = ga.to(torch::kFloat32);
    auto r = dtw_backward_full_run(costs, ga, l, d, (float)temperature, bw);
    return {std::get<0>(r), std::get<1>(r).sum().reshape({1})};
}

[[noreturn]] void cpu_unsupported() {
    TORCH_CHECK(false,
                "d2p_amd implements the MI355X (HIP) path only: move the inputs to a "
                "HIP device (device='cuda' on PyTorch-ROCm)");
}

}  // namespace

// ---------------------------------------------------------------------------
// fused squared-Euclidean costs + soft DTW (no counterpart in the reference: its
// callers form torch.cdist(x, y) ** 2 first, /root/reference/docs/algorithms/dtw.md:52)
// ---------------------------------------------------------------------------
namespace {
Dims checked_dims_xy(const Tensor& x, const Tensor& y) {
    TORCH_CHECK(x.dim() == 3 && y.dim() == 3, "x and y must be 3D (B, L, D)");
    TORCH_CHECK(x.size(0) == y.size(0), "x and y must have the same batch size, got ",
                x.size(0), " and ", y.size(0));
    TORCH_CHECK(x.size(2) == y.size(2), "x and y must have the same feature dimension, got ",
                x.size(2), " and ", y.size(2));
    TORCH_CHECK(x.size(2) >= 1 && x.size(2) <= 128, "feature dimension D must be between 1 and "
                "128, got ", x.size(2));
    TORCH_CHECK(y.device() == x.device(), "y must be on same device as x, got ", y.device(),
                " vs ", x.device());
    Dims d{checked_dim(x.size(0), "x batch dimension"), checked_dim(x.size(1), "x L1 dimension"),
           checked_dim(y.size(1), "y L2 dimension")};
    const int64_t cells = (int64_t(d.L1) + 1) * (int64_t(d.L2) + 1);
    TORCH_CHECK(cells <= std::numeric_limits<int>::max(),
                "DTW alpha table is too large for CUDA kernels: ", cells);
    return d;
}
}  // namespace

// (value [B], alignment [B, L1, L2], dvalue/dT [B]) of soft DTW over the costs
// sum_d (x[b,i,d] - y[b,j,d])^2, formed inside the forward sweep
std::tuple<Tensor, Tensor, Tensor> dtw_sqeuclid(Tensor x, Tensor y, double temperature,
                                                c10::optional<Tensor> lengths, int64_t bandwidth) {
    CHECK_INPUT_DEV(x);
    CHECK_INPUT_DEV(y);
    TORCH_CHECK(temperature > 0, "temperature must be positive, got ", temperature);
    Dims d = checked_dims_xy(x, y);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    Tensor l = resolve_lengths(lengths, d, x.device(), "x");
    const int bw = checked_bandwidth(bandwidth);
    auto opt = x.options();
    Tensor value = torch::empty({d.B}, opt), marg = torch::empty({d.B, d.L1, d.L2}, opt);
    Tensor gT = torch::empty({d.B}, opt);
    const size_t ws_bytes = d2p_dtw_workspace_bytes_banded(d.B, d.L1, d.L2, bw);
    Tensor ws = workspace(ws_bytes, x);
    D2P_CALL(d2p_dtw_sqeuclid_forward_marginals(
        x.data_ptr<float>(), y.data_ptr<float>(), lengths_ptr(l), d.B, d.L1, d.L2,
        (int)x.size(2), (float)temperature, bw, value.data_ptr<float>(), marg.data_ptr<float>(),
        gT.data_ptr<float>(), ws.data_ptr(), ws_bytes, current_stream()));
    check_status(ws, d.B);
    return {value, marg, gT};
}

// costs [B, L1, L2] = sum_d (x[b,i,d] - y[b,j,d])^2, bit-identical to the fused forward's
Tensor pairwise_sqdist(Tensor x, Tensor y) {
    CHECK_INPUT_DEV(x);
    CHECK_INPUT_DEV(y);
    Dims d = checked_dims_xy(x, y);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    Tensor out = torch::empty({d.B, d.L1, d.L2}, x.options());
    D2P_CALL(d2p_pairwise_sqdist(x.data_ptr<float>(), y.data_ptr<float>(), d.B, d.L1, d.L2,
                                 (int)x.size(2), out.data_ptr<float>(), current_stream()));
    return out;
}

// (grad_x, grad_y) through the squared-Euclidean costs from G = dL/dcosts and an
// optional per-element factor scale [B]
std::tuple<Tensor, Tensor> sqeuclid_feature_grad(Tensor G, Tensor x, Tensor y,
                                                 c10::optional<Tensor> scale) {
    CHECK_INPUT_DEV(G);
    CHECK_INPUT_DEV(x);
    CHECK_INPUT_DEV(y);
    Dims d = checked_dims_xy(x, y);
    TORCH_CHECK(G.dim() == 3 && G.size(0) == d.B && G.size(1) == d.L1 && G.size(2) == d.L2,
                "G must be [B, L1, L2] = [", d.B, ", ", d.L1, ", ", d.L2, "]");
    TORCH_CHECK(G.device() == x.device(), "G must be on same device as x");
    const float* sp = nullptr;
    Tensor sc;
    if (scale.has_value()) {
        sc = scale->contiguous();
        TORCH_CHECK(sc.scalar_type() == torch::kFloat32 && sc.numel() == d.B &&
                        sc.device() == x.device(),
                    "scale must be a float32 [B] tensor on x's device");
        sp = sc.data_ptr<float>();
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    Tensor gx = torch::empty_like(x), gy = torch::empty_like(y);
    D2P_CALL(d2p_sqeuclid_feature_grad(G.data_ptr<float>(), x.data_ptr<float>(),
                                       y.data_ptr<float>(), sp, d.B, d.L1, d.L2,
                                       (int)x.size(2), gx.data_ptr<float>(),
                                       gy.data_ptr<float>(), current_stream()));
    return {gx, gy};
}

TORCH_LIBRARY(d2p, m) {
    // /root/reference/src/sw/registry.cpp:30-44
    m.def("soft_sw(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) -> Tensor[]");
    m.def("soft_sw_float(Tensor scores, float gap, float temperature, Tensor? lengths) -> Tensor[]");
    m.def("soft_sw_with_grads(Tensor scores, float gap, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("soft_sw_hvp(Tensor scores, Tensor tangent, float gap, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_sw_param_jacobian(Tensor scores, int param_type, float gap, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_sw_backward_full(Tensor scores, Tensor grad_alignment, float gap, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor)");
    m.def("sw_forward(Tensor scores, float gap, float temp, Tensor? lengths) -> Tensor[]");
    m.def("sw_forward_t(Tensor scores, Tensor gap, Tensor temp, Tensor lengths) -> Tensor[]");
    m.def("sw_value_grad_params(Tensor scores, float gap, float temp, Tensor? lengths) -> (Tensor, Tensor)");
    m.def("sw_marginals_backward(Tensor scores, Tensor grad_marginals, float gap, float temp, Tensor? lengths) -> (Tensor, Tensor, Tensor)");
    m.def("sw_marginals_hvp(Tensor scores, Tensor v, float gap, float temp, Tensor? lengths) -> Tensor");
    m.def("sw_marginals_grad_gap(Tensor scores, float gap, float temp, Tensor? lengths) -> Tensor");
    m.def("sw_marginals_grad_temp(Tensor scores, float gap, float temp, Tensor? lengths) -> Tensor");

    // /root/reference/src/sw_affine/registry.cpp:74-89
    m.def("soft_sw_affine(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temperature, Tensor lengths) -> Tensor[]");
    m.def("soft_sw_affine_float(Tensor scores, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> Tensor[]");
    m.def("soft_sw_affine_with_grads(Tensor scores, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def("soft_sw_affine_hvp(Tensor scores, Tensor tangent, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_sw_affine_param_jacobian(Tensor scores, int param_type, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_sw_affine_backward_full(Tensor scores, Tensor grad_alignment, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("sw_affine_forward(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor[]");
    m.def("sw_affine_forward_t(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temp, Tensor lengths) -> Tensor[]");
    m.def("sw_affine_value_grad_params(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> (Tensor, Tensor, Tensor)");
    m.def("sw_affine_marginals_backward(Tensor scores, Tensor grad_marginals, float gap_open, float gap_ext, float temp, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("sw_affine_marginals_hvp(Tensor scores, Tensor v, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");
    m.def("sw_affine_marginals_grad_gap_open(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");
    m.def("sw_affine_marginals_grad_gap_ext(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");
    m.def("sw_affine_marginals_grad_temp(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");

    // /root/reference/src/nw_affine/registry.cpp:35-50
    m.def("soft_nw_affine(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temperature, Tensor lengths) -> Tensor[]");
    m.def("soft_nw_affine_float(Tensor scores, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> Tensor[]");
    m.def("soft_nw_affine_with_grads(Tensor scores, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def("soft_nw_affine_hvp(Tensor scores, Tensor tangent, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_nw_affine_param_jacobian(Tensor scores, int param_type, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_nw_affine_backward_full(Tensor scores, Tensor grad_alignment, float gap_open, float gap_ext, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("nw_affine_forward(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor[]");
    m.def("nw_affine_forward_t(Tensor scores, Tensor gap_open, Tensor gap_ext, Tensor temp, Tensor lengths) -> Tensor[]");
    m.def("nw_affine_value_grad_params(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> (Tensor, Tensor, Tensor)");
    m.def("nw_affine_marginals_backward(Tensor scores, Tensor grad_marginals, float gap_open, float gap_ext, float temp, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("nw_affine_marginals_hvp(Tensor scores, Tensor v, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");
    m.def("nw_affine_marginals_grad_gap_open(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");
    m.def("nw_affine_marginals_grad_gap_ext(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");
    m.def("nw_affine_marginals_grad_temp(Tensor scores, float gap_open, float gap_ext, float temp, Tensor? lengths) -> Tensor");

    // /root/reference/src/dtw/registry.cpp:127-132
    // /root/reference/src/nw/registry.cpp:35-45 (first-order operators)
    m.def("soft_nw(Tensor scores, Tensor gap, Tensor temperature, Tensor lengths) -> Tensor[]");
    m.def("soft_nw_float(Tensor scores, float gap, float temperature, Tensor? lengths) -> Tensor[]");
    m.def("soft_nw_with_grads(Tensor scores, float gap, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("nw_forward(Tensor scores, float gap, float temp, Tensor? lengths) -> Tensor[]");
    m.def("nw_forward_t(Tensor scores, Tensor gap, Tensor temp, Tensor lengths) -> Tensor[]");
    m.def("nw_value_grad_params(Tensor scores, float gap, float temp, Tensor? lengths) -> (Tensor, Tensor)");
    m.def("soft_nw_hvp(Tensor scores, Tensor tangent, float gap, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_nw_param_jacobian(Tensor scores, int param_type, float gap, float temperature, Tensor? lengths) -> Tensor");
    m.def("soft_nw_backward_full(Tensor scores, Tensor grad_alignment, float gap, float temperature, Tensor? lengths) -> (Tensor, Tensor, Tensor)");
    m.def("nw_marginals_backward(Tensor scores, Tensor grad_marginals, float gap, float temp, Tensor? lengths) -> (Tensor, Tensor, Tensor)");
    m.def("nw_marginals_hvp(Tensor scores, Tensor v, float gap, float temp, Tensor? lengths) -> Tensor");
    m.def("nw_marginals_grad_gap(Tensor scores, float gap, float temp, Tensor? lengths) -> Tensor");
    m.def("nw_marginals_grad_temp(Tensor scores, float gap, float temp, Tensor? lengths) -> Tensor");

    m.def("soft_dtw(Tensor costs, Tensor temperature, Tensor lengths, int bandwidth) -> Tensor[]");
    m.def("soft_dtw_float(Tensor costs, float temperature, Tensor? lengths, int? bandwidth) -> Tensor[]");
    m.def("soft_dtw_with_grads(Tensor costs, float temperature, Tensor? lengths, int? bandwidth) -> (Tensor, Tensor, Tensor)");
    m.def("soft_dtw_hvp(Tensor costs, Tensor tangent, float temperature, Tensor? lengths, int? bandwidth) -> Tensor");
    m.def("soft_dtw_param_jacobian(Tensor costs, float temperature, Tensor? lengths, int? bandwidth) -> Tensor");
    m.def("soft_dtw_backward_full(Tensor costs, Tensor grad_alignment, float temperature, Tensor? lengths, int? bandwidth) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(d2p, CUDA, m) {
    m.impl("soft_sw", soft_sw_t);
    m.impl("soft_sw_float", soft_sw_float);
    m.impl("soft_sw_with_grads", soft_sw_with_grads);
    m.impl("soft_sw_hvp", soft_sw_hvp);
    m.impl("soft_sw_param_jacobian", soft_sw_param_jacobian);
    m.impl("soft_sw_backward_full", soft_sw_backward_full);
    m.impl("sw_forward", sw_forward);
    m.impl("sw_forward_t", sw_forward_t);
    m.impl("sw_value_grad_params", sw_value_grad_params);
    m.impl("sw_marginals_backward", sw_marginals_backward);
    m.impl("sw_marginals_hvp", sw_marginals_hvp);
    m.impl("sw_marginals_grad_gap", sw_marginals_grad_gap);
    m.impl("sw_marginals_grad_temp", sw_marginals_grad_temp);

    m.impl("soft_nw", soft_nw_t);
    m.impl("soft_nw_float", soft_nw_float);
    m.impl("soft_nw_with_grads", soft_nw_with_grads);
    m.impl("nw_forward", nw_forward);
    m.impl("nw_forward_t", nw_forward_t);
    m.impl("nw_value_grad_params", nw_value_grad_params);
    m.impl("soft_nw_hvp", soft_nw_hvp);
    m.impl("soft_nw_param_jacobian", soft_nw_param_jacobian);
    m.impl("soft_nw_backward_full", soft_nw_backward_full);
    m.impl("nw_marginals_backward", nw_marginals_backward);
    m.impl("nw_marginals_hvp", nw_marginals_hvp);
    m.impl("nw_marginals_grad_gap", nw_marginals_grad_gap);
    m.impl("nw_marginals_grad_temp", nw_marginals_grad_temp);

    m.impl("soft_sw_affine", swa_t);
    m.impl("soft_sw_affine_float", swa_float);
    m.impl("soft_sw_affine_with_grads", swa_with_grads);
    m.impl("soft_sw_affine_hvp", swa_hvp);
    m.impl("soft_sw_affine_param_jacobian", swa_param_jacobian);
    m.impl("soft_sw_affine_backward_full", swa_backward_full);
    m.impl("sw_affine_forward", swa_float);
    m.impl("sw_affine_forward_t", swa_t);
    m.impl("sw_affine_value_grad_params", swa_value_grad_params);
    m.impl("sw_affine_marginals_backward", swa_backward_full);
    m.impl("sw_affine_marginals_hvp", swa_hvp);
    m.impl("sw_affine_marginals_grad_gap_open", swa_marg_grad_open);
    m.impl("sw_affine_marginals_grad_gap_ext", swa_marg_grad_ext);
    m.impl("sw_affine_marginals_grad_temp", swa_marg_grad_temp);
    m.impl("soft_nw_affine", nwa_t);
    m.impl("soft_nw_affine_float", nwa_float);
    m.impl("soft_nw_affine_with_grads", nwa_with_grads);
    m.impl("soft_nw_affine_hvp", nwa_hvp);
    m.impl("soft_nw_affine_param_jacobian", nwa_param_jacobian);
    m.impl("soft_nw_affine_backward_full", nwa_backward_full);
    m.impl("nw_affine_forward", nwa_float);
    m.impl("nw_affine_forward_t", nwa_t);
    m.impl("nw_affine_value_grad_params", nwa_value_grad_params);
    m.impl("nw_affine_marginals_backward", nwa_backward_full);
    m.impl("nw_affine_marginals_hvp", nwa_hvp);
    m.impl("nw_affine_marginals_grad_gap_open", nwa_marg_grad_open);
    m.impl("nw_affine_marginals_grad_gap_ext", nwa_marg_grad_ext);
    m.impl("nw_affine_marginals_grad_temp", nwa_marg_grad_temp);

    m.impl("soft_dtw", dtw_t);
    m.impl("soft_dtw_float", dtw_float);
    m.impl("soft_dtw_with_grads", dtw_with_grads);
    m.impl("soft_dtw_hvp", dtw_hvp);
    m.impl("soft_dtw_param_jacobian", dtw_param_jacobian);
    m.impl("soft_dtw_backward_full", dtw_backward_full);
}

// Autograd-registered ops, as in the reference
// (/root/reference/src/sw/torch_cuda.cpp:876-883 and the affine/DTW equivalents).
TORCH_LIBRARY_IMPL(d2p, AutogradCUDA, m) {
    m.impl("soft_sw", soft_sw_t);
    m.impl("soft_sw_float", soft_sw_float);
    m.impl("sw_forward", sw_forward);
    m.impl("sw_forward_t", sw_forward_t);
    m.impl("soft_sw_affine", swa_t);
    m.impl("soft_sw_affine_float", swa_float);
    m.impl("sw_affine_forward", swa_float);
    m.impl("sw_affine_forward_t", swa_t);
    m.impl("soft_dtw", dtw_t);
    m.impl("soft_dtw_float", dtw_float);
    m.impl("soft_nw", soft_nw_t);
    m.impl("soft_nw_float", soft_nw_float);
    m.impl("nw_forward", nw_forward);
    m.impl("nw_forward_t", nw_forward_t);
    m.impl("soft_nw_affine", nwa_t);
    m.impl("soft_nw_affine_float", nwa_float);
    m.impl("nw_affine_forward", nwa_float);
    m.impl("nw_affine_forward_t", nwa_t);
}

namespace {
void cpu_boxed(const c10::OperatorHandle&, torch::jit::Stack*) { cpu_unsupported(); }
const char* const kAllOps[] = {
    "soft_sw", "soft_sw_float", "soft_sw_with_grads", "soft_sw_hvp", "soft_sw_param_jacobian",
    "soft_sw_backward_full", "sw_forward", "sw_forward_t", "sw_value_grad_params",
    "sw_marginals_backward", "sw_marginals_hvp", "sw_marginals_grad_gap",
    "sw_marginals_grad_temp", "soft_sw_affine", "soft_sw_affine_float",
    "soft_sw_affine_with_grads", "soft_sw_affine_hvp", "soft_sw_affine_param_jacobian",
    "soft_sw_affine_backward_full", "sw_affine_forward", "sw_affine_forward_t",
    "sw_affine_value_grad_params", "sw_affine_marginals_backward", "sw_affine_marginals_hvp",
    "sw_affine_marginals_grad_gap_open", "sw_affine_marginals_grad_gap_ext",
    "sw_affine_marginals_grad_temp", "soft_dtw", "soft_dtw_float", "soft_dtw_with_grads",
    "soft_dtw_hvp", "soft_dtw_param_jacobian", "soft_dtw_backward_full", "soft_nw",
    "soft_nw_float", "soft_nw_with_grads", "soft_nw_hvp", "soft_nw_param_jacobian",
    "soft_nw_backward_full", "nw_forward", "nw_forward_t", "nw_value_grad_params",
    "nw_marginals_backward", "nw_marginals_hvp", "nw_marginals_grad_gap",
    "nw_marginals_grad_temp", "soft_nw_affine", "soft_nw_affine_float",
    "soft_nw_affine_with_grads", "soft_nw_affine_hvp", "soft_nw_affine_param_jacobian",
    "soft_nw_affine_backward_full", "nw_affine_forward", "nw_affine_forward_t",
    "nw_affine_value_grad_params", "nw_affine_marginals_backward", "nw_affine_marginals_hvp",
    "nw_affine_marginals_grad_gap_open", "nw_affine_marginals_grad_gap_ext",
    "nw_affine_marginals_grad_temp"};
}  // namespace

TORCH_LIBRARY_IMPL(d2p, CPU, m) {
    for (const char* name : kAllOps)
        m.impl(name, torch::CppFunction::makeFromBoxedFunction<&cpu_boxed>());
}

// Ops of this build with no counterpart in the reference live in their own namespace,
// so that d2p:: holds exactly the reference's schemas.
TORCH_LIBRARY(d2p_amd, m) {
    m.def("soft_dtw_sqeuclidean(Tensor x, Tensor y, float temperature, Tensor? lengths, "
          "int bandwidth) -> (Tensor, Tensor, Tensor)");
    m.def("pairwise_sqdist(Tensor x, Tensor y) -> Tensor");
    m.def("sqeuclid_feature_grad(Tensor G, Tensor x, Tensor y, Tensor? scale) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(d2p_amd, CUDA, m) {
    m.impl("soft_dtw_sqeuclidean", dtw_sqeuclid);
    m.impl("pairwise_sqdist", pairwise_sqdist);
    m.impl("sqeuclid_feature_grad", sqeuclid_feature_grad);
}

TORCH_LIBRARY_IMPL(d2p_amd, CPU, m) {
    m.impl("soft_dtw_sqeuclidean", torch::CppFunction::makeFromBoxedFunction<&cpu_boxed>());
    m.impl("pairwise_sqdist", torch::CppFunction::makeFromBoxedFunction<&cpu_boxed>());
    m.impl("sqeuclid_feature_grad", torch::CppFunction::makeFromBoxedFunction<&cpu_boxed>());
}
