// GroupNorm / SiLU / GNSiLU / add_tensors on libsoar_gn.so.
//
// Forward/backward structure follows src/nn/layers.cpp:483-802 and
// src/nn/blocks.cpp:17-72 of the reference: the layer allocates its output
// and saved statistics, calls the device operator, and attaches a node
// only when the output requires grad (and grad mode is on); the node's
// backward routes gradients with propagate_grad.  Differences, each
// result-preserving:
//   * parameter gradients of a leaf parameter that already has a device
//     .grad are accumulated straight into it by the kernel (the reference
//     zero-fills temporaries, then clones or adds them into .grad);
//   * the statistics are saved as mean, rstd and the mean's fp32 rounding
//     residual, so the backward's xhat is exact when std << |mean|.
#include "soar/nn.hpp"

#include "soar/autograd.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar_gn.h"

namespace soar::nn {

using autograd::GradMode;
using hip::kernels::check;

void Module::register_parameter(const std::string& name, TensorPtr p) {
    params_.emplace_back(name, std::move(p));
}

std::vector<std::pair<std::string, TensorPtr>> Module::named_parameters(
    const std::string& prefix) const {
    std::vector<std::pair<std::string, TensorPtr>> out;
    for (const auto& [n, p] : params_) out.emplace_back(prefix.empty() ? n : prefix + "." + n, p);
    return out;
}

void Module::to_device() {
    for (auto& [n, p] : params_) p->to_cuda();
}

void Module::zero_grad() {
    for (auto& [n, p] : params_) p->zero_grad();
}

namespace {

struct NCHW {
    int64_t N, C, HW;
};

NCHW nchw_of(const TensorPtr& t) {
    if (t->ndim() == 3) return {1, t->dim(0), t->dim(1) * t->dim(2)};
    if (t->ndim() == 4) return {t->dim(0), t->dim(1), t->dim(2) * t->dim(3)};
    throw ShapeError("GroupNorm expects [C,H,W] or [N,C,H,W], got " + to_string(t->shape()));
}

void* workspace(size_t bytes) {
    auto* arena = memory::DeviceArena::current();
    if (!arena) throw DeviceError("GroupNorm needs a DeviceArena for its workspace");
    return arena->allocate(bytes > 0 ? bytes : 1, {}, "gn_workspace");
}

const float* dptr(const TensorPtr& t) { return t ? t->cuda_data() : nullptr; }

// Backward node of GroupNorm and of the fused GN(+SiLU)(+residual) layer.
struct GroupNormNode : autograd::AutogradNode {
    TensorPtr input, weight, bias, mean, rstd, mean_lo;
    int64_t num_groups = 1;
    unsigned flags = 0;  // SOAR_GN_SILU / SOAR_GN_RESIDUAL of the forward

    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : {input, weight, bias})
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }

    void backward(const TensorPtr& go) override {
        const NCHW s = nchw_of(input);
        const bool want_x = input->requires_grad();
        const bool want_p = weight && weight->requires_grad();
        if (!want_x && !want_p) return;
        if (!go->is_cuda()) go->to_cuda();
        TensorPtr gx = want_x ? Tensor::create(input->shape(), false, true) : nullptr;
        TensorPtr gw, gb;
        bool direct = false;
        if (want_p) {
            const bool leaves = !weight->grad_fn() && !bias->grad_fn();
            if (leaves && weight->grad() && bias->grad() && weight->grad()->is_cuda() &&
                bias->grad()->is_cuda()) {
                gw = weight->grad();
                gb = bias->grad();
                direct = true;
            } else {
                gw = Tensor::zeros({s.C}, false, true);
                gb = Tensor::zeros({s.C}, false, true);
            }
        }
        const size_t wsb = soar_gn_workspace_bytes(s.N, s.C, s.HW, num_groups);
        check(soar_gn_silu_backward(go->cuda_data(), input->cuda_data(), dptr(weight), dptr(bias),
                                    mean->cuda_data(), rstd->cuda_data(), dptr(mean_lo),
                                    gx ? gx->cuda_data() : nullptr,
                                    gw ? gw->cuda_data() : nullptr,
                                    gb ? gb->cuda_data() : nullptr, s.N, s.C, s.HW, num_groups,
                                    flags, workspace(wsb), wsb, nullptr),
              "GroupNorm backward");
        if (want_p && !direct) {
            propagate_grad(weight, std::move(gw));
            propagate_grad(bias, std::move(gb));
        }
        if (want_x) propagate_grad(input, std::move(gx));
    }

    void release_variables() override {
        input = nullptr;
        mean = rstd = mean_lo = nullptr;
    }
};

struct SiLUNode : autograd::AutogradNode {
    TensorPtr input;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        if (input && input->grad_fn()) return {input->grad_fn()};
        return {};
    }
    void backward(const TensorPtr& go) override {
        if (!input->requires_grad()) return;
        if (!go->is_cuda()) go->to_cuda();
        TensorPtr gx = Tensor::zeros(input->shape(), false, true);
        hip::kernels::silu_backward(go->cuda_data(), input->cuda_data(), gx->cuda_data(),
                                    (size_t)input->numel());
        propagate_grad(input, std::move(gx));
    }
    void release_variables() override { input = nullptr; }
};

struct AddNode : autograd::AutogradNode {
    TensorPtr a, b;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        if (a && a->grad_fn()) r.push_back(a->grad_fn());
        if (b && b->grad_fn()) r.push_back(b->grad_fn());
        return r;
    }
    void backward(const TensorPtr& go) override {
        if (a) propagate_grad(a, go);
        if (b) propagate_grad(b, go);
    }
    void release_variables() override { a = b = nullptr; }
};

}  // namespace

GroupNorm::GroupNorm(size_t num_groups, size_t num_channels, float eps, bool affine)
    : GroupNorm("GroupNorm", num_groups, num_channels, eps, affine) {}

GroupNorm::GroupNorm(std::string name, size_t num_groups, size_t num_channels, float eps,
                     bool affine)
    : Module(std::move(name)),
      num_groups_(num_groups),
      num_channels_(num_channels),
      eps_(eps),
      affine_(affine) {
    if (num_groups == 0 || num_channels % num_groups != 0)
        throw InvalidArgument("GroupNorm: num_channels must be a multiple of num_groups");
    if (affine_) {
        weight_ = Tensor::ones({(int64_t)num_channels}, true);
        bias_ = Tensor::zeros({(int64_t)num_channels}, true);
        register_parameter("weight", weight_);
        register_parameter("bias", bias_);
    }
}

TensorPtr GroupNorm::forward(const TensorPtr& input) { return run(input, 0u); }

TensorPtr GroupNorm::run(const TensorPtr& input, unsigned flags) {
    const NCHW s = nchw_of(input);
    if (s.C != (int64_t)num_channels_)
        throw ShapeError("GroupNorm: expected " + std::to_string(num_channels_) +
                         " channels, got " + to_string(input->shape()));
    if (!input->is_cuda()) input->to_cuda();
    if (affine_) {
        weight_->to_cuda();
        bias_->to_cuda();
    }
    const int64_t G = (int64_t)num_groups_;
    const bool rg = input->requires_grad() || (affine_ && weight_->requires_grad());
    const bool record = rg && GradMode::is_enabled();
    TensorPtr out = Tensor::create(input->shape(), record, true);
    TensorPtr mean = Tensor::create({s.N * G}, false, true);
    TensorPtr rstd = Tensor::create({s.N * G}, false, true);
    TensorPtr lo = record ? Tensor::create({s.N * G}, false, true) : nullptr;
    const size_t wsb = soar_gn_workspace_bytes(s.N, s.C, s.HW, G);
    check(soar_gn_silu_forward(input->cuda_data(), dptr(weight_), dptr(bias_), out->cuda_data(),
                               mean->cuda_data(), rstd->cuda_data(),
                               lo ? lo->cuda_data() : nullptr, s.N, s.C, s.HW, G, eps_, flags,
                               workspace(wsb), wsb, nullptr),
          "GroupNorm forward");
    if (record) {
        auto node = std::make_shared<GroupNormNode>();
        node->input = input;
        node->weight = weight_;
        node->bias = bias_;
        node->mean = mean;
        node->rstd = rstd;
        node->mean_lo = lo;
        node->num_groups = G;
        node->flags = flags;
        out->set_grad_fn(node);
    }
    return out;
}

GNSiLU::GNSiLU(size_t num_groups, size_t num_channels, float eps, bool affine, bool residual)
    : GroupNorm("GNSiLU", num_groups, num_channels, eps, affine), residual_(residual) {}

TensorPtr GNSiLU::forward(const TensorPtr& input) {
    return run(input, SOAR_GN_SILU | (residual_ ? SOAR_GN_RESIDUAL : 0u));
}

TensorPtr SiLU::forward(const TensorPtr& input) {
    if (!input->is_cuda()) input->to_cuda();
    const bool record = input->requires_grad() && GradMode::is_enabled();
    TensorPtr out = Tensor::create(input->shape(), record, true);
    hip::kernels::silu_forward(input->cuda_data(), out->cuda_data(), (size_t)input->numel());
    if (record) {
        auto node = std::make_shared<SiLUNode>();
        node->input = input;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr add_tensors(const TensorPtr& a, const TensorPtr& b) {
    if (a->shape() != b->shape())
        throw ShapeError("Cannot add tensors with different shapes " + to_string(a->shape()) +
                         " and " + to_string(b->shape()));
    if (!a->is_cuda()) a->to_cuda();
    if (!b->is_cuda()) b->to_cuda();
    const bool record = (a->requires_grad() || b->requires_grad()) && GradMode::is_enabled();
    TensorPtr out = Tensor::create(a->shape(), record, true);
    hip::kernels::add_forward(a->cuda_data(), b->cuda_data(), out->cuda_data(),
                              (size_t)a->numel());
    if (record) {
        auto node = std::make_shared<AddNode>();
        node->a = a;
        node->b = b;
        out->set_grad_fn(node);
    }
    return out;
}

}  // namespace soar::nn
