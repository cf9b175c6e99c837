// GroupNorm / SiLU / GNSiLU / Conv2d / CBA / add_tensors on libsoar_gn.so.
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

#include <atomic>
#include <cmath>
#include <random>

#include "soar/autograd.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar_gn.h"
#include "soar_ops.h"

namespace soar::nn {

using autograd::GradMode;
using hip::kernels::check;

TensorPtr Module::forward(const TensorPtr& input) {
    return forward(std::vector<TensorPtr>{input});
}

TensorPtr Module::forward(const std::vector<TensorPtr>& inputs) {
    if (inputs.empty()) throw ShapeError("Module::forward needs at least one input tensor");
    return forward(inputs[0]);
}

void Module::register_parameter(const std::string& name, TensorPtr p) {
    params_[name] = std::move(p);
}

void Module::register_submodule(const std::string& name, std::shared_ptr<Module> m) {
    subs_[name] = std::move(m);
}

void Module::train(bool mode) {
    training_ = mode;
    for (auto& [n, m] : subs_) m->train(mode);
}

std::vector<std::pair<std::string, TensorPtr>> Module::named_parameters(
    const std::string& prefix) const {
    std::vector<std::pair<std::string, TensorPtr>> out;
    for (const auto& [n, p] : params_) out.emplace_back(prefix.empty() ? n : prefix + "." + n, p);
    for (const auto& [n, m] : subs_)
        for (auto& np : m->named_parameters(prefix.empty() ? n : prefix + "." + n))
            out.push_back(std::move(np));
    return out;
}

std::vector<TensorPtr> Module::parameters() const {
    std::vector<TensorPtr> out;
    for (auto& [n, p] : named_parameters()) out.push_back(p);
    return out;
}

void Module::to_device() {
    for (auto& [n, p] : params_) p->to_cuda();
    for (auto& [n, m] : subs_) m->to_device();
}

void Module::zero_grad() {
    for (auto& [n, p] : params_) p->zero_grad();
    for (auto& [n, m] : subs_) m->zero_grad();
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
// SOAR_GN_ACCUMULATE_DX when the kernel adds into a pending gradient (see
// write_target), 0 when it writes a fresh one.
unsigned dx_mode(const TensorPtr& gx, bool fresh) {
    return gx && !fresh ? SOAR_GN_ACCUMULATE_DX : 0u;
}

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
        bool fresh = false;
        TensorPtr gx = want_x ? write_target(input, &fresh) : nullptr;
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
                                    flags | dx_mode(gx, fresh), workspace(wsb), wsb, exec::stream()),
              "GroupNorm backward");
        if (want_p && !direct) {
            propagate_grad(weight, std::move(gw));
            propagate_grad(bias, std::move(gb));
        }
        if (want_x && fresh) propagate_grad(input, std::move(gx));
    }

    void release_variables() override {
        input = nullptr;
        mean = rstd = mean_lo = nullptr;
    }
};

// Gradient buffer of parameter `p` for a kernel that accumulates (+=):
// its existing device .grad when p is a leaf that has one (no temporary,
// no merge pass), else fresh zeros that the caller propagates.
// SOAR_DEFER_WEIGHT_FINISH when the weight gradients of a backward call all
// land in the parameters' own gradient buffers (direct): their final
// addition then joins the single launch the backward pass ends with
// (run_backward's soar_weight_grad_flush), and nothing reads those buffers
// before it.  A fresh gradient tensor is handed on by propagate_grad right
// after the call, so that call finishes its sums at once.
unsigned defer_finish(bool deferrable) { return deferrable ? SOAR_DEFER_WEIGHT_FINISH : 0u; }

TensorPtr param_grad_target(const TensorPtr& p, bool* direct) {
    if (!p->grad_fn() && p->grad() && p->grad()->is_cuda()) {
        *direct = true;
        return p->grad();
    }
    *direct = false;
    return Tensor::zeros(p->shape(), false, true);
}

struct ConvGeom {
    int64_t N, C_in, H, W, C_out, Ho, Wo;
};

ConvGeom conv_geom(const TensorPtr& x, const Conv2d& c) {
    ConvGeom g{};
    if (x->ndim() == 3) {
        g.N = 1;
        g.C_in = x->dim(0);
        g.H = x->dim(1);
        g.W = x->dim(2);
    } else if (x->ndim() == 4) {
        g.N = x->dim(0);
        g.C_in = x->dim(1);
        g.H = x->dim(2);
        g.W = x->dim(3);
    } else {
        throw ShapeError("Conv2d expects [C,H,W] or [N,C,H,W], got " + to_string(x->shape()));
    }
    if (g.C_in != (int64_t)c.in_channels())
        throw ShapeError("Conv2d: expected " + std::to_string(c.in_channels()) +
                         " input channels, got " + to_string(x->shape()));
    const int64_t ek = (int64_t)(c.dilation() * (c.kernel_size() - 1) + 1);
    const int64_t p2 = 2 * (int64_t)c.padding();
    if (g.H + p2 < ek || g.W + p2 < ek)
        throw ShapeError("Conv2d: input " + to_string(x->shape()) + " is smaller than the kernel");
    g.C_out = (int64_t)c.out_channels();
    g.Ho = (g.H + p2 - ek) / (int64_t)c.stride() + 1;
    g.Wo = (g.W + p2 - ek) / (int64_t)c.stride() + 1;
    return g;
}

Shape conv_out_shape(const TensorPtr& x, const ConvGeom& g) {
    if (x->ndim() == 3) return {g.C_out, g.Ho, g.Wo};
    return {g.N, g.C_out, g.Ho, g.Wo};
}

// Backward of Conv2d (layers.cpp:17-292): dx written fresh, dW and db
// accumulated by the kernels.
enum class ConvKind { Pointwise, Depthwise, General };

struct Conv2dNode : autograd::AutogradNode {
    TensorPtr input, weight, bias;
    ConvGeom g{};
    int64_t K = 1, pad = 0, stride = 1, dil = 1, groups = 1;
    ConvKind kind = ConvKind::Pointwise;

    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : {input, weight, bias})
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }

    void backward(const TensorPtr& go) override {
        const bool want_x = input->requires_grad();
        const bool want_w = weight->requires_grad();
        const bool want_b = bias && bias->requires_grad();
        if (!want_x && !want_w && !want_b) return;
        if (!go->is_cuda()) go->to_cuda();
        bool fresh = false;
        TensorPtr gx = want_x ? write_target(input, &fresh) : nullptr;
        const unsigned fl = dx_mode(gx, fresh);
        bool dw_direct = false, db_direct = false;
        TensorPtr gw = want_w ? param_grad_target(weight, &dw_direct) : nullptr;
        TensorPtr gb = want_b ? param_grad_target(bias, &db_direct) : nullptr;
        float* px = gx ? gx->cuda_data() : nullptr;
        float* pw = gw ? gw->cuda_data() : nullptr;
        float* pb = gb ? gb->cuda_data() : nullptr;
        const unsigned dfl = defer_finish((!gw || dw_direct) && (!gb || db_direct));
        if (kind == ConvKind::Pointwise) {
            const size_t wsb =
                soar_pw_conv_backward_workspace_bytes(g.N, g.C_in, g.C_out, g.H * g.W);
            check(soar_pw_conv_backward(go->cuda_data(), input->cuda_data(), weight->cuda_data(),
                                        px, pw, pb, g.N, g.C_in, g.C_out, g.H * g.W, fl | dfl,
                                        workspace(wsb), wsb, exec::stream()),
                  "pointwise convolution backward");
        } else if (kind == ConvKind::General) {
            const size_t wsb = soar_conv_backward_workspace_bytes(
                g.N, g.C_in, g.C_out, g.H, g.W, g.Ho, g.Wo, K, pad, stride, dil, groups);
            check(soar_conv_backward(go->cuda_data(), input->cuda_data(), weight->cuda_data(), px,
                                     pw, pb, g.N, g.C_in, g.C_out, g.H, g.W, g.Ho, g.Wo, K, pad,
                                     stride, dil, groups, fl, workspace(wsb), wsb, exec::stream()),
                  "convolution backward");
        } else {
            const size_t wsb = soar_dw_conv_backward_workspace_bytes(g.N, g.C_in, g.H, g.W, g.Ho,
                                                                     g.Wo, K, stride, dil);
            check(soar_dw_conv_backward(go->cuda_data(), input->cuda_data(), weight->cuda_data(),
                                        px, pw, pb, g.N, g.C_in, g.H, g.W, g.Ho, g.Wo, K, pad,
                                        stride, dil, fl | dfl, wsb ? workspace(wsb) : nullptr, wsb,
                                        exec::stream()),
                  "depthwise convolution backward");
        }
        if (gb && !db_direct) propagate_grad(bias, std::move(gb));
        if (gw && !dw_direct) propagate_grad(weight, std::move(gw));
        if (gx && fresh) propagate_grad(input, std::move(gx));
    }

    void release_variables() override { input = nullptr; }
};

// Backward of the fused pointwise CBA: the GroupNorm(+SiLU) backward at the
// saved conv output z and the conv backward in one call
// (soar_pw_cba_backward: above its size switch one kernel forms dz in
// registers and never stores it).
struct CBAPointwiseNode : autograd::AutogradNode {
    TensorPtr input, conv_w, gamma, beta, z, mean, rstd, mean_lo;
    ConvGeom g{};
    int64_t G = 1;
    unsigned flags = 0;

    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : {input, conv_w, gamma, beta})
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }

    void backward(const TensorPtr& go) override {
        const bool want_x = input->requires_grad();
        const bool want_w = conv_w->requires_grad();
        const bool want_p = gamma && gamma->requires_grad();
        if (!want_x && !want_w && !want_p) return;
        if (!go->is_cuda()) go->to_cuda();
        const int64_t HW = g.H * g.W;
        bool g_direct = false, b_direct = false, w_direct = false, fresh = false;
        TensorPtr dg = want_p ? param_grad_target(gamma, &g_direct) : nullptr;
        TensorPtr db = want_p ? param_grad_target(beta, &b_direct) : nullptr;
        TensorPtr gx = want_x ? write_target(input, &fresh) : nullptr;
        TensorPtr gw = want_w ? param_grad_target(conv_w, &w_direct) : nullptr;
        const size_t wsb = soar_pw_cba_backward_workspace_bytes(g.N, g.C_in, g.C_out, HW, G);
        check(soar_pw_cba_backward(go->cuda_data(), z->cuda_data(), input->cuda_data(),
                                   conv_w->cuda_data(), dptr(gamma), dptr(beta),
                                   mean->cuda_data(), rstd->cuda_data(), dptr(mean_lo),
                                   gx ? gx->cuda_data() : nullptr,
                                   gw ? gw->cuda_data() : nullptr,
                                   dg ? dg->cuda_data() : nullptr,
                                   db ? db->cuda_data() : nullptr, g.N, g.C_in, g.C_out, HW, G,
                                   (flags & SOAR_GN_SILU) | dx_mode(gx, fresh) |
                                       defer_finish(!gw || w_direct),
                                   workspace(wsb), wsb, exec::stream()),
              "CBA backward");
        if (dg && !g_direct) propagate_grad(gamma, std::move(dg));
        if (db && !b_direct) propagate_grad(beta, std::move(db));
        if (gw && !w_direct) propagate_grad(conv_w, std::move(gw));
        if (gx && fresh) propagate_grad(input, std::move(gx));
    }

    void release_variables() override {
        input = nullptr;
        z = mean = rstd = mean_lo = nullptr;
    }
};

// Backward of a CBA block with a depthwise conv: the GroupNorm(+SiLU)
// backward at the saved conv output z and the conv backward in one call
// (soar_dw_cba_backward: for stride 1 with "same" padding, one kernel forms
// dz over each tile in LDS and never stores it).
struct CBADepthwiseNode : autograd::AutogradNode {
    TensorPtr input, conv_w, gamma, beta, z, mean, rstd, mean_lo;
    ConvGeom g{};
    int64_t K = 1, pad = 0, stride = 1, dil = 1, G = 1;
    unsigned flags = 0;

    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : {input, conv_w, gamma, beta})
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }

    void backward(const TensorPtr& go) override {
        const bool want_x = input->requires_grad();
        const bool want_w = conv_w->requires_grad();
        const bool want_p = gamma && gamma->requires_grad();
        if (!want_x && !want_w && !want_p) return;
        if (!go->is_cuda()) go->to_cuda();
        bool g_direct = false, b_direct = false, w_direct = false, fresh = false;
        TensorPtr dg = want_p ? param_grad_target(gamma, &g_direct) : nullptr;
        TensorPtr db = want_p ? param_grad_target(beta, &b_direct) : nullptr;
        TensorPtr gx = want_x ? write_target(input, &fresh) : nullptr;
        TensorPtr gw = want_w ? param_grad_target(conv_w, &w_direct) : nullptr;
        const size_t wsb = soar_dw_cba_backward_workspace_bytes(g.N, g.C_in, g.H, g.W, g.Ho,
                                                                g.Wo, K, pad, stride, dil, G);
        check(soar_dw_cba_backward(go->cuda_data(), z->cuda_data(), input->cuda_data(),
                                   conv_w->cuda_data(), dptr(gamma), dptr(beta),
                                   mean->cuda_data(), rstd->cuda_data(), dptr(mean_lo),
                                   gx ? gx->cuda_data() : nullptr,
                                   gw ? gw->cuda_data() : nullptr,
                                   dg ? dg->cuda_data() : nullptr,
                                   db ? db->cuda_data() : nullptr, g.N, g.C_in, g.H, g.W, g.Ho,
                                   g.Wo, K, pad, stride, dil, G,
                                   (flags & SOAR_GN_SILU) | dx_mode(gx, fresh) |
                                       defer_finish(!gw || w_direct),
                                   workspace(wsb), wsb, exec::stream()),
              "depthwise CBA backward");
        if (dg && !g_direct) propagate_grad(gamma, std::move(dg));
        if (db && !b_direct) propagate_grad(beta, std::move(db));
        if (gw && !w_direct) propagate_grad(conv_w, std::move(gw));
        if (gx && fresh) propagate_grad(input, std::move(gx));
    }

    void release_variables() override {
        input = nullptr;
        z = mean = rstd = mean_lo = nullptr;
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
        bool fresh = false;
        TensorPtr gx = add_target(input, &fresh);
        hip::kernels::silu_backward(go->cuda_data(), input->cuda_data(), gx->cuda_data(),
                                    (size_t)input->numel());
        if (fresh) propagate_grad(input, std::move(gx));
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
    // go goes to both inputs unchanged.  Inputs whose pending gradient may
    // be added into directly get go added there, both in one launch; the
    // others receive go itself (kept by reference, no copy).
    void backward(const TensorPtr& go) override {
        TensorPtr sa = grad_sink(a);
        TensorPtr sb = grad_sink(b);  // (null when b is a and sa holds its sink)
        if (sa || sb) {
            if (!go->is_cuda()) go->to_cuda();
            hip::kernels::add_backward(go->cuda_data(), sa ? sa->cuda_data() : nullptr,
                                       sb ? sb->cuda_data() : nullptr, (size_t)go->numel());
        }
        if (a && !sa) propagate_grad(a, go);
        if (b && !sb) propagate_grad(b, go);
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
                               workspace(wsb), wsb, exec::stream()),
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

namespace {
std::atomic<uint64_t> g_init_counter{0x50a4c0deull};

// splitmix64 of a process-wide counter
uint64_t next_init_seed() {
    uint64_t z = (g_init_counter.fetch_add(1) + 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
}  // namespace

void set_init_seed(uint64_t seed) { g_init_counter.store(seed); }

Conv2d::Conv2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride,
               int padding, size_t dilation, size_t groups, bool bias, uint64_t seed)
    : Module("Conv2d"),
      in_(in_channels),
      out_(out_channels),
      kernel_(kernel_size),
      stride_(stride),
      padding_((size_t)(padding < 0 ? autopad((int)kernel_size, -1, (int)dilation) : padding)),
      dilation_(dilation),
      groups_(groups) {
    if (in_ == 0 || out_ == 0 || kernel_ == 0 || stride_ == 0 || dilation_ == 0 || groups_ == 0 ||
        in_ % groups_ != 0 || out_ % groups_ != 0)
        throw InvalidArgument("Conv2d: invalid channel / kernel / stride / group arguments");
    const size_t cig = in_ / groups_;
    weight_ = Tensor::create({(int64_t)out_, (int64_t)cig, (int64_t)kernel_, (int64_t)kernel_},
                             true);
    const float bound = std::sqrt(1.0f / (float)(cig * kernel_ * kernel_));
    std::mt19937_64 gen(seed ? seed : next_init_seed());
    std::uniform_real_distribution<float> dist(-bound, bound);
    float* w = weight_->data();
    for (int64_t i = 0; i < weight_->numel(); ++i) w[i] = dist(gen);
    register_parameter("weight", weight_);
    if (bias) {
        bias_ = Tensor::zeros({(int64_t)out_}, true);
        register_parameter("bias", bias_);
    }
}

TensorPtr Conv2d::forward(const TensorPtr& input) {
    const ConvGeom g = conv_geom(input, *this);
    if (!input->is_cuda()) input->to_cuda();
    weight_->to_cuda();
    if (bias_) bias_->to_cuda();
    const bool record = (input->requires_grad() || weight_->requires_grad() ||
                         (bias_ && bias_->requires_grad())) &&
                        GradMode::is_enabled();
    TensorPtr out = Tensor::create(conv_out_shape(input, g), record, true);
    const ConvKind kind = pointwise()   ? ConvKind::Pointwise
                          : depthwise() ? ConvKind::Depthwise
                                        : ConvKind::General;
    if (kind == ConvKind::Pointwise) {
        check(soar_pw_conv_forward(input->cuda_data(), weight_->cuda_data(), dptr(bias_),
                                   out->cuda_data(), g.N, g.C_in, g.C_out, g.H * g.W, exec::stream()),
              "pointwise convolution");
    } else if (kind == ConvKind::General) {
        check(soar_conv_forward(input->cuda_data(), weight_->cuda_data(), dptr(bias_),
                                out->cuda_data(), g.N, g.C_in, g.C_out, g.H, g.W, g.Ho, g.Wo,
                                (int64_t)kernel_, (int64_t)padding_, (int64_t)stride_,
                                (int64_t)dilation_, (int64_t)groups_, exec::stream()),
              "convolution");
    } else {
        check(soar_dw_conv_forward(input->cuda_data(), weight_->cuda_data(), dptr(bias_),
                                   out->cuda_data(), g.N, g.C_in, g.H, g.W, g.Ho, g.Wo,
                                   (int64_t)kernel_, (int64_t)padding_, (int64_t)stride_,
                                   (int64_t)dilation_, exec::stream()),
              "depthwise convolution");
    }
    if (record) {
        auto node = std::make_shared<Conv2dNode>();
        node->input = input;
        node->weight = weight_;
        node->bias = bias_;
        node->g = g;
        node->K = (int64_t)kernel_;
        node->pad = (int64_t)padding_;
        node->stride = (int64_t)stride_;
        node->dil = (int64_t)dilation_;
        node->groups = (int64_t)groups_;
        node->kind = kind;
        out->set_grad_fn(node);
    }
    return out;
}

CBA::CBA(size_t c1, size_t c2, size_t k, size_t s, int p, size_t d, size_t g, bool act)
    : Module("CBA"), act_(act) {
    conv_ = std::make_shared<Conv2d>(c1, c2, k, s, p, d, g, false);
    norm_ = std::make_shared<GroupNorm>((size_t)select_group_count((int)c2), c2);
    register_submodule("conv", conv_);
    register_submodule("norm", norm_);
}

TensorPtr CBA::forward(const TensorPtr& input) {
    const unsigned flags = act_ ? SOAR_GN_SILU : 0u;
    if (conv_->depthwise() && !conv_->pointwise()) return forward_depthwise(input, flags);
    if (!conv_->pointwise()) return norm_->run(conv_->forward(input), flags);
    // pointwise conv: one call, the GroupNorm statistics from the conv epilogue
    const ConvGeom g = conv_geom(input, *conv_);
    if (!input->is_cuda()) input->to_cuda();
    const TensorPtr w = conv_->weight();
    const TensorPtr gamma = norm_->weight(), beta = norm_->bias();
    w->to_cuda();
    if (gamma) {
        gamma->to_cuda();
        beta->to_cuda();
    }
    const int64_t G = (int64_t)norm_->num_groups(), HW = g.H * g.W;
    const bool record = (input->requires_grad() || w->requires_grad() ||
                         (gamma && gamma->requires_grad())) &&
                        GradMode::is_enabled();
    const Shape os = conv_out_shape(input, g);
    TensorPtr z = Tensor::create(os, false, true);
    TensorPtr y = Tensor::create(os, record, true);
    TensorPtr mean = Tensor::create({g.N * G}, false, true);
    TensorPtr rstd = Tensor::create({g.N * G}, false, true);
    TensorPtr lo = Tensor::create({g.N * G}, false, true);
    const size_t wsb = soar_pw_conv_gn_workspace_bytes(g.N, g.C_out, HW, G);
    check(soar_pw_conv_gn_silu_forward(input->cuda_data(), w->cuda_data(), nullptr, dptr(gamma),
                                       dptr(beta), z->cuda_data(), y->cuda_data(),
                                       mean->cuda_data(), rstd->cuda_data(), lo->cuda_data(), g.N,
                                       g.C_in, g.C_out, HW, G, norm_->eps(), flags,
                                       workspace(wsb), wsb, exec::stream()),
          "CBA forward");
    if (record) {
        auto node = std::make_shared<CBAPointwiseNode>();
        node->input = input;
        node->conv_w = w;
        node->gamma = gamma;
        node->beta = beta;
        node->z = z;
        node->mean = mean;
        node->rstd = rstd;
        node->mean_lo = lo;
        node->g = g;
        node->G = G;
        node->flags = flags;
        y->set_grad_fn(node);
    }
    return y;
}

// residual + forward(input) with the add done by the GroupNorm's apply pass
// (soar_pw_conv_gn_silu_add_forward) for a pointwise conv; recorded as the
// CBA node and an add node, as add_tensors(residual, forward(input)) would
// be (the CBA output tensor is allocated but never written: the add node
// only routes the gradient through it).
TensorPtr CBA::forward_residual(const TensorPtr& input, const TensorPtr& residual) {
    if (!conv_->pointwise()) return add_tensors(residual, forward(input));
    const unsigned flags = act_ ? SOAR_GN_SILU : 0u;
    const ConvGeom g = conv_geom(input, *conv_);
    if (!input->is_cuda()) input->to_cuda();
    if (!residual->is_cuda()) residual->to_cuda();
    const TensorPtr w = conv_->weight();
    const TensorPtr gamma = norm_->weight(), beta = norm_->bias();
    w->to_cuda();
    if (gamma) {
        gamma->to_cuda();
        beta->to_cuda();
    }
    const int64_t G = (int64_t)norm_->num_groups(), HW = g.H * g.W;
    const bool record_cba = (input->requires_grad() || w->requires_grad() ||
                             (gamma && gamma->requires_grad())) &&
                            GradMode::is_enabled();
    const bool record = (record_cba || residual->requires_grad()) && GradMode::is_enabled();
    const Shape os = conv_out_shape(input, g);
    if (residual->shape() != os)
        throw ShapeError("Cannot add tensors with different shapes " +
                         to_string(residual->shape()) + " and " + to_string(os));
    TensorPtr z = Tensor::create(os, false, true);
    TensorPtr y = Tensor::create(os, record, true);
    TensorPtr mean = Tensor::create({g.N * G}, false, true);
    TensorPtr rstd = Tensor::create({g.N * G}, false, true);
    TensorPtr lo = Tensor::create({g.N * G}, false, true);
    const size_t wsb = soar_pw_conv_gn_workspace_bytes(g.N, g.C_out, HW, G);
    check(soar_pw_conv_gn_silu_add_forward(
              input->cuda_data(), w->cuda_data(), nullptr, dptr(gamma), dptr(beta),
              residual->cuda_data(), z->cuda_data(), y->cuda_data(), mean->cuda_data(),
              rstd->cuda_data(), lo->cuda_data(), g.N, g.C_in, g.C_out, HW, G, norm_->eps(),
              flags, workspace(wsb), wsb, exec::stream()),
          "CBA forward + residual");
    if (record) {
        TensorPtr cba_out;  // the CBA's own output: only its gradient flows through it
        if (record_cba) {
            cba_out = Tensor::create(os, true, true);
            auto node = std::make_shared<CBAPointwiseNode>();
            node->input = input;
            node->conv_w = w;
            node->gamma = gamma;
            node->beta = beta;
            node->z = z;
            node->mean = mean;
            node->rstd = rstd;
            node->mean_lo = lo;
            node->g = g;
            node->G = G;
            node->flags = flags;
            cba_out->set_grad_fn(node);
        }
        auto add = std::make_shared<AddNode>();
        add->a = residual;
        add->b = cba_out;
        y->set_grad_fn(add);
    }
    return y;
}

// Depthwise conv: the conv and the GroupNorm forward, recorded as one node
// whose backward is soar_dw_cba_backward.
TensorPtr CBA::forward_depthwise(const TensorPtr& input, unsigned flags) {
    const ConvGeom g = conv_geom(input, *conv_);
    if (!input->is_cuda()) input->to_cuda();
    const TensorPtr w = conv_->weight();
    const TensorPtr gamma = norm_->weight(), beta = norm_->bias();
    w->to_cuda();
    if (gamma) {
        gamma->to_cuda();
        beta->to_cuda();
    }
    const int64_t G = (int64_t)norm_->num_groups();
    const int64_t K = (int64_t)conv_->kernel_size(), pad = (int64_t)conv_->padding();
    const int64_t S = (int64_t)conv_->stride(), D = (int64_t)conv_->dilation();
    const bool record = (input->requires_grad() || w->requires_grad() ||
                         (gamma && gamma->requires_grad())) &&
                        GradMode::is_enabled();
    const Shape os = conv_out_shape(input, g);
    TensorPtr z = Tensor::create(os, false, true);
    TensorPtr y = Tensor::create(os, record, true);
    TensorPtr mean = Tensor::create({g.N * G}, false, true);
    TensorPtr rstd = Tensor::create({g.N * G}, false, true);
    TensorPtr lo = Tensor::create({g.N * G}, false, true);
    // the GroupNorm statistics come from the convolution's epilogue
    const size_t wsb =
        soar_dw_conv_gn_workspace_bytes(g.N, g.C_in, g.H, g.W, g.Ho, g.Wo, K, pad, S, D, G);
    check(soar_dw_conv_gn_silu_forward(input->cuda_data(), w->cuda_data(), nullptr, dptr(gamma),
                                       dptr(beta), z->cuda_data(), y->cuda_data(),
                                       mean->cuda_data(), rstd->cuda_data(), lo->cuda_data(),
                                       g.N, g.C_in, g.H, g.W, g.Ho, g.Wo, K, pad, S, D, G,
                                       norm_->eps(), flags, workspace(wsb), wsb, exec::stream()),
          "CBA depthwise forward");
    if (record) {
        auto node = std::make_shared<CBADepthwiseNode>();
        node->input = input;
        node->conv_w = w;
        node->gamma = gamma;
        node->beta = beta;
        node->z = z;
        node->mean = mean;
        node->rstd = rstd;
        node->mean_lo = lo;
        node->g = g;
        node->K = K;
        node->pad = pad;
        node->stride = S;
        node->dil = D;
        node->G = G;
        node->flags = flags;
        y->set_grad_fn(node);
    }
    return y;
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
