// Sigmoid / PixelShuffle / Upsample / AdaptiveAvgPool2d and the tensor
// helpers of the SOAR blocks (mul_tensors, convex_combination,
// concat_channels, resize_bilinear) on libsoar_gn.so.
//
// Structure follows src/nn/layers.cpp:807-1345 and src/nn/blocks.cpp:
// 75-427 of the reference: each op allocates its output on the device,
// runs one operator of include/soar_ops.h, and records a node when the
// output requires grad and grad mode is on.  Gradients of the operators
// are accumulated into zero-filled buffers, as the reference's kernels do.
// Inputs are [C,H,W] (the reference's layout) or [N,C,H,W].
#include <algorithm>
#include <cmath>

#include "soar/autograd.hpp"
#include "soar/kernels.hpp"
#include "soar/nn.hpp"
#include "soar_gn.h"
#include "soar_ops.h"

namespace soar::nn {

using autograd::GradMode;
using hip::kernels::check;

namespace {

struct Planes {
    int64_t rows, H, W;
};

Planes planes_of(const TensorPtr& t, const char* what) {
    if (t->ndim() == 3) return {t->dim(0), t->dim(1), t->dim(2)};
    if (t->ndim() == 4) return {t->dim(0) * t->dim(1), t->dim(2), t->dim(3)};
    throw ShapeError(std::string(what) + " expects [C,H,W] or [N,C,H,W], got " +
                     to_string(t->shape()));
}

void to_dev(const TensorPtr& t) {
    if (t && !t->is_cuda()) t->to_cuda();
}

bool wants(const TensorPtr& t) { return t && t->requires_grad(); }

// Flags of the _ex backward entry points: add into a pending gradient,
// write a fresh one.
unsigned mode(bool fresh) { return fresh ? 0u : SOAR_GN_ACCUMULATE_DX; }

// One mode for a kernel with several gradient outputs (null ones ignored):
// write when every output is fresh, else zero the fresh ones and add.
unsigned joint_mode(std::initializer_list<std::pair<const TensorPtr*, bool>> outs) {
    bool all_fresh = true;
    for (const auto& [t, fresh] : outs)
        if (*t && !fresh) all_fresh = false;
    if (all_fresh) return 0u;
    for (const auto& [t, fresh] : outs)
        if (*t && fresh) (*t)->zero_();
    return SOAR_GN_ACCUMULATE_DX;
}

// ---- nodes ------------------------------------------------------------------
struct SigmoidNode : autograd::AutogradNode {
    TensorPtr input, output;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        if (input && input->grad_fn()) return {input->grad_fn()};
        return {};
    }
    void backward(const TensorPtr& go) override {
        if (!wants(input)) return;
        to_dev(go);
        bool fresh = false;
        TensorPtr gx = write_target(input, &fresh);
        check(soar_sigmoid_backward_ex(go->cuda_data(), output->cuda_data(), gx->cuda_data(),
                                       (size_t)input->numel(), mode(fresh), exec::stream()),
              "sigmoid backward");
        if (fresh) propagate_grad(input, std::move(gx));
    }
    void release_variables() override { input = output = nullptr; }
};

struct PixelShuffleNode : autograd::AutogradNode {
    TensorPtr input;
    int64_t r = 2;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        if (input && input->grad_fn()) return {input->grad_fn()};
        return {};
    }
    void backward(const TensorPtr& go) override {
        if (!wants(input)) return;
        to_dev(go);
        const Planes p = planes_of(input, "PixelShuffle");
        bool fresh = false;
        TensorPtr gx = write_target(input, &fresh);
        check(soar_pixel_shuffle_backward_ex(go->cuda_data(), gx->cuda_data(), (size_t)p.rows,
                                             (size_t)p.H, (size_t)p.W, (size_t)r, mode(fresh),
                                             exec::stream()),
              "pixel shuffle backward");
        if (fresh) propagate_grad(input, std::move(gx));
    }
    void release_variables() override { input = nullptr; }
};

struct UpsampleNode : autograd::AutogradNode {
    TensorPtr input;
    int64_t H_out = 0, W_out = 0;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        if (input && input->grad_fn()) return {input->grad_fn()};
        return {};
    }
    void backward(const TensorPtr& go) override {
        if (!wants(input)) return;
        to_dev(go);
        const Planes p = planes_of(input, "Upsample");
        bool fresh = false;
        TensorPtr gx = write_target(input, &fresh);
        check(soar_upsample_bilinear_backward_ex(go->cuda_data(), gx->cuda_data(),
                                                 (size_t)p.rows, (size_t)p.H, (size_t)p.W,
                                                 (size_t)H_out, (size_t)W_out, mode(fresh),
                                                 exec::stream()),
              "upsample backward");
        if (fresh) propagate_grad(input, std::move(gx));
    }
    void release_variables() override { input = nullptr; }
};

struct AvgPoolNode : autograd::AutogradNode {
    TensorPtr input;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        if (input && input->grad_fn()) return {input->grad_fn()};
        return {};
    }
    void backward(const TensorPtr& go) override {
        if (!wants(input)) return;
        to_dev(go);
        const Planes p = planes_of(input, "AdaptiveAvgPool2d");
        bool fresh = false;
        TensorPtr gx = write_target(input, &fresh);
        check(soar_global_avg_pool_backward_ex(go->cuda_data(), gx->cuda_data(),
                                               (size_t)p.rows, (size_t)(p.H * p.W), mode(fresh),
                                               exec::stream()),
              "average pool backward");
        if (fresh) propagate_grad(input, std::move(gx));
    }
    void release_variables() override { input = nullptr; }
};

struct MulBroadcastNode : autograd::AutogradNode {
    TensorPtr a, b;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        if (a && a->grad_fn()) r.push_back(a->grad_fn());
        if (b && b->grad_fn()) r.push_back(b->grad_fn());
        return r;
    }
    void backward(const TensorPtr& go) override {
        const bool wa = wants(a), wb = wants(b);
        if (!wa && !wb) return;
        to_dev(go);
        const Planes p = planes_of(a, "mul_tensors");
        bool fa = false, fb = false;
        TensorPtr ga = wa ? write_target(a, &fa) : nullptr;
        TensorPtr gb = wb ? write_target(b, &fb) : nullptr;
        const unsigned fl = joint_mode({{&ga, fa}, {&gb, fb}});
        check(soar_mul_broadcast_backward_ex(go->cuda_data(), a->cuda_data(), b->cuda_data(),
                                             ga ? ga->cuda_data() : nullptr,
                                             gb ? gb->cuda_data() : nullptr, (size_t)p.rows,
                                             (size_t)(p.H * p.W), fl, exec::stream()),
              "mul_broadcast backward");
        if (ga && fa) propagate_grad(a, std::move(ga));
        if (gb && fb) propagate_grad(b, std::move(gb));
    }
    void release_variables() override { a = b = nullptr; }
};

struct ConvexNode : autograd::AutogradNode {
    TensorPtr g, a, b;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : {g, a, b})
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }
    void backward(const TensorPtr& go) override {
        const bool wg = wants(g), wa = wants(a), wb = wants(b);
        if (!wg && !wa && !wb) return;
        to_dev(go);
        bool fg = false, fa = false, fb = false;
        TensorPtr gg = wg ? write_target(g, &fg) : nullptr;
        TensorPtr ga = wa ? write_target(a, &fa) : nullptr;
        TensorPtr gb = wb ? write_target(b, &fb) : nullptr;
        const unsigned fl = joint_mode({{&gg, fg}, {&ga, fa}, {&gb, fb}});
        check(soar_convex_combination_backward_ex(
                  go->cuda_data(), g->cuda_data(), a->cuda_data(), b->cuda_data(),
                  gg ? gg->cuda_data() : nullptr, ga ? ga->cuda_data() : nullptr,
                  gb ? gb->cuda_data() : nullptr, (size_t)a->numel(), fl, exec::stream()),
              "convex combination backward");
        // the reference's order (blocks.cpp:258-262): a, b, then g
        if (ga && fa) propagate_grad(a, std::move(ga));
        if (gb && fb) propagate_grad(b, std::move(gb));
        if (gg && fg) propagate_grad(g, std::move(gg));
    }
    void release_variables() override { g = a = b = nullptr; }
};

struct SigmoidConvexNode : autograd::AutogradNode {
    TensorPtr z, a, b;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : {z, a, b})
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }
    void backward(const TensorPtr& go) override {
        const bool wz = wants(z), wa = wants(a), wb = wants(b);
        if (!wz && !wa && !wb) return;
        to_dev(go);
        bool fz = false, fa = false, fb = false;
        TensorPtr gz = wz ? write_target(z, &fz) : nullptr;
        TensorPtr ga = wa ? write_target(a, &fa) : nullptr;
        TensorPtr gb = wb ? write_target(b, &fb) : nullptr;
        const unsigned fl = joint_mode({{&gz, fz}, {&ga, fa}, {&gb, fb}});
        check(soar_sigmoid_convex_backward_ex(
                  go->cuda_data(), z->cuda_data(), a->cuda_data(), b->cuda_data(),
                  gz ? gz->cuda_data() : nullptr, ga ? ga->cuda_data() : nullptr,
                  gb ? gb->cuda_data() : nullptr, (size_t)a->numel(), fl, exec::stream()),
              "sigmoid convex combination backward");
        // ConvexNode's order, the gate's (through its sigmoid) last
        if (ga && fa) propagate_grad(a, std::move(ga));
        if (gb && fb) propagate_grad(b, std::move(gb));
        if (gz && fz) propagate_grad(z, std::move(gz));
    }
    void release_variables() override { z = a = b = nullptr; }
};

struct MulSigmoidNode : autograd::AutogradNode {
    TensorPtr a, z;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        if (a && a->grad_fn()) r.push_back(a->grad_fn());
        if (z && z->grad_fn()) r.push_back(z->grad_fn());
        return r;
    }
    void backward(const TensorPtr& go) override {
        const bool wa = wants(a), wz = wants(z);
        if (!wa && !wz) return;
        to_dev(go);
        const Planes p = planes_of(a, "mul_sigmoid");
        bool fa = false, fz = false;
        TensorPtr ga = wa ? write_target(a, &fa) : nullptr;
        TensorPtr gz = wz ? write_target(z, &fz) : nullptr;
        const unsigned fl = joint_mode({{&ga, fa}, {&gz, fz}});
        check(soar_mul_sigmoid_broadcast_backward_ex(
                  go->cuda_data(), a->cuda_data(), z->cuda_data(), ga ? ga->cuda_data() : nullptr,
                  gz ? gz->cuda_data() : nullptr, (size_t)p.rows, (size_t)(p.H * p.W), fl,
                  exec::stream()),
              "mul_sigmoid backward");
        if (ga && fa) propagate_grad(a, std::move(ga));
        if (gz && fz) propagate_grad(z, std::move(gz));
    }
    void release_variables() override { a = z = nullptr; }
};

struct ConcatNode : autograd::AutogradNode {
    std::vector<TensorPtr> inputs;
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        std::vector<std::shared_ptr<AutogradNode>> r;
        for (const auto& t : inputs)
            if (t && t->grad_fn()) r.push_back(t->grad_fn());
        return r;
    }
    void backward(const TensorPtr& go) override {
        to_dev(go);
        const bool batched = go->ndim() == 4;
        const int64_t N = batched ? go->dim(0) : 1;
        const int64_t HW = go->dim(-1) * go->dim(-2);
        const size_t K = inputs.size();
        if (K > 16) throw ShapeError("concat_channels: at most 16 tensors");
        std::vector<TensorPtr> gi(K);
        std::vector<float*> ptr(K, nullptr);
        std::vector<int64_t> ch(K);
        std::vector<unsigned> fl(K, 0u);
        std::vector<bool> fresh(K, false);
        for (size_t k = 0; k < K; ++k) {
            const TensorPtr& t = inputs[k];
            ch[k] = batched ? t->dim(1) : t->dim(0);
            if (!wants(t)) continue;
            bool f = false;
            gi[k] = write_target(t, &f);
            fresh[k] = f;
            fl[k] = mode(f);
            ptr[k] = gi[k]->cuda_data();
        }
        check(soar_concat_channels_backward(go->cuda_data(), ptr.data(), ch.data(), fl.data(),
                                            (int)K, N, HW, exec::stream()),
              "concat backward");
        for (size_t k = 0; k < K; ++k)
            if (gi[k] && fresh[k]) propagate_grad(inputs[k], std::move(gi[k]));
    }
    void release_variables() override { inputs.clear(); }
};

bool recording(std::initializer_list<TensorPtr> ts) {
    if (!GradMode::is_enabled()) return false;
    for (const auto& t : ts)
        if (t && t->requires_grad()) return true;
    return false;
}

}  // namespace

TensorPtr Sigmoid::forward(const TensorPtr& input) {
    to_dev(input);
    const bool record = recording({input});
    TensorPtr out = Tensor::create(input->shape(), record, true);
    check(soar_sigmoid_forward(input->cuda_data(), out->cuda_data(), (size_t)input->numel(),
                               exec::stream()),
          "sigmoid");
    if (record) {
        auto node = std::make_shared<SigmoidNode>();
        node->input = input;
        node->output = out;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr PixelShuffle::forward(const TensorPtr& input) {
    const Planes p = planes_of(input, "PixelShuffle");
    const int64_t r = (int64_t)r_, r2 = r * r;
    const int64_t C_in = input->ndim() == 4 ? input->dim(1) : input->dim(0);
    if (r <= 0 || C_in % r2 != 0)
        throw ShapeError("PixelShuffle: the channel count is not a multiple of r*r");
    to_dev(input);
    Shape os = input->shape();
    const size_t cdim = input->ndim() == 4 ? 1 : 0;
    os[cdim] = C_in / r2;
    os[cdim + 1] = p.H * r;
    os[cdim + 2] = p.W * r;
    const bool record = recording({input});
    TensorPtr out = Tensor::create(os, record, true);
    check(soar_pixel_shuffle_forward(input->cuda_data(), out->cuda_data(), (size_t)p.rows,
                                     (size_t)p.H, (size_t)p.W, (size_t)r, exec::stream()),
          "pixel shuffle");
    if (record) {
        auto node = std::make_shared<PixelShuffleNode>();
        node->input = input;
        node->r = r;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr Upsample::forward(const TensorPtr& input) {
    const Planes p = planes_of(input, "Upsample");
    // layers.cpp:1078-1079: round(H_in * scale) in float
    const int64_t H_out = (int64_t)std::round((float)p.H * scale_);
    const int64_t W_out = (int64_t)std::round((float)p.W * scale_);
    if (H_out <= 0 || W_out <= 0) throw ShapeError("Upsample: empty output");
    to_dev(input);
    Shape os = input->shape();
    os[os.size() - 2] = H_out;
    os[os.size() - 1] = W_out;
    const bool record = recording({input});
    TensorPtr out = Tensor::create(os, record, true);
    check(soar_upsample_bilinear_forward(input->cuda_data(), out->cuda_data(), (size_t)p.rows,
                                         (size_t)p.H, (size_t)p.W, (size_t)H_out, (size_t)W_out,
                                         exec::stream()),
          "upsample");
    if (record) {
        auto node = std::make_shared<UpsampleNode>();
        node->input = input;
        node->H_out = H_out;
        node->W_out = W_out;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr AdaptiveAvgPool2d::forward(const TensorPtr& input) {
    const Planes p = planes_of(input, "AdaptiveAvgPool2d");
    to_dev(input);
    Shape os = input->shape();
    os[os.size() - 2] = 1;
    os[os.size() - 1] = 1;
    const bool record = recording({input});
    TensorPtr out = Tensor::create(os, record, true);
    check(soar_global_avg_pool_forward(input->cuda_data(), out->cuda_data(), (size_t)p.rows,
                                       (size_t)(p.H * p.W), exec::stream()),
          "average pool");
    if (record) {
        auto node = std::make_shared<AvgPoolNode>();
        node->input = input;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr mul_tensors(const TensorPtr& a, const TensorPtr& b) {
    const Planes p = planes_of(a, "mul_tensors");
    if (b->numel() != p.rows)
        throw ShapeError("mul_tensors: b " + to_string(b->shape()) +
                         " must hold one value per channel of " + to_string(a->shape()));
    to_dev(a);
    to_dev(b);
    const bool record = recording({a, b});
    TensorPtr out = Tensor::create(a->shape(), record, true);
    check(soar_mul_broadcast_forward(a->cuda_data(), b->cuda_data(), out->cuda_data(),
                                     (size_t)p.rows, (size_t)(p.H * p.W), exec::stream()),
          "mul_broadcast");
    if (record) {
        auto node = std::make_shared<MulBroadcastNode>();
        node->a = a;
        node->b = b;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr convex_combination(const TensorPtr& g, const TensorPtr& a, const TensorPtr& b) {
    if (g->shape() != a->shape() || a->shape() != b->shape())
        throw ShapeError("convex_combination: shapes differ");
    to_dev(g);
    to_dev(a);
    to_dev(b);
    const bool record = recording({g, a, b});
    TensorPtr out = Tensor::create(a->shape(), record, true);
    check(soar_convex_combination_forward(g->cuda_data(), a->cuda_data(), b->cuda_data(),
                                          out->cuda_data(), (size_t)a->numel(), exec::stream()),
          "convex combination");
    if (record) {
        auto node = std::make_shared<ConvexNode>();
        node->g = g;
        node->a = a;
        node->b = b;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr sigmoid_convex_combination(const TensorPtr& z, const TensorPtr& a,
                                     const TensorPtr& b) {
    if (z->shape() != a->shape() || a->shape() != b->shape())
        throw ShapeError("sigmoid_convex_combination: shapes differ");
    to_dev(z);
    to_dev(a);
    to_dev(b);
    const bool record = recording({z, a, b});
    TensorPtr out = Tensor::create(a->shape(), record, true);
    check(soar_sigmoid_convex_forward(z->cuda_data(), a->cuda_data(), b->cuda_data(),
                                      out->cuda_data(), (size_t)a->numel(), exec::stream()),
          "sigmoid convex combination");
    if (record) {
        auto node = std::make_shared<SigmoidConvexNode>();
        node->z = z;
        node->a = a;
        node->b = b;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr mul_sigmoid(const TensorPtr& a, const TensorPtr& z) {
    const Planes p = planes_of(a, "mul_sigmoid");
    if (z->numel() != p.rows)
        throw ShapeError("mul_sigmoid: z " + to_string(z->shape()) +
                         " must hold one value per channel of " + to_string(a->shape()));
    to_dev(a);
    to_dev(z);
    const bool record = recording({a, z});
    TensorPtr out = Tensor::create(a->shape(), record, true);
    check(soar_mul_sigmoid_broadcast_forward(a->cuda_data(), z->cuda_data(), out->cuda_data(),
                                             (size_t)p.rows, (size_t)(p.H * p.W),
                                             exec::stream()),
          "mul_sigmoid");
    if (record) {
        auto node = std::make_shared<MulSigmoidNode>();
        node->a = a;
        node->z = z;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr concat_channels(const std::vector<TensorPtr>& tensors) {
    if (tensors.empty()) throw ShapeError("concat: no tensors given");
    const TensorPtr& t0 = tensors[0];
    const bool batched = t0->ndim() == 4;
    if (t0->ndim() != 3 && !batched)
        throw ShapeError("concat_channels expects [C,H,W] or [N,C,H,W] tensors");
    const int64_t N = batched ? t0->dim(0) : 1;
    const int64_t H = t0->dim(-2), W = t0->dim(-1);
    int64_t C_total = 0;
    for (const auto& t : tensors) {
        if (t->ndim() != t0->ndim() || t->dim(-2) != H || t->dim(-1) != W ||
            (batched && t->dim(0) != N))
            throw ShapeError("concat_channels: tensors differ in batch or spatial size");
        C_total += batched ? t->dim(1) : t->dim(0);
        to_dev(t);
    }
    const bool record = GradMode::is_enabled() &&
                        std::any_of(tensors.begin(), tensors.end(),
                                    [](const TensorPtr& t) { return t->requires_grad(); });
    if (tensors.size() > 16) throw ShapeError("concat_channels: at most 16 tensors");
    Shape os = batched ? Shape{N, C_total, H, W} : Shape{C_total, H, W};
    TensorPtr out = Tensor::create(os, record, true);
    std::vector<const float*> src;
    std::vector<int64_t> ch;
    for (const auto& t : tensors) {
        src.push_back(t->cuda_data());
        ch.push_back(batched ? t->dim(1) : t->dim(0));
    }
    check(soar_concat_channels_forward(src.data(), ch.data(), (int)tensors.size(),
                                       out->cuda_data(), N, H * W, exec::stream()),
          "concat");
    if (record) {
        auto node = std::make_shared<ConcatNode>();
        node->inputs = tensors;
        out->set_grad_fn(node);
    }
    return out;
}

TensorPtr resize_bilinear(const TensorPtr& input, size_t target_h, size_t target_w) {
    if (input->dim(-2) == (int64_t)target_h && input->dim(-1) == (int64_t)target_w) return input;
    const float scale = (float)target_h / (float)input->dim(-2);
    Upsample up(scale);
    return up.forward(input);
}

}  // namespace soar::nn
