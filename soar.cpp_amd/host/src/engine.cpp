// Dice+BCE loss, AdamW, Trainer and Predictor on the MI355X kernels.
// Semantics follow src/losses/losses.cpp:458-563,1087-1219,
// src/optim/adamw.cpp:7-108, src/engine/trainer.cpp:33-245 and
// src/engine/predictor.cpp:7-85 of the reference.
#include "soar/engine.hpp"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstring>
#include <sstream>
#include <vector>

#include "soar/autograd.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar_gn.h"
#include "soar_ops.h"

namespace soar {

using hip::kernels::check;

namespace losses {

namespace {

// Backward of the Dice+BCE loss (losses.cpp:481-561): the fused device
// kernel with the statistics saved by the forward.
struct DiceBCENode : autograd::AutogradNode {
    TensorPtr logits, targets;
    float w = 1, bw = 1, dw = 1, pos_weight = 1, smooth = 1;
    float inter = 0, sum_p = 0, sum_y = 0;
    const double* sums = nullptr;  // device loss sums (forward_device), else null

    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        if (logits && logits->grad_fn()) return {logits->grad_fn()};
        return {};
    }
    void backward(const TensorPtr& grad_output) override {
        if (!logits || !logits->requires_grad()) return;
        const float go = grad_output->to_host()[0];
        bool fresh = false;
        TensorPtr gz = write_target(logits, &fresh);
        const unsigned fl = fresh ? 0u : SOAR_GN_ACCUMULATE_DX;
        if (sums)
            check(soar_dice_bce_loss_backward_device(logits->cuda_data(), targets->cuda_data(),
                                                     gz->cuda_data(), go, w, bw, dw, pos_weight,
                                                     smooth, sums, (size_t)logits->numel(), fl,
                                                     exec::stream()),
                  "Dice+BCE backward");
        else
            check(soar_dice_bce_loss_backward_ex(logits->cuda_data(), targets->cuda_data(),
                                                 gz->cuda_data(), go, w, bw, dw, pos_weight,
                                                 smooth, inter, sum_p, sum_y,
                                                 (size_t)logits->numel(), fl, exec::stream()),
                  "Dice+BCE backward");
        if (fresh) propagate_grad(logits, std::move(gz));
    }
    void release_variables() override { logits = targets = nullptr; }
};

}  // namespace

DiceBCELoss::DiceBCELoss(float weight, float dice_weight, float bce_weight, float bce_pos_weight,
                         float smooth)
    : weight_(weight),
      dice_weight_(dice_weight),
      bce_weight_(bce_weight),
      pos_weight_(bce_pos_weight),
      smooth_(smooth) {}

TensorPtr DiceBCELoss::forward(const TensorPtr& logits, const TensorPtr& targets) {
    if (logits->numel() != targets->numel())
        throw ShapeError("DiceBCELoss: shape mismatch between logits and targets");
    if (!logits->is_cuda()) logits->to_cuda();
    if (!targets->is_cuda()) targets->to_cuda();
    float out[6];
    check(soar_dice_bce_loss_forward(logits->cuda_data(), targets->cuda_data(),
                                     (size_t)logits->numel(), weight_, bce_weight_, dice_weight_,
                                     pos_weight_, smooth_, out, exec::stream()),
          "Dice+BCE forward");
    last_bce_ = out[1];
    last_dice_ = out[2];
    inter_ = out[3];
    sum_p_ = out[4];
    sum_y_ = out[5];
    const bool record = logits->requires_grad() && autograd::GradMode::is_enabled();
    TensorPtr total = Tensor::create({1}, record);
    total->data()[0] = out[0];
    if (record) {
        auto node = std::make_shared<DiceBCENode>();
        node->logits = logits;
        node->targets = targets;
        node->w = weight_;
        node->bw = bce_weight_;
        node->dw = dice_weight_;
        node->pos_weight = pos_weight_;
        node->smooth = smooth_;
        node->inter = inter_;
        node->sum_p = sum_p_;
        node->sum_y = sum_y_;
        total->set_grad_fn(node);
    }
    return total;
}

TensorPtr DiceBCELoss::forward_device(const TensorPtr& logits, const TensorPtr& targets,
                                      double* sums) {
    if (logits->numel() != targets->numel())
        throw ShapeError("DiceBCELoss: shape mismatch between logits and targets");
    if (!logits->is_cuda() || !targets->is_cuda())
        throw InvalidArgument("DiceBCELoss::forward_device needs device tensors");
    auto* arena = memory::DeviceArena::current();
    if (!arena) throw DeviceError("DiceBCELoss::forward_device needs a DeviceArena");
    const size_t n = (size_t)logits->numel();
    const size_t wsb = soar_dice_bce_loss_workspace_bytes(n);
    void* ws = wsb ? arena->allocate(wsb, {}, "loss_ws") : nullptr;
    check(soar_dice_bce_loss_sums_device(logits->cuda_data(), targets->cuda_data(), n,
                                         pos_weight_, sums, ws, wsb, exec::stream()),
          "Dice+BCE sums");
    const bool record = logits->requires_grad() && autograd::GradMode::is_enabled();
    TensorPtr total = Tensor::create({1}, record);
    total->data()[0] = 0.0f;
    if (record) {
        auto node = std::make_shared<DiceBCENode>();
        node->logits = logits;
        node->targets = targets;
        node->w = weight_;
        node->bw = bce_weight_;
        node->dw = dice_weight_;
        node->pos_weight = pos_weight_;
        node->smooth = smooth_;
        node->sums = sums;
        total->set_grad_fn(node);
    }
    return total;
}

SegmentationLoss::SegmentationLoss(float bce_weight, float dice_weight, float pos_weight,
                                   float dice_smooth, float cldice_weight)
    : bce_weight_(bce_weight),
      dice_weight_(dice_weight),
      pos_weight_(pos_weight),
      region_(1.0f, dice_weight, bce_weight, pos_weight, dice_smooth) {
    if (cldice_weight > 0.0f)
        throw InvalidArgument("SegmentationLoss: the clDice structure term is not built here");
}

TensorPtr SegmentationLoss::forward(const TensorPtr& logits, const TensorPtr& targets,
                                    float& out_bce, float& out_dice) {
    TensorPtr t = region_.forward(logits, targets);
    out_bce = region_.last_bce();
    out_dice = region_.last_dice();
    return t;
}

}  // namespace losses

namespace optim {

AdamW::AdamW(std::vector<TensorPtr> params, AdamWOptions options)
    : params_(std::move(params)), options_(options) {
    auto* arena = memory::DeviceArena::current();
    if (!arena) throw DeviceError("AdamW allocates its state from a DeviceArena: install one");
    const size_t n = params_.size();
    std::vector<int64_t> numel(n);
    for (size_t i = 0; i < n; ++i) {
        TensorPtr& p = params_[i];
        if (!p) throw InvalidArgument("AdamW: null parameter");
        if (!p->is_cuda()) p->to_cuda();
        if (!p->grad() || !p->grad()->is_cuda())
            p->set_grad(Tensor::zeros(p->shape(), false, true));
        m_.push_back(Tensor::zeros(p->shape(), false, true));
        v_.push_back(Tensor::zeros(p->shape(), false, true));
        numel[i] = p->numel();
    }
    if (n == 0) return;
    table_ = arena->allocate(5 * n * sizeof(void*), {}, "adamw_table");
    norm_ = static_cast<double*>(arena->allocate(sizeof(double), {}, "grad_norm"));
    norm_ws_bytes_ = soar_multi_tensor_norm_workspace_bytes();
    norm_ws_ = arena->allocate(norm_ws_bytes_, {}, "grad_norm_ws");
    std::vector<void*> host(5 * n);
    for (size_t i = 0; i < n; ++i) {
        host[i] = params_[i]->cuda_data();
        host[2 * n + i] = m_[i]->cuda_data();
        host[3 * n + i] = v_[i]->cuda_data();
        std::memcpy(&host[4 * n + i], &numel[i], sizeof(int64_t));
    }
    check(soar_memcpy_h2d(table_, host.data(), host.size() * sizeof(void*), exec::stream()),
          "AdamW table");
    grad_ptrs_.assign(n, nullptr);
    sync_tables();
}

// (Re)uploads the gradient pointers when a parameter's .grad buffer changed.
void AdamW::sync_tables() {
    const size_t n = params_.size();
    bool changed = false;
    for (size_t i = 0; i < n; ++i) {
        if (!params_[i]->grad() || !params_[i]->grad()->is_cuda())
            params_[i]->set_grad(Tensor::zeros(params_[i]->shape(), false, true));
        float* g = params_[i]->grad()->cuda_data();
        if (g != grad_ptrs_[i]) {
            grad_ptrs_[i] = g;
            changed = true;
        }
    }
    if (changed)
        check(soar_memcpy_h2d(static_cast<char*>(table_) + n * sizeof(void*), grad_ptrs_.data(),
                              n * sizeof(void*), exec::stream()),
              "AdamW gradient table");
}

// One fill launch over the gradient table (the reference zeroes each
// gradient in turn, adamw.cpp:20-26).
void AdamW::zero_grad() {
    const int n = (int)params_.size();
    if (n == 0) return;
    sync_tables();
    auto* t = static_cast<char*>(table_);
    const size_t nb = (size_t)n * sizeof(void*);
    check(soar_multi_tensor_fill_device(reinterpret_cast<float* const*>(t + nb),
                                        reinterpret_cast<const int64_t*>(t + 4 * nb), n, 0.0f,
                                        exec::stream()),
          "zero_grad");
}

float AdamW::clip_grad_norm(float max_norm) {
    const int n = (int)params_.size();
    if (n == 0) return 0.0f;
    sync_tables();
    auto* t = static_cast<char*>(table_);
    const size_t nb = (size_t)n * sizeof(void*);
    check(soar_multi_tensor_norm_sq_device(reinterpret_cast<const float* const*>(t + nb),
                                           reinterpret_cast<const int64_t*>(t + 4 * nb), n, norm_,
                                           norm_ws_, norm_ws_bytes_, exec::stream()),
          "gradient norm");
    double sq = 0.0;
    check(soar_memcpy_d2h(&sq, norm_, sizeof sq, exec::stream()), "gradient norm read-back");
    const float total_norm = static_cast<float>(std::sqrt(sq));
    if (total_norm > max_norm && total_norm > 1e-6f) {
        const float clip_coef = max_norm / total_norm;
        check(soar_multi_tensor_scale_device(reinterpret_cast<float* const*>(t + nb),
                                             reinterpret_cast<const int64_t*>(t + 4 * nb), n,
                                             clip_coef, exec::stream()),
              "gradient clip");
    }
    return total_norm;
}

void AdamW::clip_grad_norm_device(float max_norm) {
    const int n = (int)params_.size();
    if (n == 0) return;
    sync_tables();
    auto* t = static_cast<char*>(table_);
    const size_t nb = (size_t)n * sizeof(void*);
    check(soar_multi_tensor_norm_sq_device(reinterpret_cast<const float* const*>(t + nb),
                                           reinterpret_cast<const int64_t*>(t + 4 * nb), n, norm_,
                                           norm_ws_, norm_ws_bytes_, exec::stream()),
          "gradient norm");
    check(soar_multi_tensor_clip_device(reinterpret_cast<float* const*>(t + nb),
                                        reinterpret_cast<const int64_t*>(t + 4 * nb), n, norm_,
                                        max_norm, exec::stream()),
          "gradient clip");
}

void AdamW::next_scalars(float out[3]) {
    step_count_++;
    // adamw.cpp:67-70, in fp32, as step()
    const float beta1 = options_.beta1, beta2 = options_.beta2;
    const float bias_correction1 = 1.0f - std::pow(beta1, static_cast<float>(step_count_));
    const float bias_correction2 = 1.0f - std::pow(beta2, static_cast<float>(step_count_));
    out[0] = options_.lr;
    out[1] = options_.lr / bias_correction1;
    out[2] = std::sqrt(bias_correction2);
}

void AdamW::step_device(const float* scalars) {
    const int n = (int)params_.size();
    if (n == 0) return;
    sync_tables();
    auto* t = static_cast<char*>(table_);
    const size_t nb = (size_t)n * sizeof(void*);
    check(soar_adamw_multi_tensor_device_scalars(
              reinterpret_cast<float* const*>(t), reinterpret_cast<const float* const*>(t + nb),
              reinterpret_cast<float* const*>(t + 2 * nb),
              reinterpret_cast<float* const*>(t + 3 * nb),
              reinterpret_cast<const int64_t*>(t + 4 * nb), n, scalars, options_.beta1,
              options_.beta2, options_.eps, options_.weight_decay, exec::stream()),
          "AdamW step");
}

void AdamW::clip_step_zero_device(float max_norm, const float* scalars) {
    const int n = (int)params_.size();
    if (n == 0) return;
    sync_tables();
    auto* t = static_cast<char*>(table_);
    const size_t nb = (size_t)n * sizeof(void*);
    check(soar_multi_tensor_norm_sq_partials_device(
              reinterpret_cast<const float* const*>(t + nb),
              reinterpret_cast<const int64_t*>(t + 4 * nb), n, norm_ws_, norm_ws_bytes_,
              exec::stream()),
          "gradient norm");
    check(soar_adamw_clip_multi_tensor_device(
              reinterpret_cast<float* const*>(t), reinterpret_cast<float* const*>(t + nb),
              reinterpret_cast<float* const*>(t + 2 * nb),
              reinterpret_cast<float* const*>(t + 3 * nb),
              reinterpret_cast<const int64_t*>(t + 4 * nb), n, scalars, options_.beta1,
              options_.beta2, options_.eps, options_.weight_decay, norm_ws_, norm_ws_bytes_,
              max_norm, norm_, SOAR_ADAMW_ZERO_GRAD, exec::stream()),
          "clip + AdamW step");
}

void AdamW::step() {
    step_count_++;
    const int n = (int)params_.size();
    if (n == 0) return;
    sync_tables();
    const float lr = options_.lr, beta1 = options_.beta1, beta2 = options_.beta2;
    // adamw.cpp:67-70, in fp32
    const float bias_correction1 = 1.0f - std::pow(beta1, static_cast<float>(step_count_));
    const float bias_correction2 = 1.0f - std::pow(beta2, static_cast<float>(step_count_));
    const float sqrt_bc2 = std::sqrt(bias_correction2);
    const float step_size = lr / bias_correction1;
    auto* t = static_cast<char*>(table_);
    const size_t nb = (size_t)n * sizeof(void*);
    check(soar_adamw_multi_tensor_device(
              reinterpret_cast<float* const*>(t), reinterpret_cast<const float* const*>(t + nb),
              reinterpret_cast<float* const*>(t + 2 * nb),
              reinterpret_cast<float* const*>(t + 3 * nb),
              reinterpret_cast<const int64_t*>(t + 4 * nb), n, lr, beta1, beta2, options_.eps,
              options_.weight_decay, step_size, sqrt_bc2, exec::stream()),
          "AdamW step");
}

}  // namespace optim

namespace engine {

Trainer::Trainer(std::shared_ptr<nn::SOARModel> model, losses::CompositeLoss loss_fn,
                 std::unique_ptr<optim::AdamW> optimizer, size_t accumulate_grad_batches,
                 float grad_clip)
    : model_(std::move(model)),
      loss_fn_(std::move(loss_fn)),
      optimizer_(std::move(optimizer)),
      accumulate_(std::max<size_t>(1, accumulate_grad_batches)),
      grad_clip_(grad_clip) {
    if (!model_ || !optimizer_) throw InvalidArgument("Trainer needs a model and an optimizer");
}

StepMetrics Trainer::forward_backward(const TensorPtr& image, const TensorPtr& mask,
                                      float scale) {
    image->set_requires_grad(false);
    TensorPtr logits = model_->forward(image);
    float bce = 0.0f, dice = 0.0f;
    TensorPtr loss = loss_fn_.forward(logits, mask, bce, dice);
    TensorPtr grad_out = Tensor::create({1});
    grad_out->data()[0] = scale;
    loss->backward(grad_out);
    StepMetrics m;
    m.loss = loss->data()[0];
    m.bce_loss = bce;
    m.dice_loss = dice;
    // device-path metrics (trainer.cpp:80-86)
    const float d = std::max(0.0f, std::min(1.0f, 1.0f - dice));
    m.dice_score = d;
    m.iou_score = d / (2.0f - d + 1e-7f);
    m.lr = optimizer_->get_lr();
    logits->set_grad_fn(nullptr);
    loss->set_grad_fn(nullptr);
    return m;
}

namespace {
// Sample b of a [B,C,H,W] device tensor as [C,H,W] (a copy).
TensorPtr sample(const TensorPtr& t, int64_t b) {
    const int64_t C = t->dim(1), H = t->dim(2), W = t->dim(3);
    TensorPtr s = Tensor::create({C, H, W}, false, true);
    check(soar_memcpy_d2d(s->cuda_data(), t->cuda_data() + b * C * H * W,
                          (size_t)(C * H * W) * sizeof(float), exec::stream()),
          "sample slice");
    return s;
}
}  // namespace

StepMetrics Trainer::train_step(const TensorPtr& images, const TensorPtr& masks,
                                bool is_accumulating) {
    model_->train(true);
    if (!images->is_cuda()) images->to_cuda();
    if (!masks->is_cuda()) masks->to_cuda();
    const int64_t B = images->ndim() == 4 ? images->dim(0) : 1;
    StepMetrics m;
    if (B <= 1) {
        TensorPtr img = images->ndim() == 4 ? sample(images, 0) : images;
        TensorPtr msk = masks->ndim() == 4 ? sample(masks, 0) : masks;
        m = forward_backward(img, msk, 1.0f / (float)accumulate_);
    } else {
        // micro-batches of one sample (trainer.cpp:174-226)
        double loss = 0, bce = 0, dice = 0, iou = 0, dsc = 0;
        for (int64_t b = 0; b < B; ++b) {
            const StepMetrics s = forward_backward(
                sample(images, b), masks->ndim() == 4 ? sample(masks, b) : masks,
                1.0f / (float)((size_t)B * accumulate_));
            loss += s.loss;
            bce += s.bce_loss;
            dice += s.dice_loss;
            iou += s.iou_score;
            dsc += s.dice_score;
        }
        m.loss = (float)(loss / (double)B);
        m.bce_loss = (float)(bce / (double)B);
        m.dice_loss = (float)(dice / (double)B);
        m.iou_score = (float)(iou / (double)B);
        m.dice_score = (float)(dsc / (double)B);
    }
    if (!is_accumulating) {
        m.grad_norm = optimizer_->clip_grad_norm(grad_clip_);
        optimizer_->step();
        optimizer_->zero_grad();
    }
    m.lr = optimizer_->get_lr();
    return m;
}

void Trainer::train_step_device(const TensorPtr& image, const TensorPtr& mask,
                                double* loss_sums, float* pinned_scalars, float* dev_scalars) {
    model_->train(true);
    if (!image->is_cuda() || !mask->is_cuda())
        throw InvalidArgument("Trainer::train_step_device needs device tensors");
    image->set_requires_grad(false);
    TensorPtr logits = model_->forward(image);
    TensorPtr loss = loss_fn_.forward_device(logits, mask, loss_sums);
    TensorPtr grad_out = Tensor::create({1});
    grad_out->data()[0] = 1.0f / (float)accumulate_;
    loss->backward(grad_out);
    logits->set_grad_fn(nullptr);
    loss->set_grad_fn(nullptr);
    // clip, step, zero_grad (trainer.cpp:110-220), the last three in one launch
    optimizer_->next_scalars(pinned_scalars);
    check(soar_memcpy_async(dev_scalars, pinned_scalars, 3 * sizeof(float), 0, exec::stream()),
          "AdamW scalars");
    optimizer_->clip_step_zero_device(grad_clip_, dev_scalars);
}

StepMetrics Trainer::device_step_metrics(const double loss_sums[4], double norm_sq,
                                         size_t numel) const {
    const losses::DiceBCELoss& r = loss_fn_.region();
    float out[6];
    check(soar_dice_bce_loss_from_sums(loss_sums, numel, r.weight(), r.bce_weight(),
                                       r.dice_weight(), r.smooth(), out),
          "Dice+BCE finish");
    StepMetrics m;
    m.loss = out[0];
    m.bce_loss = out[1];
    m.dice_loss = out[2];
    // device-path metrics (trainer.cpp:80-86), as forward_backward
    const float d = std::max(0.0f, std::min(1.0f, 1.0f - out[2]));
    m.dice_score = d;
    m.iou_score = d / (2.0f - d + 1e-7f);
    m.grad_norm = static_cast<float>(std::sqrt(norm_sq));
    m.lr = optimizer_->get_lr();
    return m;
}

Predictor::Predictor(std::shared_ptr<nn::SOARModel> model, float threshold)
    : model_(std::move(model)), threshold_(threshold) {}

namespace {
// High bit of each byte of v set where that byte is nonzero.
inline uint64_t nonzero_bytes(uint64_t v) {
    const uint64_t lo7 = 0x7f7f7f7f7f7f7f7fULL;
    return (((v & lo7) + lo7) | v) & ~lo7;
}
}  // namespace

// Column-major (Fortran order), 1-indexed runs of nonzero pixels,
// "start len start len ..." (predictor.cpp:10-47; a run may continue from
// the bottom of one column into the top of the next).  The mask is read
// once in row order: comparing each row with the one above it (8 columns
// per word) gives, per column, the rows where the pixel turns on or off
// (row -1 and row H count as off).  A counting sort by column puts those
// transitions in column order, and consecutive on/off pairs are the runs;
// a run that ends at the bottom of a column and one that starts at the top
// of the next are joined, as the column-order scan would see them.
std::string Predictor::encode_rle(const uint8_t* mask, size_t height, size_t width) {
    const size_t H = height, W = width;
    if (H == 0 || W == 0) return std::string();
    std::vector<uint32_t> tcol, trow;  // transitions, in row order
    std::vector<size_t> first(W + 1, 0);
    auto add = [&](size_t x, size_t y) {
        tcol.push_back((uint32_t)x);
        trow.push_back((uint32_t)y);
        ++first[x + 1];
    };
    const size_t W8 = W / 8 * 8;
    for (size_t y = 0; y <= H; ++y) {
        const uint8_t* cur = y < H ? mask + y * W : nullptr;
        const uint8_t* above = y > 0 ? mask + (y - 1) * W : nullptr;
        size_t x = 0;
        for (; x < W8; x += 8) {
            uint64_t a = 0, b = 0;
            if (cur) std::memcpy(&a, cur + x, 8);
            if (above) std::memcpy(&b, above + x, 8);
            for (uint64_t d = nonzero_bytes(a) ^ nonzero_bytes(b); d; d &= d - 1)
                add(x + (size_t)(__builtin_ctzll(d) >> 3), y);
        }
        for (; x < W; ++x)
            if ((cur && cur[x]) != (above && above[x])) add(x, y);
    }
    for (size_t x = 0; x < W; ++x) first[x + 1] += first[x];
    std::vector<uint32_t> rows(tcol.size());
    {
        std::vector<size_t> next(first.begin(), first.end() - 1);
        for (size_t i = 0; i < tcol.size(); ++i) rows[next[tcol[i]]++] = trow[i];
    }
    std::string out;
    char num[24];
    auto emit = [&](size_t s, size_t e) {  // run [s, e) of column-order indices
        if (!out.empty()) out.push_back(' ');
        out.append(num, std::to_chars(num, num + sizeof num, s + 1).ptr);
        out.push_back(' ');
        out.append(num, std::to_chars(num, num + sizeof num, e - s).ptr);
    };
    size_t ps = 0, pe = 0;
    bool pending = false;
    for (size_t x = 0; x < W; ++x) {
        for (size_t k = first[x]; k < first[x + 1]; k += 2) {  // on, off
            const size_t s = x * H + rows[k], e = x * H + rows[k + 1];
            if (pending && s == pe) {
                pe = e;
                continue;
            }
            if (pending) emit(ps, pe);
            ps = s;
            pe = e;
            pending = true;
        }
    }
    if (pending) emit(ps, pe);
    return out;
}

std::pair<int64_t, int64_t> Predictor::predict_device(const TensorPtr& image, float* probs,
                                                      uint8_t* mask) {
    autograd::NoGradGuard guard;
    model_->eval();
    TensorPtr logits = model_->forward(image);
    const int64_t H = logits->dim(-2), W = logits->dim(-1);
    check(soar_sigmoid_threshold(logits->cuda_data(), probs, mask, (size_t)(H * W), threshold_,
                                 exec::stream()),
          "sigmoid threshold");
    return {H, W};
}

PredictionResult Predictor::predict(const TensorPtr& image) {
    autograd::NoGradGuard guard;
    model_->eval();
    TensorPtr logits = model_->forward(image);
    const int64_t H = logits->dim(-2), W = logits->dim(-1);
    const int64_t n = H * W;
    TensorPtr probs = Tensor::create({1, H, W}, false, true);
    auto* arena = memory::DeviceArena::current();
    if (!arena) throw DeviceError("Predictor needs a DeviceArena");
    auto* mask_dev = static_cast<uint8_t*>(arena->allocate((size_t)n, {}, "mask"));
    check(soar_sigmoid_threshold(logits->cuda_data(), probs->cuda_data(), mask_dev, (size_t)n,
                                 threshold_, exec::stream()),
          "sigmoid threshold");
    PredictionResult r;
    r.height = (size_t)H;
    r.width = (size_t)W;
    r.probabilities = probs->to_host();
    r.binary_mask.resize((size_t)n);
    check(soar_memcpy_d2h(r.binary_mask.data(), mask_dev, (size_t)n, exec::stream()), "mask read-back");
    for (uint8_t v : r.binary_mask) r.foreground_pixels += v;
    r.rle_string = encode_rle(r.binary_mask.data(), r.height, r.width);
    return r;
}

}  // namespace engine
}  // namespace soar
