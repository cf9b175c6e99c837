// engine.hpp - training and inference around SOARModel on the MI355X
// kernels: the Dice+BCE segmentation loss (include/soar/losses/
// losses.hpp:123-148,226-272), AdamW with gradient-norm clipping
// (include/soar/optim/adamw.hpp:10-60), Trainer::train_step
// (include/soar/engine/trainer.hpp:40-105) and Predictor with the
// column-major RLE encoder (include/soar/engine/predictor.hpp).
//
// Everything stays on the device except the scalars the reference returns
// on the host (loss values, the gradient norm) and the Predictor's result.
// The device work of one step allocates from the current DeviceArena; the
// optimizer's state (moments, parameter tables) is allocated when AdamW is
// constructed, so construct it under the arena that holds the parameters.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "soar/model.hpp"

namespace soar::losses {

// weight * (bce_weight * BCEWithLogits(pos_weight) + dice_weight *
// SoftDice(smooth)) with the fused device backward of losses.cpp:464-561.
class DiceBCELoss {
public:
    explicit DiceBCELoss(float weight = 1.0f, float dice_weight = 1.0f, float bce_weight = 1.0f,
                         float bce_pos_weight = 1.0f, float smooth = 1.0f);
    // Scalar loss tensor [1] on the host, with a backward node to logits.
    TensorPtr forward(const TensorPtr& logits, const TensorPtr& targets);
    // The same with nothing read back (capture-safe): the loss sums go to
    // `sums` (device, 4 doubles; workspace from the current arena), the
    // returned scalar holds 0, and its backward reads the sums on the
    // device.  soar_dice_bce_loss_from_sums finishes them into the values
    // forward() returns.
    TensorPtr forward_device(const TensorPtr& logits, const TensorPtr& targets, double* sums);
    [[nodiscard]] float weight() const noexcept { return weight_; }
    [[nodiscard]] float dice_weight() const noexcept { return dice_weight_; }
    [[nodiscard]] float bce_weight() const noexcept { return bce_weight_; }
    [[nodiscard]] float smooth() const noexcept { return smooth_; }

    [[nodiscard]] float last_bce() const noexcept { return last_bce_; }
    [[nodiscard]] float last_dice() const noexcept { return last_dice_; }
    [[nodiscard]] float last_inter() const noexcept { return inter_; }
    [[nodiscard]] float last_sum_p() const noexcept { return sum_p_; }
    [[nodiscard]] float last_sum_y() const noexcept { return sum_y_; }

private:
    float weight_, dice_weight_, bce_weight_, pos_weight_, smooth_;
    float last_bce_ = 0.0f, last_dice_ = 0.0f, inter_ = 0.0f, sum_p_ = 0.0f, sum_y_ = 0.0f;
};

// SegmentationLoss(bce_weight, dice_weight, pos_weight = 3, dice_smooth =
// 1, cldice_weight = 0) (losses.cpp:1090-1099): the region term only.  The
// boundary and clDice terms of the reference are not part of this build
// (cldice_weight > 0 throws InvalidArgument); with their default weight 0
// the loss is the reference's.
class SegmentationLoss {
public:
    SegmentationLoss(float bce_weight, float dice_weight, float pos_weight = 3.0f,
                     float dice_smooth = 1.0f, float cldice_weight = 0.0f);
    TensorPtr forward(const TensorPtr& logits, const TensorPtr& targets, float& out_bce,
                      float& out_dice);
    // Capture-safe form of forward (DiceBCELoss::forward_device).
    TensorPtr forward_device(const TensorPtr& logits, const TensorPtr& targets, double* sums) {
        return region_.forward_device(logits, targets, sums);
    }
    [[nodiscard]] const DiceBCELoss& region() const noexcept { return region_; }
    [[nodiscard]] float bce_weight() const noexcept { return bce_weight_; }
    [[nodiscard]] float dice_weight() const noexcept { return dice_weight_; }
    [[nodiscard]] float pos_weight() const noexcept { return pos_weight_; }

private:
    float bce_weight_, dice_weight_, pos_weight_;
    DiceBCELoss region_;
};
using CompositeLoss = SegmentationLoss;

}  // namespace soar::losses

namespace soar::optim {

struct AdamWOptions {
    float lr{1e-3f};
    float beta1{0.9f};
    float beta2{0.999f};
    float eps{1e-8f};
    float weight_decay{1e-2f};
};

// AdamW (adamw.cpp:7-108) over device parameters: one multi-tensor launch
// per step, moments in device memory, the parameter / gradient / moment
// tables resident on the device.  Every parameter gets a zeroed device
// gradient at construction.
class AdamW {
public:
    AdamW(std::vector<TensorPtr> params, AdamWOptions options = {});
    void zero_grad();
    // Global L2 norm of the gradients (fp64 accumulation); when it exceeds
    // max_norm (and 1e-6) every gradient is scaled by max_norm / norm
    // (adamw.cpp:28-57).  Returns the norm before clipping.
    float clip_grad_norm(float max_norm);
    void step();
    // Capture-safe forms: nothing is read back and nothing step-dependent is
    // baked into a launch.  clip_grad_norm_device leaves the squared norm in
    // norm_sq() (device) and takes the clip decision on the device.
    // next_scalars advances the step count and writes the step's lr, step
    // size and sqrt of bias correction 2 (as step() computes them) to
    // out[3]; step_device runs the update with those three read from the
    // device array `scalars` when the kernel executes.
    void clip_grad_norm_device(float max_norm);
    void next_scalars(float out[3]);
    void step_device(const float* scalars);
    // clip_grad_norm_device, step_device and zero_grad in two launches (the
    // norm's partials, then its finish + clip + update + zero in one), the
    // same values; norm_sq() receives the squared norm.
    void clip_step_zero_device(float max_norm, const float* scalars);
    [[nodiscard]] const double* norm_sq() const noexcept { return norm_; }
    // Puts the squared norm at `p` (a device double the caller keeps), e.g.
    // next to other values read back together with it.
    void set_norm_sq_buffer(double* p) noexcept {
        if (p) norm_ = p;
    }
    [[nodiscard]] float get_lr() const noexcept { return options_.lr; }
    void set_lr(float lr) noexcept { options_.lr = lr; }
    [[nodiscard]] const AdamWOptions& options() const noexcept { return options_; }
    [[nodiscard]] int64_t step_count() const noexcept { return step_count_; }
    // (to undo next_scalars of a step that was captured but never ran)
    void set_step_count(int64_t n) noexcept { step_count_ = n; }
    [[nodiscard]] const std::vector<TensorPtr>& params() const noexcept { return params_; }

private:
    void sync_tables();

    std::vector<TensorPtr> params_, m_, v_;
    AdamWOptions options_;
    int64_t step_count_ = 0;
    // device tables: params, grads, m, v (pointer arrays) and numel
    void* table_ = nullptr;
    std::vector<float*> grad_ptrs_;
    double* norm_ = nullptr;
    void* norm_ws_ = nullptr;
    size_t norm_ws_bytes_ = 0;
};

}  // namespace soar::optim

namespace soar::engine {

struct StepMetrics {
    float loss{0.0f};
    float bce_loss{0.0f};
    float dice_loss{0.0f};
    float dice_score{0.0f};
    float iou_score{0.0f};
    float lr{0.0f};
    float grad_norm{0.0f};  // before clipping (AdamW::clip_grad_norm's return)
};

// Trainer::train_step of trainer.cpp:110-245: forward, loss, backward with
// gradient scale 1/(B * accumulate_grad_batches), then (unless
// accumulating) clip, AdamW step and zero_grad.  A [B,C,H,W] batch runs
// sample by sample.  Metrics are those of the reference's device path
// (trainer.cpp:80-86): dice_score = clamp(1 - dice_loss), iou = d/(2-d).
class Trainer {
public:
    Trainer(std::shared_ptr<nn::SOARModel> model, losses::CompositeLoss loss_fn,
            std::unique_ptr<optim::AdamW> optimizer, size_t accumulate_grad_batches = 1,
            float grad_clip = 2.0f);
    StepMetrics train_step(const TensorPtr& images, const TensorPtr& masks,
                           bool is_accumulating = false);
    // Forward, loss and backward only (gradients accumulate; no step).
    StepMetrics forward_backward(const TensorPtr& image, const TensorPtr& mask, float scale);
    // One step of one [C,H,W] sample with every scalar kept on the device,
    // so the whole step can be captured into a graph and replayed: forward,
    // loss sums to loss_sums (device, 4 doubles), backward, the clip
    // decided on the device, the AdamW scalars written to pinned_scalars
    // (host, pinned) and copied from there to dev_scalars (device) on the
    // stream, the update, zero_grad.  Same arithmetic as train_step.  Read
    // loss_sums and optimizer().norm_sq() back afterwards and pass them to
    // device_step_metrics.
    void train_step_device(const TensorPtr& image, const TensorPtr& mask, double* loss_sums,
                           float* pinned_scalars, float* dev_scalars);
    [[nodiscard]] StepMetrics device_step_metrics(const double loss_sums[4], double norm_sq,
                                                  size_t numel) const;

    [[nodiscard]] optim::AdamW& optimizer() noexcept { return *optimizer_; }
    [[nodiscard]] losses::CompositeLoss& loss_fn() noexcept { return loss_fn_; }
    [[nodiscard]] size_t accumulate_grad_batches() const noexcept { return accumulate_; }
    void set_accumulate_grad_batches(size_t n) noexcept { accumulate_ = n ? n : 1; }
    [[nodiscard]] float grad_clip() const noexcept { return grad_clip_; }
    void set_grad_clip(float c) noexcept { grad_clip_ = c; }

private:
    std::shared_ptr<nn::SOARModel> model_;
    losses::CompositeLoss loss_fn_;
    std::unique_ptr<optim::AdamW> optimizer_;
    size_t accumulate_;
    float grad_clip_;
};

struct PredictionResult {
    std::vector<float> probabilities;  // [H*W] (first class), host
    std::vector<uint8_t> binary_mask;  // [H*W] 0/1, host
    size_t height{0}, width{0};
    size_t foreground_pixels{0};
    std::string rle_string;
};

// Predictor::predict of predictor.cpp:50-85: no-grad forward, sigmoid,
// threshold (prob >= threshold), RLE of the mask.
class Predictor {
public:
    Predictor(std::shared_ptr<nn::SOARModel> model, float threshold = 0.5f);
    PredictionResult predict(const TensorPtr& image);
    // The device part of predict on exec::stream(): no-grad forward, then
    // probabilities (H*W floats) and the 0/1 mask (H*W bytes) into the
    // given device buffers; nothing is read back (capturable).  Returns
    // (H, W) of the logits.
    std::pair<int64_t, int64_t> predict_device(const TensorPtr& image, float* probs,
                                               uint8_t* mask);
    // Column-major, 1-indexed "start length" pairs of the non-zero runs
    // (predictor.cpp:10-48).
    static std::string encode_rle(const uint8_t* mask, size_t height, size_t width);

private:
    std::shared_ptr<nn::SOARModel> model_;
    float threshold_;
};

}  // namespace soar::engine
