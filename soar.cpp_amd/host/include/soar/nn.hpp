// nn.hpp - the GroupNorm / SiLU layers, the pointwise and depthwise
// convolutions, the CBA block and the residual add of the SOAR blocks,
// running on the MI355X kernels of libsoar_gn.so.
//
// Mirrors include/soar/nn/layers.hpp:9-14,61-91 and src/nn/blocks.cpp:
// 17-72,429-445 of the reference: GroupNorm(num_groups, num_channels,
// eps = 1e-5, affine = true) with parameters "weight" (ones) and "bias"
// (zeros), SiLU, add_tensors.  Inputs are [C,H,W] (the reference's layout)
// or [N,C,H,W] (all samples in one launch; parameter gradients are summed
// over samples exactly as the reference's per-sample loop accumulates
// them).  GNSiLU is the fused GroupNorm -> SiLU pair (optionally with the
// residual add x + silu(gn(x)) of a SOAR block): one forward saves only x
// and the statistics, one backward recomputes SiLU.
//
// These layers run on device tensors only; there is no host fallback (a
// host tensor is moved to the device on entry, as the reference's layers
// do when a parameter lives on the device).
//
// Also here: the other layers and tensor helpers of the SOAR blocks
// (layers.hpp:96-159, blocks.hpp:10-14): Sigmoid, PixelShuffle, Upsample
// (bilinear), AdaptiveAvgPool2d, mul_tensors (channel broadcast),
// convex_combination, concat_channels and resize_bilinear.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "soar/tensor.hpp"

namespace soar::nn {

// Largest divisor of `channels` not above max_groups (layers.hpp:9-14).
inline int select_group_count(int channels, int max_groups = 8) {
    for (int g = std::min(max_groups, channels); g > 0; --g)
        if (channels % g == 0) return g;
    return 1;
}

// Autopadding of Conv2d (layers.hpp:16-19): half the dilated kernel.
inline int autopad(int k, int p = -1, int d = 1) {
    if (d > 1) k = d * (k - 1) + 1;
    return p < 0 ? k / 2 : p;
}

// Module base (module.hpp:15-137): parameters and submodules live in
// name-sorted maps, so parameters() / named_parameters() list a module's own
// parameters by name, then each submodule's by submodule name, recursively,
// in the reference's order (which is also the order of a .soar file).
class Module {
public:
    explicit Module(std::string name) : name_(std::move(name)) {}
    virtual ~Module() = default;
    // Single- and multi-input forward; each defaults to the other
    // (module.hpp:21-29), so a module overrides at least one.
    virtual TensorPtr forward(const TensorPtr& input);
    virtual TensorPtr forward(const std::vector<TensorPtr>& inputs);

    void register_parameter(const std::string& name, TensorPtr p);
    // Parameters of a submodule are named "<name>.<parameter>"
    // (the reference's register_submodule naming).
    void register_submodule(const std::string& name, std::shared_ptr<Module> m);
    [[nodiscard]] std::vector<std::pair<std::string, TensorPtr>> named_parameters(
        const std::string& prefix = "") const;
    [[nodiscard]] std::vector<TensorPtr> parameters() const;
    // Moves every parameter to the device (allocated from the current
    // arena: do this before freeze_static_parameters()).
    void to_device();
    void zero_grad();
    virtual void train(bool mode = true);
    void eval() { train(false); }
    [[nodiscard]] bool is_training() const noexcept { return training_; }
    [[nodiscard]] const std::string& name() const noexcept { return name_; }

private:
    std::string name_;
    bool training_ = true;
    std::map<std::string, TensorPtr> params_;
    std::map<std::string, std::shared_ptr<Module>> subs_;
};

class GroupNorm : public Module {
public:
    GroupNorm(size_t num_groups, size_t num_channels, float eps = 1e-5f, bool affine = true);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

    [[nodiscard]] size_t num_groups() const noexcept { return num_groups_; }
    [[nodiscard]] size_t num_channels() const noexcept { return num_channels_; }
    [[nodiscard]] float eps() const noexcept { return eps_; }
    [[nodiscard]] TensorPtr weight() const { return weight_; }
    [[nodiscard]] TensorPtr bias() const { return bias_; }

    // The layer with the soar_gn_silu_forward flags (SOAR_GN_SILU,
    // SOAR_GN_RESIDUAL): GroupNorm -> SiLU in one pass for CBA.
    TensorPtr run(const TensorPtr& input, unsigned flags);

protected:
    GroupNorm(std::string name, size_t num_groups, size_t num_channels, float eps, bool affine);

    size_t num_groups_;
    size_t num_channels_;
    float eps_;
    bool affine_;
    TensorPtr weight_;
    TensorPtr bias_;
};

class SiLU : public Module {
public:
    SiLU() : Module("SiLU") {}
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;
};

// silu(group_norm(x)), or x + silu(group_norm(x)) with residual = true.
class GNSiLU : public GroupNorm {
public:
    GNSiLU(size_t num_groups, size_t num_channels, float eps = 1e-5f, bool affine = true,
           bool residual = false);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;
    [[nodiscard]] bool residual() const noexcept { return residual_; }

private:
    bool residual_;
};

// Conv2d(in, out, kernel_size, stride = 1, padding = -1 (autopad),
// dilation = 1, groups = 1, bias = true) of layers.hpp:24-58: weight
// [out][in/groups][k][k] with Kaiming-uniform initialisation
// U(-1/sqrt(fan_in), 1/sqrt(fan_in)) (layers.cpp:303-317; drawn from a
// seeded generator, where the reference seeds from std::random_device:
// seed 0 takes the next seed of a process-wide sequence started by
// set_init_seed, so layers of one model differ and a model is reproducible),
// bias zeros.  Three device paths, chosen as the reference chooses its
// kernels (layers.cpp:59-72): pointwise (k = 1, stride 1, no padding,
// groups 1) on the MFMA kernel, depthwise (groups = in = out) on the tiled
// depthwise kernels, anything else on the general grouped convolution.
// Input [C,H,W] or [N,C,H,W]; the output size is (H + 2p - d(k-1) - 1)/s + 1
// (layers.cpp:330-332).
// Restarts the sequence of initialisation seeds of Conv2d(seed = 0).
void set_init_seed(uint64_t seed);

class Conv2d : public Module {
public:
    Conv2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride = 1,
           int padding = -1, size_t dilation = 1, size_t groups = 1, bool bias = true,
           uint64_t seed = 0);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

    [[nodiscard]] bool pointwise() const noexcept {
        return groups_ == 1 && kernel_ == 1 && stride_ == 1 && padding_ == 0;
    }
    [[nodiscard]] bool depthwise() const noexcept {
        return !pointwise() && groups_ == in_ && in_ == out_;
    }
    [[nodiscard]] size_t groups() const noexcept { return groups_; }
    [[nodiscard]] TensorPtr weight() const { return weight_; }
    [[nodiscard]] TensorPtr bias() const { return bias_; }
    [[nodiscard]] size_t in_channels() const noexcept { return in_; }
    [[nodiscard]] size_t out_channels() const noexcept { return out_; }
    [[nodiscard]] size_t kernel_size() const noexcept { return kernel_; }
    [[nodiscard]] size_t stride() const noexcept { return stride_; }
    [[nodiscard]] size_t padding() const noexcept { return padding_; }
    [[nodiscard]] size_t dilation() const noexcept { return dilation_; }

private:
    size_t in_, out_, kernel_, stride_, padding_, dilation_, groups_;
    TensorPtr weight_;
    TensorPtr bias_;
};

// CBA(c1, c2, k = 1, s = 1, p = -1, d = 1, g = 1, act = true) of
// blocks.cpp:429-445: Conv2d (no bias) -> GroupNorm(select_group_count(c2),
// c2) -> SiLU when act.  Submodules "conv" and "norm" as in the reference.
// With a pointwise conv the whole block is one forward call whose GroupNorm
// statistics come from the conv's epilogue, and one backward node; with a
// depthwise conv the conv runs, then GroupNorm(+SiLU) in one pass.
class CBA : public Module {
public:
    CBA(size_t c1, size_t c2, size_t k = 1, size_t s = 1, int p = -1, size_t d = 1,
        size_t g = 1, bool act = true);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;
    // residual + forward(input) (the LKR block's skip), the add in the
    // GroupNorm's apply pass for a pointwise conv
    TensorPtr forward_residual(const TensorPtr& input, const TensorPtr& residual);

    [[nodiscard]] std::shared_ptr<Conv2d> conv() const { return conv_; }
    [[nodiscard]] std::shared_ptr<GroupNorm> norm() const { return norm_; }
    [[nodiscard]] bool act() const noexcept { return act_; }

private:
    TensorPtr forward_depthwise(const TensorPtr& input, unsigned flags);

    std::shared_ptr<Conv2d> conv_;
    std::shared_ptr<GroupNorm> norm_;
    bool act_;
};

// y = a + b (blocks.cpp:39-72); shapes must match (ShapeError otherwise).
TensorPtr add_tensors(const TensorPtr& a, const TensorPtr& b);

// y = 1 / (1 + exp(-x)) (layers.cpp:807-870).
class Sigmoid : public Module {
public:
    Sigmoid() : Module("Sigmoid") {}
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;
};

// [C*r*r, H, W] -> [C, H*r, W*r] (layers.cpp:875-989).
class PixelShuffle : public Module {
public:
    explicit PixelShuffle(size_t upscale_factor = 2)
        : Module("PixelShuffle"), r_(upscale_factor) {}
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;
    [[nodiscard]] size_t upscale_factor() const noexcept { return r_; }

private:
    size_t r_;
};

// Bilinear resize to round(H*scale) x round(W*scale), half-pixel centres
// (layers.cpp:991-1150).
class Upsample : public Module {
public:
    explicit Upsample(float scale_factor = 2.0f) : Module("Upsample"), scale_(scale_factor) {}
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

private:
    float scale_;
};

// [C, H, W] -> [C, 1, 1] plane means (layers.cpp:1274-1345).
class AdaptiveAvgPool2d : public Module {
public:
    AdaptiveAvgPool2d() : Module("AdaptiveAvgPool2d") {}
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;
};

// a [C,H,W] times b [C,1,1] (or [C]) per channel (blocks.cpp:148-212; the
// elementwise branch of the reference's CPU path is not used by the model).
TensorPtr mul_tensors(const TensorPtr& a, const TensorPtr& b);
// g*a + (1-g)*b (blocks.cpp:280-320).
TensorPtr convex_combination(const TensorPtr& g, const TensorPtr& a, const TensorPtr& b);
// The same two gates with the gate's sigmoid folded in: convex_combination
// (sigmoid(z), a, b) and mul_tensors(a, sigmoid(z)), the same values in one
// launch per direction instead of two.
TensorPtr sigmoid_convex_combination(const TensorPtr& z, const TensorPtr& a,
                                     const TensorPtr& b);
TensorPtr mul_sigmoid(const TensorPtr& a, const TensorPtr& z);
// Channel concatenation of [C_i, H, W] tensors (blocks.cpp:363-418).
TensorPtr concat_channels(const std::vector<TensorPtr>& tensors);
// Bilinear resize to target_h x target_w through Upsample(target_h / H)
// (blocks.cpp:420-427); the input itself when the size already matches.
TensorPtr resize_bilinear(const TensorPtr& input, size_t target_h, size_t target_w);

}  // namespace soar::nn
