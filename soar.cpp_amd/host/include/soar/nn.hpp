// nn.hpp - the GroupNorm / SiLU layers and the residual add of the SOAR
// blocks, running on the MI355X kernels of libsoar_gn.so.
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
#pragma once

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

class Module {
public:
    explicit Module(std::string name) : name_(std::move(name)) {}
    virtual ~Module() = default;
    virtual TensorPtr forward(const TensorPtr& input) = 0;

    void register_parameter(const std::string& name, TensorPtr p);
    [[nodiscard]] std::vector<std::pair<std::string, TensorPtr>> named_parameters(
        const std::string& prefix = "") const;
    // Moves every parameter to the device (allocated from the current
    // arena: do this before freeze_static_parameters()).
    void to_device();
    void zero_grad();
    [[nodiscard]] const std::string& name() const noexcept { return name_; }

private:
    std::string name_;
    std::vector<std::pair<std::string, TensorPtr>> params_;
};

class GroupNorm : public Module {
public:
    GroupNorm(size_t num_groups, size_t num_channels, float eps = 1e-5f, bool affine = true);
    TensorPtr forward(const TensorPtr& input) override;

    [[nodiscard]] size_t num_groups() const noexcept { return num_groups_; }
    [[nodiscard]] size_t num_channels() const noexcept { return num_channels_; }
    [[nodiscard]] float eps() const noexcept { return eps_; }
    [[nodiscard]] TensorPtr weight() const { return weight_; }
    [[nodiscard]] TensorPtr bias() const { return bias_; }

protected:
    GroupNorm(std::string name, size_t num_groups, size_t num_channels, float eps, bool affine);
    TensorPtr run(const TensorPtr& input, unsigned flags);

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
    TensorPtr forward(const TensorPtr& input) override;
};

// silu(group_norm(x)), or x + silu(group_norm(x)) with residual = true.
class GNSiLU : public GroupNorm {
public:
    GNSiLU(size_t num_groups, size_t num_channels, float eps = 1e-5f, bool affine = true,
           bool residual = false);
    TensorPtr forward(const TensorPtr& input) override;
    [[nodiscard]] bool residual() const noexcept { return residual_; }

private:
    bool residual_;
};

// y = a + b (blocks.cpp:39-72); shapes must match (ShapeError otherwise).
TensorPtr add_tensors(const TensorPtr& a, const TensorPtr& b);

}  // namespace soar::nn
