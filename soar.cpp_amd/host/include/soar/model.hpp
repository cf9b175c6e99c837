// model.hpp - the SOAR segmentation network on the MI355X kernels: the
// blocks of include/soar/nn/blocks.hpp:36-124 (Down, LKR, Ctx, Fuse, Agg,
// SegHead) and SOARModel of include/soar/nn/soar_model.hpp:9-66 with its
// five width/depth variants and the .soar weight format
// (src/nn/soar_model.cpp:175-523).
//
// Submodule and parameter names follow the reference exactly (e.g.
// "l2_lkr.pw2.norm.weight"), so .soar files are interchangeable.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "soar/nn.hpp"

namespace soar::nn {

// Depthwise stride-2 CBA then pointwise CBA (blocks.cpp:447-458).
class Down : public Module {
public:
    Down(size_t c1, size_t c2);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

private:
    std::shared_ptr<CBA> dw_, pw_;
};

// x + pw2(pw1(dw(x))), hidden width max(c*e, 8); pw2's GroupNorm weight
// starts at zero so the block starts as the identity (blocks.cpp:463-481).
class LKR : public Module {
public:
    LKR(size_t c, size_t k = 7, float e = 2.0f);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

private:
    std::shared_ptr<CBA> dw_, pw1_, pw2_;
};

// Multi-scale context: cv1, dilated depthwise branches, cv2 over the
// concatenation, gated by sigmoid(gate_conv(avg_pool(x))), plus x when
// c1 == c2 (blocks.cpp:486-519).
class Ctx : public Module {
public:
    Ctx(size_t c1, size_t c2, const std::vector<size_t>& dilations = {1, 3, 5});
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

private:
    bool add_;
    std::shared_ptr<CBA> cv1_;
    std::vector<std::shared_ptr<CBA>> branches_;
    std::shared_ptr<CBA> cv2_;
    std::shared_ptr<AdaptiveAvgPool2d> pool_;
    std::shared_ptr<Conv2d> gate_conv_;
    std::shared_ptr<Sigmoid> gate_sig_;
};

// Gated convex fusion of an upsampled low-resolution input with a skip
// input (blocks.cpp:524-559); forward({low, skip}).
class Fuse : public Module {
public:
    Fuse(size_t c_low, size_t c_skip, size_t c2);
    using Module::forward;
    TensorPtr forward(const std::vector<TensorPtr>& inputs) override;

private:
    std::shared_ptr<CBA> low_, skip_, gate_dw_;
    std::shared_ptr<Conv2d> gate_conv_;
    std::shared_ptr<Sigmoid> gate_sig_;
    std::shared_ptr<CBA> out_dw_, out_pw_;
};

// Projects each input to max(c2/2, 8) channels, resizes to the first
// input's size, concatenates and fuses (blocks.cpp:564-591).
class Agg : public Module {
public:
    Agg(const std::vector<size_t>& chs, size_t c2);
    using Module::forward;
    TensorPtr forward(const std::vector<TensorPtr>& inputs) override;

private:
    std::vector<std::shared_ptr<CBA>> proj_;
    std::shared_ptr<CBA> fuse_;
};

// Sub-pixel head: depthwise + pointwise refine, a 1x1 prediction of
// nc*r*r channels (bias -log((1-prior)/prior)), PixelShuffle(r)
// (blocks.cpp:596-620).
class SegHead : public Module {
public:
    SegHead(size_t c1, size_t nc, size_t mid = 32, size_t r = 2, float prior = 0.01f);
    using Module::forward;
    TensorPtr forward(const TensorPtr& input) override;

private:
    std::shared_ptr<CBA> refine_dw_, refine_pw_;
    std::shared_ptr<Conv2d> pred_;
    std::shared_ptr<PixelShuffle> shuffle_;
};

enum class ModelVariant { Nano = 0, Small = 1, Medium = 2, Large = 3, XLarge = 4 };

// Pads [C,H,W] up to multiples of `divisor` by reflection (or edge
// repetition when the pad is not smaller than the image) and crops back
// (soar_model.cpp:15-172); both differentiable.
TensorPtr pad_spatial(const TensorPtr& input, size_t ph, size_t pw);
TensorPtr unpad_spatial(const TensorPtr& input, size_t orig_h, size_t orig_w);

class SOARModel : public Module {
public:
    SOARModel(size_t in_channels = 1, size_t num_classes = 1,
              ModelVariant variant = ModelVariant::Nano);
    using Module::forward;
    // [C,H,W] -> logits [num_classes,H,W]; [B,C,H,W] runs sample by sample
    // (soar_model.cpp:258-314).  H and W are padded to multiples of 32.
    TensorPtr forward(const TensorPtr& input) override;

    [[nodiscard]] size_t in_channels() const noexcept { return in_channels_; }
    [[nodiscard]] size_t num_classes() const noexcept { return num_classes_; }
    [[nodiscard]] ModelVariant variant() const noexcept { return variant_; }
    [[nodiscard]] size_t parameter_count() const;

    // The .soar format (soar_model.cpp:427-523): u32 magic 0x534F4152
    // ("SOAR" little-endian), u32 version 1, u32 variant, u32 tensor count,
    // then per tensor: name[128] (NUL-padded), u32 ndim, u32 shape[4]
    // (unused dims 1), u64 byte count, raw fp32 data; tensors in
    // named_parameters() order.  Loading matches by name; a tensor whose
    // byte count differs, or whose name is unknown, is skipped.  Device
    // parameters are read back / written through.
    void save_weights(const std::string& path) const;
    // Returns the number of tensors loaded.
    size_t load_weights(const std::string& path);

private:
    TensorPtr forward_one(const TensorPtr& input);

    size_t in_channels_, num_classes_;
    ModelVariant variant_;
    std::shared_ptr<CBA> l0_cba_;
    std::shared_ptr<Down> l1_down_, l3_down_, l5_down_, l7_down_;
    std::vector<std::shared_ptr<LKR>> l2_, l4_, l6_, l8_, l11_, l13_;
    std::shared_ptr<Ctx> l9_ctx_;
    std::shared_ptr<Fuse> l10_fuse_, l12_fuse_, l14_fuse_, l16_fuse_;
    std::shared_ptr<Agg> l15_agg_;
    std::shared_ptr<SegHead> l17_head_;
};

}  // namespace soar::nn
