// tensor.hpp - the Tensor of the host layer: shape, storage on the host or
// in device memory from the current DeviceArena, and autograd state
// (requires_grad, grad, grad_fn).  Mirrors the reference's Tensor API
// (include/soar/tensor/tensor.hpp:28-130, src/tensor/tensor.cpp:17-271)
// for the operations the GroupNorm path uses.  A device tensor has no host
// shadow (the reference zero-fills one for every device tensor,
// tensor.cpp:19-23).
#pragma once

#include <memory>
#include <vector>

#include "soar/core.hpp"

namespace soar {

namespace autograd {
struct AutogradNode;
}

class Tensor;
using TensorPtr = std::shared_ptr<Tensor>;

class Tensor : public std::enable_shared_from_this<Tensor> {
public:
    // Uninitialised storage (host tensors are zero-filled).
    static TensorPtr create(const Shape& shape, bool requires_grad = false,
                            bool on_device = false);
    static TensorPtr zeros(const Shape& shape, bool requires_grad = false,
                           bool on_device = false);
    static TensorPtr ones(const Shape& shape, bool requires_grad = false,
                          bool on_device = false);
    static TensorPtr full(const Shape& shape, float value, bool requires_grad = false,
                          bool on_device = false);
    // Copies `count` = numel(shape) floats from host memory.
    static TensorPtr from_blob(const float* host, const Shape& shape,
                               bool requires_grad = false, bool on_device = false);

    ~Tensor();

    [[nodiscard]] const Shape& shape() const noexcept { return shape_; }
    [[nodiscard]] int64_t ndim() const noexcept { return (int64_t)shape_.size(); }
    [[nodiscard]] int64_t dim(int64_t i) const;
    [[nodiscard]] int64_t numel() const noexcept { return numel_; }
    [[nodiscard]] size_t bytes() const noexcept { return (size_t)numel_ * sizeof(float); }

    // Device-resident (the reference's name for it).
    [[nodiscard]] bool is_cuda() const noexcept { return dev_ != nullptr; }
    // Host storage; throws DeviceError for a device tensor.
    float* data();
    const float* data() const;
    // Device storage; throws DeviceError for a host tensor.
    float* cuda_data();
    const float* cuda_data() const;

    // Moves a host tensor to the device (storage from the current arena).
    void to_cuda();
    // Copy of the values on the host (synchronous).
    [[nodiscard]] std::vector<float> to_host() const;
    // Overwrites the values from numel() host floats (device or host).
    void copy_from_host(const float* src);
    [[nodiscard]] TensorPtr clone() const;
    void zero_();
    void fill_(float value);

    [[nodiscard]] bool requires_grad() const noexcept { return requires_grad_; }
    void set_requires_grad(bool r) noexcept { requires_grad_ = r; }
    [[nodiscard]] TensorPtr grad() const noexcept { return grad_; }
    void set_grad(TensorPtr g) noexcept { grad_ = std::move(g); }
    void zero_grad();
    // First arrival keeps a copy, later arrivals accumulate in place, so
    // the gradient buffer keeps its address (tensor.cpp:173-192).  The
    // rvalue overload adopts the incoming tensor instead of copying it when
    // the caller gives up the only reference.
    void add_grad(const TensorPtr& incoming);
    void add_grad(TensorPtr&& incoming);

    [[nodiscard]] std::shared_ptr<autograd::AutogradNode> grad_fn() const noexcept {
        return grad_fn_;
    }
    void set_grad_fn(std::shared_ptr<autograd::AutogradNode> fn) noexcept {
        grad_fn_ = std::move(fn);
    }
    // Runs the engine from this tensor's grad_fn with `gradient` (ones of
    // this shape when null).
    void backward(TensorPtr gradient = nullptr);

private:
    Tensor(Shape shape, bool requires_grad, bool on_device);

    Shape shape_;
    int64_t numel_ = 0;
    std::vector<float> host_;
    float* dev_ = nullptr;  // owned by the arena it came from
    bool requires_grad_ = false;
    TensorPtr grad_;
    std::shared_ptr<autograd::AutogradNode> grad_fn_;
};

}  // namespace soar
