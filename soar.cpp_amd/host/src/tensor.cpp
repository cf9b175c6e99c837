#include "soar/tensor.hpp"

#include <algorithm>
#include <cstring>

#include "soar/autograd.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar_gn.h"

namespace soar {

namespace {
float* device_storage(int64_t n, const Shape& shape) {
    auto* arena = memory::DeviceArena::current();
    if (!arena)
        throw DeviceError("device tensors are allocated from a DeviceArena: install one with "
                          "memory::ArenaScope");
    return arena->allocate_floats(std::max<int64_t>(n, 1), shape, "tensor");
}
}  // namespace

Tensor::Tensor(Shape shape, bool requires_grad, bool on_device)
    : shape_(std::move(shape)), numel_(soar::numel(shape_)), requires_grad_(requires_grad) {
    if (on_device)
        dev_ = device_storage(numel_, shape_);
    else
        host_.assign((size_t)numel_, 0.0f);
}

Tensor::~Tensor() = default;  // device storage belongs to its arena

TensorPtr Tensor::create(const Shape& shape, bool requires_grad, bool on_device) {
    return TensorPtr(new Tensor(shape, requires_grad, on_device));
}

TensorPtr Tensor::zeros(const Shape& shape, bool requires_grad, bool on_device) {
    TensorPtr t = create(shape, requires_grad, on_device);
    if (on_device) t->zero_();
    return t;
}

TensorPtr Tensor::ones(const Shape& shape, bool requires_grad, bool on_device) {
    return full(shape, 1.0f, requires_grad, on_device);
}

TensorPtr Tensor::full(const Shape& shape, float value, bool requires_grad, bool on_device) {
    TensorPtr t = create(shape, requires_grad, on_device);
    t->fill_(value);
    return t;
}

TensorPtr Tensor::from_blob(const float* host, const Shape& shape, bool requires_grad,
                            bool on_device) {
    TensorPtr t = create(shape, requires_grad, on_device);
    if (t->numel_ == 0) return t;
    if (on_device)
        hip::kernels::check(soar_memcpy_h2d(t->dev_, host, t->bytes(), exec::stream()), "from_blob");
    else
        std::memcpy(t->host_.data(), host, t->bytes());
    return t;
}

int64_t Tensor::dim(int64_t i) const {
    if (i < 0) i += ndim();
    if (i < 0 || i >= ndim()) throw ShapeError("dimension index out of range for " + to_string(shape_));
    return shape_[(size_t)i];
}

float* Tensor::data() {
    if (dev_) throw DeviceError("data(): tensor lives on the device");
    return host_.data();
}
const float* Tensor::data() const {
    if (dev_) throw DeviceError("data(): tensor lives on the device");
    return host_.data();
}
float* Tensor::cuda_data() {
    if (!dev_) throw DeviceError("cuda_data(): tensor lives on the host");
    return dev_;
}
const float* Tensor::cuda_data() const {
    if (!dev_) throw DeviceError("cuda_data(): tensor lives on the host");
    return dev_;
}

void Tensor::to_cuda() {
    if (dev_) return;
    float* d = device_storage(numel_, shape_);
    if (numel_)
        hip::kernels::check(soar_memcpy_h2d(d, host_.data(), bytes(), exec::stream()), "to_cuda");
    dev_ = d;
    host_.clear();
    host_.shrink_to_fit();
}

std::vector<float> Tensor::to_host() const {
    if (!dev_) return host_;
    std::vector<float> out((size_t)numel_);
    if (numel_)
        hip::kernels::check(soar_memcpy_d2h(out.data(), dev_, bytes(), exec::stream()), "to_host");
    return out;
}

void Tensor::copy_from_host(const float* src) {
    if (numel_ == 0) return;
    if (dev_)
        hip::kernels::check(soar_memcpy_h2d(dev_, src, bytes(), exec::stream()), "copy_from_host");
    else
        std::memcpy(host_.data(), src, bytes());
}

TensorPtr Tensor::clone() const {
    TensorPtr t = create(shape_, false, dev_ != nullptr);
    if (numel_ == 0) return t;
    if (dev_)
        hip::kernels::check(soar_memcpy_d2d(t->dev_, dev_, bytes(), exec::stream()), "clone");
    else
        t->host_ = host_;
    return t;
}

void Tensor::zero_() { fill_(0.0f); }

void Tensor::fill_(float value) {
    if (dev_)
        hip::kernels::cuda_fill(dev_, value, (size_t)numel_);
    else
        std::fill(host_.begin(), host_.end(), value);
}

void Tensor::zero_grad() {
    if (grad_) grad_->zero_();
}

namespace autograd {
// acc += inc, elementwise; both on the device (kernel) or both on the host.
void accumulate_into(const TensorPtr& acc, const TensorPtr& inc) {
    if (acc->numel() != inc->numel())
        throw ShapeError("gradient shape " + to_string(inc->shape()) + " does not match " +
                         to_string(acc->shape()));
    if (acc->is_cuda() && inc->is_cuda()) {
        hip::kernels::add_backward(inc->cuda_data(), acc->cuda_data(), nullptr,
                                   (size_t)acc->numel());
    } else if (!acc->is_cuda() && !inc->is_cuda()) {
        float* a = acc->data();
        const float* b = inc->data();
        for (int64_t i = 0; i < acc->numel(); ++i) a[i] += b[i];
    } else {
        throw DeviceError("cannot accumulate a host gradient into a device one (or back)");
    }
}

// a + b into a new tensor, elementwise; both on the device or both on the
// host.
TensorPtr sum_of(const TensorPtr& a, const TensorPtr& b) {
    if (a->numel() != b->numel())
        throw ShapeError("gradient shape " + to_string(b->shape()) + " does not match " +
                         to_string(a->shape()));
    if (a->is_cuda() != b->is_cuda())
        throw DeviceError("cannot add a host gradient to a device one (or back)");
    TensorPtr out = Tensor::create(a->shape(), false, a->is_cuda());
    if (a->is_cuda()) {
        hip::kernels::add_forward(a->cuda_data(), b->cuda_data(), out->cuda_data(),
                                  (size_t)a->numel());
    } else {
        const float* x = a->data();
        const float* y = b->data();
        float* o = out->data();
        for (int64_t i = 0; i < a->numel(); ++i) o[i] = x[i] + y[i];
    }
    return out;
}

// First arrival of a handed-over tensor: adopt it when nobody else holds
// it, else copy, so later in-place accumulation never changes a tensor
// someone else still reads.
TensorPtr adopt_or_copy(TensorPtr&& incoming) {
    if (incoming.use_count() == 1) return std::move(incoming);
    return incoming->clone();
}
}  // namespace autograd

void Tensor::add_grad(const TensorPtr& incoming) {
    if (!incoming) return;
    if (!grad_) {
        grad_ = incoming->clone();
        return;
    }
    autograd::accumulate_into(grad_, incoming);
}

void Tensor::add_grad(TensorPtr&& incoming) {
    if (!incoming) return;
    if (!grad_) {
        grad_ = autograd::adopt_or_copy(std::move(incoming));
        return;
    }
    autograd::accumulate_into(grad_, incoming);
}

void Tensor::backward(TensorPtr gradient) {
    if (!requires_grad_) throw InvalidArgument("backward() on a tensor that does not require grad");
    if (!gradient) gradient = Tensor::ones(shape_, false, is_cuda());
    if (grad_fn_)
        run_backward(grad_fn_, gradient);
    else
        add_grad(std::move(gradient));
}

}  // namespace soar
