// autograd.hpp - reverse-mode execution over AutogradNodes, with the
// reference's semantics (include/soar/autograd/node.hpp:15-77,
// engine.hpp:70-176, src/autograd/engine.cpp:126-224,
// src/tensor/tensor.cpp:173-246):
//   * dependency counting over get_inputs() edges, then a FIFO ready queue;
//   * a node's incoming gradients are merged in add_grad_output (first
//     arrival kept by reference, later arrivals added);
//   * release_variables() right after a node's backward (eager release).
#pragma once

#include <memory>
#include <unordered_map>
#include <vector>

#include "soar/tensor.hpp"

namespace soar::autograd {

struct AutogradNode : std::enable_shared_from_this<AutogradNode> {
    virtual ~AutogradNode() = default;
    virtual void backward(const TensorPtr& grad_output) = 0;
    [[nodiscard]] virtual std::vector<std::shared_ptr<AutogradNode>> get_inputs() const = 0;
    virtual void release_variables() {}
    // Later arrivals are added to the first (tensor.cpp:194-213).  The
    // first is kept by reference, not copied, so backward() must treat its
    // grad_output as read-only; a later arrival adds in place only while
    // this node holds the sole reference, else it sums into a new buffer.
    void add_grad_output(const TensorPtr& incoming);
    void add_grad_output(TensorPtr&& incoming);

    TensorPtr grad_output_;
};

// Leaf accumulation node (engine.hpp:70-88): backward adds into the
// variable's gradient in place.
struct AccumulateGradNode : AutogradNode {
    explicit AccumulateGradNode(TensorPtr v) : variable(std::move(v)) {}
    void backward(const TensorPtr& grad_output) override;
    [[nodiscard]] std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override {
        return {};
    }
    TensorPtr variable;
};

class Engine {
public:
    static Engine& get_default_engine();

    void compute_dependencies(
        AutogradNode* root, std::unordered_map<AutogradNode*, size_t>& dependencies,
        std::unordered_map<AutogradNode*, std::vector<std::shared_ptr<AutogradNode>>>& edges);
    void execute(std::shared_ptr<AutogradNode> root, const TensorPtr& root_grad);

    void set_eager_activation_release(bool on) noexcept { eager_release_ = on; }

private:
    bool eager_release_ = true;
};

// Grad mode: nodes are recorded only while enabled (node.hpp:57-77).
class GradMode {
public:
    static bool is_enabled() noexcept;
    static void set_enabled(bool on) noexcept;
};

class NoGradGuard {
public:
    NoGradGuard() noexcept : prev_(GradMode::is_enabled()) { GradMode::set_enabled(false); }
    ~NoGradGuard() { GradMode::set_enabled(prev_); }

private:
    bool prev_;
};

}  // namespace soar::autograd

namespace soar {
using autograd::AutogradNode;
// Routes a gradient to a tensor: its grad_fn when it has one, else its
// own .grad (tensor.cpp:215-224).  Nothing happens unless the tensor
// requires grad.
void propagate_grad(const TensorPtr& tensor, const TensorPtr& incoming);
// Same, handing over `incoming` (adopted without a copy on first arrival
// when the caller held the only reference).
void propagate_grad(const TensorPtr& tensor, TensorPtr&& incoming);
void run_backward(std::shared_ptr<AutogradNode> root, const TensorPtr& root_grad);
// The pending gradient of `tensor` when a kernel may add into it directly,
// in place of making a fresh gradient and propagating it (which costs a
// separate merge pass): the grad_output of tensor's producing node, if
// that node holds the only reference to it and it is a device tensor of
// tensor's size.  nullptr otherwise (and for leaves).
TensorPtr grad_sink(const TensorPtr& tensor);
// Gradient buffer for a kernel that adds (+=) into it: grad_sink(tensor)
// when there is one (*fresh = false), else fresh device zeros
// (*fresh = true) that the caller hands to propagate_grad.
TensorPtr add_target(const TensorPtr& tensor, bool* fresh);
// Gradient buffer for a kernel that can write or add its result:
// grad_sink(tensor) when there is one (*fresh = false: the kernel adds),
// else a new uninitialised device tensor (*fresh = true: the kernel
// writes, and the caller hands the tensor to propagate_grad).
TensorPtr write_target(const TensorPtr& tensor, bool* fresh);
}  // namespace soar
