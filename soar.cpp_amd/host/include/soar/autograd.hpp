// autograd.hpp - reverse-mode execution over AutogradNodes, with the
// reference's semantics (include/soar/autograd/node.hpp:15-77,
// engine.hpp:70-176, src/autograd/engine.cpp:126-224,
// src/tensor/tensor.cpp:173-246):
//   * dependency counting over get_inputs() edges, then a FIFO ready queue;
//   * a node's incoming gradients are merged in add_grad_output (first
//     arrival kept, later arrivals accumulated);
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
    // First arrival kept (a copy; the rvalue overload adopts a sole-owner
    // tensor), later arrivals accumulated (tensor.cpp:194-213).
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
}  // namespace soar
