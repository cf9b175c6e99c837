#include "soar/autograd.hpp"

#include "soar/core.hpp"
#include "soar/kernels.hpp"
#include "soar_gn.h"

#include <queue>
#include <unordered_set>

namespace soar::autograd {

void accumulate_into(const TensorPtr& acc, const TensorPtr& inc);
TensorPtr sum_of(const TensorPtr& a, const TensorPtr& b);

// A node's first incoming gradient is kept by reference, without a copy:
// backward implementations only read their grad_output.  A later arrival
// adds in place when the node holds the only reference to its buffer, and
// otherwise (another node or the caller still reads that buffer) writes the
// sum to a new buffer, which costs one pass where a copy on first arrival
// plus an in-place add cost two.
void AutogradNode::add_grad_output(const TensorPtr& incoming) {
    if (!incoming) return;
    if (!grad_output_)
        grad_output_ = incoming;
    else if (grad_output_.use_count() == 1)
        accumulate_into(grad_output_, incoming);
    else
        grad_output_ = sum_of(grad_output_, incoming);
}

void AutogradNode::add_grad_output(TensorPtr&& incoming) {
    if (!incoming) return;
    if (!grad_output_) {
        grad_output_ = std::move(incoming);
    } else if (grad_output_.use_count() > 1 && incoming.use_count() == 1) {
        accumulate_into(incoming, grad_output_);  // the sum lands in the sole-owner buffer
        grad_output_ = std::move(incoming);
    } else {
        add_grad_output(static_cast<const TensorPtr&>(incoming));
    }
}

void AccumulateGradNode::backward(const TensorPtr& grad_output) {
    if (variable && grad_output) variable->add_grad(grad_output);
}

Engine& Engine::get_default_engine() {
    static Engine engine;
    return engine;
}

void Engine::compute_dependencies(
    AutogradNode* root, std::unordered_map<AutogradNode*, size_t>& dependencies,
    std::unordered_map<AutogradNode*, std::vector<std::shared_ptr<AutogradNode>>>& edges) {
    if (!root) return;
    std::vector<AutogradNode*> stack{root};
    std::unordered_set<AutogradNode*> seen{root};
    while (!stack.empty()) {
        AutogradNode* fn = stack.back();
        stack.pop_back();
        for (const auto& next : fn->get_inputs()) {
            if (!next) continue;
            edges[fn].push_back(next);
            dependencies[next.get()] += 1;
            if (seen.insert(next.get()).second) stack.push_back(next.get());
        }
    }
}

void Engine::execute(std::shared_ptr<AutogradNode> root, const TensorPtr& root_grad) {
    if (!root) return;
    std::unordered_map<AutogradNode*, size_t> deps;
    std::unordered_map<AutogradNode*, std::vector<std::shared_ptr<AutogradNode>>> edges;
    compute_dependencies(root.get(), deps, edges);
    root->add_grad_output(root_grad);
    std::queue<std::shared_ptr<AutogradNode>> ready;
    ready.push(root);
    while (!ready.empty()) {
        auto node = ready.front();
        ready.pop();
        TensorPtr go = std::move(node->grad_output_);
        node->grad_output_ = nullptr;
        if (go) node->backward(go);
        go.reset();
        if (eager_release_) node->release_variables();
        auto it = edges.find(node.get());
        if (it == edges.end()) continue;
        for (const auto& next : it->second) {
            auto d = deps.find(next.get());
            if (d != deps.end() && --d->second == 0) ready.push(next);
        }
    }
    if (!eager_release_) {
        // release everything reached, after the whole pass
        for (auto& [fn, outs] : edges)
            for (auto& n : outs) n->release_variables();
        root->release_variables();
    }
}

namespace {
thread_local bool g_grad_enabled = true;
}

bool GradMode::is_enabled() noexcept { return g_grad_enabled; }
void GradMode::set_enabled(bool on) noexcept { g_grad_enabled = on; }

}  // namespace soar::autograd

namespace soar {

void propagate_grad(const TensorPtr& tensor, const TensorPtr& incoming) {
    if (!tensor || !incoming || !tensor->requires_grad()) return;
    if (auto fn = tensor->grad_fn())
        fn->add_grad_output(incoming);
    else
        tensor->add_grad(incoming);
}

void propagate_grad(const TensorPtr& tensor, TensorPtr&& incoming) {
    if (!tensor || !incoming || !tensor->requires_grad()) return;
    if (auto fn = tensor->grad_fn())
        fn->add_grad_output(std::move(incoming));
    else
        tensor->add_grad(std::move(incoming));
}

TensorPtr grad_sink(const TensorPtr& tensor) {
    if (!tensor || !tensor->requires_grad()) return nullptr;
    const auto fn = tensor->grad_fn();
    if (!fn || !fn->grad_output_ || fn->grad_output_.use_count() != 1) return nullptr;
    const TensorPtr& g = fn->grad_output_;
    if (!g->is_cuda() || g->numel() != tensor->numel()) return nullptr;
    return g;
}

TensorPtr add_target(const TensorPtr& tensor, bool* fresh) {
    if (TensorPtr s = grad_sink(tensor)) {
        *fresh = false;
        return s;
    }
    *fresh = true;
    return Tensor::zeros(tensor->shape(), false, true);
}

TensorPtr write_target(const TensorPtr& tensor, bool* fresh) {
    if (TensorPtr s = grad_sink(tensor)) {
        *fresh = false;
        return s;
    }
    *fresh = true;
    return Tensor::create(tensor->shape(), false, true);
}

void run_backward(std::shared_ptr<AutogradNode> root, const TensorPtr& root_grad) {
    try {
        autograd::Engine::get_default_engine().execute(std::move(root), root_grad);
        // the convolution weight gradients whose final addition the layers
        // left pending (SOAR_DEFER_WEIGHT_FINISH), in one launch
        if (soar_weight_grad_pending() > 0)
            hip::kernels::check(soar_weight_grad_flush(exec::stream()), "weight-gradient finish");
    } catch (...) {
        // An abandoned pass (e.g. OutOfMemory, after which the caller frees
        // the activation arena holding the queued partials and runs the
        // step again): its pending finishes must never run.
        soar_weight_grad_discard();
        throw;
    }
}

}  // namespace soar
