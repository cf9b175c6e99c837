// Host-only tests of the C++ layer (no device needed):
//  * DeviceSlabSubAllocator against the reference's slab test
//    (tests/test_palloc_memory.cpp:74-115 of pomagrenate/soar.cpp);
//  * the autograd engine against the reference's engine test
//    (tests/test_autograd_engine.cpp:28-102): in-degree counting on a DAG
//    with a shared leaf, in-place gradient accumulation with a stable
//    gradient buffer;
//  * gradient routing (first arrival kept or copied, later ones summed),
//    grad mode, and that the layers refuse to run without a device.
#include <cstdio>
#include <memory>

#include "check.hpp"
#include "soar/autograd.hpp"
#include "soar/kernels.hpp"
#include "soar/memory.hpp"
#include "soar/nn.hpp"

using namespace soar;
using namespace soar::autograd;
using soar::memory::DataType;
using soar::memory::DeviceSlabSubAllocator;

// Test-only node: passes its gradient to two input nodes.
struct PairNode : AutogradNode {
    std::shared_ptr<AutogradNode> lhs, rhs;
    PairNode(std::shared_ptr<AutogradNode> l, std::shared_ptr<AutogradNode> r)
        : lhs(std::move(l)), rhs(std::move(r)) {}
    void backward(const TensorPtr& g) override {
        if (lhs) lhs->add_grad_output(g);
        if (rhs) rhs->add_grad_output(g);
    }
    std::vector<std::shared_ptr<AutogradNode>> get_inputs() const override { return {lhs, rhs}; }
};

static void test_device_slab_sub_allocator() {
    DeviceSlabSubAllocator slab(256u * 1024 * 1024, 256);
    auto w1 = slab.sub_allocate(1024 * 1024 * 4, Shape{64, 3, 3, 3}, DataType::Float32, "w1");
    CHECK(w1.ok() && w1.value().offset % 256 == 0);
    auto w2 = slab.sub_allocate(1024 * 1024 * 8 + 3, Shape{128, 64, 3, 3}, DataType::Float32, "w2");
    CHECK(w2.ok() && w2.value().offset % 256 == 0);
    slab.freeze_static_parameters();
    const size_t sb = slab.static_boundary();
    CHECK(sb > 0 && sb % 256 == 0 && slab.current_offset() == sb);
    auto a1 = slab.sub_allocate(512 * 512 * 64 * 2, Shape{1, 64, 512, 512}, DataType::Float16, "a1");
    CHECK(a1.ok() && a1.value().offset >= sb && a1.value().offset % 256 == 0);
    auto a2 = slab.sub_allocate(256 * 256 * 128 * 2, Shape{1, 128, 256, 256}, DataType::Float16, "a2");
    CHECK(a2.ok() && a2.value().offset % 256 == 0);
    CHECK(slab.allocations().size() == 4);
    slab.reset_dynamic_allocations();
    CHECK(slab.current_offset() == sb && slab.allocations().size() == 2);
    auto a1b = slab.sub_allocate(512 * 512 * 64 * 2, Shape{1, 64, 512, 512}, DataType::Float16, "a1b");
    CHECK(a1b.ok() && a1b.value().offset == a1.value().offset);
    auto zero = slab.sub_allocate(0);
    CHECK(!zero.ok() && zero.status().code() == StatusCode::InvalidArgument);
    auto big = slab.sub_allocate(300u * 1024 * 1024);
    CHECK(!big.ok() && big.status().code() == StatusCode::OutOfMemory);
}

static void test_dag_dependency_counting() {
    auto a = Tensor::create({2}, true), b = Tensor::create({2}, true), c = Tensor::create({2}, true);
    auto acc_a = std::make_shared<AccumulateGradNode>(a);
    auto acc_b = std::make_shared<AccumulateGradNode>(b);
    auto acc_c = std::make_shared<AccumulateGradNode>(c);
    auto add1 = std::make_shared<PairNode>(acc_a, acc_b);
    auto add2 = std::make_shared<PairNode>(acc_b, acc_c);
    auto root = std::make_shared<PairNode>(add1, add2);
    std::unordered_map<AutogradNode*, size_t> deps;
    std::unordered_map<AutogradNode*, std::vector<std::shared_ptr<AutogradNode>>> edges;
    Engine::get_default_engine().compute_dependencies(root.get(), deps, edges);
    CHECK(deps[add1.get()] == 1 && deps[add2.get()] == 1);
    CHECK(deps[acc_a.get()] == 1 && deps[acc_b.get()] == 2 && deps[acc_c.get()] == 1);
    // and the whole DAG runs: b receives the root gradient twice
    auto g = Tensor::full({2}, 1.0f);
    Engine::get_default_engine().execute(root, g);
    CHECK(a->grad()->data()[0] == 1.0f && b->grad()->data()[0] == 2.0f &&
          c->grad()->data()[1] == 1.0f);
}

static void test_accumulation_keeps_buffer() {
    auto w = Tensor::create({2}, true);
    w->data()[0] = 3.0f;
    w->data()[1] = -2.0f;
    auto acc_w = std::make_shared<AccumulateGradNode>(w);
    auto root = std::make_shared<PairNode>(acc_w, acc_w);
    auto g = Tensor::full({2}, 1.0f);
    Engine::get_default_engine().execute(root, g);
    CHECK(w->grad() && w->grad()->data()[0] == 2.0f && w->grad()->data()[1] == 2.0f);
    const float* first = w->grad()->data();
    auto root2 = std::make_shared<PairNode>(acc_w, acc_w);
    Engine::get_default_engine().execute(root2, g);
    CHECK(w->grad()->data() == first);
    CHECK(w->grad()->data()[0] == 4.0f && w->grad()->data()[1] == 4.0f);
    // the caller's gradient tensor was never modified in place
    CHECK(g->data()[0] == 1.0f);
}

static void test_propagate_grad_routing() {
    auto leaf = Tensor::create({3}, true);
    auto frozen = Tensor::create({3}, false);
    auto g = Tensor::full({3}, 2.0f);
    propagate_grad(frozen, g);
    CHECK(!frozen->grad());
    propagate_grad(leaf, g);  // passed by reference -> a copy is kept
    CHECK(leaf->grad() && leaf->grad() != g);
    g->data()[0] = 100.0f;
    CHECK(leaf->grad()->data()[0] == 2.0f);
    auto tmp = Tensor::full({3}, 1.0f);
    auto leaf2 = Tensor::create({3}, true);
    Tensor* raw = tmp.get();
    leaf2->add_grad(std::move(tmp));  // sole owner hands it over
    CHECK(leaf2->grad().get() == raw);
    CHECK_THROWS(leaf2->add_grad(Tensor::full({4}, 1.0f)), ShapeError);
}

static void test_grad_mode() {
    CHECK(GradMode::is_enabled());
    {
        NoGradGuard g;
        CHECK(!GradMode::is_enabled());
        {
            NoGradGuard g2;
            CHECK(!GradMode::is_enabled());
        }
        CHECK(!GradMode::is_enabled());
    }
    CHECK(GradMode::is_enabled());
}

static void test_layers_need_a_device() {
    CHECK(nn::select_group_count(32) == 8 && nn::select_group_count(12) == 6 &&
          nn::select_group_count(7) == 7 && nn::select_group_count(9, 8) == 3);
    CHECK_THROWS(nn::GroupNorm(3, 8), InvalidArgument);
    nn::GroupNorm gn(2, 4);
    auto names = gn.named_parameters("norm");
    // name-sorted like the reference's std::map (module.hpp:133-134)
    CHECK(names.size() == 2 && names[0].first == "norm.bias" && names[1].first == "norm.weight");
    CHECK(names[1].second->data()[3] == 1.0f && names[0].second->data()[0] == 0.0f);
    auto x = Tensor::create({4, 8, 8}, true);
    CHECK_THROWS(gn.forward(Tensor::create({3, 8, 8})), ShapeError);
    if (!hip::kernels::is_cuda_available()) {
        // no host fallback: a layer on a machine without a device fails
        // loudly (no arena can even be created)
        CHECK_THROWS(memory::DeviceArena(1 << 20), DeviceError);
        CHECK_THROWS(gn.forward(x), DeviceError);
    }
    CHECK_THROWS(nn::add_tensors(Tensor::create({2}), Tensor::create({3})), ShapeError);
}

int main() {
    std::printf("=== host layer: CPU tests ===\n");
    int fails = 0;
    fails += run_test("device_slab_sub_allocator", test_device_slab_sub_allocator);
    fails += run_test("dag_dependency_counting", test_dag_dependency_counting);
    fails += run_test("accumulation_keeps_buffer", test_accumulation_keeps_buffer);
    fails += run_test("propagate_grad_routing", test_propagate_grad_routing);
    fails += run_test("grad_mode", test_grad_mode);
    fails += run_test("layers_need_a_device", test_layers_need_a_device);
    std::printf("%s (%d failed)\n", fails ? "FAILED" : "ALL PASSED", fails);
    return fails ? 1 : 0;
}
