// memory.hpp - device memory for tensors: a bump-allocated slab with a
// static region (parameters and their gradients) and a dynamic region
// (activations, statistics, workspaces) reset in O(1) per step.
//
// DeviceSlabSubAllocator keeps the reference's bookkeeping and API
// (include/soar/memory/device_slab.hpp:21-47, src/memory/device_slab.cpp:
// 6-56); DeviceArena backs it with one device allocation from
// libsoar_gn.so in place of the reference's VulkanBuffer / CudaMemoryPool
// storage (src/vulkan/buffer.cpp:8-75, src/cuda/cuda_allocator.cpp:24-77).
#pragma once

#include <cstddef>
#include <string>
#include <string_view>
#include <vector>

#include "soar/core.hpp"

struct soar_arena;

namespace soar::memory {

enum class DataType { Float32, Float16 };

struct SubAllocation {
    size_t offset{0};
    size_t size{0};
    Shape shape{};
    DataType dtype{DataType::Float32};
    std::string tag{};
};

class DeviceSlabSubAllocator {
public:
    explicit DeviceSlabSubAllocator(size_t total_capacity_bytes, size_t alignment = 256) noexcept
        : total_capacity_(total_capacity_bytes), alignment_(alignment) {}

    // Zero bytes -> InvalidArgument; past capacity -> OutOfMemory.
    Result<SubAllocation> sub_allocate(size_t size_bytes, Shape shape = {},
                                       DataType dtype = DataType::Float32,
                                       std::string_view tag = "") noexcept;
    // Everything allocated so far becomes the static region.
    void freeze_static_parameters() noexcept;
    // Drops every allocation past the static boundary; the next step's
    // allocations land at the same offsets.
    void reset_dynamic_allocations() noexcept;

    [[nodiscard]] size_t total_capacity() const noexcept { return total_capacity_; }
    [[nodiscard]] size_t current_offset() const noexcept { return current_offset_; }
    [[nodiscard]] size_t static_boundary() const noexcept { return static_boundary_; }
    [[nodiscard]] size_t alignment() const noexcept { return alignment_; }
    [[nodiscard]] const std::vector<SubAllocation>& allocations() const noexcept {
        return allocations_;
    }

private:
    size_t total_capacity_{0};
    size_t alignment_{256};
    size_t current_offset_{0};
    size_t static_boundary_{0};
    std::vector<SubAllocation> allocations_{};
};

class DeviceArena {
public:
    explicit DeviceArena(size_t capacity_bytes, size_t alignment = 256);
    ~DeviceArena();
    DeviceArena(const DeviceArena&) = delete;
    DeviceArena& operator=(const DeviceArena&) = delete;

    void* allocate(size_t bytes, const Shape& shape = {}, std::string_view tag = "");
    float* allocate_floats(int64_t n, const Shape& shape = {}, std::string_view tag = "");
    void freeze_static_parameters() noexcept { slab_.freeze_static_parameters(); }
    void reset_dynamic_allocations() noexcept { slab_.reset_dynamic_allocations(); }

    [[nodiscard]] const DeviceSlabSubAllocator& slab() const noexcept { return slab_; }
    [[nodiscard]] void* base() const noexcept { return base_; }

    // The arena device tensors are allocated from on this thread (null if
    // none is installed).
    static DeviceArena* current() noexcept;

private:
    friend class ArenaScope;
    soar_arena* handle_ = nullptr;
    void* base_ = nullptr;
    DeviceSlabSubAllocator slab_;
};

// Installs an arena as the current one for the scope's lifetime.
class ArenaScope {
public:
    explicit ArenaScope(DeviceArena& arena) noexcept;
    ~ArenaScope();
    ArenaScope(const ArenaScope&) = delete;
    ArenaScope& operator=(const ArenaScope&) = delete;

private:
    DeviceArena* prev_;
};

}  // namespace soar::memory
