#include "soar/memory.hpp"

#include <algorithm>

#include "soar/kernels.hpp"
#include "soar_gn.h"

namespace soar::memory {

Result<SubAllocation> DeviceSlabSubAllocator::sub_allocate(size_t size_bytes, Shape shape,
                                                           DataType dtype,
                                                           std::string_view tag) noexcept {
    if (size_bytes == 0)
        return Status(StatusCode::InvalidArgument, "device slab: a sub-allocation needs a nonzero size");
    const size_t aligned = (current_offset_ + alignment_ - 1) & ~(alignment_ - 1);
    if (aligned < current_offset_ || aligned > total_capacity_ ||
        total_capacity_ - aligned < size_bytes)
        return Status(StatusCode::OutOfMemory, "Device slab capacity exceeded");
    SubAllocation a;
    a.offset = aligned;
    a.size = size_bytes;
    a.shape = std::move(shape);
    a.dtype = dtype;
    a.tag = std::string(tag);
    allocations_.push_back(a);
    current_offset_ = aligned + size_bytes;
    return a;
}

void DeviceSlabSubAllocator::freeze_static_parameters() noexcept {
    static_boundary_ = std::min((current_offset_ + alignment_ - 1) & ~(alignment_ - 1),
                                total_capacity_);
    current_offset_ = static_boundary_;
}

void DeviceSlabSubAllocator::reset_dynamic_allocations() noexcept {
    current_offset_ = static_boundary_;
    std::erase_if(allocations_, [this](const SubAllocation& a) { return a.offset >= static_boundary_; });
}

namespace {
thread_local DeviceArena* g_current = nullptr;
}

DeviceArena::DeviceArena(size_t capacity_bytes, size_t alignment)
    : slab_(capacity_bytes, alignment) {
    if (alignment == 0 || (alignment & (alignment - 1)))
        throw InvalidArgument("arena alignment must be a power of two");
    hip::kernels::check(soar_arena_create(capacity_bytes, alignment, &handle_), "arena create");
    // One device block; DeviceSlabSubAllocator hands out offsets inside it.
    int rc = soar_arena_alloc(handle_, capacity_bytes, &base_, nullptr);
    if (rc != SOAR_OK) {
        soar_arena_destroy(handle_);
        hip::kernels::check(rc, "arena block");
    }
}

DeviceArena::~DeviceArena() {
    if (g_current == this) g_current = nullptr;
    if (handle_) soar_arena_destroy(handle_);
}

void* DeviceArena::allocate(size_t bytes, const Shape& shape, std::string_view tag) {
    auto r = slab_.sub_allocate(bytes, shape, DataType::Float32, tag);
    if (!r.ok()) {
        if (r.status().code() == StatusCode::OutOfMemory) throw OutOfMemory(r.status().message());
        throw InvalidArgument(r.status().message());
    }
    return static_cast<char*>(base_) + r.value().offset;
}

float* DeviceArena::allocate_floats(int64_t n, const Shape& shape, std::string_view tag) {
    if (n <= 0) throw InvalidArgument("allocate_floats needs a positive count");
    return static_cast<float*>(allocate((size_t)n * sizeof(float), shape, tag));
}

DeviceArena* DeviceArena::current() noexcept { return g_current; }

ArenaScope::ArenaScope(DeviceArena& arena) noexcept : prev_(g_current) { g_current = &arena; }
ArenaScope::~ArenaScope() { g_current = prev_; }

}  // namespace soar::memory
