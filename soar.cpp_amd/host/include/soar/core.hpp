// core.hpp - shapes, status codes and the exception hierarchy of the host
// layer (the parts of the reference's include/soar/core/error.hpp:11-107
// and shape.hpp:14-87 that the GroupNorm path's boundary uses).
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace soar {

using Shape = std::vector<int64_t>;

int64_t numel(const Shape& s);
std::string to_string(const Shape& s);

enum class StatusCode { Ok = 0, InvalidArgument, OutOfMemory, DeviceError, ShapeError };

class Status {
public:
    Status() = default;
    Status(StatusCode code, std::string message) : code_(code), message_(std::move(message)) {}
    [[nodiscard]] bool ok() const noexcept { return code_ == StatusCode::Ok; }
    [[nodiscard]] StatusCode code() const noexcept { return code_; }
    [[nodiscard]] const std::string& message() const noexcept { return message_; }

private:
    StatusCode code_ = StatusCode::Ok;
    std::string message_;
};

template <typename T>
class Result {
public:
    Result(T value) : value_(std::move(value)) {}  // NOLINT: implicit like the reference
    Result(Status status) : status_(std::move(status)) {}  // NOLINT
    [[nodiscard]] bool ok() const noexcept { return status_.ok(); }
    [[nodiscard]] const Status& status() const noexcept { return status_; }
    [[nodiscard]] const T& value() const {
        if (!ok()) throw std::logic_error("Result::value() on error: " + status_.message());
        return value_;
    }

private:
    Status status_;
    T value_{};
};

class SoarError : public std::runtime_error {
public:
    SoarError(StatusCode code, const std::string& what) : std::runtime_error(what), code_(code) {}
    [[nodiscard]] StatusCode code() const noexcept { return code_; }

private:
    StatusCode code_;
};

struct InvalidArgument : SoarError {
    explicit InvalidArgument(const std::string& w) : SoarError(StatusCode::InvalidArgument, w) {}
};
struct OutOfMemory : SoarError {
    explicit OutOfMemory(const std::string& w) : SoarError(StatusCode::OutOfMemory, w) {}
};
struct DeviceError : SoarError {
    explicit DeviceError(const std::string& w) : SoarError(StatusCode::DeviceError, w) {}
};
struct ShapeError : SoarError {
    explicit ShapeError(const std::string& w) : SoarError(StatusCode::ShapeError, w) {}
};

// The stream (a hipStream_t) that the host layer's device work goes to:
// every C-ABI call of the layers, the autograd nodes, the loss and the
// optimizer passes exec::stream().  Thread-local; null (the device's
// default stream) unless a StreamScope is active, as during a model
// handle's training step, which runs on its own stream so that it can be
// captured into a graph.
namespace exec {
void* stream() noexcept;
class StreamScope {
public:
    explicit StreamScope(void* stream) noexcept;
    ~StreamScope();
    StreamScope(const StreamScope&) = delete;
    StreamScope& operator=(const StreamScope&) = delete;

private:
    void* prev_;
};
}  // namespace exec

}  // namespace soar
