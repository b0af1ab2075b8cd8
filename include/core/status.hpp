#pragma once

// sci::Status / sci::Result<T>: the error-carrying types of the attention stack's public API.
//
// Same API shape as the SciComputeInfra types the reference's public headers are written against
// (reference stub/include/core/status.hpp:13-161): no exceptions, Status carries a code plus a
// message, Result<T> holds either a value or a Status.

#include <cstdint>
#include <new>
#include <string>
#include <type_traits>
#include <utility>

namespace sci {

// Code values are part of the interface shared with SciComputeInfra callers.
enum class StatusCode : int32_t {
    kOk = 0,
    kError = 1,
    kNotFound = 2,
    kInvalidArgument = 4,
    kNotImplemented = 5,
    kOutOfMemory = 6,
    kResourceExhausted = 7,
    kInvalidOperation = 10,
    kInternal = 12,
    kCudaError = 100,        // device runtime error (HIP on this build)
    kCudaNotAvailable = 101, // no usable GPU
    kCudaOutOfMemory = 102,  // device allocation failed
    kDeviceError = 500,
};

inline const char* StatusCodeToString(StatusCode code) noexcept {
    switch (code) {
        case StatusCode::kOk: return "OK";
        case StatusCode::kError: return "Error";
        case StatusCode::kNotFound: return "Not Found";
        case StatusCode::kInvalidArgument: return "Invalid Argument";
        case StatusCode::kNotImplemented: return "Not Implemented";
        case StatusCode::kOutOfMemory: return "Out of Memory";
        case StatusCode::kResourceExhausted: return "Resource Exhausted";
        case StatusCode::kInvalidOperation: return "Invalid Operation";
        case StatusCode::kInternal: return "Internal Error";
        case StatusCode::kCudaError: return "GPU Runtime Error";
        case StatusCode::kCudaNotAvailable: return "GPU Not Available";
        case StatusCode::kCudaOutOfMemory: return "GPU Out of Memory";
        case StatusCode::kDeviceError: return "Device Error";
    }
    return "Unknown";
}

class Status {
public:
    Status() = default;
    Status(StatusCode code, std::string message = {}) : code_(code), message_(std::move(message)) {}

    static Status Ok() { return Status(); }
    static Status Error(const std::string& m = "Unknown error") { return {StatusCode::kError, m}; }
    static Status InvalidArgument(const std::string& m = "Invalid argument") {
        return {StatusCode::kInvalidArgument, m};
    }
    static Status NotImplemented(const std::string& m = "Not implemented") {
        return {StatusCode::kNotImplemented, m};
    }
    static Status InvalidOperation(const std::string& m = "Invalid operation") {
        return {StatusCode::kInvalidOperation, m};
    }
    static Status OutOfMemory(const std::string& m = "Out of memory") {
        return {StatusCode::kOutOfMemory, m};
    }
    static Status CudaError(const std::string& m = "GPU runtime error") {
        return {StatusCode::kCudaError, m};
    }
    static Status CudaNotAvailable(const std::string& m = "GPU not available") {
        return {StatusCode::kCudaNotAvailable, m};
    }
    static Status CudaOutOfMemory(const std::string& m = "GPU out of memory") {
        return {StatusCode::kCudaOutOfMemory, m};
    }

    bool ok() const { return code_ == StatusCode::kOk; }
    StatusCode code() const { return code_; }
    const std::string& message() const { return message_; }
    explicit operator bool() const { return ok(); }
    bool operator==(const Status& other) const { return code_ == other.code_; }
    bool operator!=(const Status& other) const { return code_ != other.code_; }
    std::string ToString() const {
        if (ok()) return "OK";
        return std::string(StatusCodeToString(code_)) + ": " + message_;
    }

private:
    StatusCode code_{StatusCode::kOk};
    std::string message_;
};

struct Unexpected {
    explicit Unexpected(Status s) : error_(std::move(s)) {}
    const Status& error() const { return error_; }
    Status error_;
};

// Value-or-status. Implemented over a tagged union so that T needs no default constructor
// and move-only types (sci::Tensor) are supported.
template <typename T>
class Expected {
public:
    Expected() : has_value_(true) { new (&storage_) T(); }
    explicit Expected(T value) : has_value_(true) { new (&storage_) T(std::move(value)); }
    explicit Expected(Unexpected u) : has_value_(false) { new (&storage_) Status(std::move(u.error_)); }
    Expected(Expected&& other) noexcept : has_value_(other.has_value_) {
        if (has_value_) new (&storage_) T(std::move(*other.ValuePtr()));
        else new (&storage_) Status(std::move(*other.ErrorPtr()));
    }
    Expected(const Expected& other) : has_value_(other.has_value_) {
        if (has_value_) CopyValue(other);
        else new (&storage_) Status(*other.ErrorPtr());
    }
    Expected& operator=(Expected&& other) noexcept {
        if (this != &other) {
            Destroy();
            has_value_ = other.has_value_;
            if (has_value_) new (&storage_) T(std::move(*other.ValuePtr()));
            else new (&storage_) Status(std::move(*other.ErrorPtr()));
        }
        return *this;
    }
    Expected& operator=(const Expected& other) {
        if (this != &other) {
            Destroy();
            has_value_ = other.has_value_;
            if (has_value_) CopyValue(other);
            else new (&storage_) Status(*other.ErrorPtr());
        }
        return *this;
    }
    ~Expected() { Destroy(); }

    bool ok() const noexcept { return has_value_; }
    explicit operator bool() const noexcept { return has_value_; }
    T& value() & { return *ValuePtr(); }
    const T& value() const& { return *ValuePtr(); }
    T* operator->() { return ValuePtr(); }
    const T* operator->() const { return ValuePtr(); }
    T& operator*() { return *ValuePtr(); }
    const T& operator*() const { return *ValuePtr(); }
    Status error() const { return has_value_ ? Status::Ok() : *ErrorPtr(); }
    const std::string& message() const {
        static const std::string kEmpty;
        return has_value_ ? kEmpty : ErrorPtr()->message();
    }

private:
    void CopyValue(const Expected& other) {
        if constexpr (std::is_copy_constructible<T>::value) {
            new (&storage_) T(*other.ValuePtr());
        } else {
            static_assert(std::is_copy_constructible<T>::value,
                          "Expected<T> of a move-only T cannot be copied");
        }
    }
    void Destroy() {
        if (has_value_) ValuePtr()->~T();
        else ErrorPtr()->~Status();
    }
    T* ValuePtr() { return std::launder(reinterpret_cast<T*>(&storage_)); }
    const T* ValuePtr() const { return std::launder(reinterpret_cast<const T*>(&storage_)); }
    Status* ErrorPtr() { return std::launder(reinterpret_cast<Status*>(&storage_)); }
    const Status* ErrorPtr() const { return std::launder(reinterpret_cast<const Status*>(&storage_)); }

    alignas(T) alignas(Status) unsigned char storage_[sizeof(T) > sizeof(Status) ? sizeof(T) : sizeof(Status)];
    bool has_value_{true};
};

template <typename T>
using Result = Expected<T>;

template <typename T>
Expected<T> MakeUnexpected(Status s) {
    return Expected<T>(Unexpected(std::move(s)));
}

template <typename T>
inline Result<T> Ok(T value) {
    return Result<T>(std::move(value));
}

}  // namespace sci
