// status.hpp -- error model of the executor contract.
//
// Same classes and semantics as AIR's air::Status / air::Result
// (include/air/status.hpp:8-57, include/air/result.hpp:11-49) so code written
// against the reference contract compiles unchanged: nothing throws across
// the contract except Result::value() on a failed result.
#pragma once

#include <optional>
#include <stdexcept>
#include <string>
#include <utility>

namespace air {

enum class ErrorCode {
    ok = 0,
    invalid_argument,
    invalid_state,
    io_error,
    cancelled,
    data_error,
    unsupported,
    internal_error,
};

class Status {
public:
    Status() = default;
    static Status ok() { return {}; }
    static Status invalid_argument(std::string m) { return {ErrorCode::invalid_argument, std::move(m)}; }
    static Status invalid_state(std::string m) { return {ErrorCode::invalid_state, std::move(m)}; }
    static Status io_error(std::string m) { return {ErrorCode::io_error, std::move(m)}; }
    static Status cancelled(std::string m) { return {ErrorCode::cancelled, std::move(m)}; }
    static Status data_error(std::string m) { return {ErrorCode::data_error, std::move(m)}; }
    static Status unsupported(std::string m) { return {ErrorCode::unsupported, std::move(m)}; }
    static Status internal_error(std::string m) { return {ErrorCode::internal_error, std::move(m)}; }

    [[nodiscard]] bool is_ok() const noexcept { return code_ == ErrorCode::ok; }
    [[nodiscard]] explicit operator bool() const noexcept { return is_ok(); }
    [[nodiscard]] ErrorCode code() const noexcept { return code_; }
    [[nodiscard]] const std::string& message() const noexcept { return message_; }

private:
    Status(ErrorCode code, std::string message) : code_(code), message_(std::move(message)) {}
    ErrorCode code_{ErrorCode::ok};
    std::string message_;
};

template <typename T>
class Result {
public:
    Result(T value) : value_(std::move(value)) {}
    Result(Status status) : status_(std::move(status)) {
        if (status_.is_ok()) throw std::invalid_argument("Result error constructor requires a non-ok status");
    }
    [[nodiscard]] bool is_ok() const noexcept { return value_.has_value(); }
    [[nodiscard]] explicit operator bool() const noexcept { return is_ok(); }
    [[nodiscard]] const Status& status() const noexcept { return status_; }
    [[nodiscard]] const T& value() const& { check(); return *value_; }
    [[nodiscard]] T& value() & { check(); return *value_; }
    [[nodiscard]] T&& value() && { check(); return std::move(*value_); }

private:
    void check() const {
        if (!value_) throw std::logic_error("attempted to read value from failed Result");
    }
    std::optional<T> value_;
    Status status_{};
};

} // namespace air
