#pragma once

// Error values without exceptions. Same contract as the reference's
// include/minicompiler/result.hpp:14-69: a fallible call returns Status (ok or
// an Error) or Result<T> (a T or an Error) and the caller checks ok().

#include <cassert>
#include <string>
#include <utility>
#include <variant>

namespace minicompiler {

struct Error {
    std::string message;
};

class [[nodiscard]] Status {
public:
    Status() = default;
    Status(Error error) : failed_(true), error_(std::move(error)) {}

    bool ok() const { return !failed_; }
    const Error& error() const {
        assert(failed_);
        return error_;
    }
    const std::string& message() const { return error().message; }

private:
    bool failed_ = false;
    Error error_;
};

template <typename T>
class [[nodiscard]] Result {
public:
    Result(T value) : v_(std::in_place_index<0>, std::move(value)) {}
    Result(Error error) : v_(std::in_place_index<1>, std::move(error)) {}

    bool ok() const { return v_.index() == 0; }

    T& value() & {
        assert(ok());
        return std::get<0>(v_);
    }
    const T& value() const& {
        assert(ok());
        return std::get<0>(v_);
    }
    T&& value() && {
        assert(ok());
        return std::get<0>(std::move(v_));
    }
    const Error& error() const {
        assert(!ok());
        return std::get<1>(v_);
    }

    T* operator->() { return &value(); }
    const T* operator->() const { return &value(); }
    T& operator*() & { return value(); }
    const T& operator*() const& { return value(); }

    Status status() const { return ok() ? Status() : Status(error()); }

private:
    std::variant<T, Error> v_;
};

}  // namespace minicompiler
