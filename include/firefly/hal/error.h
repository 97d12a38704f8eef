// error.h - status values of the HAL layer (reference include/firefly/hal/error.h:20-212).
//
// Callers of the reference use these names: `Result<T>` (has_value(), explicit operator bool, value(), error()),
// `Status` = Result<void>, `Error` (code, category, message, location, name(), description()), `unexpected(...)`
// to return a failure, and FIREFLY_TRY to propagate one.  The engine's decode-graph code, for example, does
// `auto result = graph.capture(...); if (!result) ... result.error().description()` (src/engine.cc:137-166,
// :329-333).  Errors of the HIP runtime carry the hipError_t code and describe themselves with
// hipGetErrorString; other errors carry their own message.
//
// No exceptions are thrown.  Asking a failed Result for its value, or a successful one for its error, is a
// programming error: the message is printed and the process aborts.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <new>
#include <source_location>
#include <string>
#include <string_view>
#include <type_traits>
#include <utility>

namespace firefly::hal
{

enum class ErrorCategory
{
    CUDA,  // the GPU runtime (HIP here); the reference's name is kept for source compatibility
    Runtime,
    System
};

struct Error
{
    int                  code = 0;
    ErrorCategory        category = ErrorCategory::Runtime;
    std::string          message;
    std::source_location location;

    // A HIP runtime failure: description() is the runtime's text for `c`.
    Error(hipError_t c, std::string_view msg = "", std::source_location loc = std::source_location::current())
        : code(static_cast<int>(c)), category(ErrorCategory::CUDA), message(msg), location(loc)
    {
    }

    // Any other failure: description() is `msg`.
    Error(int c, ErrorCategory cat, std::string_view msg = "",
          std::source_location loc = std::source_location::current())
        : code(c), category(cat), message(msg), location(loc)
    {
    }

    [[nodiscard]] const char* name() const
    {
        return category == ErrorCategory::CUDA ? hipGetErrorName(static_cast<hipError_t>(code)) : "RuntimeError";
    }

    // The runtime's text for HIP errors (the context, if any, is in `message`); the message otherwise.
    [[nodiscard]] const char* description() const
    {
        return category == ErrorCategory::CUDA ? hipGetErrorString(static_cast<hipError_t>(code)) : message.c_str();
    }
};

// Marks a value as the failure of a Result; built by unexpected(...).
template <typename E>
struct Unexpected
{
    E error;
    explicit Unexpected(E e) : error(std::move(e)) {}
};

template <typename E>
Unexpected(E) -> Unexpected<E>;

template <typename E>
[[nodiscard]] Unexpected<std::decay_t<E>> unexpected(E&& e)
{
    return Unexpected<std::decay_t<E>>(std::forward<E>(e));
}

namespace detail
{
[[noreturn]] inline void bad_access(const char* what, const Error* err)
{
    std::fprintf(stderr, "firefly::hal::Result: %s%s%s\n", what, err ? ": " : "", err ? err->description() : "");
    std::abort();
}
}  // namespace detail

// A value of type T or an Error.  Default construction value-initialises T (success).
template <typename T>
class Result
{
public:
    Result() : ok_(true) { new (&slot_.value) T(); }
    Result(T v) : ok_(true) { new (&slot_.value) T(std::move(v)); }
    Result(Unexpected<Error> u) : ok_(false) { new (&slot_.error) Error(std::move(u.error)); }
    Result(const Result& o) : ok_(o.ok_) { o.ok_ ? construct(o.slot_.value) : construct_error(o.slot_.error); }
    Result(Result&& o) noexcept : ok_(o.ok_)
    {
        o.ok_ ? construct(std::move(o.slot_.value)) : construct_error(std::move(o.slot_.error));
    }
    Result& operator=(Result o)
    {
        reset();
        ok_ = o.ok_;
        o.ok_ ? construct(std::move(o.slot_.value)) : construct_error(std::move(o.slot_.error));
        return *this;
    }
    ~Result() { reset(); }

    [[nodiscard]] bool has_value() const { return ok_; }
    explicit           operator bool() const { return ok_; }

    T& value() &
    {
        if (!ok_) detail::bad_access("value() of a failed result", &slot_.error);
        return slot_.value;
    }
    const T& value() const&
    {
        if (!ok_) detail::bad_access("value() of a failed result", &slot_.error);
        return slot_.value;
    }
    T&& value() &&
    {
        if (!ok_) detail::bad_access("value() of a failed result", &slot_.error);
        return std::move(slot_.value);
    }
    T value_or(T fallback) const { return ok_ ? slot_.value : std::move(fallback); }

    const Error& error() const
    {
        if (ok_) detail::bad_access("error() of a successful result", nullptr);
        return slot_.error;
    }
    Error& error()
    {
        if (ok_) detail::bad_access("error() of a successful result", nullptr);
        return slot_.error;
    }

private:
    template <typename U>
    void construct(U&& v)
    {
        new (&slot_.value) T(std::forward<U>(v));
    }
    template <typename U>
    void construct_error(U&& e)
    {
        new (&slot_.error) Error(std::forward<U>(e));
    }
    void reset()
    {
        if (ok_)
            slot_.value.~T();
        else
            slot_.error.~Error();
    }

    union Slot
    {
        Slot() {}
        ~Slot() {}
        T     value;
        Error error;
    } slot_;
    bool ok_;
};

// Success, or an Error.
template <>
class Result<void>
{
public:
    Result() = default;
    Result(Unexpected<Error> u) : failed_(true), error_(std::move(u.error)) {}

    [[nodiscard]] bool has_value() const { return !failed_; }
    explicit           operator bool() const { return !failed_; }

    void value() const
    {
        if (failed_) detail::bad_access("value() of a failed status", &error_);
    }

    const Error& error() const
    {
        if (!failed_) detail::bad_access("error() of a successful status", nullptr);
        return error_;
    }

private:
    bool  failed_ = false;
    Error error_{0, ErrorCategory::Runtime};
};

using Status = Result<void>;

// Evaluates `expression` (a Result); on failure returns its error from the enclosing function, otherwise the
// expression's value is the macro's value.  A GNU statement expression, as in the reference.
#define FIREFLY_TRY(expression)                                                         \
    ({                                                                                  \
        auto&& ff_try_result_ = (expression);                                           \
        if (!ff_try_result_.has_value()) return ::firefly::hal::unexpected(ff_try_result_.error()); \
        std::forward<decltype(ff_try_result_)>(ff_try_result_).value();                \
    })

// A HIP runtime call's status as a Status.
inline Status check_hip(hipError_t err, std::source_location loc = std::source_location::current())
{
    if (err != hipSuccess) return unexpected(Error{err, "", loc});
    return {};
}

// For failures that cannot be reported (destructors): print and abort.
inline void check_hip_fatal(hipError_t err, std::source_location loc = std::source_location::current())
{
    if (err != hipSuccess)
    {
        std::fprintf(stderr, "fatal HIP error at %s:%u: %s (%s)\n", loc.file_name(), static_cast<unsigned>(loc.line()),
                     hipGetErrorString(err), hipGetErrorName(err));
        std::abort();
    }
}

}  // namespace firefly::hal
