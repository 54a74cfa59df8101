// Result<T> = expected<T, Error>, the error convention of the reference
// (compiler/include/mlk/core/result.h:48-96). Uses <expected> where the
// standard library has it; libstdc++ 11 (this toolchain) does not, so a
// minimal stand-in with the same surface (has_value, value, error,
// operator*, operator->, unexpected) is provided. No exceptions, no RTTI.
#pragma once

#include <string>
#include <utility>

#if defined(__has_include)
#if __has_include(<expected>) && __cplusplus > 202002L
#include <expected>
#if defined(__cpp_lib_expected)
#define MLK_HAVE_STD_EXPECTED 1
#endif
#endif
#endif

namespace mlk {

/// ErrorCode values of compiler/include/mlk/core/result.h:23-41.
enum class ErrorCode : unsigned {
    Ok = 0,
    InvalidArgument,
    InvalidGraph,
    InvalidArtifact,
    UnsupportedCapability,
    Unimplemented,
    BudgetExceeded,
    VerificationFailed,
    ProofInvalid,
    AccuracyViolation,
    EffectIllegal,
    CacheInvalid,
    ParseError,
    IoError,
    Cancelled,
    ResourceExhausted,
    Internal,
};

struct Error {
    ErrorCode code{ErrorCode::Internal};
    std::string message{};
};

#ifdef MLK_HAVE_STD_EXPECTED
template <class T>
using Result = std::expected<T, Error>;
inline std::unexpected<Error> err(ErrorCode c, std::string m) {
    return std::unexpected<Error>(Error{c, std::move(m)});
}
#else
struct Unexpected {
    Error e;
};
inline Unexpected err(ErrorCode c, std::string m) { return Unexpected{Error{c, std::move(m)}}; }

template <class T>
class Result {
public:
    Result(T v) : ok_(true), v_(std::move(v)) {}
    Result(Unexpected u) : ok_(false), e_(std::move(u.e)) {}
    bool has_value() const { return ok_; }
    explicit operator bool() const { return ok_; }
    T& value() { return v_; }
    const T& value() const { return v_; }
    T& operator*() { return v_; }
    const T& operator*() const { return v_; }
    T* operator->() { return &v_; }
    const T* operator->() const { return &v_; }
    const Error& error() const { return e_; }

private:
    bool ok_;
    T v_{};
    Error e_{};
};

template <>
class Result<void> {
public:
    Result() : ok_(true) {}
    Result(Unexpected u) : ok_(false), e_(std::move(u.e)) {}
    bool has_value() const { return ok_; }
    explicit operator bool() const { return ok_; }
    const Error& error() const { return e_; }

private:
    bool ok_;
    Error e_{};
};
#endif

}  // namespace mlk

/// Propagates an error Result (MLK_TRYV of result.h).
#define MLK_TRYV(expr)                                         \
    do {                                                       \
        auto mlk_tryv_r = (expr);                              \
        if (!mlk_tryv_r.has_value()) return mlk::err(mlk_tryv_r.error().code, mlk_tryv_r.error().message); \
    } while (0)
