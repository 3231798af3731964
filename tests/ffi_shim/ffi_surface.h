// Test scaffolding, not XLA: the part of XLA's FFI C++ API (xla/ffi/api/ffi.h,
// as jax.ffi.include_dir() ships it) that the handler shim of INTEGRATION.md
// uses, declared from that API's published types so that a CPU test can
// compile the shim here, where jax is absent.  What the compile checks: every
// call from the shim into include/nanorts_amd.h (names, argument counts and
// types), and each handler's parameter list against its binding (Bind's
// Ctx / Arg / Ret / RemainingArgs / RemainingRets / Attr, decoded in order, as
// XLA decodes them).  What it does not check: that these declarations match
// XLA's header; a maintainer's build against jax's headers does that.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <type_traits>

namespace xla::ffi {

enum class DataType : uint8_t { INVALID, PRED, S8, S16, S32, S64, U8, U16, U32, U64, F16, F32, F64, BF16 };
inline constexpr DataType PRED = DataType::PRED;
inline constexpr DataType S8 = DataType::S8;
inline constexpr DataType S16 = DataType::S16;
inline constexpr DataType S32 = DataType::S32;
inline constexpr DataType U8 = DataType::U8;
inline constexpr DataType U32 = DataType::U32;

template <DataType dtype> struct Native;
template <> struct Native<DataType::PRED> { using type = bool; };
template <> struct Native<DataType::S8> { using type = int8_t; };
template <> struct Native<DataType::S16> { using type = int16_t; };
template <> struct Native<DataType::S32> { using type = int32_t; };
template <> struct Native<DataType::U8> { using type = uint8_t; };
template <> struct Native<DataType::U32> { using type = uint32_t; };

class Dimensions {
 public:
  size_t size() const { return n_; }
  int64_t operator[](size_t i) const { return p_[i]; }
  const int64_t* begin() const { return p_; }
  const int64_t* end() const { return p_ + n_; }

 private:
  const int64_t* p_ = nullptr;
  size_t n_ = 0;
};

class AnyBuffer {
 public:
  DataType element_type() const { return type_; }
  Dimensions dimensions() const { return dims_; }
  size_t size_bytes() const { return bytes_; }
  size_t element_count() const { return count_; }
  void* untyped_data() const { return data_; }

 private:
  DataType type_ = DataType::INVALID;
  size_t count_ = 0;
  Dimensions dims_;
  size_t bytes_ = 0;
  void* data_ = nullptr;
};

template <DataType dtype>
class Buffer {
 public:
  using T = typename Native<dtype>::type;
  DataType element_type() const { return dtype; }
  Dimensions dimensions() const { return dims_; }
  size_t size_bytes() const { return bytes_; }
  void* untyped_data() const { return data_; }
  T* typed_data() const { return static_cast<T*>(data_); }

 private:
  Dimensions dims_;
  size_t bytes_ = 0;
  void* data_ = nullptr;
};

template <typename T>
class Result {
 public:
  T& operator*() { return value_; }
  T* operator->() { return &value_; }

 private:
  T value_;
};

class Error {
 public:
  static Error Success() { return Error(true); }
  static Error InvalidArgument(std::string) { return Error(false); }
  static Error Internal(std::string) { return Error(false); }
  bool success() const { return ok_; }
  bool failure() const { return !ok_; }

 private:
  explicit Error(bool ok) : ok_(ok) {}
  bool ok_;
};

template <typename T>
class ErrorOr {
 public:
  bool has_error() const { return false; }
  Error error() const { return Error::Success(); }
  T& operator*() { return value_; }
  T* operator->() { return &value_; }

 private:
  T value_;
};

class RemainingArgs {
 public:
  size_t size() const { return 0; }
  template <typename T>
  ErrorOr<T> get(size_t) const { return {}; }
};

class RemainingRets {
 public:
  size_t size() const { return 0; }
  template <typename T>
  ErrorOr<Result<T>> get(size_t) const { return {}; }
};

template <typename T>
struct PlatformStream {};

enum class Traits : uint32_t { kCmdBufferCompatible = 1 };

// What the handler receives for each binding step, in order.
template <typename... Decoded>
struct Binding {
  template <typename C> struct CtxOf;
  template <typename T> struct CtxOf<PlatformStream<T>> { using type = T; };

  template <typename C>
  Binding<Decoded..., typename CtxOf<C>::type> Ctx() const { return {}; }
  template <typename T>
  Binding<Decoded..., T> Arg() const { return {}; }
  template <typename T>
  Binding<Decoded..., Result<T>> Ret() const { return {}; }
  Binding<Decoded..., xla::ffi::RemainingArgs> RemainingArgs() const { return {}; }
  Binding<Decoded..., xla::ffi::RemainingRets> RemainingRets() const { return {}; }
  template <typename T>
  Binding<Decoded..., T> Attr(std::string_view) const { return {}; }

  template <typename F>
  int To(F) const {
    static_assert(std::is_invocable_r_v<Error, F, Decoded...>,
                  "the handler's parameters do not match its binding");
    return 0;
  }
};

struct Ffi {
  static Binding<> Bind() { return {}; }
};

}  // namespace xla::ffi

// One exported handler symbol per target, whose binding is checked against
// its implementation.
#define XLA_FFI_DEFINE_HANDLER_SYMBOL(fn, impl, binding, ...) \
  extern "C" int fn() { return (binding).To(impl); }
