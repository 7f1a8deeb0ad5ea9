// Host-side dtype dispatch: calls fn(T{}) with the element type of `dt`.
#pragma once

#include "common.h"

namespace ntops {

template <typename Fn>
int dispatch_float(int dt, const char* what, Fn&& fn) {
  switch (dt) {
    case NTOPS_F32: return fn(float{});
    case NTOPS_F16: return fn(_Float16{});
    case NTOPS_BF16: return fn(__bf16{});
    case NTOPS_F64: return fn(double{});
    default: return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unsupported floating dtype %d", what, dt);
  }
}

template <typename Fn>
int dispatch_float16_32(int dt, const char* what, Fn&& fn) {
  switch (dt) {
    case NTOPS_F32: return fn(float{});
    case NTOPS_F16: return fn(_Float16{});
    case NTOPS_BF16: return fn(__bf16{});
    default: return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unsupported dtype %d (F32/F16/BF16 only)", what, dt);
  }
}

template <typename Fn>
int dispatch_integral(int dt, const char* what, Fn&& fn) {
  switch (dt) {
    case NTOPS_BOOL: return fn(bool{});
    case NTOPS_U8: return fn(uint8_t{});
    case NTOPS_I8: return fn(int8_t{});
    case NTOPS_I16: return fn(int16_t{});
    case NTOPS_I32: return fn(int32_t{});
    case NTOPS_I64: return fn(int64_t{});
    default: return set_error(NTOPS_ERR_UNSUPPORTED, "%s: unsupported integral dtype %d", what, dt);
  }
}

template <typename Fn>
int dispatch_all(int dt, const char* what, Fn&& fn) {
  if (dtype_is_float(dt)) return dispatch_float(dt, what, fn);
  return dispatch_integral(dt, what, fn);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace ntops
