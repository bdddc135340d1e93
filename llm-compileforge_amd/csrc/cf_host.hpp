// Host-side helpers for the cf_hip C ABI: error state, descriptor checks,
// kernel-launch profiling.  Internal to libcf_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "cf_hip.h"

namespace cf {

// ---- error state --------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const std::string& last_error();

struct Status {
  int32_t code = CF_OK;
  bool ok() const { return code == CF_OK; }
};

#define CF_CHECK(cond, ...)            \
  do {                                 \
    if (!(cond)) {                     \
      ::cf::set_error(__VA_ARGS__);    \
      return CF_ERR_INVALID;           \
    }                                  \
  } while (0)

#define CF_HIP_CHECK(expr)                                                    \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess) {                                                   \
      ::cf::set_error("%s failed: %s", #expr, hipGetErrorString(e_));         \
      return CF_ERR_HIP;                                                      \
    }                                                                         \
  } while (0)

// ---- descriptor view ----------------------------------------------------
struct View {
  char* base = nullptr;  // aligned pointer + offset, in bytes
  int rank = 0;
  int dtype = -1;
  int elem = 0;
  int64_t size[4] = {0, 0, 0, 0};
  int64_t stride[4] = {0, 0, 0, 0};  // elements
};

inline int dtype_bytes(int dt) {
  switch (dt) {
    case CF_F32: return 4;
    case CF_F16: return 2;
    case CF_BF16: return 2;
    case CF_I64: return 8;
    case CF_I32: return 4;
    case CF_I8: return 1;
    case CF_U8: return 1;
    case CF_F8E4M3FN: return 1;
    default: return 0;
  }
}

inline const char* dtype_name(int dt) {
  switch (dt) {
    case CF_F32: return "f32";
    case CF_F16: return "f16";
    case CF_BF16: return "bf16";
    case CF_I64: return "i64";
    case CF_I32: return "i32";
    case CF_I8: return "i8";
    case CF_U8: return "u8";
    case CF_F8E4M3FN: return "f8e4m3fn";
    default: return "?";
  }
}

// Unpacks a CfTensor into a View, checking what every kernel relies on.
int32_t view_of(const CfTensor* t, const char* name, int rank, View* v);

// ---- launch profiling ---------------------------------------------------
bool profiling_enabled();
// Records the "begin" event for a launch of kernel `name` on `stream` and
// returns a slot id (or -1 when disabled); profile_end records the "end".
int profile_begin(const char* name, hipStream_t stream);
void profile_end(int slot, hipStream_t stream);

struct ProfileScope {
  int slot;
  hipStream_t stream;
  ProfileScope(const char* name, hipStream_t s) : slot(profile_begin(name, s)), stream(s) {}
  ~ProfileScope() { profile_end(slot, stream); }
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace cf
