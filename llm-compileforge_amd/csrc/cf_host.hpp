// Host-side helpers for the cf_hip C ABI: error state, descriptor checks,
// kernel-launch profiling.  Internal to libcf_hip.so.
#pragma once

#include <hip/hip_ext.h>
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
// While the timing hook (cf_profile_enable) is on, a ProfileScope arms a
// pair of HIP events for the next CF_LAUNCH on this thread.  The launch
// hands them to hipExtLaunchKernel, which records them at the kernel's
// start and end on its stream; the pair becomes a launch record only when
// the runtime accepted the launch, and goes back to the pool otherwise.
bool profiling_enabled();
// Arms events for kernel `name` (no-op when profiling is off).
void profile_arm(const char* name);
// Disarms events the launch did not consume (error paths).
void profile_disarm();

struct ArmedEvents {
  const char* name = nullptr;
  hipEvent_t begin = nullptr, end = nullptr;
};
// Hands over this thread's armed events (all null when none are armed).
ArmedEvents profile_take();
// Registers the launch record when `launched`, else returns the events to
// the pool.  No-op for an empty pair.
void profile_commit(const ArmedEvents& ev, bool launched);

struct ProfileScope {
  ProfileScope(const char* name, hipStream_t) { profile_arm(name); }
  ~ProfileScope() { profile_disarm(); }
};

// Kernel launch on `stream`: an ordinary launch (what stream capture
// records), or, when timing events are armed, hipExtLaunchKernel carrying
// them.  The launch's error stays pending for the caller's hipGetLastError
// check.
#define CF_LAUNCH(kernel, grid, block, lds, stream, ...)                                                  \
  do {                                                                                                   \
    const ::cf::ArmedEvents cf_ev_ = ::cf::profile_take();                                               \
    if (cf_ev_.begin) {                                                                                  \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, cf_ev_.begin, cf_ev_.end, 0, __VA_ARGS__); \
      ::cf::profile_commit(cf_ev_, hipPeekAtLastError() == hipSuccess);                                  \
    } else {                                                                                             \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                                 \
    }                                                                                                    \
  } while (0)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (cached per device; 256 if unknown).
int device_cu_count();

}  // namespace cf
