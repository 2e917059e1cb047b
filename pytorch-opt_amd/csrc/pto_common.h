// Shared definitions for the gfx950 kernels behind pytorch_opt.ops:
// dtype codes, error reporting, workspace carving and small device helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <string>

#include "pytorch_opt_hip.h"  // the exported C ABI; definitions must match it

namespace pto {

// dtype codes shared with the C ABI (include/pytorch_opt_hip.h).
enum Dtype : int { kF32 = 0, kF64 = 1, kBF16 = 2 };

typedef __bf16 bf16;

// Every operand buffer the kernels read along K has its leading dimension
// padded to a multiple of this many elements, with the pad columns zeroed:
// four 64-byte K tiles of bf16 (eight of fp32), the MFMA core's unroll.
constexpr int kPadK = 128;

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Thread-local message for the last failing call (read by pto_last_error).
void set_error(const std::string& msg);

#define PTO_HIP(expr)                                                                \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess) {                                                          \
      ::pto::set_error(std::string(#expr) + " failed: " + hipGetErrorString(e_));    \
      return -1;                                                                     \
    }                                                                                \
  } while (0)

#define PTO_REQUIRE(cond, msg)               \
  do {                                       \
    if (!(cond)) {                           \
      ::pto::set_error(std::string(msg));    \
      return -2;                             \
    }                                        \
  } while (0)

// Check for an asynchronous launch error right after a kernel launch.
#define PTO_LAUNCHED(name)                                                           \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess) {                                                          \
      ::pto::set_error(std::string("launch of ") + (name) + " failed: " +            \
                       hipGetErrorString(e_));                                       \
      return -1;                                                                     \
    }                                                                                \
  } while (0)

// Bump allocator over a caller-provided workspace. Every block starts at a
// 256-byte aligned address, whatever the workspace pointer's alignment, so
// 16-byte vector loads are always legal on workspace operands; the
// workspace-size queries include 256 bytes of slack for the first block.
struct Carver {
  char* base;
  size_t cap;
  size_t used = 0;
  bool overflow = false;
  Carver(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
  template <typename T>
  T* take(int64_t count) {
    size_t bytes = static_cast<size_t>(count) * sizeof(T);
    const size_t addr = reinterpret_cast<uintptr_t>(base) + used;
    size_t at = used + ((256 - (addr & 255)) & 255);
    used = at + bytes;
    if (used > cap || base == nullptr) {
      overflow = true;
      return nullptr;
    }
    return reinterpret_cast<T*>(base + at);
  }
};

// Per-launch profiling hooks (HIP events around selected launches).
bool prof_enabled();  // false on a thread inside a ProfSuspend scope
void prof_suspend(int delta);
void prof_begin(const char* name, hipStream_t stream, void** token);
void prof_end(void* token, hipStream_t stream);

// Keeps kernel timing off on this thread for the scope (the timing creates
// events, which a caller that may not allocate cannot have).
struct ProfSuspend {
  ProfSuspend() { prof_suspend(1); }
  ~ProfSuspend() { prof_suspend(-1); }
};

struct ProfScope {
  void* tok = nullptr;
  hipStream_t s;
  ProfScope(const char* name, hipStream_t st) : s(st) {
    if (prof_enabled()) prof_begin(name, st, &tok);
  }
  ~ProfScope() {
    if (tok) prof_end(tok, s);
  }
};

// ---------------------------------------------------------------- device side

template <typename T>
struct AccOf {
  typedef float type;
};
template <>
struct AccOf<double> {
  typedef double type;
};

template <typename T>
__device__ __forceinline__ T cvt_to(float v);
template <>
__device__ __forceinline__ float cvt_to<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 cvt_to<bf16>(float v) { return static_cast<bf16>(v); }
template <>
__device__ __forceinline__ double cvt_to<double>(float v) { return static_cast<double>(v); }

template <typename T>
__device__ __forceinline__ T cvt_to_d(double v);
template <>
__device__ __forceinline__ double cvt_to_d<double>(double v) { return v; }
template <>
__device__ __forceinline__ float cvt_to_d<float>(double v) { return static_cast<float>(v); }
template <>
__device__ __forceinline__ bf16 cvt_to_d<bf16>(double v) { return static_cast<bf16>(static_cast<float>(v)); }

__device__ __forceinline__ float to_f(bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ double to_f(double v) { return v; }

// Generic convert between the three element types, computing in the
// destination's accumulation precision.
template <typename To, typename From>
__device__ __forceinline__ To convert(From v) {
  return static_cast<To>(to_f(v));
}
template <>
__device__ __forceinline__ bf16 convert<bf16, double>(double v) {
  return static_cast<bf16>(static_cast<float>(v));
}
template <>
__device__ __forceinline__ bf16 convert<bf16, bf16>(bf16 v) {
  return v;
}

}  // namespace pto
