// Host-side helpers shared by the entry points: error state, argument checks, launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdint.h>

#include "../../include/mimo_moe.h"

namespace mimo {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Launch-error check after a kernel launch.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MIMO_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MIMO_OK;
}

// Opt-in per-kernel timing: when enabled (mimo_profile_enable), every launch site brackets its kernel with
// HIP events on the launch stream; mimo_profile_read aggregates durations per kernel name.
void prof_begin(hipStream_t st, const char* name);
void prof_end(hipStream_t st);
void prof_chain(bool on);
// While a ProfSuspend lives on this thread, launches are not timed (no events are created or recorded).
void prof_suspend(bool on);
struct ProfSuspend {
  ProfSuspend() { prof_suspend(true); }
  ~ProfSuspend() { prof_suspend(false); }
};
// Multi-kernel entry points time their kernels back to back: each begin is the previous kernel's end event.
struct ProfChain {
  ProfChain() { prof_chain(true); }
  ~ProfChain() { prof_chain(false); }
};
struct ProfScope {
  hipStream_t st;
  ProfScope(hipStream_t s, const char* name) : st(s) { prof_begin(s, name); }
  ~ProfScope() { prof_end(st); }
};

// Device address of the bf16 sigmoid table on the current device (compile-time data; no stream work).
const uint16_t* sigtab_device(int* err);

// Bump allocator over a caller workspace.
struct Carve {
  char* base;
  size_t cap, off = 0;
  Carve(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
  template <class T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off = align256(off + count * sizeof(T));
    return p;
  }
  bool fits() const { return off <= cap; }
};

}  // namespace mimo

#define MIMO_REQUIRE(cond, code, ...) \
  do { if (!(cond)) return ::mimo::set_error((code), __VA_ARGS__); } while (0)
#define MIMO_HIP(call) \
  do { hipError_t e_ = (call); if (e_ != hipSuccess) return ::mimo::set_error(MIMO_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); } while (0)
