// mkv_host.h — host-side helpers for the extern "C" entry points: argument
// checks, the per-thread error message, and launch-status translation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mkv.h"

namespace mkv {

// Records a formatted message for mkv_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the message (called at the start of every entry point).
void clear_error();

// Translates hipGetLastError() after a launch into MKV_OK / MKV_E_LAUNCH.
int check_launch(const char* kernel);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// 16-byte vector moved by every streaming kernel (global_load/store_dwordx4).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 wave64s per workgroup

}  // namespace mkv

#define MKV_REQUIRE(cond, code, ...)              \
  do {                                            \
    if (!(cond)) return mkv::set_error((code), __VA_ARGS__); \
  } while (0)
