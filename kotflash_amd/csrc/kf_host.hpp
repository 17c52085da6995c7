// Host-side helpers shared by the C-ABI entry points: error reporting and
// launch checks. Every entry point returns 0 on success or one of the KF_E*
// codes declared in include/kotflash_amd.h; the message is kept per thread and
// read back through kf_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kotflash_amd.h"

namespace kf {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Translate the last HIP launch status into an error code.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Padded head-dim tile (multiple of 32) for a real head dim D in [8, 128].
inline int head_tile(int64_t D) {
  if (D <= 32) return 32;
  if (D <= 64) return 64;
  if (D <= 96) return 96;
  return 128;
}

}  // namespace kf
