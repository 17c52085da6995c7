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

// The split forms of the forward and dQ kernels (32-row workgroups whose
// waves split the key range) run when a grid of 128-row tiles would leave
// most of the 256 CUs idle and a tile sees more than two K/V tiles: config
// 1's 64 workgroups, for instance, become 256 with chains of at most two
// tiles. The split grid (four times the tiles, one workgroup per CU) fits
// one round of the CUs up to 64 tiles; causal grids, whose tiles differ in
// length, still gain up to 128. Measured on MI355X for the forward against
// the tiled form: config 1 -37%; 256 tiles, or non-causal D >= 96 at 96-128
// tiles, 5-20% slower split.
constexpr int64_t kSplitMaxTiles = 64;
constexpr int64_t kSplitMaxTilesCausal = 128;

inline bool attn_use_split(int64_t B, int64_t Hq, int64_t Sq, int64_t Sk, bool causal) {
  const int64_t tiles = (Sq + 127) / 128 * B * Hq;
  return Sk > 128 && tiles <= (causal ? kSplitMaxTilesCausal : kSplitMaxTiles);
}

}  // namespace kf
