// Measurement probes for the decode floor (not part of the attention
// library): the least any design with one or two launches per call can take
// to read a config 2 call's K/V. bench.py --decode-floor runs them in the same
// HIP-graph setting as its decode figure.
//
//  * kfp_stream: the split-KV decode's memory traffic and nothing else. One
//    workgroup per (KV group, split) reads its chunk of K and V (16-byte
//    loads, every load in flight before any is used), folds the data with
//    XOR and writes one word, so no load can be optimised away.
//  * kfp_merge_like: a second launch of the merge's shape, one 64-lane
//    workgroup per output row reading that row's fp32 partials (num_splits x
//    D floats) and writing D floats.
//  * kfp_empty: an empty kernel (the cost of a launch in the graph).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kf_common.hpp"

namespace {

using kf::buf_load16;
using kf::make_rsrc;
using kf::u32x4;

constexpr int kLoadsPerLane = 16;  // 8 of K, 8 of V: 32 KB of each per workgroup
constexpr int kMergeLoads = 16;    // partial rows per lane in the merge-shaped launch

// Every load is a raw buffer load whose out-of-range lanes read zero, so all
// of them issue back to back with no branch and one wait covers them.
__global__ __launch_bounds__(256) void stream_kernel(const uint16_t* k, const uint16_t* v,
                                                     uint32_t* out, int64_t chunk_bytes,
                                                     int64_t group_bytes, int num_splits) {
  const int split = blockIdx.x % num_splits, grp = blockIdx.x / num_splits;
  const int64_t base = grp * group_bytes + split * chunk_bytes;
  // Bytes of this split inside its group (the last split may be short).
  const int64_t left = group_bytes - split * chunk_bytes;
  const uint32_t ext = (uint32_t)(left < chunk_bytes ? left : chunk_bytes);
  const auto kr = make_rsrc(reinterpret_cast<const char*>(k) + base, ext);
  const auto vr = make_rsrc(reinterpret_cast<const char*>(v) + base, ext);
  u32x4 a[kLoadsPerLane];
  constexpr int half = kLoadsPerLane / 2;
#pragma unroll
  for (int i = 0; i < half; ++i) {
    const uint32_t off = (uint32_t)(i * 256 + threadIdx.x) * 16u;
    a[i] = buf_load16(kr, off);
    a[half + i] = buf_load16(vr, off);
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < kLoadsPerLane; ++i) x ^= a[i][0] ^ a[i][1] ^ a[i][2] ^ a[i][3];
  x ^= __shfl_xor(x, 32);
  x ^= __shfl_xor(x, 16);
  x ^= __shfl_xor(x, 8);
  x ^= __shfl_xor(x, 4);
  x ^= __shfl_xor(x, 2);
  x ^= __shfl_xor(x, 1);
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = x;
}

// Row blockIdx.x holds num_splits x d4 float4 partials; lane = (split slice,
// column), kMergeLoads splits per lane, all loads in flight at once.
__global__ __launch_bounds__(64) void merge_like_kernel(const float* part, float* out,
                                                        int num_splits, int d4) {
  const int64_t row_bytes = (int64_t)num_splits * d4 * 16;
  const auto pr = make_rsrc(reinterpret_cast<const char*>(part) + blockIdx.x * row_bytes,
                            (uint32_t)row_bytes);
  const int per = 64 / d4;  // split slices (d4 divides 64)
  const int col = threadIdx.x % d4, s0 = threadIdx.x / d4;
  u32x4 p[kMergeLoads];
#pragma unroll
  for (int u = 0; u < kMergeLoads; ++u)
    p[u] = buf_load16(pr, (uint32_t)((s0 + per * u) * d4 + col) * 16u);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kMergeLoads; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __uint_as_float(p[u][e]);
  for (int off = d4; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], off);
  if (threadIdx.x < d4)
#pragma unroll
    for (int e = 0; e < 4; ++e) out[((int64_t)blockIdx.x * d4 + col) * 4 + e] = acc[e];
}

__global__ void empty_kernel() {}

}  // namespace

// k, v: [groups][group_keys][D] fp16/bf16 contiguous, read as 16-byte
// vectors; each of the num_splits splits of a group covers chunk_keys keys.
// out: groups * num_splits * 4 words. Returns 0 or 1 (launch error / bad size).
extern "C" int kfp_stream(const void* k, const void* v, void* out, int64_t groups,
                          int64_t group_keys, int64_t D, int64_t chunk_keys, int num_splits,
                          void* stream) {
  const int64_t chunk_bytes = chunk_keys * D * 2, group_bytes = group_keys * D * 2;
  if (chunk_bytes > 256 * 16 * (kLoadsPerLane / 2) || chunk_keys * num_splits < group_keys ||
      group_bytes > 0x7fffffff)
    return 1;
  hipLaunchKernelGGL(stream_kernel, dim3((unsigned)(groups * num_splits)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)k, (const uint16_t*)v, (uint32_t*)out,
                     chunk_bytes, group_bytes, num_splits);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

// part: rows x num_splits x D fp32; out: rows x D fp32. D / 4 divides 64 and
// num_splits <= 16 (64 / (D / 4)).
extern "C" int kfp_merge_like(const void* part, void* out, int64_t rows, int num_splits,
                              int64_t D, void* stream) {
  const int d4 = (int)(D / 4);
  if (D % 4 || d4 <= 0 || d4 > 64 || 64 % d4 || num_splits > (64 / d4) * kMergeLoads) return 1;
  hipLaunchKernelGGL(merge_like_kernel, dim3((unsigned)rows), dim3(64), 0, (hipStream_t)stream,
                     (const float*)part, (float*)out, num_splits, d4);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

extern "C" int kfp_empty(void* stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
