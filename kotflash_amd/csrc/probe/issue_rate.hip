// Measurement probe (not part of the attention library): how many other
// instructions one wave can issue beside a v_mfma_f32_32x32x16_f16 before the
// MFMA stream slows down. bench.py --issue-rates runs it.
//
// Every SIMD of the GPU runs one wave (1024 one-wave workgroups). The wave
// issues N rounds of two MFMAs on two independent accumulators, each MFMA
// followed by `nv` instructions of one kind on registers the MFMAs do not
// touch, with a scheduling fence between rounds. The wave's own shader-clock
// span (s_memtime) divided by the MFMA count is the cost of one MFMA plus its
// companions; s_memrealtime (100 MHz) over the same span gives the clock.
//
// Kinds: 0 v_fma_f32, 1 v_exp_f32, 2 ds_read_b128, 3 ds_read_b64_tr_b16;
// mixed slots, `nv` v_fma_f32 after 4 one ds_read_b128, 5 two
// ds_read_b64_tr_b16, 6 one v_exp_f32 (the shapes of the attention kernels'
// MFMA slots); scalar-side instructions, 7 s_add_u32, 8 s_waitcnt
// lgkmcnt(15) (nothing to wait for), 9 s_nop 0. The LDS reads address 16 (or 8) consecutive bytes per lane of
// a 1 KB (512 B) block of this workgroup's LDS, every read in bounds.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRounds = 512;

template <int KIND, int NV>
__global__ __launch_bounds__(64) void issue_kernel(float* sink, uint64_t* ticks, float seed) {
  __shared__ u32x4 lds[64];
  lds[threadIdx.x] = u32x4{threadIdx.x, 1u, 2u, 3u};
  __syncthreads();
  half8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(seed * i);
    b[i] = (_Float16)(seed + i);
  }
  f32x16 c0 = {}, c1 = {};
  float v[8];
  u32x4 r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = seed + threadIdx.x + i;
    r[i] = u32x4{(unsigned)i, 0u, 0u, 0u};
  }
  const unsigned a16 = (unsigned)(uintptr_t)&lds[threadIdx.x];
  const unsigned a8 = (unsigned)(uintptr_t)lds + 8u * threadIdx.x;
  const float c = seed * 0.5f;
  unsigned sreg = 0u;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kRounds; ++it) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 0)
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
      else
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
      if constexpr (KIND == 4) asm volatile("ds_read_b128 %0, %1" : "+v"(r[7]) : "v"(a16));
      if constexpr (KIND == 5) {
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "+v"(*reinterpret_cast<uint64_t*>(&r[6])) : "v"(a8));
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "+v"(*reinterpret_cast<uint64_t*>(&r[7])) : "v"(a8));
      }
      if constexpr (KIND == 6) asm volatile("v_exp_f32 %0, %0" : "+v"(v[7]));
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if constexpr (KIND == 0 || (KIND >= 4 && KIND <= 6))
          asm volatile("v_fma_f32 %0, %0, %1, %1" : "+v"(v[KIND == 6 ? j % 7 : j & 7]) : "v"(c));
        else if constexpr (KIND == 1)
          asm volatile("v_exp_f32 %0, %0" : "+v"(v[j & 7]));
        else if constexpr (KIND == 2)
          asm volatile("ds_read_b128 %0, %1" : "+v"(r[j & 7]) : "v"(a16));
        else if constexpr (KIND == 7)
          asm volatile("s_add_u32 %0, %0, 1" : "+s"(sreg));
        else if constexpr (KIND == 8)
          asm volatile("s_waitcnt lgkmcnt(15)" ::: "memory");
        else if constexpr (KIND == 9)
          asm volatile("s_nop 0");
        else
          asm volatile("ds_read_b64_tr_b16 %0, %1" : "+v"(*reinterpret_cast<uint64_t*>(&r[j & 7])) : "v"(a8));
      }
      if constexpr (KIND == 2 || KIND == 3 || KIND == 4 || KIND == 5) asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i] + (float)r[i][0] + (float)r[i][1];
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i];
  sink[blockIdx.x * 64 + threadIdx.x] = s + (float)sreg;
  if (threadIdx.x == 0) {
    ticks[2 * blockIdx.x] = t1 - t0;
    ticks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

template <int KIND>
hipError_t launch_kind(int nv, int blocks, float* sink, uint64_t* ticks, hipStream_t s) {
  switch (nv) {
    case 0: hipLaunchKernelGGL((issue_kernel<KIND, 0>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    case 2: hipLaunchKernelGGL((issue_kernel<KIND, 2>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    case 3: hipLaunchKernelGGL((issue_kernel<KIND, 3>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    case 4: hipLaunchKernelGGL((issue_kernel<KIND, 4>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    case 5: hipLaunchKernelGGL((issue_kernel<KIND, 5>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    case 6: hipLaunchKernelGGL((issue_kernel<KIND, 6>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    case 8: hipLaunchKernelGGL((issue_kernel<KIND, 8>), dim3(blocks), dim3(64), 0, s, sink, ticks, 0.001f); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" {

// One launch of `blocks` one-wave workgroups (the caller passes the GPU's
// SIMD count) with `nv` in {0, 2, 3, 4, 5, 6, 8} instructions of `kind`
// after each MFMA (kinds as above). sink holds blocks x 64 floats; ticks receives, per
// workgroup, the s_memtime span and the s_memrealtime span (2 x uint64).
// Rounds per wave: kfp_issue_rounds(). Returns a hipError_t.
int kfp_issue_rate(int kind, int nv, int blocks, float* sink, uint64_t* ticks, void* stream) {
  if (blocks <= 0 || !sink || !ticks) return (int)hipErrorInvalidValue;
  const hipStream_t s = (hipStream_t)stream;
  switch (kind) {
    case 0: return (int)launch_kind<0>(nv, blocks, sink, ticks, s);
    case 1: return (int)launch_kind<1>(nv, blocks, sink, ticks, s);
    case 2: return (int)launch_kind<2>(nv, blocks, sink, ticks, s);
    case 3: return (int)launch_kind<3>(nv, blocks, sink, ticks, s);
    case 4: return (int)launch_kind<4>(nv, blocks, sink, ticks, s);
    case 5: return (int)launch_kind<5>(nv, blocks, sink, ticks, s);
    case 6: return (int)launch_kind<6>(nv, blocks, sink, ticks, s);
    case 7: return (int)launch_kind<7>(nv, blocks, sink, ticks, s);
    case 8: return (int)launch_kind<8>(nv, blocks, sink, ticks, s);
    case 9: return (int)launch_kind<9>(nv, blocks, sink, ticks, s);
    default: return (int)hipErrorInvalidValue;
  }
}

int kfp_issue_rounds(void) { return kRounds; }

}  // extern "C"
