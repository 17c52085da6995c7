// Shared device primitives for the gfx950 (CDNA4) attention kernels.
//
// Conventions used by every kernel in this directory:
//  * Tensors are [batch, heads, sequence, head_dim] with a unit head_dim stride;
//    the batch/head/sequence strides are passed in elements (int64).
//  * Head dims are padded at compile time to DT (a multiple of 32). The real
//    head_dim D is a multiple of 8, so a 16-byte chunk of 8 elements is either
//    entirely inside [0, D) or entirely padding (zero-filled).
//  * MFMA is v_mfma_f32_32x32x16_{f16,bf16}. Its operand/result layout, checked
//    on the device with an in-bounds probe:
//      A (32 x 16):  lane l holds row  i = l % 32, eight k slots (h = l / 32, t = 0..7)
//      B (16 x 32):  lane l holds col  j = l % 32, the same eight k slots
//      C (32 x 32):  lane l, register r holds C[8*(r/4) + 4*(l/32) + r%4][l % 32]
//    Only the agreement of the A and B k-slots matters, so every kernel assigns
//    slot (h, t) to whatever contraction index is cheapest to load.
//  * ds_read_b64_tr_b16 (gfx950), checked the same way: inside each 16-lane
//    group, lane i element e is element (i % 4) of the 8-byte piece addressed by
//    lane (i / 4 + 4 e). Giving lane p the address of row (p / 4), columns
//    4 (p % 4) .. +3 of a row-major 4 x 16 block therefore returns column i of
//    that block (rows 0..3) to lane i: a transposed read of 16-bit data.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace kf {

// Compile-time loop: calls f(std::integral_constant<int, I>) for I in [B, E).
// Used where every iteration must see its index as a constant (register
// arrays indexed by it stay in registers).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

#define KF_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// Element traits: storage type, MFMA, float conversion.
template <typename T> struct Elem;

template <> struct Elem<_Float16> {
  using v8 = f16x8;
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // v_mfma_f32_16x16x32_f16: A lane l holds row l % 16, B lane l column l % 16,
  // both with the eight k slots of lane group l / 16; C lane l register r holds
  // C[4 (l / 16) + r][l % 16].
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint16_t bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
};

template <> struct Elem<__bf16> {
  using v8 = bf16x8;
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint16_t bits(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  __device__ static inline float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, ((uint32_t)b) << 16);
  }
};

// Two floats -> two packed 16-bit elements, round to nearest even, in one
// v_cvt_pk_{f16,bf16}_f32.
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ inline uint32_t pack2(float lo, float hi) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  const f32x2 x = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, t2));
}

// Eight consecutive accumulator registers -> one 8-element MFMA operand.
template <typename T>
__device__ inline u32x4 pack8(const f32x16& acc, int r0) {
  u32x4 out;
  out[0] = pack2<T>(acc[r0 + 0], acc[r0 + 1]);
  out[1] = pack2<T>(acc[r0 + 2], acc[r0 + 3]);
  out[2] = pack2<T>(acc[r0 + 4], acc[r0 + 5]);
  out[3] = pack2<T>(acc[r0 + 6], acc[r0 + 7]);
  return out;
}

__device__ inline f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ inline u32x4 zero_u4() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return z;
}

__device__ inline u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Raw buffer loads: a wave-uniform resource (base, byte extent) plus a per-lane
// byte offset. Offsets at or beyond the extent read as zero, so tails of the
// key/query range and head-dim padding need no branches: invalid lanes pass
// kOOB. The extent is limited to 2^31 - 1 bytes (checked on the host).
constexpr uint32_t kOOB = 0x80000000u;

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ inline u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// Byte extent of rows [0, n) of a [rows, D] slice with a row stride of
// `stride` elements (16-bit): the last row ends at (n - 1) * stride + D.
__device__ inline uint32_t rows_extent(int n, int64_t stride, int D) {
  return n > 0 ? (uint32_t)((((int64_t)(n - 1)) * stride + D) * 2) : 0u;
}

// Wave-uniform "any lane" for a per-lane predicate.
__device__ inline bool wave_any(bool pred) { return __builtin_amdgcn_ballot_w64(pred) != 0; }

// Lazy rescaling threshold of the online softmax (log2 units): the reference
// max m of a row is only moved (and O, l rescaled) when a new score exceeds it
// by more than this, so P = 2^(s - m) stays <= 2^8 -- exact in fp32 and
// representable in fp16/bf16 -- and most tiles skip the O rescale entirely.
constexpr float kRescaleThreshold = 8.f;
__device__ inline void stg16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

__device__ inline u32x4 lds_read16(const uint16_t* p) {
  return *(const KF_LDS u32x4*)(p);
}
__device__ inline void lds_write16(uint16_t* p, u32x4 v) { *(KF_LDS u32x4*)(p) = v; }

// Transposed LDS read of a 4 x 16 block of 16-bit elements (see header comment).
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((KF_LDS s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// The same read at an LDS byte address.
__device__ inline u32x2 lds_read_tr16_at(uint32_t addr) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((KF_LDS s16x4*)(uintptr_t)addr);
  return __builtin_bit_cast(u32x2, r);
}

// MFMA A operand of a transposed row-major LDS tile: lane (i = l % 32, h = l / 32)
// receives X[row0 + 8u + 4h + e][col0 + i] for slots t = 4u + e.  The row index
// of slot (h, t) is therefore 8 (t / 4) + 4 h + t % 4 -- the same contraction
// index an f32x16 accumulator register r = t (+ 8) carries in its row, which is
// what lets a softmax result feed the next MFMA as a B operand without any data
// movement.
__device__ inline u32x4 lds_read_tr_operand(const uint16_t* tile, int stride, int row0, int col0,
                                            int lane) {
  const int p = lane & 15;
  const int h = lane >> 5;
  const int g = (lane >> 4) & 1;
  const uint16_t* base = tile + (row0 + 4 * h + (p >> 2)) * stride + col0 + 16 * g + 4 * (p & 3);
  u32x2 lo = lds_read_tr16(base);
  u32x2 hi = lds_read_tr16(base + 8 * stride);
  u32x4 out = {lo[0], lo[1], hi[0], hi[1]};
  return out;
}

// Direct-to-LDS buffer loads (gfx950): every lane reads `size` bytes at its own
// byte offset and the data lands at lds_base + size * lane, with lds_base
// wave-uniform (M0). Checked on the device with an in-bounds probe. Offsets
// beyond the resource extent (kOOB) deposit zeros, like register loads.
//
// They are issued as inline assembly on purpose: the compiler cannot tell
// which LDS bytes an in-flight load of this kind writes, so for the builtin it
// waits for all of them (vmcnt(0)) before any later LDS read, which would
// drain a multi-stage ring every step. Callers therefore wait for these loads
// themselves (KF_WAIT_VMCNT + barrier). The compiler's own waits on other
// vector-memory loads stay correct: the counter completes in order, so extra
// younger loads it does not know of only make its waits longer.
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const KF_LDS void*)p;
}
__device__ inline void dma16(__amdgpu_buffer_rsrc_t r, uint16_t* lds_base, uint32_t byte_off) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds_base))), "v"(byte_off), "s"(r)
      : "memory", "m0");
}
__device__ inline void dma4(__amdgpu_buffer_rsrc_t r, float* lds_base, uint32_t byte_off) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds_base))), "v"(byte_off), "s"(r)
      : "memory", "m0");
}

// The same loads with the LDS destination given as a wave-uniform LDS byte
// address (M0) and a wave-uniform byte offset added to every lane's (soffset).
// Both are plain integers here, so callers that compute them from uniform
// values keep the whole address computation on the scalar unit. A lane's
// voffset + soffset must stay below 2^32: with voffset < 2^31 (or kOOB) and
// soffset < 2^31 it does.
__device__ inline void dma16_s(__amdgpu_buffer_rsrc_t r, uint32_t lds_m0, uint32_t voff,
                               uint32_t soff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_m0)), "v"(voff), "s"(r),
        "s"(__builtin_amdgcn_readfirstlane(soff))
      : "memory", "m0");
}
__device__ inline void dma4_s(__amdgpu_buffer_rsrc_t r, uint32_t lds_m0, uint32_t voff,
                              uint32_t soff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, %3 offen lds"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_m0)), "v"(voff), "s"(r),
        "s"(__builtin_amdgcn_readfirstlane(soff))
      : "memory", "m0");
}

// s_waitcnt that waits until at most n vector-memory operations of the wave
// are outstanding (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt and
// lgkmcnt left at their maxima). n must be a compile-time constant < 64.
#define KF_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | ((((n) >> 4) & 3) << 14) | (7 << 4) | (15 << 8)))

// Row-major 16-bit tile of `rows` x (8 cpr) elements stored without padding,
// 16-byte chunks XOR-swizzled within each row: logical chunk c of row r lives
// at physical chunk c ^ key(r). The LDS serves a b128 read 16 lanes per pass
// and a ds_read_b64_tr_b16 read 32 lanes per pass over 64 four-byte banks, and
// the kernels read these tiles both ways:
//   - b128 rows: 16 lanes read 16 consecutive rows at one logical chunk, so
//     key(r) must differ across any 16 consecutive rows (mod 16);
//   - transposed: 32 lanes read 4 consecutive rows (from a multiple of 4) x 4
//     consecutive chunks (from a multiple of 4), so the keys of those 4 rows
//     must differ in the bits above the chunk's low two.
// key(r) = rotate(r mod 16) by two bits meets both at 16 chunks per row
// (measured: 4 passes per b128 read and 2 per transposed read, the minimum;
// the plain key r mod 16 costs 8 passes per transposed read). Narrower rows
// use the largest key that keeps c ^ key inside the row.
template <int CPR>
struct SwizzledTile {
  static constexpr int SW = (CPR % 16 == 0) ? 16 : (CPR % 8 == 0) ? 8 : 4;
  __device__ static inline int key(int r) {
    if constexpr (SW == 16) return ((r & 3) << 2) | ((r >> 2) & 3);
    else if constexpr (SW == 8) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else return (r >> 2) & 3;
  }
  __device__ static inline int chunk(int r, int c) { return r * CPR + (c ^ key(r)); }
  // Element offset of element col (any in [0, 8 cpr)) of row r.
  __device__ static inline int elem(int r, int col) { return chunk(r, col >> 3) * 8 + (col & 7); }
};

// Transposed MFMA A operand (as lds_read_tr_operand) from a swizzled tile.
template <int CPR>
__device__ inline u32x4 lds_read_tr_operand_sw(const uint16_t* tile, int row0, int col0, int lane) {
  const int p = lane & 15;
  const int h = lane >> 5;
  const int g = (lane >> 4) & 1;
  const int r = row0 + 4 * h + (p >> 2);
  const int col = col0 + 16 * g + 4 * (p & 3);
  u32x2 lo = lds_read_tr16(tile + SwizzledTile<CPR>::elem(r, col));
  u32x2 hi = lds_read_tr16(tile + SwizzledTile<CPR>::elem(r + 8, col));
  u32x4 out = {lo[0], lo[1], hi[0], hi[1]};
  return out;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Combine the two 32-lane halves of a wave. v_permlane32_swap (gfx950, VALU)
// exchanges the upper half of its first operand with the lower half of its
// second; with both operands x the two results hold (x_lo, x_lo) and
// (x_hi, x_hi), so max/sum of the pair is the cross-half reduction in every
// lane, bit-identical in both halves.
__device__ inline float wave_xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Combine the four 16-lane groups of a wave (lanes i, i + 16, i + 32, i + 48):
// v_permlane16_swap pairs groups (0, 1) and (2, 3) the same way
// v_permlane32_swap pairs the two halves, so both steps leave every lane of
// the four groups with the same, bit-identical result.
__device__ inline float wave_group16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return wave_xor32_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ inline float wave_group16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return wave_xor32_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

// Wave index inside the workgroup as a wave-uniform (scalar) value, so that
// conditions built from it compile to scalar branches.
__device__ inline int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Wait for every outstanding memory operation of the wave. Placed after
// prologue loads whose completion the compiler cannot otherwise prove on all
// paths into a loop; without it, the loop waits on them (and on every load
// issued after them) at its first use of those registers in each iteration.
__device__ inline void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }

// acc + x.lo + x.hi for two packed 16-bit elements, accumulated in fp32
// (v_dot2c_f32_f16 / _bf16 against (1, 1)).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <typename T> __device__ inline float sum2_acc(uint32_t x, float acc);
template <> __device__ inline float sum2_acc<_Float16>(uint32_t x, float acc) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), one, acc, false);
}
template <> __device__ inline float sum2_acc<__bf16>(uint32_t x, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), one, acc, false);
}

__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace kf
