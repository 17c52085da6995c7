// Split-KV decode for gfx950 (short query, long KV cache, non-causal).
//
// Layout of the work:
//  * The Hq/Hkv query heads of a KV group and the Sq query positions are packed
//    into R = G * Sq rows (row = g * Sq + i). A workgroup owns up to 32 * QB of
//    those rows for one (batch, kv_head) and one KV chunk, so every K/V byte of
//    the chunk is read from HBM once for all rows of the group (the reference
//    re-reads K/V once per query head, triton_decode.py:16-104).
//  * The chunk is streamed in stages of 128 keys; the 4 waves each take 32 keys
//    of a stage and all rows, keeping their own online-softmax state
//    (S^T = K Q^T per 32 keys, P^T feeding O^T += V^T P^T as in the forward).
//  * At the end the 4 per-wave states are merged in LDS in a fixed order
//    (deterministic), and the workgroup writes either the final O/LSE (one
//    split) or an fp32 partial (O_s, LSE_s) for merge_kernel.
//  * Keys at or beyond the per-batch visible length L_b are masked; a split
//    with no visible key writes O_s = 0, LSE_s = -inf (weight 0 in the merge),
//    as the reference does (triton_forward.py:240-246).
// merge_kernel combines the partials with LSE weights
//   w_s = exp(LSE_s - max) / sum_t exp(LSE_t - max),  LSE = max + ln(sum)
// guarded for all -inf (reference triton_forward.py:269-349).
#include "kf_common.hpp"
#include "kf_host.hpp"

namespace kf {

int check_attn_common(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                      int64_t D, int dtype);
int check_tensor(const char* what, const char* name, const void* ptr, const int64_t* strides);

struct DecParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  float* part_o;
  float* part_lse;
  const int32_t* seqlens;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t rows;  // B * Hq * Sq
  int B, Hq, Hkv, Sq, Sk, D, G;
  int nsplit, chunk, nrb;
  float scale_log2;
};

template <typename T, int DT, int QB>
__global__ __launch_bounds__(256, 1) void decode_kernel(const DecParams p) {
  constexpr int NKEY = 128;  // keys per stage, 32 per wave
  constexpr int KSTR = DT + 8;
  constexpr int VSTR = DT + 16;
  constexpr int KT = NKEY * KSTR;
  constexpr int STAGE = KT + NKEY * VSTR;
  constexpr int CPR = DT / 8;
  constexpr int CPT = NKEY * CPR / 256;
  constexpr int NKS = DT / 16;
  constexpr int NDB = DT / 32;
  constexpr int RB = 32 * QB;  // rows per workgroup
  // Stage buffers, reused at the end for the cross-wave merge.
  constexpr int MERGE_BYTES = (RB * DT + RB + 4 * RB) * 4;
  constexpr int SMEM_ELEMS = (STAGE * 2 > MERGE_BYTES ? STAGE * 2 : MERGE_BYTES) / 2;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h32 = lane >> 5;

  int bid = blockIdx.x;
  const int split = bid % p.nsplit;
  bid /= p.nsplit;
  const int rb = bid % p.nrb;
  bid /= p.nrb;
  const int kvh = bid % p.Hkv;
  const int b = bid / p.Hkv;
  const int R = p.G * p.Sq;

  const int L = p.seqlens ? min(max(p.seqlens[b], 0), p.Sk) : p.Sk;
  const int c0 = split * p.chunk;
  const int c1 = min(c0 + p.chunk, L);
  const int nst = c1 > c0 ? cdiv(c1 - c0, NKEY) : 0;

  const uint16_t* Kp = p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t* Vp = p.v + b * p.v_sb + kvh * p.v_sh;

  // Q rows as MFMA B operands (lane = packed row).
  u32x4 qf[QB][NKS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int rho = rb * RB + qb * 32 + l32;
    const bool ok = rho < R;
    const int g = ok ? rho / p.Sq : 0, i = ok ? rho % p.Sq : 0;
    const uint16_t* Qp = p.q + b * p.q_sb + (kvh * p.G + g) * p.q_sh + i * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = 16 * ks + 8 * h32;
      qf[qb][ks] = (ok && d < p.D) ? ldg16(Qp + d) : zero_u4();
    }
  }

  f32x16 oacc[QB][NDB];
  float m_i[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = kNegInf;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = zero16();
  }

  u32x4 kreg[CPT], vreg[CPT];
  auto gload = [&](int st) {
    const int kbase = c0 + st * NKEY;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + 256 * c;
      const int row = e / CPR, col = e % CPR;
      const int key = kbase + row;
      const bool ok = key < c1 && col * 8 < p.D;
      kreg[c] = ok ? ldg16(Kp + key * p.k_ss + col * 8) : zero_u4();
      vreg[c] = ok ? ldg16(Vp + key * p.v_ss + col * 8) : zero_u4();
    }
  };

  if (nst > 0) gload(0);
  for (int st = 0; st < nst; ++st) {
    {
      uint16_t* Ks = smem;
      uint16_t* Vs = smem + KT;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int e = tid + 256 * c;
        const int row = e / CPR, col = e % CPR;
        lds_write16(Ks + row * KSTR + col * 8, kreg[c]);
        lds_write16(Vs + row * VSTR + col * 8, vreg[c]);
      }
    }
    __syncthreads();
    if (st + 1 < nst) gload(st + 1);
    const int kbase = c0 + st * NKEY + wave * 32;
    if (kbase < c1) {
      const uint16_t* Ks = smem + wave * 32 * KSTR;
      const uint16_t* Vs = smem + KT + wave * 32 * VSTR;
      f32x16 s[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[qb] = zero16();
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const u32x4 a = lds_read16(Ks + l32 * KSTR + 16 * ks + 8 * h32);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) s[qb] = Elem<T>::mfma(a, qf[qb][ks], s[qb]);
      }
      const bool need_mask = kbase + 32 > c1;
      u32x4 pk[QB][2];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mx = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[qb][r] * p.scale_log2;
          if (need_mask) {
            const int key = kbase + 8 * (r >> 2) + 4 * h32 + (r & 3);
            if (key >= c1) x = kNegInf;
          }
          s[qb][r] = x;
          mx = fmaxf(mx, x);
        }
        mx = wave_xor32_max(mx);
        const float m_new = fmaxf(m_i[qb], mx);
        const float msub = (m_new == kNegInf) ? 0.f : m_new;
        const float alpha = fast_exp2(m_i[qb] - msub);
        float rs = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = fast_exp2(s[qb][r] - msub);
          s[qb][r] = e;
          rs += e;
        }
        l_i[qb] = l_i[qb] * alpha + rs;
        m_i[qb] = m_new;
#pragma unroll
        for (int db = 0; db < NDB; ++db) oacc[qb][db] *= alpha;
        pk[qb][0] = pack8<T>(s[qb], 0);
        pk[qb][1] = pack8<T>(s[qb], 8);
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int stp = 0; stp < 2; ++stp) {
          const u32x4 a = lds_read_tr_operand(Vs, VSTR, 16 * stp, 32 * db, lane);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) oacc[qb][db] = Elem<T>::mfma(a, pk[qb][stp], oacc[qb][db]);
        }
      }
    }
    __syncthreads();
  }

  // Cross-wave merge: M = max_w m_w, O = sum_w 2^(m_w - M) O_w, l likewise.
  float* obuf = reinterpret_cast<float*>(smem);  // [RB][DT]
  float* lbuf = obuf + RB * DT;                  // [RB]
  float* mbuf = lbuf + RB;                       // [4][RB]
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    l_i[qb] = wave_xor32_sum(l_i[qb]);
    if (h32 == 0) mbuf[wave * RB + qb * 32 + l32] = m_i[qb];
  }
  __syncthreads();
  float cw[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = qb * 32 + l32;
    const float M = fmaxf(fmaxf(mbuf[r], mbuf[RB + r]), fmaxf(mbuf[2 * RB + r], mbuf[3 * RB + r]));
    cw[qb] = (M == kNegInf) ? 0.f : fast_exp2(m_i[qb] - M);
  }
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int r = qb * 32 + l32;
        float* orow = obuf + r * DT;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int d = 32 * db + 8 * (rr >> 2) + 4 * h32 + (rr & 3);
            const float val = cw[qb] * oacc[qb][db][rr];
            orow[d] = (w == 0) ? val : orow[d] + val;
          }
        }
        if (h32 == 0) lbuf[r] = (w == 0) ? cw[qb] * l_i[qb] : lbuf[r] + cw[qb] * l_i[qb];
      }
    }
    __syncthreads();
  }

  // Write out: thread -> (row, 4 consecutive d).
  const bool final_out = p.nsplit == 1;
  constexpr int QPR = DT / 4;
  for (int e = tid; e < RB * QPR; e += 256) {
    const int r = e / QPR, d = (e % QPR) * 4;
    const int rho = rb * RB + r;
    if (rho >= R || d >= p.D) continue;
    const int g = rho / p.Sq, i = rho % p.Sq;
    const int h = kvh * p.G + g;
    const float lt = lbuf[r];
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float4 ov = *reinterpret_cast<const float4*>(obuf + r * DT + d);
    const int64_t rowlin = ((int64_t)b * p.Hq + h) * p.Sq + i;
    float M = fmaxf(fmaxf(mbuf[r], mbuf[RB + r]), fmaxf(mbuf[2 * RB + r], mbuf[3 * RB + r]));
    const float lse_val = lt > 0.f ? (M + fast_log2(lt)) * kLn2 : kNegInf;
    if (final_out) {
      uint16_t* Op = p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss + d;
      u32x2 w;
      w[0] = pack2<T>(ov.x * inv, ov.y * inv);
      w[1] = pack2<T>(ov.z * inv, ov.w * inv);
      *reinterpret_cast<u32x2*>(Op) = w;
      if (d == 0 && p.lse) p.lse[rowlin] = lse_val;
    } else {
      float* po = p.part_o + ((int64_t)split * p.rows + rowlin) * p.D + d;
      *reinterpret_cast<float4*>(po) = make_float4(ov.x * inv, ov.y * inv, ov.z * inv, ov.w * inv);
      if (d == 0) p.part_lse[(int64_t)split * p.rows + rowlin] = lse_val;
    }
  }
}

struct MergeParams {
  const float* part_o;
  const float* part_lse;
  uint16_t* o;
  float* lse;
  int64_t o_sb, o_sh, o_ss;
  int64_t rows;
  int Hq, Sq, D, nsplit;
};

// One wave per output row.
template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(const MergeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  float M = kNegInf;
  for (int s = lane; s < p.nsplit; s += 64) M = fmaxf(M, p.part_lse[(int64_t)s * p.rows + row]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  const float Ms = (M == kNegInf) ? 0.f : M;
  float den = 0.f;
  for (int s = lane; s < p.nsplit; s += 64)
    den += fast_exp2((p.part_lse[(int64_t)s * p.rows + row] - Ms) * kLog2e);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off);
  const float inv = den > 0.f ? 1.f / den : 0.f;

  const int64_t bh = row / p.Sq;
  const int i = (int)(row - bh * p.Sq);
  const int b = (int)(bh / p.Hq), h = (int)(bh % p.Hq);
  uint16_t* Op = p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss;
  for (int d = lane * 2; d < p.D; d += 128) {
    float a0 = 0.f, a1 = 0.f;
    for (int s = 0; s < p.nsplit; ++s) {
      const float w = fast_exp2((p.part_lse[(int64_t)s * p.rows + row] - Ms) * kLog2e);
      const float2 v = *reinterpret_cast<const float2*>(p.part_o + ((int64_t)s * p.rows + row) * p.D + d);
      a0 += w * v.x;
      a1 += w * v.y;
    }
    *reinterpret_cast<uint32_t*>(Op + d) = pack2<T>(a0 * inv, a1 * inv);
  }
  if (lane == 0 && p.lse) p.lse[row] = den > 0.f ? M + fast_log2(den) * kLn2 : kNegInf;
}

static int decode_rows_per_wg(int64_t G, int64_t Sq) { return G * Sq <= 32 ? 32 : 64; }

template <typename T, int DT>
static int launch_decode(DecParams p, hipStream_t stream) {
  const int R = p.G * p.Sq;
  const bool qb2 = R > 32;
  p.nrb = cdiv(R, qb2 ? 64 : 32);
  const int64_t grid = (int64_t)p.nsplit * p.nrb * p.B * p.Hkv;
  if (grid > 0x7fffffff) return set_error(KF_EUNSUPPORTED, "kf_attn_decode: grid too large");
  if (qb2)
    hipLaunchKernelGGL((decode_kernel<T, DT, 2>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_kernel<T, DT, 1>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  int rc = check_launch("kf_attn_decode(split)");
  if (rc || p.nsplit == 1) return rc;
  MergeParams m{};
  m.part_o = p.part_o;
  m.part_lse = p.part_lse;
  m.o = p.o;
  m.lse = p.lse;
  m.o_sb = p.o_sb; m.o_sh = p.o_sh; m.o_ss = p.o_ss;
  m.rows = p.rows;
  m.Hq = p.Hq; m.Sq = p.Sq; m.D = p.D; m.nsplit = p.nsplit;
  hipLaunchKernelGGL((merge_kernel<T>), dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, stream, m);
  return check_launch("kf_attn_decode(merge)");
}

template <typename T>
static int dispatch_decode(const DecParams& p, hipStream_t stream) {
  switch (head_tile(p.D)) {
    case 32: return launch_decode<T, 32>(p, stream);
    case 64: return launch_decode<T, 64>(p, stream);
    case 96: return launch_decode<T, 96>(p, stream);
    default: return launch_decode<T, 128>(p, stream);
  }
}

}  // namespace kf

using namespace kf;

extern "C" int kf_decode_num_splits(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                                    int64_t D) {
  (void)D;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Sk <= 0 || Hq % Hkv) return 1;
  const int64_t G = Hq / Hkv;
  const int64_t nrb = (G * Sq + decode_rows_per_wg(G, Sq) - 1) / decode_rows_per_wg(G, Sq);
  const int64_t units = B * Hkv * nrb;
  // Aim for about two workgroups per CU (256 CUs), with at least one 128-key
  // stage per split.
  const int64_t target = 512;
  int64_t ns = (target + units - 1) / units;
  const int64_t max_ns = (Sk + 127) / 128;
  if (ns > max_ns) ns = max_ns;
  if (ns < 1) ns = 1;
  // Round the chunk to whole stages and recount.
  const int64_t chunk = ((Sk + ns - 1) / ns + 127) / 128 * 128;
  ns = (Sk + chunk - 1) / chunk;
  return (int)ns;
}

extern "C" size_t kf_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Sq, int64_t D,
                                            int num_splits) {
  if (B <= 0 || Hq <= 0 || Sq <= 0 || D <= 0 || num_splits <= 1) return 0;
  const size_t rows = (size_t)B * Hq * Sq;
  const size_t bytes = (size_t)num_splits * rows * ((size_t)D + 1) * sizeof(float);
  return (bytes + 255) / 256 * 256 + 256;
}

extern "C" int kf_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse,
                              const int32_t* seqlens_k, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides,
                              const int64_t* k_strides, const int64_t* v_strides,
                              const int64_t* o_strides, float scale, int num_splits, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kf_attn_decode";
  int rc = check_attn_common(what, B, Hq, Hkv, Sq, Sk, D, dtype);
  if (rc) return rc;
  if ((rc = check_tensor(what, "q", q, q_strides)) || (rc = check_tensor(what, "k", k, k_strides)) ||
      (rc = check_tensor(what, "v", v, v_strides)) || (rc = check_tensor(what, "o", o, o_strides)))
    return rc;
  if (!(scale == scale) || scale - scale != 0.f) return set_error(KF_EINVAL, "%s: scale must be finite", what);
  if (num_splits < 1) return set_error(KF_EINVAL, "%s: num_splits must be >= 1", what);
  const int64_t chunk = ((Sk + num_splits - 1) / num_splits + 127) / 128 * 128;
  if ((Sk + chunk - 1) / chunk != num_splits)
    return set_error(KF_EINVAL, "%s: num_splits=%d does not partition Sk=%lld into 128-key stages "
                     "(use kf_decode_num_splits)", what, num_splits, (long long)Sk);
  const size_t need = kf_decode_workspace_bytes(B, Hq, Sq, D, num_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return set_error(KF_EINVAL, "%s: workspace of %zu bytes required, got %zu", what, need,
                     workspace == nullptr ? (size_t)0 : workspace_bytes);
  DecParams p{};
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k; p.v = (const uint16_t*)v;
  p.o = (uint16_t*)o; p.lse = lse; p.seqlens = seqlens_k;
  p.rows = B * Hq * Sq;
  if (need > 0) {
    p.part_o = (float*)workspace;
    const size_t obytes = ((size_t)num_splits * p.rows * D * sizeof(float) + 255) / 256 * 256;
    p.part_lse = (float*)((char*)workspace + obytes);
  }
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Sq = (int)Sq; p.Sk = (int)Sk; p.D = (int)D;
  p.G = (int)(Hq / Hkv);
  p.nsplit = num_splits;
  p.chunk = (int)chunk;
  p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  return dtype == KF_F16 ? dispatch_decode<_Float16>(p, s) : dispatch_decode<__bf16>(p, s);
}
