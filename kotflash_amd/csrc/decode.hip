// Split-KV decode for gfx950 (short query, long KV cache, non-causal).
//
// Layout of the work:
//  * The Hq/Hkv query heads of a KV group and the Sq query positions are packed
//    into R = G * Sq rows (row = g * Sq + i). A workgroup owns up to 32 * QB of
//    those rows for one (batch, kv_head) and one KV chunk, so every K/V byte of
//    the chunk is read from HBM once for all rows of the group (the reference
//    re-reads K/V once per query head, triton_decode.py:16-104).
//  * The chunk is streamed in stages of NKEY keys (all of a stage's loads are
//    issued together, and the next stage's loads are in flight while the
//    current one is computed); the 4 waves each take NKEY / 4 keys of a stage
//    and all rows, keeping their own online-softmax state (S^T = K Q^T per 32
//    keys, P^T feeding O^T += V^T P^T as in the forward).
//  * At the end the 4 per-wave states are merged in LDS in a fixed order
//    (deterministic), and the workgroup writes either the final O/LSE (one
//    split) or an fp32 partial (O_s, LSE_s) of its row block.
//  * Keys at or beyond the per-batch visible length L_b are masked; a split
//    with no visible key writes O_s = 0, LSE_s = -inf (weight 0 in the merge),
//    as the reference does (triton_forward.py:240-246).
//  * merge_kernel (second launch, one workgroup per output row) combines the
//    partials with LSE weights
//      w_s = exp(LSE_s - max) / sum_t exp(LSE_t - max),  LSE = max + ln(sum)
//    guarded for all -inf (reference triton_forward.py:269-349). Each of its
//    threads issues all of its partial loads before using any, so the merge
//    costs about one memory latency. (A single-launch merge by the last
//    arriving workgroup needs an agent-scope release fence per workgroup; on
//    this part those fences cost more than the second launch.)
#include "kf_common.hpp"
#include "kf_host.hpp"

namespace kf {

int check_attn_common(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                      int64_t D, int dtype);
int check_tensor(const char* what, const char* name, const void* ptr, const int64_t* strides);
int check_extent(const char* what, const char* name, int64_t rows, int64_t stride, int64_t D);

struct DecParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  float* part_o;    // [ngroups][nsplit][RB][D]
  float* part_lse;  // [ngroups][nsplit][RB]
  const int32_t* seqlens;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, Sq, Sk, D, G;
  int nsplit, chunk, nrb, rb_rows;
  float scale_log2;
};

// Keys per stage: 256 for head dims up to 64 (64 KiB of K/V per stage), 128
// above (the stage buffers then take 72 KiB of LDS).
template <int DT> struct DecodeStage { static constexpr int NKEY = DT <= 64 ? 256 : 128; };

template <typename T, int DT, int QB>
__global__ __launch_bounds__(256, 2) void decode_kernel(const DecParams p) {
  constexpr int NKEY = DecodeStage<DT>::NKEY;
  constexpr int KPW = NKEY / 4;  // keys per wave and stage
  constexpr int KSTR = DT + 8;
  constexpr int VSTR = DT + 16;
  constexpr int KT = NKEY * KSTR;
  constexpr int STAGE = KT + NKEY * VSTR;
  constexpr int CPR = DT / 8;
  constexpr int CPT = NKEY * CPR / 256;
  constexpr int NKS = DT / 16;
  constexpr int NDB = DT / 32;
  constexpr int RB = 32 * QB;  // rows per workgroup
  constexpr int OSTR = DT + 1;
  // Stage buffer, reused at the end for the cross-wave merge.
  constexpr int MERGE_BYTES = (4 * RB + 2 * RB + 2 * RB * OSTR) * 4;
  constexpr int SMEM_ELEMS = (STAGE * 2 > MERGE_BYTES ? STAGE * 2 : MERGE_BYTES) / 2;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
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

  const auto kr = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, rows_extent(p.Sk, p.k_ss, p.D));
  const auto vr = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, rows_extent(p.Sk, p.v_ss, p.D));

  u32x4 kreg[CPT], vreg[CPT];
  auto gload = [&](int st) {
    const int kbase = c0 + st * NKEY;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + 256 * c;
      const int row = e / CPR, col = e % CPR;
      const int key = kbase + row;
      const bool ok = key < c1 && col * 8 < p.D;
      kreg[c] = buf_load16(kr, ok ? (uint32_t)(key * p.k_ss + col * 8) * 2u : kOOB);
      vreg[c] = buf_load16(vr, ok ? (uint32_t)(key * p.v_ss + col * 8) * 2u : kOOB);
    }
  };
  if (nst > 0) gload(0);

  // Q rows as MFMA B operands (lane = packed row).
  u32x4 qf[QB][NKS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int rho = rb * RB + qb * 32 + l32;
    const bool ok = rho < R;
    const int g = ok ? rho / p.Sq : 0, i = ok ? rho % p.Sq : 0;
    const auto qr = make_rsrc(p.q + b * p.q_sb + kvh * p.G * p.q_sh,
                              (uint32_t)((((int64_t)p.G - 1) * p.q_sh + ((int64_t)p.Sq - 1) * p.q_ss + p.D) * 2));
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = 16 * ks + 8 * h32;
      qf[qb][ks] = buf_load16(qr, (ok && d < p.D) ? (uint32_t)(g * p.q_sh + i * p.q_ss + d) * 2u : kOOB);
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
  wait_all_memory();

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
#pragma unroll
    for (int kb = 0; kb < KPW / 32; ++kb) {
      const int kbase = c0 + st * NKEY + wave * KPW + kb * 32;
      if (kbase < c1) {
        const uint16_t* Ks = smem + (wave * KPW + kb * 32) * KSTR;
        const uint16_t* Vs = smem + KT + (wave * KPW + kb * 32) * VSTR;
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
              x = key >= c1 ? kNegInf : x;
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
    }
    __syncthreads();
  }

  // Cross-wave merge: M = max_w m_w, O = sum_w 2^(m_w - M) O_w, l likewise.
  // Waves 0/1 write their rescaled state into LDS slots 0/1, then waves 2/3
  // add theirs (fixed order: deterministic). Slot rows are padded by one float
  // so the 32 lanes writing one column of 32 rows hit 32 different banks.
  float* mbuf = reinterpret_cast<float*>(smem);  // [4][RB] per-wave row max
  float* lbuf = mbuf + 4 * RB;                   // [2][RB]
  float* obuf = lbuf + 2 * RB;                   // [2][RB][OSTR]
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
  for (int round = 0; round < 2; ++round) {
    if ((wave >> 1) == round) {
      const int slot = wave & 1;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int r = qb * 32 + l32;
        float* orow = obuf + (slot * RB + r) * OSTR;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int d = 32 * db + 8 * (rr >> 2) + 4 * h32 + (rr & 3);
            const float val = cw[qb] * oacc[qb][db][rr];
            orow[d] = round == 0 ? val : orow[d] + val;
          }
        }
        if (h32 == 0) {
          float* lp = lbuf + slot * RB + r;
          *lp = round == 0 ? cw[qb] * l_i[qb] : *lp + cw[qb] * l_i[qb];
        }
      }
    }
    __syncthreads();
  }

  // Output: final O/LSE (one split) or this split's fp32 partial.
  const int nrow = min(RB, R - rb * RB);
  const int DQ = p.D / 4;
  const int grp = (b * p.Hkv + kvh) * p.nrb + rb;
  const int64_t pbase = ((int64_t)grp * p.nsplit + split) * RB;
  for (int e = tid; e < nrow * DQ; e += 256) {
    const int r = e / DQ, d = (e % DQ) * 4;
    const float M = fmaxf(fmaxf(mbuf[r], mbuf[RB + r]), fmaxf(mbuf[2 * RB + r], mbuf[3 * RB + r]));
    const float lt = lbuf[r] + lbuf[RB + r];
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const float* o0 = obuf + r * OSTR + d;
    const float* o1 = obuf + (RB + r) * OSTR + d;
    const float4 ov = make_float4((o0[0] + o1[0]) * inv, (o0[1] + o1[1]) * inv,
                                  (o0[2] + o1[2]) * inv, (o0[3] + o1[3]) * inv);
    const float lse_val = lt > 0.f ? (M + fast_log2(lt)) * kLn2 : kNegInf;
    if (p.nsplit == 1) {
      const int rho = rb * RB + r;
      const int g = rho / p.Sq, i = rho % p.Sq;
      const int h = kvh * p.G + g;
      u32x2 w;
      w[0] = pack2<T>(ov.x, ov.y);
      w[1] = pack2<T>(ov.z, ov.w);
      *reinterpret_cast<u32x2*>(p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss + d) = w;
      if (d == 0 && p.lse) p.lse[((int64_t)b * p.Hq + h) * p.Sq + i] = lse_val;
    } else {
      *reinterpret_cast<float4*>(p.part_o + (pbase + r) * p.D + d) = ov;
      if (d == 0) p.part_lse[pbase + r] = lse_val;
    }
  }
}

// Merge of the split partials: one workgroup per output row.
template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(const DecParams p) {
  const int tid = threadIdx.x;
  const int RB = p.rb_rows;
  const int r = blockIdx.x % RB;
  const int grp = blockIdx.x / RB;
  const int rb = grp % p.nrb;
  const int bk = grp / p.nrb;
  const int kvh = bk % p.Hkv, b = bk / p.Hkv;
  const int rho = rb * RB + r;
  if (rho >= p.G * p.Sq) return;
  const int g = rho / p.Sq, i = rho % p.Sq;
  const int h = kvh * p.G + g;
  const float* plse = p.part_lse + (int64_t)grp * p.nsplit * RB + r;
  const float* po = p.part_o + (int64_t)grp * p.nsplit * RB * p.D + (int64_t)r * p.D;
  __shared__ float red[8];
  __shared__ float4 acc4[256];

  // Max and weight sum of the split LSEs (block reduction).
  float mx = kNegInf;
  for (int sp = tid; sp < p.nsplit; sp += 256) mx = fmaxf(mx, plse[(int64_t)sp * RB]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float ms = (mx == kNegInf) ? 0.f : mx;
  float den = 0.f;
  for (int sp = tid; sp < p.nsplit; sp += 256)
    den += fast_exp2((plse[(int64_t)sp * RB] - ms) * kLog2e);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = den;
  __syncthreads();
  den = red[4] + red[5] + red[6] + red[7];

  // Weighted sum: thread -> (4-column group q, split lane sl); all of a
  // thread's loads are issued before they are consumed.
  const int DQ = p.D / 4;
  const int SL = 256 / DQ;
  const int q = tid % DQ, sl = tid / DQ;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (sl < SL) {
    constexpr int UNR = 4;
    for (int sp = sl; sp < p.nsplit; sp += SL * UNR) {
      float4 v[UNR];
      float w[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int s2 = sp + SL * u;
        const bool ok = s2 < p.nsplit;
        v[u] = ok ? *reinterpret_cast<const float4*>(po + (int64_t)s2 * RB * p.D + 4 * q)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
        w[u] = ok ? plse[(int64_t)s2 * RB] : kNegInf;
      }
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const float wt = fast_exp2((w[u] - ms) * kLog2e);
        acc.x += wt * v[u].x;
        acc.y += wt * v[u].y;
        acc.z += wt * v[u].z;
        acc.w += wt * v[u].w;
      }
    }
  }
  acc4[tid] = acc;
  __syncthreads();
  if (tid < DQ) {
    for (int s2 = 1; s2 < SL; ++s2) {
      const float4 o2 = acc4[s2 * DQ + tid];
      acc.x += o2.x; acc.y += o2.y; acc.z += o2.z; acc.w += o2.w;
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    u32x2 wv;
    wv[0] = pack2<T>(acc.x * inv, acc.y * inv);
    wv[1] = pack2<T>(acc.z * inv, acc.w * inv);
    *reinterpret_cast<u32x2*>(p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss + 4 * tid) = wv;
    if (tid == 0 && p.lse)
      p.lse[((int64_t)b * p.Hq + h) * p.Sq + i] = den > 0.f ? mx + fast_log2(den) * kLn2 : kNegInf;
  }
}

static int decode_rows_per_wg(int64_t G, int64_t Sq) { return G * Sq <= 32 ? 32 : 64; }

template <typename T, int DT>
static int launch_decode(DecParams p, hipStream_t stream) {
  const int R = p.G * p.Sq;
  const bool qb2 = R > 32;
  p.rb_rows = qb2 ? 64 : 32;
  p.nrb = cdiv(R, p.rb_rows);
  const int64_t grid = (int64_t)p.nsplit * p.nrb * p.B * p.Hkv;
  if (grid > 0x7fffffff) return set_error(KF_EUNSUPPORTED, "kf_attn_decode: grid too large");
  if (qb2)
    hipLaunchKernelGGL((decode_kernel<T, DT, 2>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_kernel<T, DT, 1>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  int rc = check_launch("kf_attn_decode(split)");
  if (rc || p.nsplit == 1) return rc;
  const int64_t mgrid = (int64_t)p.B * p.Hkv * p.nrb * p.rb_rows;
  hipLaunchKernelGGL((merge_kernel<T>), dim3((unsigned)mgrid), dim3(256), 0, stream, p);
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
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Sk <= 0 || Hq % Hkv) return 1;
  const int64_t G = Hq / Hkv;
  const int64_t nrb = (G * Sq + decode_rows_per_wg(G, Sq) - 1) / decode_rows_per_wg(G, Sq);
  const int64_t units = B * Hkv * nrb;
  // About one workgroup per CU (256 CUs, two resident each), each streaming
  // whole stages; splits only add merge traffic beyond that.
  const int64_t stage = D <= 64 ? 256 : 128;
  const int64_t target = 256;
  int64_t ns = (target + units - 1) / units;
  const int64_t max_ns = (Sk + stage - 1) / stage;
  if (ns > max_ns) ns = max_ns;
  if (ns < 1) ns = 1;
  // Chunks are whole stages; recount so that every split is non-empty.
  const int64_t chunk = ((Sk + ns - 1) / ns + stage - 1) / stage * stage;
  ns = (Sk + chunk - 1) / chunk;
  return (int)ns;
}

static int64_t decode_row_blocks(int64_t G, int64_t Sq) {
  const int rb = decode_rows_per_wg(G, Sq);
  return (G * Sq + rb - 1) / rb;
}

extern "C" size_t kf_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                            int64_t D, int num_splits) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || D <= 0 || Hq % Hkv || num_splits <= 1) return 0;
  const int64_t G = Hq / Hkv;
  const size_t slots = (size_t)(B * Hkv * decode_row_blocks(G, Sq)) * num_splits *
                       decode_rows_per_wg(G, Sq);
  return (slots * (size_t)D * sizeof(float) + 255) / 256 * 256 + (slots * sizeof(float) + 255) / 256 * 256;
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
  const int64_t stage = D <= 64 ? 256 : 128;
  const int64_t chunk = ((Sk + num_splits - 1) / num_splits + stage - 1) / stage * stage;
  if ((Sk + chunk - 1) / chunk != num_splits)
    return set_error(KF_EINVAL, "%s: num_splits=%d does not partition Sk=%lld into whole %lld-key "
                     "stages (use kf_decode_num_splits)", what, num_splits, (long long)Sk,
                     (long long)stage);
  if (((Hq / Hkv - 1) * q_strides[1] + (Sq - 1) * q_strides[2] + D) * 2 > 0x7fffffffLL)
    return set_error(KF_EUNSUPPORTED, "%s: one KV group of q spans more than 2 GiB", what);
  const size_t need = kf_decode_workspace_bytes(B, Hq, Hkv, Sq, D, num_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return set_error(KF_EINVAL, "%s: workspace of %zu bytes required, got %zu", what, need,
                     workspace == nullptr ? (size_t)0 : workspace_bytes);
  if ((rc = check_extent(what, "k", Sk, k_strides[2], D)) || (rc = check_extent(what, "v", Sk, v_strides[2], D)))
    return rc;
  DecParams p{};
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k; p.v = (const uint16_t*)v;
  p.o = (uint16_t*)o; p.lse = lse; p.seqlens = seqlens_k;
  if (need > 0) {
    const int64_t G = Hq / Hkv;
    const size_t slots = (size_t)(B * Hkv * decode_row_blocks(G, Sq)) * num_splits *
                         decode_rows_per_wg(G, Sq);
    p.part_o = (float*)workspace;
    p.part_lse = (float*)((char*)workspace + (slots * (size_t)D * sizeof(float) + 255) / 256 * 256);
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
