// Split-KV decode for gfx950 (short query, long KV cache, non-causal).
//
// Layout of the work:
//  * The Hq/Hkv query heads of a KV group and the Sq query positions are packed
//    into R = G * Sq rows (row = g * Sq + i). A workgroup owns up to 32 * QB of
//    those rows for one (batch, kv_head) and one KV chunk, so every K/V byte of
//    the chunk is read from HBM once for all rows of the group (the reference
//    re-reads K/V once per query head, triton_decode.py:16-104).
//  * The chunk is cut into 32-key steps that the 4 waves take in turn (so
//    chunks are whole 128-key granules). Each wave streams its own steps with
//    no workgroup barrier: its K and V tiles go into a wave-private LDS ring
//    by direct-to-LDS loads (two steps in flight), and the wave keeps its own
//    online-softmax state
//    (S^T = K Q^T per step, P^T feeding O^T += V^T P^T as in the forward).
//  * At the end the 4 per-wave states are merged in LDS in one pass with a
//    fixed order (deterministic), and the workgroup writes either the final
//    O/LSE (one split) or an fp32 partial (O_s, LSE_s) of its row block.
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

// Keys per split granule: the four waves of a workgroup take 32-key steps in
// turn, so chunks are whole multiples of 128 keys.
constexpr int kDecGranule = 128;

template <typename T, int DT, int QB>
__global__ __launch_bounds__(256, 2) void decode_kernel(const DecParams p) {
  constexpr int CPR = DT / 8;
  constexpr int NKS = DT / 16;
  constexpr int NDB = DT / 32;
  constexpr int RB = 32 * QB;          // rows per workgroup
  constexpr int RING = 2;              // 32-key steps in flight per wave
  constexpr int VT = 32 * DT;          // elements of one K (or V) step tile
  constexpr int NVI = 32 * CPR / 64;   // 1 KB DMA instructions per step tile
  constexpr int NL = 2 * NVI;          // memory instructions per step (K and V)
  constexpr int OSTR = DT + 1;         // padded rows of the merge buffer
  using Tile = SwizzledTile<CPR>;
  static_assert(32 * CPR % 64 == 0, "V step tiles must split into whole DMA instructions");
  // Per wave: RING (K, V) step tiles; reused at the end for the cross-wave merge.
  constexpr int VBYTES = 4 * RING * 2 * VT * 2;
  constexpr int MBYTES = (4 * RB * OSTR + 8 * RB) * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[VBYTES > MBYTES ? VBYTES : MBYTES];

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
  // This wave's steps: 32-key blocks c0 + 32 (wave + 4 j), j = 0 .. nst - 1.
  const int nst = c1 > c0 + 32 * wave ? cdiv(c1 - c0 - 32 * wave, 128) : 0;

  const auto kr = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, rows_extent(p.Sk, p.k_ss, p.D));
  const auto vr = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, rows_extent(p.Sk, p.v_ss, p.D));
  uint16_t* kvring = reinterpret_cast<uint16_t*>(smem) + wave * RING * 2 * VT;  // [slot][K | V]

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
  const float sl2 = fabsf(p.scale_log2);
  // Per-lane DMA plan: the tile row this lane fills in each instruction
  // (huge for head-dim padding) and its chunk's byte offset in the row.
  int vrow[NVI];
  uint32_t vcol[NVI];
#pragma unroll
  for (int k = 0; k < NVI; ++k) {
    const int pc = k * 64 + lane;
    const int r = pc / CPR;
    const int c = (pc % CPR) ^ Tile::key(r);
    vrow[k] = c * 8 < p.D ? r : 0x7fffffff;
    vcol[k] = (uint32_t)c * 16u;
  }
  // Step j of this wave: its K and V tiles (32 keys) into the wave's LDS
  // ring by direct-to-LDS loads. Every load of the loop is of this kind, so
  // the compiler tracks none of them and the explicit waits below are the
  // only ones (a compiler wait on a register load would drain the ring).
  auto issue = [&](int j, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int kb0 = c0 + 32 * (wave + 4 * j);
#pragma unroll
    for (int k = 0; k < NVI; ++k) {
      const bool ok = vrow[k] < c1 - kb0;
      const uint32_t row = (uint32_t)(kb0 + vrow[k]);
      dma16(kr, kvring + slot * 2 * VT + k * 512, ok ? row * (uint32_t)(p.k_ss * 2) + vcol[k] : kOOB);
      dma16(vr, kvring + slot * 2 * VT + VT + k * 512, ok ? row * (uint32_t)(p.v_ss * 2) + vcol[k] : kOOB);
    }
  };

  f32x16 oacc[QB][NDB];
  float m_i[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = kNegInf;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = zero16();
  }

  // One 32-key step from ring slot `slot`.
  auto step = [&](int j, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int kb0 = c0 + 32 * (wave + 4 * j);
    const uint16_t* Ks = kvring + slot * 2 * VT;
    const uint16_t* Vs = Ks + VT;
    u32x4 ka[NKS];  // K rows as MFMA A operands: lane = key, slots = head_dim
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) ka[ks] = lds_read16(Ks + Tile::chunk(l32, 2 * ks + h32) * 8);
    f32x16 s[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      s[qb] = zero16();
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) s[qb] = Elem<T>::mfma(ka[ks], qf[qb][ks], s[qb]);
    }
    // S^T layout: lane = row, register r = key kb0 + 8 (r/4) + 4 h + r % 4.
    const int lim = c1 - kb0;  // keys c < lim are visible
    u32x4 pk[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (lim < 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = 8 * (r >> 2) + 4 * h32 + (r & 3);
          s[qb][r] = c < lim ? s[qb][r] : kNegInf;
        }
      }
      float mx = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][r]);
      mx = wave_xor32_max(mx) * sl2;
      if (m_i[qb] == kNegInf) {
        m_i[qb] = mx;
      } else {
        const bool grow = mx > m_i[qb] + kRescaleThreshold;
        if (wave_any(grow)) {
          const float alpha = grow ? fast_exp2(m_i[qb] - mx) : 1.f;
          l_i[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < NDB; ++db) oacc[qb][db] *= alpha;
          m_i[qb] = grow ? mx : m_i[qb];
        }
      }
      const float msub = (m_i[qb] == kNegInf) ? 0.f : m_i[qb];
#pragma unroll
      for (int r = 0; r < 16; ++r) s[qb][r] = fast_exp2(fmaf(s[qb][r], sl2, -msub));
      pk[qb][0] = pack8<T>(s[qb], 0);
      pk[qb][1] = pack8<T>(s[qb], 8);
      // The denominator sums the rounded P that the PV product consumes.
      float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < 2; ++w2) {
        rs0 = sum2_acc<T>(pk[qb][w2][0], rs0);
        rs1 = sum2_acc<T>(pk[qb][w2][1], rs1);
        rs0 = sum2_acc<T>(pk[qb][w2][2], rs0);
        rs1 = sum2_acc<T>(pk[qb][w2][3], rs1);
      }
      l_i[qb] += rs0 + rs1;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int stp = 0; stp < 2; ++stp) {
        const u32x4 a = lds_read_tr_operand_sw<CPR>(Vs, 16 * stp, 32 * db, lane);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) oacc[qb][db] = Elem<T>::mfma(a, pk[qb][stp], oacc[qb][db]);
      }
    }
  };

  // Ring: steps j .. j + RING - 1 are in flight; before step j the wave waits
  // for its loads (those of later steps may remain outstanding), and after it
  // refills the slot with step j + RING. A wave only ever reads its own LDS
  // slots, so no workgroup barrier is needed until the merge.
  static_for<0, RING>([&](auto sc) {
    if (decltype(sc)::value < nst) issue(decltype(sc)::value, sc);
  });
  // Q (issued first) is needed from the first step on; waiting for it only
  // now overlaps its latency with that of the ring's first loads.
  wait_all_memory();
  // Scores are reduced before scaling, which needs a positive scale: for a
  // negative one Q is negated (exact) and |scale| (sl2) used.
  if (p.scale_log2 < 0.f) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) qf[qb][ks] ^= 0x80008000u;
  }
  for (int j0 = 0; j0 < nst; j0 += RING) {
    static_for<0, RING>([&](auto sc) {
      constexpr int slot = decltype(sc)::value;
      const int j = j0 + slot;
      if (j < nst) {
        const int later = min(RING - 1, nst - 1 - j);  // steps issued after j
        if (later >= 1) KF_WAIT_VMCNT(NL);
        else KF_WAIT_VMCNT(0);
        step(j, sc);
        if (j + RING < nst) issue(j + RING, sc);
      }
    });
  }
  static_assert(RING == 2, "the waits above assume at most one later step in flight");

  // Cross-wave merge in one pass: every wave stores (m, l, O) of its rows;
  // then each output element combines the four waves in a fixed order.
  __syncthreads();  // all waves are done with their V rings
  float* obuf = reinterpret_cast<float*>(smem);  // [4][RB][OSTR]
  float* mbuf = obuf + 4 * RB * OSTR;            // [4][RB]
  float* lbuf = mbuf + 4 * RB;                   // [4][RB]
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int r = qb * 32 + l32;
    const float lt = wave_xor32_sum(l_i[qb]);
    if (h32 == 0) {
      mbuf[wave * RB + r] = m_i[qb];
      lbuf[wave * RB + r] = lt;
    }
    float* orow = obuf + (wave * RB + r) * OSTR;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) orow[32 * db + 8 * (rr >> 2) + 4 * h32 + (rr & 3)] = oacc[qb][db][rr];
  }
  __syncthreads();

  // Output: final O/LSE (one split) or this split's fp32 partial.
  const int nrow = min(RB, R - rb * RB);
  const int DQ = p.D / 4;
  const int grp = (b * p.Hkv + kvh) * p.nrb + rb;
  const int64_t pbase = ((int64_t)grp * p.nsplit + split) * RB;
  for (int e = tid; e < nrow * DQ; e += 256) {
    const int r = e / DQ, d = (e % DQ) * 4;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, mbuf[w * RB + r]);
    const float Ms = M == kNegInf ? 0.f : M;
    float lt = 0.f;
    float4 ov = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float cw = fast_exp2(mbuf[w * RB + r] - Ms);
      const float* o = obuf + (w * RB + r) * OSTR + d;
      lt += cw * lbuf[w * RB + r];
      ov.x += cw * o[0]; ov.y += cw * o[1]; ov.z += cw * o[2]; ov.w += cw * o[3];
    }
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    ov.x *= inv; ov.y *= inv; ov.z *= inv; ov.w *= inv;
    const float lse_val = lt > 0.f ? (M + fast_log2(lt)) * kLn2 : kNegInf;
    if (p.nsplit == 1) {
      const int rho = rb * RB + r;
      const int g = rho / p.Sq, i = rho % p.Sq;
      const int h = kvh * p.G + g;
      u32x2 w2;
      w2[0] = pack2<T>(ov.x, ov.y);
      w2[1] = pack2<T>(ov.z, ov.w);
      *reinterpret_cast<u32x2*>(p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss + d) = w2;
      if (d == 0 && p.lse) p.lse[((int64_t)b * p.Hq + h) * p.Sq + i] = lse_val;
    } else {
      *reinterpret_cast<float4*>(p.part_o + (pbase + r) * p.D + d) = ov;
      if (d == 0) p.part_lse[pbase + r] = lse_val;
    }
  }
}

// Merge of the split partials: one workgroup per output row. Thread
// (q = tid % DQ, sl = tid / DQ) owns 4 columns of splits sl, sl + SL, ...; it
// issues the loads of up to kMergeU of its splits (LSE and O) before using
// any, so a chunk of kMergeU * SL splits costs one memory round trip: the
// common case (nsplit <= kMergeU * SL) reads everything in one trip.
constexpr int kMergeU = 8;

template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(const DecParams p) {
  const int tid = threadIdx.x;
  const int RB = p.rb_rows;
  const int R = p.G * p.Sq;
  // blockIdx -> (b, kvh, packed row rho); partial rows are grouped by row block.
  const int rho_all = blockIdx.x % R;
  const int bk = blockIdx.x / R;
  const int kvh = bk % p.Hkv, b = bk / p.Hkv;
  const int rb = rho_all / RB, r = rho_all % RB;
  const int grp = (b * p.Hkv + kvh) * p.nrb + rb;
  const int g = rho_all / p.Sq, i = rho_all % p.Sq;
  const int h = kvh * p.G + g;
  const float* plse = p.part_lse + (int64_t)grp * p.nsplit * RB + r;
  const float* po = p.part_o + (int64_t)grp * p.nsplit * RB * p.D + (int64_t)r * p.D;
  __shared__ float red[8];
  __shared__ float4 acc4[256];

  const int DQ = p.D / 4;
  const int SL = 256 / DQ;
  const int q = tid % DQ, sl = tid / DQ;
  const bool active = sl < SL;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float den = 0.f, mrun = kNegInf;  // running reference max of this thread's chunks
  for (int c0 = 0; c0 < p.nsplit; c0 += kMergeU * SL) {
    float4 v[kMergeU];
    float w[kMergeU];
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      const int s2 = c0 + sl + SL * u;
      const bool ok = active && s2 < p.nsplit;
      v[u] = ok ? *reinterpret_cast<const float4*>(po + (int64_t)s2 * RB * p.D + 4 * q)
                : make_float4(0.f, 0.f, 0.f, 0.f);
      w[u] = ok ? plse[(int64_t)s2 * RB] * kLog2e : kNegInf;
    }
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) mx = fmaxf(mx, w[u]);
    // Thread-local online rescale across chunks (one chunk in the common case).
    const float mnew = fmaxf(mrun, mx);
    const float ms = mnew == kNegInf ? 0.f : mnew;
    const float alpha = fast_exp2(mrun - ms);
    acc.x *= alpha; acc.y *= alpha; acc.z *= alpha; acc.w *= alpha;
    den *= alpha;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      const float wt = fast_exp2(w[u] - ms);
      den += wt;
      acc.x += wt * v[u].x; acc.y += wt * v[u].y; acc.z += wt * v[u].z; acc.w += wt * v[u].w;
    }
    mrun = mnew;
  }
  // Block-wide max of the per-thread reference maxima, then rescale.
  float mx = mrun;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float Ms = M == kNegInf ? 0.f : M;
  const float sc = fast_exp2(mrun - Ms);
  acc.x *= sc; acc.y *= sc; acc.z *= sc; acc.w *= sc;
  den *= sc;
  // Every split's weight was counted once per column group; use q == 0's.
  float dsum = q == 0 ? den : 0.f;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = dsum;
  acc4[tid] = acc;
  __syncthreads();
  const float dtot = red[4] + red[5] + red[6] + red[7];
  if (tid < DQ) {
    for (int s2 = 1; s2 < SL; ++s2) {
      const float4 o2 = acc4[s2 * DQ + tid];
      acc.x += o2.x; acc.y += o2.y; acc.z += o2.z; acc.w += o2.w;
    }
    const float inv = dtot > 0.f ? 1.f / dtot : 0.f;
    u32x2 wv;
    wv[0] = pack2<T>(acc.x * inv, acc.y * inv);
    wv[1] = pack2<T>(acc.z * inv, acc.w * inv);
    *reinterpret_cast<u32x2*>(p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss + 4 * tid) = wv;
    if (tid == 0 && p.lse)
      p.lse[((int64_t)b * p.Hq + h) * p.Sq + i] = dtot > 0.f ? (M + fast_log2(dtot)) * kLn2 : kNegInf;
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
  const int64_t mgrid = (int64_t)p.B * p.Hkv * R;
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
  // whole 128-key granules; splits only add merge traffic beyond that.
  const int64_t stage = kDecGranule;
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
  const int64_t stage = kDecGranule;
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
