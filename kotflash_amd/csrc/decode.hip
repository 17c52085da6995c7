// Split-KV decode for gfx950 (short query, long KV cache, non-causal).
//
// Layout of the work:
//  * The Hq/Hkv query heads of a KV group and the Sq query positions are packed
//    into R = G * Sq rows (row = g * Sq + i). A workgroup owns up to 16 * QB of
//    those rows (QB = 1, 2, 4) for one (batch, kv_head) and one KV chunk, so
//    every K/V byte of the chunk is read from HBM once for all rows of the
//    group (the reference re-reads K/V once per query head,
//    triton_decode.py:16-104). Rows come in 16-row blocks because the products
//    are v_mfma_f32_16x16x32: a decode step has few rows (4 at G = 4, Sq = 1),
//    of which a 16-row block computes a quarter usefully and a 32-row block an
//    eighth, so 16-row blocks take half as long per key.
//  * The chunk is cut into 32-key steps that the 4 waves take in turn (so
//    chunks are whole 128-key granules). Each wave streams its own steps with
//    no workgroup barrier: its K and V tiles go into a wave-private LDS ring
//    by direct-to-LDS loads (two steps in flight), and the wave keeps its own
//    online-softmax state
//    (S^T = K Q^T per step, P^T feeding O^T += V^T P^T as in the forward).
//    The Q tile is loaded the same way, so a wave starts on its first step as
//    soon as that step has landed while its later loads are still in flight.
//  * At the end the 4 per-wave states are merged in LDS in one pass with a
//    fixed order (deterministic), and the workgroup writes either the final
//    O/LSE (one split) or an fp32 partial (O_s, LSE_s) of its row block.
//  * Keys at or beyond the per-batch visible length L_b are masked; a split
//    with no visible key writes O_s = 0, LSE_s = -inf (weight 0 in the merge),
//    as the reference does (triton_forward.py:240-246).
//  * merge_kernel (second launch, one wave per output row) combines the
//    partials with LSE weights
//      w_s = exp(LSE_s - max) / sum_t exp(LSE_t - max),  LSE = max + ln(sum)
//    guarded for all -inf (reference triton_forward.py:269-349). Each lane
//    issues all of its partial loads before using any, so the merge costs
//    about one memory latency. (A single-launch merge by the last arriving
//    workgroup was measured slower: either agent-scope release fences or
//    agent-scope stores plus a counter atomic per workgroup cost more than
//    the second launch.)
#include <atomic>
#include <mutex>

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
  // Fused append (decode_kernel<..., true>): the new tokens [B][Hkv][nnew][D];
  // k/v above are then the caches themselves.
  const uint16_t* nk;
  const uint16_t* nv;
  int64_t nk_sb, nk_sh, nk_ss;
  int64_t nv_sb, nv_sh, nv_ss;
  int nnew;
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

template <typename T, int DT, int QB, bool APPEND>
__global__ __launch_bounds__(256, 2) void decode_kernel(const DecParams p) {
  constexpr int CPR = DT / 8;          // 16-byte chunks per row
  constexpr int NDC = DT / 32;         // 32-wide head-dim chunks (S contraction)
  constexpr int NDB = DT / 16;         // 16-wide head-dim blocks of O^T
  constexpr int RB = 16 * QB;          // packed rows per workgroup
  constexpr int RING = 2;              // 32-key steps in flight per wave
  constexpr int VT = 32 * DT;          // elements of one K (or V) step tile
  constexpr int NVI = 32 * CPR / 64;   // 1 KB DMA instructions per step tile
  constexpr int NL = 2 * NVI;          // memory instructions per step (K and V)
  constexpr int QT = RB * DT;          // elements of the Q tile
  constexpr int NQI = RB * CPR / 64;   // DMA instructions of the Q tile
  constexpr int OSTR = DT + 1;         // padded rows of the merge buffer
  using Tile = SwizzledTile<CPR>;
  static_assert(32 * CPR % 64 == 0 && RB * CPR % 64 == 0, "tiles must split into whole DMA instructions");
  // Q tile, then per wave RING (K, V) step tiles; reused at the end for the
  // cross-wave merge.
  constexpr int VBYTES = (QT + 4 * RING * 2 * VT) * 2;
  constexpr int MBYTES = (4 * RB * OSTR + 8 * RB) * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[VBYTES > MBYTES ? VBYTES : MBYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int l16 = lane & 15, g16 = lane >> 4;

  int bid = blockIdx.x;
  int split;
  if constexpr (APPEND) {
    // The new tokens' workgroups (split nsplit - 1 of every row group) come
    // first in the grid: they are short, and dispatched last they would end
    // the launch.
    const int ngrp = p.B * p.Hkv * p.nrb;
    if (bid < ngrp) {
      split = p.nsplit - 1;
    } else {
      bid -= ngrp;
      split = bid % (p.nsplit - 1);
      bid /= p.nsplit - 1;
    }
  } else {
    split = bid % p.nsplit;
    bid /= p.nsplit;
  }
  const int rb = bid % p.nrb;
  bid /= p.nrb;
  const int kvh = bid % p.Hkv;
  const int b = bid / p.Hkv;
  const int R = p.G * p.Sq;

  const int L = p.seqlens ? min(max(p.seqlens[b], 0), p.Sk) : p.Sk;
  // With APPEND, the last split attends to the nnew new tokens, read from
  // their own buffer (keys [0, nnew) of it); the others cover the cache's
  // keys [0, L_b) as without it. No workgroup of the launch reads cache rows
  // [L_b, L_b + nnew), so the new split's copy into them races with nothing.
  const bool fresh = APPEND && split == p.nsplit - 1;
  const int c0 = fresh ? 0 : split * p.chunk;
  const int c1 = fresh ? p.nnew : min(c0 + p.chunk, L);
  const uint16_t* kbase = fresh ? p.nk + b * p.nk_sb + kvh * p.nk_sh : p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t* vbase = fresh ? p.nv + b * p.nv_sb + kvh * p.nv_sh : p.v + b * p.v_sb + kvh * p.v_sh;
  const int64_t kss = fresh ? p.nk_ss : p.k_ss;
  const int64_t vss = fresh ? p.nv_ss : p.v_ss;
  // This wave's steps: 32-key blocks c0 + 32 (wave + 4 j), j = 0 .. nst - 1.
  const int nst = c1 > c0 + 32 * wave ? cdiv(c1 - c0 - 32 * wave, 128) : 0;
  const int nrow = min(RB, R - rb * RB);
  const int grp = (b * p.Hkv + kvh) * p.nrb + rb;
  const int64_t pbase = ((int64_t)grp * p.nsplit + split) * RB;
  if (c1 <= c0 && p.nsplit > 1) {
    // A split past this sequence's visible length (ragged batches): weight 0
    // in the merge, written without loading anything.
    for (int e = tid; e < nrow * (p.D / 4); e += 256) {
      const int r = e / (p.D / 4), d = (e % (p.D / 4)) * 4;
      *reinterpret_cast<float4*>(p.part_o + (pbase + r) * p.D + d) = make_float4(0.f, 0.f, 0.f, 0.f);
      if (d == 0) p.part_lse[pbase + r] = kNegInf;
    }
    return;
  }

  // K/V resources end at the chunk's last visible key: keys at or beyond c1
  // (the range check includes the scalar offset) load as zeros.
  const auto kr = make_rsrc(kbase, rows_extent(c1, kss, p.D));
  const auto vr = make_rsrc(vbase, rows_extent(c1, vss, p.D));
  const auto qr = make_rsrc(p.q + b * p.q_sb + kvh * p.G * p.q_sh,
                            (uint32_t)((((int64_t)p.G - 1) * p.q_sh + ((int64_t)p.Sq - 1) * p.q_ss + p.D) * 2));
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem);                 // [RB][DT], swizzled
  uint16_t* kvring = qs + QT + wave * RING * 2 * VT;                // [slot][K | V]

  // The Q tile goes to LDS by direct-to-LDS loads too (the waves share its
  // instructions), so that no register load is pending when the ring starts:
  // the compiler would otherwise wait for every load at the first use of Q.
#pragma unroll
  for (int k = 0; k < NQI; ++k) {
    if (k % 4 != wave) continue;
    const int pc = k * 64 + lane;
    const int r = pc / CPR;
    const int c = (pc % CPR) ^ Tile::key(r);
    const int rho = rb * RB + r;
    const bool ok = rho < R && c * 8 < p.D;
    const int g = ok ? rho / p.Sq : 0, i = ok ? rho % p.Sq : 0;
    dma16(qr, qs + k * 512, ok ? (uint32_t)(g * p.q_sh + i * p.q_ss + c * 8) * 2u : kOOB);
  }
  // Per-lane DMA plan of a K/V step tile: the byte offset of this lane's
  // 16-byte chunk within the tile's rows (kOOB for head-dim padding). The
  // step's first key enters as the scalar offset, so issuing a step costs no
  // vector instructions.
  uint32_t koff[NVI], voff[NVI];
#pragma unroll
  for (int k = 0; k < NVI; ++k) {
    const int pc = k * 64 + lane;
    const int r = pc / CPR;
    const int c = (pc % CPR) ^ Tile::key(r);
    const bool ok = c * 8 < p.D;
    koff[k] = ok ? (uint32_t)(r * kss + c * 8) * 2u : kOOB;
    voff[k] = ok ? (uint32_t)(r * vss + c * 8) * 2u : kOOB;
  }
  const uint32_t ring0 = lds_addr(kvring);
  // Step j of this wave: its K and V tiles (32 keys) into the wave's LDS
  // ring. Every load of the kernel is a direct-to-LDS load, so the explicit
  // waits below are the only ones.
  auto issue = [&](int j, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int kb0 = c0 + 32 * (wave + 4 * j);
    const uint32_t kso = (uint32_t)kb0 * (uint32_t)(kss * 2);
    const uint32_t vso = (uint32_t)kb0 * (uint32_t)(vss * 2);
    const uint32_t m0 = ring0 + (uint32_t)(slot * 2 * VT * 2);
#pragma unroll
    for (int k = 0; k < NVI; ++k) {
      dma16_s(kr, m0 + k * 1024u, koff[k], kso);
      dma16_s(vr, m0 + VT * 2 + k * 1024u, voff[k], vso);
    }
  };
  static_for<0, RING>([&](auto sc) {
    if (decltype(sc)::value < nst) issue(decltype(sc)::value, sc);
  });

  f32x4 oacc[QB][NDB];  // O^T: lane l, register r = head-dim 16 db + 4 (l / 16) + r of row l % 16
  float m_i[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = kNegInf;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Q and step 0 have landed once at most one later step is outstanding (the
  // counter completes in order); the barrier publishes every wave's share of
  // the Q tile. Waves without steps pass it too.
  if (nst >= 2) KF_WAIT_VMCNT(NL);
  else KF_WAIT_VMCNT(0);
  __syncthreads();
  // Q rows as MFMA B operands: lane l = packed row qb * 16 + l % 16, k slots =
  // head dims 32 dc + 8 (l / 16) .. + 7.
  u32x4 qf[QB][NDC];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int dc = 0; dc < NDC; ++dc) qf[qb][dc] = lds_read16(qs + Tile::chunk(qb * 16 + l16, 4 * dc + g16) * 8);
  const float sl2 = fabsf(p.scale_log2);
  // Scores are reduced before scaling, which needs a positive scale: for a
  // negative one Q is negated (exact) and |scale| (sl2) used.
  if (p.scale_log2 < 0.f) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) qf[qb][dc] ^= 0x80008000u;
  }

  // One 32-key step from ring slot `slot`, as two 16-key blocks kb.
  auto step = [&](int j, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int kb0 = c0 + 32 * (wave + 4 * j);
    const uint16_t* Ks = kvring + slot * 2 * VT;
    const uint16_t* Vs = Ks + VT;
    // K rows as MFMA A operands: lane = key kb * 16 + l % 16, slots = head dims.
    u32x4 ka[2][NDC];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) ka[kb][dc] = lds_read16(Ks + Tile::chunk(kb * 16 + l16, 4 * dc + g16) * 8);
    // S^T: lane l, register r = key kb * 16 + 4 (l / 16) + r of row l % 16.
    f32x4 s[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dc = 0; dc < NDC; ++dc) s[qb][kb] = Elem<T>::mfma16(ka[kb][dc], qf[qb][dc], s[qb][kb]);
      }
    const int lim = c1 - kb0;  // keys c < lim are visible
    u32x4 pk[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (lim < 32) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int c = 16 * kb + 4 * g16 + r;
            s[qb][kb][r] = c < lim ? s[qb][kb][r] : kNegInf;
          }
      }
      float mx = kNegInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[qb][kb][r]);
      mx = wave_group16_max(mx) * sl2;
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
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[qb][kb][r] = fast_exp2(fmaf(s[qb][kb][r], sl2, -msub));
      // P^T as the B operand of O^T += V^T P^T: slot t of lane group g holds
      // key 4 g + t (t < 4) or 16 + 4 g + t - 4 (t >= 4).
      pk[qb][0] = pack2<T>(s[qb][0][0], s[qb][0][1]);
      pk[qb][1] = pack2<T>(s[qb][0][2], s[qb][0][3]);
      pk[qb][2] = pack2<T>(s[qb][1][0], s[qb][1][1]);
      pk[qb][3] = pack2<T>(s[qb][1][2], s[qb][1][3]);
      // The denominator sums the rounded P that the PV product consumes.
      l_i[qb] += sum2_acc<T>(pk[qb][0], sum2_acc<T>(pk[qb][1], 0.f)) +
                 sum2_acc<T>(pk[qb][2], sum2_acc<T>(pk[qb][3], 0.f));
    }
    // V^T A operands by transposed reads: lane (g, i) receives V[key][16 db + i]
    // for the keys of slot t above (rows 4 g .. 4 g + 3 and 16 + 4 g .. + 3).
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int col = 16 * db + 4 * (l16 & 3);
      const u32x2 lo = lds_read_tr16(Vs + Tile::elem(4 * g16 + (l16 >> 2), col));
      const u32x2 hi = lds_read_tr16(Vs + Tile::elem(16 + 4 * g16 + (l16 >> 2), col));
      const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) oacc[qb][db] = Elem<T>::mfma16(a, pk[qb], oacc[qb][db]);
    }
  };

  // Ring: steps j .. j + RING - 1 are in flight; before step j the wave waits
  // for its loads (those of later steps may remain outstanding), and after it
  // refills the slot with step j + RING. A wave only ever reads its own ring
  // slots, so no workgroup barrier is needed until the merge.
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
  __syncthreads();  // all waves are done with the Q tile and their rings
  float* obuf = reinterpret_cast<float*>(smem);  // [4][RB][OSTR]
  float* mbuf = obuf + 4 * RB * OSTR;            // [4][RB]
  float* lbuf = mbuf + 4 * RB;                   // [4][RB]
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if (qb * 16 >= nrow) break;
    const int r = qb * 16 + l16;
    const float lt = wave_group16_sum(l_i[qb]);
    if (g16 == 0) {
      mbuf[wave * RB + r] = m_i[qb];
      lbuf[wave * RB + r] = lt;
    }
    float* orow = obuf + (wave * RB + r) * OSTR + 4 * g16;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) orow[16 * db + rr] = oacc[qb][db][rr];
  }
  __syncthreads();

  // Output: final O/LSE (one split) or this split's fp32 partial.
  const int DQ = p.D / 4;
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
  if constexpr (APPEND) {
    // The single owner of the append: the new split of row block 0 stores
    // new[b, kvh, t, :] to cache position seqlens[b] + t (t < nnew) in
    // 16-byte vectors, after its own loads of the new tokens (bit-exact copy).
    // The host checked max_length + nnew <= capacity; a device length outside
    // [0, max_length] breaks that promise and its tokens are not written.
    if (fresh && rb == 0) {
      const int start = p.seqlens ? p.seqlens[b] : p.Sk;
      if (start < 0 || start > p.Sk) return;
      const int cpr = p.D / 8;
      uint16_t* kc = const_cast<uint16_t*>(p.k) + b * p.k_sb + kvh * p.k_sh;
      uint16_t* vc = const_cast<uint16_t*>(p.v) + b * p.v_sb + kvh * p.v_sh;
      for (int e = tid; e < p.nnew * cpr; e += 256) {
        const int t = e / cpr, d = (e % cpr) * 8;
        const uint4 kv4 = *reinterpret_cast<const uint4*>(kbase + t * kss + d);
        const uint4 vv4 = *reinterpret_cast<const uint4*>(vbase + t * vss + d);
        *reinterpret_cast<uint4*>(kc + (int64_t)(start + t) * p.k_ss + d) = kv4;
        *reinterpret_cast<uint4*>(vc + (int64_t)(start + t) * p.v_ss + d) = vv4;
      }
    }
  }
}

// Merge of the split partials: one wave per output row, no LDS and no
// barrier. Lane l = (q = l % QL, sl = l / QL) owns the 4 head-dim columns
// 4q .. 4q + 3 (QL = 16 or 32 lanes cover D / 4 <= QL) of splits sl, sl + SW,
// sl + 2 SW, ... (SW = 64 / QL). Its loads are buffer loads whose
// out-of-range lanes read zero, so no branch separates them and all kMergeU
// of a chunk (O and LSE) are in flight before the first is used: the common
// case (nsplit <= kMergeU * SW) costs one memory round trip. The SW lanes of
// a column then combine with lane swaps (v_permlane16/32_swap).
constexpr int kMergeU = 16;

// One output row: orr / lrr address split s's O row at s * ostride floats
// and its LSE at s * lstride floats; every offset must fit 32 bits (checked
// by the callers' hosts).
template <typename T, int QL>
__device__ inline void merge_row(__amdgpu_buffer_rsrc_t orr, __amdgpu_buffer_rsrc_t lrr,
                                 uint32_t ostride, uint32_t lstride, int nsplit, int D,
                                 uint16_t* out_row, float* lse_out) {
  constexpr int SW = 64 / QL;
  const int lane = threadIdx.x;
  const int q = lane % QL, sl = lane / QL;
  const bool col = 4 * q < D;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float den = 0.f, mrun = kNegInf;  // running reference max of this lane's chunks (log2 units)
  for (int c0 = 0; c0 < nsplit; c0 += kMergeU * SW) {
    u32x4 v[kMergeU];
    float w[kMergeU];
    uint32_t lw[kMergeU];
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      const int s2 = c0 + sl + SW * u;
      lw[u] = __builtin_amdgcn_raw_buffer_load_b32(lrr, s2 < nsplit ? (uint32_t)s2 * lstride * 4u : kOOB, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      const int s2 = c0 + sl + SW * u;
      v[u] = buf_load16(orr, s2 < nsplit && col ? ((uint32_t)s2 * ostride + 4u * q) * 4u : kOOB);
    }
    // Keep every load of the chunk ahead of the first use: left alone, the
    // scheduler recycles early result registers and waits for them mid-batch.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kMergeU; ++u)
      w[u] = c0 + sl + SW * u < nsplit ? __uint_as_float(lw[u]) * kLog2e : kNegInf;
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) mx = fmaxf(mx, w[u]);
    // Lane-local online rescale across chunks (one chunk in the common case).
    const float mnew = fmaxf(mrun, mx);
    const float ms = mnew == kNegInf ? 0.f : mnew;
    const float alpha = fast_exp2(mrun - ms);
    acc *= alpha;
    den *= alpha;
#pragma unroll
    for (int u = 0; u < kMergeU; ++u) {
      const float wt = fast_exp2(w[u] - ms);
      den += wt;
      acc[0] += wt * __uint_as_float(v[u][0]); acc[1] += wt * __uint_as_float(v[u][1]);
      acc[2] += wt * __uint_as_float(v[u][2]); acc[3] += wt * __uint_as_float(v[u][3]);
    }
    mrun = mnew;
  }
  // Combine the SW split lanes of each column: common reference max, then sums.
  const float M = QL == 16 ? wave_group16_max(mrun) : wave_xor32_max(mrun);
  const float Ms = M == kNegInf ? 0.f : M;
  const float sc = fast_exp2(mrun - Ms);
  float dtot = den * sc;
  dtot = QL == 16 ? wave_group16_sum(dtot) : wave_xor32_sum(dtot);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x = acc[e] * sc;
    acc[e] = QL == 16 ? wave_group16_sum(x) : wave_xor32_sum(x);
  }
  if (sl == 0 && col) {
    const float inv = dtot > 0.f ? 1.f / dtot : 0.f;
    u32x2 wv;
    wv[0] = pack2<T>(acc[0] * inv, acc[1] * inv);
    wv[1] = pack2<T>(acc[2] * inv, acc[3] * inv);
    *reinterpret_cast<u32x2*>(out_row + 4 * q) = wv;
    if (q == 0 && lse_out) *lse_out = dtot > 0.f ? (M + fast_log2(dtot)) * kLn2 : kNegInf;
  }
}

template <typename T, int QL>
__global__ __launch_bounds__(64) void merge_kernel(const DecParams p) {
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
  // Row r of every split's partial: O at (s * RB + r) * D floats, LSE at s * RB + r.
  const auto orr = make_rsrc(p.part_o + ((int64_t)grp * p.nsplit * RB + r) * p.D,
                             (uint32_t)(((int64_t)(p.nsplit - 1) * RB * p.D + p.D) * 4));
  const auto lrr = make_rsrc(p.part_lse + (int64_t)grp * p.nsplit * RB + r,
                             (uint32_t)(((int64_t)(p.nsplit - 1) * RB + 1) * 4));
  merge_row<T, QL>(orr, lrr, (uint32_t)(RB * p.D), (uint32_t)RB, p.nsplit, p.D,
                   p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss,
                   p.lse ? p.lse + ((int64_t)b * p.Hq + h) * p.Sq + i : nullptr);
}

// Standalone merge of split partials in the reference's layout
// (triton_forward.py:269-349): part_o [nsplit][B][H][S][D] and part_lse
// [nsplit][B][H][S], fp32 and contiguous; one wave per output row.
struct MergeParams {
  const float* part_o;
  const float* part_lse;
  uint16_t* o;
  float* lse;
  int64_t o_sb, o_sh, o_ss;
  int B, H, S, D, nsplit;
};

template <typename T, int QL>
__global__ __launch_bounds__(64) void lse_merge_kernel(const MergeParams p) {
  const int64_t rows = (int64_t)p.B * p.H * p.S;
  const int64_t row = blockIdx.x;
  const int i = (int)(row % p.S);
  const int64_t bh = row / p.S;
  const int h = (int)(bh % p.H), b = (int)(bh / p.H);
  const auto orr = make_rsrc(p.part_o + row * p.D,
                             (uint32_t)(((int64_t)(p.nsplit - 1) * rows * p.D + p.D) * 4));
  const auto lrr = make_rsrc(p.part_lse + row, (uint32_t)(((int64_t)(p.nsplit - 1) * rows + 1) * 4));
  merge_row<T, QL>(orr, lrr, (uint32_t)(rows * p.D), (uint32_t)rows, p.nsplit, p.D,
                   p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss, p.lse ? p.lse + row : nullptr);
}

// Packed rows per workgroup: 16-row MFMA blocks, up to four of them.
static int decode_rows_per_wg(int64_t G, int64_t Sq) {
  const int64_t R = G * Sq;
  return R <= 16 ? 16 : R <= 32 ? 32 : 64;
}

template <typename T, int DT, bool APPEND>
static int launch_decode(DecParams p, hipStream_t stream) {
  const int R = p.G * p.Sq;
  p.rb_rows = decode_rows_per_wg(p.G, p.Sq);
  p.nrb = cdiv(R, p.rb_rows);
  const int64_t grid = (int64_t)p.nsplit * p.nrb * p.B * p.Hkv;
  if (grid > 0x7fffffff) return set_error(KF_EUNSUPPORTED, "kf_attn_decode: grid too large");
  switch (p.rb_rows) {
    case 16: hipLaunchKernelGGL((decode_kernel<T, DT, 1, APPEND>), dim3((unsigned)grid), dim3(256), 0, stream, p); break;
    case 32: hipLaunchKernelGGL((decode_kernel<T, DT, 2, APPEND>), dim3((unsigned)grid), dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL((decode_kernel<T, DT, 4, APPEND>), dim3((unsigned)grid), dim3(256), 0, stream, p); break;
  }
  int rc = check_launch("kf_attn_decode(split)");
  if (rc || p.nsplit == 1) return rc;
  const int64_t mgrid = (int64_t)p.B * p.Hkv * R;
  if (p.D <= 64)
    hipLaunchKernelGGL((merge_kernel<T, 16>), dim3((unsigned)mgrid), dim3(64), 0, stream, p);
  else
    hipLaunchKernelGGL((merge_kernel<T, 32>), dim3((unsigned)mgrid), dim3(64), 0, stream, p);
  return check_launch("kf_attn_decode(merge)");
}

template <typename T, bool APPEND>
static int dispatch_decode(const DecParams& p, hipStream_t stream) {
  switch (head_tile(p.D)) {
    case 32: return launch_decode<T, 32, APPEND>(p, stream);
    case 64: return launch_decode<T, 64, APPEND>(p, stream);
    case 96: return launch_decode<T, 96, APPEND>(p, stream);
    default: return launch_decode<T, 128, APPEND>(p, stream);
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

// Ragged batches: non-empty workgroups the planner aims for. Swept on MI355X
// over 256-1024 at config 5's shapes (B=8, Hkv=8, Hq=32, n = 1-16 new rows
// per step) for three length spreads (1K-8K, 4K-28K, 16K-31K): 384 was the
// fastest or within 0.4% of it in each, 5-9% ahead of 1024, whose smaller
// chunks write and merge more fp32 partials; 448 and 512 were not monotone
// in between (up to 14% behind 384).
constexpr int64_t kDecRaggedWGs = 384;

static int64_t decode_row_blocks(int64_t G, int64_t Sq) {
  const int rb = decode_rows_per_wg(G, Sq);
  return (G * Sq + rb - 1) / rb;
}

extern "C" int kf_decode_num_splits_ragged(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                           const int32_t* lengths, int64_t D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || D <= 0 || Hq % Hkv || lengths == nullptr) return 1;
  int64_t maxlen = 0, total = 0;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t L = lengths[b] > 0 ? lengths[b] : 0;
    maxlen = L > maxlen ? L : maxlen;
    total += L;
  }
  if (maxlen <= 0) return 1;
  // Chunk from the total visible work: the non-empty splits of all sequences
  // add up to about kDecRaggedWGs workgroups. Splits past a sequence's length
  // are empty and end at once.
  const int64_t stage = kDecGranule;
  const int64_t units = Hkv * decode_row_blocks(Hq / Hkv, Sq);
  int64_t chunk = (units * total + kDecRaggedWGs - 1) / kDecRaggedWGs;
  chunk = (chunk < stage ? stage : chunk + stage - 1) / stage * stage;
  int64_t ns = (maxlen + chunk - 1) / chunk;
  // Normalise the way kf_attn_decode derives the chunk from the count.
  chunk = ((maxlen + ns - 1) / ns + stage - 1) / stage * stage;
  ns = (maxlen + chunk - 1) / chunk;
  return (int)ns;
}

extern "C" size_t kf_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                            int64_t D, int num_splits) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || D <= 0 || Hq % Hkv || num_splits <= 1) return 0;
  const int64_t G = Hq / Hkv;
  const size_t slots = (size_t)(B * Hkv * decode_row_blocks(G, Sq)) * num_splits *
                       decode_rows_per_wg(G, Sq);
  return (slots * (size_t)D * sizeof(float) + 255) / 256 * 256 + (slots * sizeof(float) + 255) / 256 * 256;
}

// Argument checks and launch of kf_attn_decode and kf_attn_decode_noalloc
// (`what` names the entry point in error messages).
static int decode_entry(const char* what, const void* q, const void* k, const void* v, void* o,
                        float* lse, const int32_t* seqlens_k, int64_t B, int64_t Hq, int64_t Hkv,
                        int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides,
                        const int64_t* o_strides, float scale, int num_splits, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
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
  return dtype == KF_F16 ? dispatch_decode<_Float16, false>(p, s) : dispatch_decode<__bf16, false>(p, s);
}

extern "C" int kf_lse_merge(const float* part_o, const float* part_lse, void* o, float* lse,
                            int64_t num_splits, int64_t B, int64_t H, int64_t S, int64_t D,
                            const int64_t* o_strides, int dtype, void* stream) {
  const char* what = "kf_lse_merge";
  if (part_o == nullptr || part_lse == nullptr)
    return set_error(KF_EINVAL, "%s: part_o and part_lse must be non-null", what);
  if (num_splits < 1 || B <= 0 || H <= 0 || S <= 0)
    return set_error(KF_EINVAL, "%s: num_splits and all sizes must be positive", what);
  if (D % 4 != 0 || D <= 0 || D > 128)
    return set_error(KF_EUNSUPPORTED, "%s: head_dim must be a multiple of 4 in [4, 128], got %lld",
                     what, (long long)D);
  if (dtype != KF_F16 && dtype != KF_BF16)
    return set_error(KF_EINVAL, "%s: dtype must be KF_F16 or KF_BF16", what);
  if (o == nullptr || o_strides == nullptr) return set_error(KF_EINVAL, "%s: o is null", what);
  if (!aligned8(o) || o_strides[0] % 4 || o_strides[1] % 4 || o_strides[2] % 4 ||
      o_strides[0] < 0 || o_strides[1] < 0 || o_strides[2] < 0)
    return set_error(KF_EINVAL, "%s: o must be 8-byte aligned with strides that are non-negative "
                     "multiples of 4 elements", what);
  if (!aligned16(part_o) || (reinterpret_cast<uintptr_t>(part_lse) & 3u) != 0)
    return set_error(KF_EINVAL, "%s: part_o must be 16-byte and part_lse 4-byte aligned", what);
  const int64_t rows = B * H * S;
  if (rows > 0x7fffffff || num_splits * rows * D * 4 > 0x7fffffffLL)
    return set_error(KF_EUNSUPPORTED, "%s: partials beyond 2 GiB", what);
  MergeParams p{};
  p.part_o = part_o; p.part_lse = part_lse; p.o = (uint16_t*)o; p.lse = lse;
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = (int)B; p.H = (int)H; p.S = (int)S; p.D = (int)D; p.nsplit = (int)num_splits;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows);
  if (dtype == KF_F16) {
    if (D <= 64) hipLaunchKernelGGL((lse_merge_kernel<_Float16, 16>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((lse_merge_kernel<_Float16, 32>), grid, dim3(64), 0, s, p);
  } else {
    if (D <= 64) hipLaunchKernelGGL((lse_merge_kernel<__bf16, 16>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((lse_merge_kernel<__bf16, 32>), grid, dim3(64), 0, s, p);
  }
  return check_launch(what);
}

extern "C" int kf_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse,
                              const int32_t* seqlens_k, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides,
                              const int64_t* k_strides, const int64_t* v_strides,
                              const int64_t* o_strides, float scale, int num_splits, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  return decode_entry("kf_attn_decode", q, k, v, o, lse, seqlens_k, B, Hq, Hkv, Sq, Sk, D,
                      q_strides, k_strides, v_strides, o_strides, scale, num_splits, dtype,
                      workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// kf_attn_decode_noalloc: kf_attn_decode for callers that cannot allocate
// device memory (code under HIP graph capture, serving loops). Its split
// partials go to `scratch`, a fixed device array that every GPU the library
// runs on holds until the process ends. In host code the name `scratch` is
// only a stand-in for the device symbol: its device address is resolved once
// per device with hipGetSymbolAddress (with that device current) and kept in
// g_scratch_ptr; the kernels only ever receive that address.
//
// The decode kernels write every partial slot they later read (a split with
// no visible key writes O_s = 0, LSE_s = -inf), so nothing is cleared
// between calls. All calls on one GPU share its array: calls that overlap in
// time on one GPU (concurrent streams or threads) race on it.
constexpr size_t kDecodeScratchBytes = KF_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mutex;
}  // namespace

// Device address of `scratch` on the current device (resolved on the first
// call for that device).
static int decode_scratch(const char* what, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(KF_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(KF_EUNSUPPORTED, "%s: device index %d beyond the %d supported", what, dev,
                     kMaxScratchDevices);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || ptr == nullptr)
        return set_error(KF_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s",
                         what, dev, hipGetErrorString(e));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return KF_OK;
}

extern "C" int kf_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o,
                                      float* lse, const int32_t* seqlens_k, int64_t B, int64_t Hq,
                                      int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                                      const int64_t* q_strides, const int64_t* k_strides,
                                      const int64_t* v_strides, const int64_t* o_strides,
                                      float scale, int num_splits, int dtype, void* stream) {
  const char* what = "kf_attn_decode_noalloc";
  if (num_splits < 1) return set_error(KF_EINVAL, "%s: num_splits must be >= 1", what);
  const size_t need = kf_decode_workspace_bytes(B, Hq, Hkv, Sq, D, num_splits);
  if (need > kDecodeScratchBytes)
    return set_error(KF_EINVAL, "%s: this problem needs %zu bytes of split partials, more than "
                     "the %zu-byte static scratch; use kf_attn_decode with a workspace", what,
                     need, kDecodeScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = decode_scratch(what, &ws);
    if (rc) return rc;
  }
  return decode_entry(what, q, k, v, o, lse, seqlens_k, B, Hq, Hkv, Sq, Sk, D, q_strides,
                      k_strides, v_strides, o_strides, scale, num_splits, dtype, ws,
                      kDecodeScratchBytes, stream);
}

extern "C" int kf_attn_append_decode(const void* q, void* k_cache, void* v_cache, const void* new_k,
                                     const void* new_v, void* o, float* lse,
                                     const int32_t* lengths, int64_t past_length, int64_t B,
                                     int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Snew,
                                     int64_t max_length, int64_t capacity, int64_t D,
                                     const int64_t* q_strides, const int64_t* k_cache_strides,
                                     const int64_t* v_cache_strides, const int64_t* new_k_strides,
                                     const int64_t* new_v_strides, const int64_t* o_strides,
                                     float scale, int num_splits, int dtype, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  const char* what = "kf_attn_append_decode";
  // Sizes are checked as for kf_attn_decode with the cache's own keys
  // (max_length, at least 1 for the check) and the new tokens both present.
  int rc = check_attn_common(what, B, Hq, Hkv, Sq, max_length > 0 ? max_length : 1, D, dtype);
  if (rc) return rc;
  if ((rc = check_tensor(what, "q", q, q_strides)) ||
      (rc = check_tensor(what, "k_cache", k_cache, k_cache_strides)) ||
      (rc = check_tensor(what, "v_cache", v_cache, v_cache_strides)) ||
      (rc = check_tensor(what, "new_k", new_k, new_k_strides)) ||
      (rc = check_tensor(what, "new_v", new_v, new_v_strides)) ||
      (rc = check_tensor(what, "o", o, o_strides)))
    return rc;
  if (!(scale == scale) || scale - scale != 0.f) return set_error(KF_EINVAL, "%s: scale must be finite", what);
  if (Snew <= 0 || Snew > 0x3fffffff) return set_error(KF_EINVAL, "%s: Snew must be positive", what);
  if (max_length < 0 || capacity <= 0 || capacity > 0x3fffffff || max_length > capacity)
    return set_error(KF_EINVAL, "%s: need 0 <= max_length <= capacity", what);
  // max_length bounds every lengths[b] (the host's promise), so the append
  // range of every sequence fits iff this does (kv_append_cuda.cu:72-73).
  if (max_length + Snew > capacity)
    return set_error(KF_EINVAL, "%s: append range exceeds cache capacity (max_length %lld + %lld "
                     "new tokens > capacity %lld)", what, (long long)max_length, (long long)Snew,
                     (long long)capacity);
  if (lengths == nullptr && (past_length != max_length || past_length + Snew > capacity))
    return set_error(KF_EINVAL, "%s: past_length %lld + %lld new tokens must fit capacity %lld "
                     "(and equal max_length without per-sequence lengths)", what,
                     (long long)past_length, (long long)Snew, (long long)capacity);
  if (num_splits < 1) return set_error(KF_EINVAL, "%s: num_splits must be >= 1", what);
  const int64_t stage = kDecGranule;
  const int64_t Sk = max_length > 0 ? max_length : 1;
  const int64_t chunk = ((Sk + num_splits - 1) / num_splits + stage - 1) / stage * stage;
  if ((Sk + chunk - 1) / chunk != num_splits)
    return set_error(KF_EINVAL, "%s: num_splits=%d does not partition max_length=%lld into whole "
                     "%lld-key stages (use kf_decode_num_splits)", what, num_splits,
                     (long long)max_length, (long long)stage);
  if (((Hq / Hkv - 1) * q_strides[1] + (Sq - 1) * q_strides[2] + D) * 2 > 0x7fffffffLL)
    return set_error(KF_EUNSUPPORTED, "%s: one KV group of q spans more than 2 GiB", what);
  // One more split (the new tokens) than the cache's own.
  const size_t need = kf_decode_workspace_bytes(B, Hq, Hkv, Sq, D, num_splits + 1);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(KF_EINVAL, "%s: workspace of %zu bytes required, got %zu", what, need,
                     workspace == nullptr ? (size_t)0 : workspace_bytes);
  if ((rc = check_extent(what, "k_cache", capacity, k_cache_strides[2], D)) ||
      (rc = check_extent(what, "v_cache", capacity, v_cache_strides[2], D)) ||
      (rc = check_extent(what, "new_k", Snew, new_k_strides[2], D)) ||
      (rc = check_extent(what, "new_v", Snew, new_v_strides[2], D)))
    return rc;
  DecParams p{};
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k_cache; p.v = (const uint16_t*)v_cache;
  p.nk = (const uint16_t*)new_k; p.nv = (const uint16_t*)new_v;
  p.o = (uint16_t*)o; p.lse = lse; p.seqlens = lengths;
  const int64_t G = Hq / Hkv;
  const size_t slots = (size_t)(B * Hkv * decode_row_blocks(G, Sq)) * (num_splits + 1) *
                       decode_rows_per_wg(G, Sq);
  p.part_o = (float*)workspace;
  p.part_lse = (float*)((char*)workspace + (slots * (size_t)D * sizeof(float) + 255) / 256 * 256);
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_cache_strides[0]; p.k_sh = k_cache_strides[1]; p.k_ss = k_cache_strides[2];
  p.v_sb = v_cache_strides[0]; p.v_sh = v_cache_strides[1]; p.v_ss = v_cache_strides[2];
  p.nk_sb = new_k_strides[0]; p.nk_sh = new_k_strides[1]; p.nk_ss = new_k_strides[2];
  p.nv_sb = new_v_strides[0]; p.nv_sh = new_v_strides[1]; p.nv_ss = new_v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Sq = (int)Sq; p.D = (int)D;
  p.Sk = (int)max_length;  // per-sequence lengths are clamped to it; 0 = no cache keys
  p.G = (int)G;
  p.nsplit = num_splits + 1;
  p.chunk = (int)chunk;
  p.nnew = (int)Snew;
  p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  return dtype == KF_F16 ? dispatch_decode<_Float16, true>(p, s) : dispatch_decode<__bf16, true>(p, s);
}
