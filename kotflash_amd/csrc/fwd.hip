// Attention forward for gfx950: online softmax with MFMA QK^T and PV.
//
// Work decomposition. One workgroup (4 waves) owns BM = 4 * QB * 32 query rows
// of one (batch, q_head). Each wave owns QB blocks of 32 rows and keeps them
// for the whole kernel:
//   - Q rows in registers as MFMA B operands,
//   - the running max m, the running denominator l and the output accumulator
//     O^T (head_dim x rows) in registers.
// The workgroup streams K/V in tiles of BN = 64 keys through a two-stage LDS
// ring filled by direct-to-LDS loads one tile ahead, so one barrier per tile
// suffices. Short problems take the split form (SPLIT, below): 32 rows per
// workgroup, the four waves splitting the key range.
//
// Per tile and 32-row block the wave computes S^T = K Q^T (keys x rows), so a
// lane owns one query row and 32 of the tile's 64 scores in registers: the row
// max/sum are in-lane reductions plus one exchange with lane^32. P^T is then
// already laid out as the B operand of O^T += V^T P^T, and V^T is read from the
// row-major V tile with ds_read_b64_tr_b16.
//
// Semantics follow the reference forward (kotflash/kernels/triton_forward.py
// :20-165): scores scaled before masking (:104,:116), mask (i < Sq, j < Sk,
// causal j <= i) (:118-121), causal tile skip end = min(Sk, Sq, (tile+1) BM)
// (:69-76), P rounded to the input dtype before the PV product (:131,:135),
// O stored in the input dtype (:139-158), LSE = m + ln(l) in fp32 (:160-165).
// exp/log use the hardware base-2 instructions with the scale folded into
// log2(e). One deliberate difference: the denominator l accumulates the
// rounded P that the PV product consumes (fp32 dot2 sums of the packed
// values), where the reference sums P before rounding (:128); the two differ
// by far less than the rounding of O itself.
#include "kf_common.hpp"
#include "kf_host.hpp"

namespace kf {

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, Sq, Sk, D;
  int nqt;
  float scale_log2;
};

// Block -> (q tile, batch, q head). Tiles are issued longest first (causal
// tiles near the end of the sequence see the most keys). When the number of KV
// groups is a multiple of the 8 XCDs, the workgroups of one KV group are kept
// on one XCD (the dispatcher assigns block i to XCD i % 8) so its L2 serves the
// group's K/V to all of them.
__device__ inline void fwd_map_block(int bid, int nqt, int B, int Hq, int Hkv, int& qt, int& b,
                                     int& h) {
  const int G = Hq / Hkv;
  const int ngroups = B * Hkv;
  if ((ngroups & 7) == 0) {
    const int x = bid & 7, j = bid >> 3;
    const int gpx = ngroups >> 3;
    const int per_tile = G * gpx;
    const int t = j / per_tile, r = j - t * per_tile;
    qt = nqt - 1 - t;
    const int grp = x + 8 * (r / G);
    const int g = r % G;
    b = grp / Hkv;
    h = (grp % Hkv) * G + g;
  } else {
    const int bh = B * Hq;
    const int t = bid / bh, r = bid - t * bh;
    qt = nqt - 1 - t;
    b = r / Hq;
    h = r % Hq;
  }
}

// KS is the number of 16-column k-steps of the S = K Q^T contraction: DT / 16,
// or fewer when the head dim ends earlier inside the tile (D <= 80 in a
// 96-wide tile needs 5): the skipped columns are zero padding on both sides.
//
// SPLIT (short problems, where 128-row tiles leave most CUs idle): the
// workgroup owns 32 query rows and its four waves split the key range
// instead, wave w taking K/V tiles w, w + 4, ... through a ring of its own in
// LDS (no workgroup barrier per tile). Each wave ends with its own (m, l, O)
// over its tiles; they are combined through LDS with the LSE weights
// 2^(m_w - M) / sum_w l_w 2^(m_w - M), as split-KV partials are (reference
// triton_forward.py:269-349). The longest chain of dependent tiles is a
// quarter of the unsplit kernel's, and the grid four times as large.
//
// Occupancy: two workgroups per CU, or three for the 96-wide tile (48 KB of
// LDS each, and 168 VGPRs with a 16-byte spill outside the tile loop). Three
// took the config 4 forward (768 equal tiles, one and a half rounds at two
// per CU) 3.5-5% faster at D = 72 and 96 and a causal D = 96 grid of 1024
// tiles 3% faster, bit-identical; the 64- and 32-wide tiles fit three too
// but ran within 0.2% of two, and the 128-wide tile's LDS does not fit.
template <typename T, int DT, int KS, int QB, bool CAUSAL, bool SPLIT>
__global__ __launch_bounds__(256, ((QB == 1 && !SPLIT) ? (DT == 96 ? 3 : 2) : 1)) void fwd_kernel(const FwdParams p) {
  static_assert(!SPLIT || QB == 1, "the split form has one 32-row block per workgroup");
  constexpr int BM = SPLIT ? 32 : 4 * QB * 32;
  constexpr int BN = 64;
  constexpr int CPR = DT / 8;           // 16-byte chunks per row
  constexpr int NKS = KS;               // MFMA k-steps over head_dim
  static_assert(KS * 16 <= DT && KS * 16 > DT - 32, "KS covers the tile's head_dim");
  // Head dims up to 80 in the 96-wide tile (TAIL): O^T columns 0-63 in two
  // 32-wide blocks and 64-79 as a 16-wide tail of v_mfma_f32_16x16x32
  // products, so the PV product runs 80 columns instead of 96 (the S product
  // already stops at 80 through KS). The tiled form only; the split form
  // keeps three 32-wide blocks.
  constexpr bool TAIL = DT == 96 && KS == 5 && !SPLIT;
  constexpr int NDB = TAIL ? 2 : DT / 32;  // 32-wide head_dim blocks of O^T
  constexpr int TB = BN * DT * 2;       // bytes of one K (or V) tile
  constexpr int STAGE_B = 2 * TB;       // K | V
  // Ring stages: two, shared by the workgroup; in the split form one ring per
  // wave, of two stages where four of them fit the LDS (head dims up to 64).
  constexpr int NST = (SPLIT && DT > 64) ? 1 : 2;
  // 1 KB loads per wave per tile and matrix: a quarter of the tile, or all of
  // it in the split form.
  constexpr int NKI = BN * CPR / (SPLIT ? 64 : 256);
  static_assert(BN * CPR == (SPLIT ? 64 : 256) * NKI, "tile chunks must split into whole loads");
  constexpr int RING_B = (SPLIT ? 4 : 1) * NST * STAGE_B;
  // Split form: the merge buffer (per wave O^T rows padded to DT + 1 floats,
  // then m and l per row) overlays the rings after the last tile.
  constexpr int OSTR = DT + 1;
  constexpr int MERGE_B = SPLIT ? (4 * 32 * OSTR + 2 * 4 * 32) * 4 : 0;
  constexpr int SMEM_B = RING_B > MERGE_B ? RING_B : MERGE_B;
  using Tile = SwizzledTile<CPR>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM_B / 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int l32 = lane & 31, h32 = lane >> 5;

  int qt, b, h;
  fwd_map_block(blockIdx.x, p.nqt, p.B, p.Hq, p.Hkv, qt, b, h);
  const int kvh = h / (p.Hq / p.Hkv);
  const int q0 = qt * BM;
  const int wq0 = SPLIT ? q0 : q0 + wave * QB * 32;

  const auto qr = make_rsrc(p.q + b * p.q_sb + h * p.q_sh, rows_extent(p.Sq, p.q_ss, p.D));
  const auto kr = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, rows_extent(p.Sk, p.k_ss, p.D));
  const auto vr = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, rows_extent(p.Sk, p.v_ss, p.D));

  u32x4 qf[QB][NKS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = wq0 + qb * 32 + l32;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = 16 * ks + 8 * h32;
      const uint32_t off = (row < p.Sq && d < p.D) ? (uint32_t)(row * p.q_ss + d) * 2u : kOOB;
      qf[qb][ks] = buf_load16(qr, off);
    }
  }
  // Scores are reduced (row max) before scaling, which needs a positive scale:
  // for a negative one, Q is negated (an exact sign flip of every element) and
  // |scale| used, giving the same scaled scores.
  const float sl2 = fabsf(p.scale_log2);
  if (p.scale_log2 < 0.f) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) qf[qb][ks] ^= 0x80008000u;
  }

  f32x16 oacc[QB][NDB];
  // TAIL: O^T head dims 64-79 for query rows 16 hf .. 16 hf + 15 of the
  // block; lane l, register r holds head dim 64 + 4 (l / 16) + r of row
  // 16 hf + l % 16 (the 16x16x32 result layout).
  f32x4 otail[QB][2];
  float m_i[QB], l_i[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = kNegInf;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = zero16();
    otail[qb][0] = otail[qb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int nkeys = CAUSAL ? min(p.Sk, q0 + BM) : p.Sk;
  const int ntiles = cdiv(nkeys, BN);
  // This wave's tiles: all of them, or every fourth from tile `wave`.
  const int nl = SPLIT ? (ntiles > wave ? (ntiles - wave + 3) / 4 : 0) : ntiles;
  auto tile_of = [&](int li) { return SPLIT ? wave + 4 * li : li; };

  // K/V tiles stream into a two-stage LDS ring by direct-to-LDS loads, stored
  // unpadded with the swizzle of SwizzledTile (conflict-free for both the
  // b128 row reads of K and the transposed reads of V). Per-lane load plan:
  // for each of this wave's NKI 1 KB blocks of a tile, the byte offset of
  // this lane's 16-byte chunk within the tile's rows (kOOB for head-dim
  // padding); the tile's first key enters as soffset, and keys past Sk fall
  // beyond the resource extent and load as zeros.
  uint32_t koff[NKI], voff[NKI];
#pragma unroll
  for (int k = 0; k < NKI; ++k) {
    const int pc = ((SPLIT ? 0 : wave * NKI) + k) * 64 + lane;
    const int r = pc / CPR;
    const int c = (pc % CPR) ^ Tile::key(r);
    const bool ok = c * 8 < p.D;
    koff[k] = ok ? (uint32_t)(r * p.k_ss + c * 8) * 2u : kOOB;
    voff[k] = ok ? (uint32_t)(r * p.v_ss + c * 8) * 2u : kOOB;
  }
  const uint32_t lds0 = lds_addr(smem) + (SPLIT ? (uint32_t)(wave * NST * STAGE_B) : 0u);
  auto tile_load = [&](int tile, int st) {
    const uint32_t kso = (uint32_t)(tile * BN * p.k_ss) * 2u;
    const uint32_t vso = (uint32_t)(tile * BN * p.v_ss) * 2u;
    const uint32_t m0 = lds0 + (uint32_t)st * STAGE_B + (SPLIT ? 0u : (uint32_t)(wave * NKI) * 1024u);
#pragma unroll
    for (int k = 0; k < NKI; ++k) {
      dma16_s(kr, m0 + k * 1024u, koff[k], kso);
      dma16_s(vr, m0 + TB + k * 1024u, voff[k], vso);
    }
  };
  // The one-stage ring of the split form loads a tile's K and V separately,
  // each once the previous tile's reads of it are done.
  auto tile_load_k = [&](int tile) {
    const uint32_t kso = (uint32_t)(tile * BN * p.k_ss) * 2u;
#pragma unroll
    for (int k = 0; k < NKI; ++k) dma16_s(kr, lds0 + k * 1024u, koff[k], kso);
  };
  auto tile_load_v = [&](int tile) {
    const uint32_t vso = (uint32_t)(tile * BN * p.v_ss) * 2u;
#pragma unroll
    for (int k = 0; k < NKI; ++k) dma16_s(vr, lds0 + TB + k * 1024u, voff[k], vso);
  };
  // LDS read bases (bytes, stage 0, key block 0). K rows for S^T: lane row
  // l32, logical chunk 2 ks + h32. V^T transposed reads: the lo / hi rows
  // 4 h + p / 4 (+ 8) of a 16-key step at head-dim block db. Other stages,
  // key blocks and key steps are whole multiples of 16 rows away, which keep
  // the swizzle key, so they are immediate offsets.
  uint32_t rd[NKS], trv[NDB][2], trt = 0;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) rd[ks] = lds0 + (uint32_t)Tile::chunk(l32, 2 * ks + h32) * 16u;
  {
    const int pl = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int r = 4 * h32 + (pl >> 2) + 8 * hi;
        const int col = 32 * db + 16 * g + 4 * (pl & 3);
        trv[db][hi] = lds0 + TB + (uint32_t)Tile::elem(r, col) * 2u;
      }
    // TAIL: the A operand V^T[64 + i][keys] of a 32-key block for lane
    // (i = l % 16, g4 = l / 16). Its k slots t are the keys the B operand
    // (P^T after the lane swaps below) holds there: keys c4 + t (t < 4) and
    // c4 + 16 + t - 4 (t >= 4) of the block, with c4 = 8 (g4 & 1) + 4 (g4 >> 1).
    // Two transposed reads, the second 16 rows on (an immediate offset).
    // Pairing rows c4 and c4 + 8 in one 32-lane pass keeps it conflict-free.
    if constexpr (TAIL) {
      const int g4 = lane >> 4;
      const int r = 8 * (g4 & 1) + 4 * (g4 >> 1) + (pl >> 2);
      trt = lds0 + TB + (uint32_t)Tile::elem(r, 64 + 4 * (pl & 3)) * 2u;
    }
  }

  if (nl > 0) tile_load(tile_of(0), 0);
  wait_all_memory();
  if constexpr (!SPLIT) __syncthreads();

  // This wave's li-th tile on ring stage ST (a compile-time constant, so
  // every LDS offset in the body is an immediate).
  auto tile_body = [&](int li, auto stc) {
    constexpr int ST = decltype(stc)::value;
    if constexpr (NST == 2) {
      if (li + 1 < nl) tile_load(tile_of(li + 1), ST ^ 1);
    }
    const int kbase = tile_of(li) * BN;
    // A causal tile whose first key is beyond every row of the wave is fully
    // masked for it. The split form's tiles all hold visible keys (its
    // ntiles ends at the block's last row), and its one-stage ring relies on
    // every tile body issuing the next tile's loads.
    const bool active = SPLIT || !CAUSAL || kbase <= wq0 + QB * 32 - 1;
    if (active) {
      // S^T = K Q^T as a stream of 2 NKS MFMA slots (key block kb = m / NKS,
      // k-step ks = m % NKS); each slot also issues the LDS read of the
      // operand LA slots ahead, the last ones reading the first V^T operands
      // of the PV product. Fences pin the order: without them the reads are
      // issued one slot ahead and every MFMA waits for its operand.
      constexpr int NS = 2 * NKS;   // S slots
      // PV slots: db = j / 4, key step st = j % 4 for j < 4 NDB; then, with
      // TAIL, four 16x16x32 slots (key block kb = u / 2, row half hf = u % 2
      // for u = j - 4 NDB).
      constexpr int NPV = 4 * NDB + (TAIL ? 4 : 0);
      // Operand read-ahead in slots. For the 128-wide tile (16 S slots) 8 is
      // the measured optimum at config 3 (A/B in one process, fp16 -3.2%,
      // bf16 -3.4% against 4; 5, 6, 10 and 12 are slower and 16 spills);
      // the narrower tiles are fastest at 4 (6 cost 1-7% there).
      constexpr int LA = DT == 128 ? 8 : 4;
      u32x4 kop[NS], vop[NPV];
      auto read_k = [&](int m) {
        const uint32_t off = ST * STAGE_B + (m / NKS) * 32 * CPR * 16;
        kop[m] = *(const KF_LDS u32x4*)(uintptr_t)(rd[m % NKS] + off);
      };
      auto read_v = [&](int j) {
        if (j < 4 * NDB) {
          const uint32_t off = ST * STAGE_B + 16 * (j % 4) * CPR * 16;
          const u32x2 lo = lds_read_tr16_at(trv[j / 4][0] + off);
          const u32x2 hi = lds_read_tr16_at(trv[j / 4][1] + off);
          vop[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else if (((j - 4 * NDB) & 1) == 0) {
          // One tail operand per key block, shared by its two row halves.
          const uint32_t off = ST * STAGE_B + 32 * ((j - 4 * NDB) >> 1) * CPR * 16;
          const u32x2 lo = lds_read_tr16_at(trt + off);
          const u32x2 hi = lds_read_tr16_at(trt + off + 16 * CPR * 16);
          vop[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      };
      f32x16 s[QB][2];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        s[qb][0] = zero16();
        s[qb][1] = zero16();
      }
      static_for<0, LA>([&](auto mc) { read_k(decltype(mc)::value); });
      __builtin_amdgcn_sched_barrier(0);
      // Raised priority while this wave issues MFMAs (S here, PV below), so
      // that the other wave on the SIMD runs its softmax in the gaps instead
      // of competing for them.
      __builtin_amdgcn_s_setprio(1);
      static_for<0, NS>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          s[qb][m / NKS] = Elem<T>::mfma(kop[m], qf[qb][m % NKS], s[qb][m / NKS]);
        if constexpr (m + LA < NS) read_k(m + LA);
        else if constexpr (m + LA - NS < NPV) {
          // One stage: this tile's V was loaded after the previous tile's PV.
          if constexpr (NST == 1 && m + LA == NS) KF_WAIT_VMCNT(0);
          read_v(m + LA - NS);
        }
        __builtin_amdgcn_sched_barrier(0);
      });

      __builtin_amdgcn_s_setprio(0);
      if constexpr (NST == 1) {
        // Every K read of this tile fed an S product: the next K can land
        // while the softmax and the PV product run.
        if (li + 1 < nl) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          tile_load_k(tile_of(li + 1));
        }
      }
      const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && kbase + BN - 1 > wq0);
      u32x4 pk[QB][4];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        if (need_mask) {
          // Key kbase + c is visible iff c < lim (c < Sk - kbase, and c <= row
          // - kbase when causal).
          const int qrow = wq0 + qb * 32 + l32;
          const int lim = CAUSAL ? min(p.Sk - kbase, qrow - kbase + 1) : p.Sk - kbase;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int c = 32 * kb + 8 * (r >> 2) + 4 * h32 + (r & 3);
              s[qb][kb][r] = c < lim ? s[qb][kb][r] : kNegInf;
            }
          }
        }
        float mx = kNegInf;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qb][kb][r]);
        }
        mx = wave_xor32_max(mx) * sl2;
        // Lazy rescale: move the reference max only when a score exceeds it
        // by more than kRescaleThreshold (O and l are still zero while the
        // max is -inf, so the first finite max is adopted without rescaling).
        if (m_i[qb] == kNegInf) {
          m_i[qb] = mx;
        } else {
          const bool grow = mx > m_i[qb] + kRescaleThreshold;
          if (wave_any(grow)) {
            const float alpha = grow ? fast_exp2(m_i[qb] - mx) : 1.f;
            l_i[qb] *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db) oacc[qb][db] *= alpha;
            if constexpr (TAIL) {
              // Tail half hf holds rows 16 hf + l % 16: their alphas.
              const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(alpha),
                                                               __float_as_uint(alpha), false, false);
              otail[qb][0] *= __uint_as_float(sw[0]);
              otail[qb][1] *= __uint_as_float(sw[1]);
            }
            m_i[qb] = grow ? mx : m_i[qb];
          }
        }
        const float msub = (m_i[qb] == kNegInf) ? 0.f : m_i[qb];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) s[qb][kb][r] = fast_exp2(fmaf(s[qb][kb][r], sl2, -msub));
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) pk[qb][st] = pack8<T>(s[qb][st >> 1], 8 * (st & 1));
        // The denominator sums the rounded P that the PV product consumes.
        float rs0 = 0.f, rs1 = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          rs0 = sum2_acc<T>(pk[qb][st][0], rs0);
          rs1 = sum2_acc<T>(pk[qb][st][1], rs1);
          rs0 = sum2_acc<T>(pk[qb][st][2], rs0);
          rs1 = sum2_acc<T>(pk[qb][st][3], rs1);
        }
        l_i[qb] += rs0 + rs1;
      }

      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      static_for<0, NPV>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if constexpr (j < 4 * NDB) {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            oacc[qb][j / 4] = Elem<T>::mfma(vop[j], pk[qb][j % 4], oacc[qb][j / 4]);
        } else {
          constexpr int u = j - 4 * NDB, kb = u >> 1, hf = u & 1;
          if constexpr (hf == 0) {
            // The B operand of a 16x16x32 product for 16 query rows: lane
            // (n = l % 16, g4 = l / 16) holds row 16 hf + n at 8 keys. Block
            // kb's P^T has row l % 32 in lane l, with keys 8 (r / 4) + 4 h32
            // + r % 4 in register r; packing registers {0-3, 8-11} as X and
            // {4-7, 12-15} as Y, v_permlane16_swap(X, Y) (odd 16-lane groups
            // of X <-> even groups of Y) leaves rows 0-15 in X and rows 16-31
            // in Y, with the key slots the tail A operand reads. The PV
            // products of the 32-wide blocks have consumed pk by now.
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
              for (int w = 0; w < 2; ++w)
#pragma unroll
                for (int hs = 0; hs < 2; ++hs) {
                  const auto sw = __builtin_amdgcn_permlane16_swap(
                      pk[qb][2 * kb + hs][w], pk[qb][2 * kb + hs][w + 2], false, false);
                  pk[qb][2 * kb + hs][w] = sw[0];
                  pk[qb][2 * kb + hs][w + 2] = sw[1];
                }
          }
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            const u32x4 bop = hf == 0
                ? u32x4{pk[qb][2 * kb][0], pk[qb][2 * kb][1], pk[qb][2 * kb + 1][0], pk[qb][2 * kb + 1][1]}
                : u32x4{pk[qb][2 * kb][2], pk[qb][2 * kb][3], pk[qb][2 * kb + 1][2], pk[qb][2 * kb + 1][3]};
            otail[qb][hf] = Elem<T>::mfma16(vop[j - hf], bop, otail[qb][hf]);
          }
        }
        if constexpr (j + LA < NPV) read_v(j + LA);
        __builtin_amdgcn_sched_barrier(0);
      });
      __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (NST == 1) {
      // Every V read fed a PV product: the next V lands during the next S
      // product.
      if (li + 1 < nl) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        tile_load_v(tile_of(li + 1));
      }
    }
    // This wave's loads of the next tile (one stage: its K; its V is waited
    // for before the first V read).
    KF_WAIT_VMCNT(NST == 1 ? NKI : 0);
    // Every wave's loads landed; stage ST is free again. The split form's
    // rings are per wave, and the wave's own wait suffices.
    if constexpr (!SPLIT) __syncthreads();
  };
  if constexpr (NST == 2) {
    for (int li = 0; li < nl; li += 2) {
      tile_body(li, std::integral_constant<int, 0>{});
      if (li + 1 < nl) tile_body(li + 1, std::integral_constant<int, 1>{});
    }
  } else {
    for (int li = 0; li < nl; ++li) tile_body(li, std::integral_constant<int, 0>{});
  }

  if constexpr (SPLIT) {
    // Merge the four waves' (m, l, O) of the same 32 rows. The buffer
    // overlays the other waves' rings, hence the barrier first.
    __syncthreads();
    float* ob = reinterpret_cast<float*>(smem);  // [wave][row][OSTR]
    float* mb = ob + 4 * 32 * OSTR;              // [wave][row]
    float* lb = mb + 4 * 32;                     // [wave][row]
    {
      const float lt = wave_xor32_sum(l_i[0]);
      float* orow = ob + (wave * 32 + l32) * OSTR;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) orow[32 * db + 8 * (r >> 2) + 4 * h32 + (r & 3)] = oacc[0][db][r];
      if (h32 == 0) {
        mb[wave * 32 + l32] = m_i[0];
        lb[wave * 32 + l32] = lt;
      }
    }
    __syncthreads();
    // Wave w stores head-dim columns [w DT/4, (w + 1) DT/4) of the 32 rows;
    // a lane takes row l32 and half h32 of those columns.
    constexpr int CW = DT / 4, CH = CW / 2;
    static_assert(CH % 4 == 0, "stores are 4 columns wide");
    const int row = l32;
    float mw[4], M = kNegInf;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = mb[w * 32 + row];
      M = fmaxf(M, mw[w]);
    }
    float sc[4], L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      // A wave with no tile (or only masked keys) for this row has m = -inf
      // and weight 0.
      sc[w] = mw[w] == kNegInf ? 0.f : fast_exp2(mw[w] - M);
      L += lb[w * 32 + row] * sc[w];
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) sc[w] *= inv;
    const int qrow = q0 + row;
    if (qrow < p.Sq) {
      uint16_t* Op = p.o + b * p.o_sb + h * p.o_sh + qrow * p.o_ss;
      const int c0 = wave * CW + h32 * CH;
#pragma unroll
      for (int j = 0; j < CH; j += 4) {
        const int d = c0 + j;
        if (d < p.D) {
          float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float* src = ob + (w * 32 + row) * OSTR + d;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = fmaf(src[e], sc[w], o[e]);
          }
          u32x2 wv;
          wv[0] = pack2<T>(o[0], o[1]);
          wv[1] = pack2<T>(o[2], o[3]);
          *reinterpret_cast<u32x2*>(Op + d) = wv;
        }
      }
      if (wave == 0 && h32 == 0)
        p.lse[((int64_t)b * p.Hq + h) * p.Sq + qrow] = L > 0.f ? (M + fast_log2(L)) * kLn2 : kNegInf;
    }
    return;
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qrow = wq0 + qb * 32 + l32;
    const float lt = wave_xor32_sum(l_i[qb]);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (qrow < p.Sq) {
      uint16_t* Op = p.o + b * p.o_sb + h * p.o_sh + qrow * p.o_ss;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d = 32 * db + 8 * g4 + 4 * h32;
          if (d < p.D) {
            u32x2 w;
            w[0] = pack2<T>(oacc[qb][db][4 * g4 + 0] * inv, oacc[qb][db][4 * g4 + 1] * inv);
            w[1] = pack2<T>(oacc[qb][db][4 * g4 + 2] * inv, oacc[qb][db][4 * g4 + 3] * inv);
            *reinterpret_cast<u32x2*>(Op + d) = w;
          }
        }
      }
      if (h32 == 0) {
        p.lse[((int64_t)b * p.Hq + h) * p.Sq + qrow] =
            lt > 0.f ? (m_i[qb] + fast_log2(lt)) * kLn2 : kNegInf;
      }
    }
    if constexpr (TAIL) {
      // Tail half hf: lane l holds head dims 64 + 4 (l / 16) .. + 3 of row
      // 16 hf + l % 16; the rows' 1 / l come over by the same lane swap.
      const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(inv), __float_as_uint(inv),
                                                       false, false);
      const int d = 64 + 4 * (lane >> 4);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int row = wq0 + qb * 32 + 16 * hf + (lane & 15);
        const float iv = __uint_as_float(sw[hf]);
        if (row < p.Sq && d < p.D) {
          u32x2 w;
          w[0] = pack2<T>(otail[qb][hf][0] * iv, otail[qb][hf][1] * iv);
          w[1] = pack2<T>(otail[qb][hf][2] * iv, otail[qb][hf][3] * iv);
          *reinterpret_cast<u32x2*>(p.o + b * p.o_sb + h * p.o_sh + row * p.o_ss + d) = w;
        }
      }
    }
  }
}

template <typename T, int DT, int KS, int QB>
static int launch_fwd(const FwdParams& prm, bool causal, hipStream_t stream) {
  FwdParams p = prm;
  const bool split = QB == 1 && attn_use_split(p.B, p.Hq, p.Sq, p.Sk, causal);
  const int BM = split ? 32 : 4 * QB * 32;
  p.nqt = cdiv(p.Sq, BM);
  const int64_t grid = (int64_t)p.nqt * p.B * p.Hq;
  if (grid > 0x7fffffff) return set_error(KF_EUNSUPPORTED, "kf_attn_fwd: grid too large");
  const dim3 g((unsigned)grid), blk(256);
  if (split) {
    if (causal)
      hipLaunchKernelGGL((fwd_kernel<T, DT, KS, 1, true, true>), g, blk, 0, stream, p);
    else
      hipLaunchKernelGGL((fwd_kernel<T, DT, KS, 1, false, true>), g, blk, 0, stream, p);
  } else if (causal) {
    hipLaunchKernelGGL((fwd_kernel<T, DT, KS, QB, true, false>), g, blk, 0, stream, p);
  } else {
    hipLaunchKernelGGL((fwd_kernel<T, DT, KS, QB, false, false>), g, blk, 0, stream, p);
  }
  return check_launch("kf_attn_fwd");
}

template <typename T>
static int dispatch_fwd(const FwdParams& p, bool causal, hipStream_t stream) {
  // One 32-row block per wave at two waves per SIMD: while one wave runs its
  // softmax on the VALU the other keeps the MFMA pipe busy.
  switch (head_tile(p.D)) {
    case 32: return launch_fwd<T, 32, 2, 1>(p, causal, stream);
    case 64: return launch_fwd<T, 64, 4, 1>(p, causal, stream);
    case 96:
      // Head dims 72 and 80 end 16 columns before the tile does.
      return p.D <= 80 ? launch_fwd<T, 96, 5, 1>(p, causal, stream)
                       : launch_fwd<T, 96, 6, 1>(p, causal, stream);
    default: return launch_fwd<T, 128, 8, 1>(p, causal, stream);
  }
}

// Shared argument checks of the attention entry points.
int check_attn_common(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                      int64_t D, int dtype) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Sk <= 0 || D <= 0)
    return set_error(KF_EINVAL, "%s: all sizes must be positive", what);
  if (Hq % Hkv != 0)
    return set_error(KF_EINVAL, "%s: num_query_heads must be divisible by num_kv_heads", what);
  if (D % 8 != 0 || D > 128)
    return set_error(KF_EUNSUPPORTED, "%s: head_dim must be a multiple of 8 in [8, 128], got %lld",
                     what, (long long)D);
  if (dtype != KF_F16 && dtype != KF_BF16)
    return set_error(KF_EINVAL, "%s: dtype must be KF_F16 or KF_BF16", what);
  if (Sq > 0x3fffffff || Sk > 0x3fffffff || B * Hq > 0x3fffffff)
    return set_error(KF_EUNSUPPORTED, "%s: sizes exceed the kernels' 32-bit row indexing", what);
  return KF_OK;
}

// The kernels address one (batch, head) slice through a 32-bit buffer
// resource: its byte extent must stay below 2^31.
int check_extent(const char* what, const char* name, int64_t rows, int64_t stride, int64_t D) {
  if (rows > 0 && ((rows - 1) * stride + D) * 2 > 0x7fffffffLL)
    return set_error(KF_EUNSUPPORTED, "%s: one head of %s spans more than 2 GiB", what, name);
  return KF_OK;
}

int check_tensor(const char* what, const char* name, const void* ptr, const int64_t* strides) {
  if (ptr == nullptr) return set_error(KF_EINVAL, "%s: %s is null", what, name);
  if (strides == nullptr) return set_error(KF_EINVAL, "%s: %s strides are null", what, name);
  if (!aligned16(ptr)) return set_error(KF_EINVAL, "%s: %s must be 16-byte aligned", what, name);
  for (int i = 0; i < 3; ++i)
    if (strides[i] < 0 || strides[i] % 8 != 0)
      return set_error(KF_EINVAL, "%s: %s strides must be non-negative multiples of 8 elements",
                       what, name);
  return KF_OK;
}

}  // namespace kf

using namespace kf;

extern "C" int kf_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                           const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* o_strides, float scale,
                           int causal, int dtype, void* stream) {
  const char* what = "kf_attn_fwd";
  int rc = check_attn_common(what, B, Hq, Hkv, Sq, Sk, D, dtype);
  if (rc) return rc;
  if ((rc = check_tensor(what, "q", q, q_strides)) || (rc = check_tensor(what, "k", k, k_strides)) ||
      (rc = check_tensor(what, "v", v, v_strides)) || (rc = check_tensor(what, "o", o, o_strides)))
    return rc;
  if (lse == nullptr) return set_error(KF_EINVAL, "%s: lse is null", what);
  if (!(scale == scale) || scale - scale != 0.f) return set_error(KF_EINVAL, "%s: scale must be finite", what);
  if ((rc = check_extent(what, "q", Sq, q_strides[2], D)) || (rc = check_extent(what, "k", Sk, k_strides[2], D)) ||
      (rc = check_extent(what, "v", Sk, v_strides[2], D)))
    return rc;
  FwdParams p{};
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.o = (uint16_t*)o;
  p.lse = lse;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Sq = (int)Sq; p.Sk = (int)Sk; p.D = (int)D;
  p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  return dtype == KF_F16 ? dispatch_fwd<_Float16>(p, causal != 0, s)
                         : dispatch_fwd<__bf16>(p, causal != 0, s);
}
