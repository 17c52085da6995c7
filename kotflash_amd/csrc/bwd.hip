// Attention backward for gfx950.
//
// Launches on one stream, no atomics, deterministic:
//   1. delta_kernel: delta[i] = sum_d O[i,d] * dO[i,d] from the stored
//      low-precision O (reference triton_backward.py:45), stored negated,
//      and LSE[i] log2(e), for the dK/dV kernel, which loads both rows
//      straight into LDS and starts its dP accumulators at -delta.
//      (When dq_kernel runs it computes both itself, and the separate launch
//      is skipped.)
//   2. dq_kernel (query-stationary, same layout as the forward, two waves per
//      SIMD): per key tile it recomputes S^T = K Q^T and dP^T = V dO^T, forms
//      dS^T = P^T (dP^T - delta) with P = exp(scale S - LSE), and accumulates
//      dQ^T += K^T dS^T; dQ = scale * dQ (reference :17-91). Short problems
//      take a split form: 32 rows per workgroup, the waves splitting the key
//      range, their dQ summed through LDS.
//   3. dkdv_kernel (key-stationary, 4 waves, one per SIMD): a key tile is 128
//      keys of one (batch, kv_head); wave w keeps keys 32 w .. +31 in
//      registers. For every query head of the GQA group and every 64-row query
//      tile the kernel recomputes S = Q K^T and dP = dO V^T and accumulates
//      dV^T += dO^T P and dK^T += Q^T dS in registers, so the group sum over
//      query heads happens in registers (reference :94-195, group loop
//      :136-137, products :183-184). Work is split stream-K style: the
//      (KV group, key tile, head, query tile) units of all tiles are laid end
//      to end and every workgroup takes an equal share of the cost, so causal
//      tiles of very different sizes still keep every CU busy until the end;
//      a group's key tiles are walked long and short alternately, so that
//      shares cut few tiles; the shares of one XCD are consecutive, so its
//      CUs stream the same KV group's Q/dO rows through one L2. A tile shared
//      by several workgroups is written as fp32 partials and
//   4. dkdv_fixup_kernel sums those partials (and zero-fills keys that no query
//      can see); the reference instead splits long query ranges into a fixed
//      number of fp32 partial copies plus a reduction pass (:198-332).
// P and dS are rounded to the input dtype before the products that consume
// them, as in the reference (:85, :183-184).
#include <algorithm>
#include <cstring>

#include "kf_common.hpp"
#include "kf_host.hpp"

namespace kf {

int check_attn_common(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                      int64_t D, int dtype);
int check_tensor(const char* what, const char* name, const void* ptr, const int64_t* strides);
int check_extent(const char* what, const char* name, int64_t rows, int64_t stride, int64_t D);

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  float* delta;  // -rowsum(O * dO), written by delta_kernel
  float* lse2;   // LSE * log2(e), written by delta_kernel
  float* part;  // dK/dV fp32 partials: [2 * nwg][2][128][DT]
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t do_sb, do_sh, do_ss;
  int64_t dq_sb, dq_sh, dq_ss;
  int64_t dk_sb, dk_sh, dk_ss;
  int64_t dv_sb, dv_sh, dv_ss;
  int B, Hq, Hkv, Sq, Sk, D;
  int G, ngroups;
  int nqt, nkt;    // dq: 128-row query tiles; dkdv: 64-row query tiles, 128-key tiles
  int nwg;         // dkdv workgroups (stream-K share count)
  int64_t units;   // dkdv: total (KV group, key tile, head, query tile) units
  float scale, scale_log2;
};

// Key-stationary tiling shared by dkdv_kernel, the fixup and the host.
constexpr int kBNK = 128;  // keys per tile
constexpr int kBMQ = 64;   // query rows per unit

__host__ __device__ inline int dkdv_qstart(int kt, bool causal) {
  // Under the upper-left causal mask, query i sees key j iff j <= i, so no
  // query before the tile's first key (kt * 128) contributes.
  return causal ? kt * (kBNK / kBMQ) : 0;
}
__host__ __device__ inline int dkdv_nq(int kt, int nqt, bool causal) {
  const int n = nqt - dkdv_qstart(kt, causal);
  return n > 0 ? n : 0;
}
// Key tiles that hold any visible (query, key) pair: all of them, or under
// the causal mask those before ceil(nqt / 2) (dkdv_nq is zero from there).
__host__ __device__ inline int dkdv_seen_tiles(int nqt, int nkt, bool causal) {
  // dkdv_nq(kt) = nqt - 2 kt under the causal mask: zero from ceil(nqt / 2).
  const int m = causal ? (nqt + 1) / 2 : nkt;
  return m < nkt ? m : nkt;
}
// Order of the key tiles within a KV group: position pos holds tile
// dkdv_tile_at(pos). The seen tiles alternate from both ends (0, m - 1, 1,
// m - 2, ...), so that under the causal mask a long tile row is followed by
// a short one; tiles that see no query come last. With the causal triangle's
// rows, 256 - 8 kt units at config 3, each pair then costs about two
// workgroups, and the stream-K boundaries cut every pair once, in its long
// tile: at most two shares per tile and two segments per workgroup.
__host__ __device__ inline int dkdv_tile_at(int pos, int m) {
  if (pos >= m) return pos;
  return (pos & 1) ? m - 1 - (pos >> 1) : pos >> 1;
}
__host__ __device__ inline int dkdv_pos_of(int kt, int m) {
  if (kt >= m) return kt;
  return kt < (m + 1) / 2 ? 2 * kt : 2 * (m - 1 - kt) + 1;
}
// Stream-K shares: workgroup w owns units [start[w], start[w + 1]). The host
// places the boundaries by cost rather than by unit count: every key-tile row
// a workgroup enters (a "segment") costs about kSegmentCost units on top of
// its units (loading the keys' K/V rows, filling the LDS ring, flushing the
// accumulators), and the short rows of the causal triangle's far end would
// otherwise pile many segments onto the last workgroups.
constexpr int kMaxDkdvWG = 512;
struct DkdvSplit {
  int start[kMaxDkdvWG + 1];
};
// Units are ordered (KV group, key tile in dkdv_tile_at order, query head,
// query tile), and the
// shares are laid out so that XCD x (the dispatcher sends workgroup i to XCD
// i % 8) runs shares [x nwg / 8, (x + 1) nwg / 8): one XCD's CUs then work on
// the same KV group(s), whose Q/dO rows they all stream, and share its L2.
__device__ inline int dkdv_share_of_block(int block, int nwg) {
  return (nwg & 7) == 0 ? (block & 7) * (nwg >> 3) + (block >> 3) : block;
}

// The share (stream-K range) that owns unit u (start[] is non-decreasing,
// start[0] = 0).
__device__ inline int dkdv_owner(const DkdvSplit& sp, int nwg, int64_t u) {
  int lo = 0, hi = nwg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (sp.start[mid] <= u) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// 1. delta = rowsum(O * dO): 16 lanes per row (one 16-byte chunk of each
// matrix per lane and row), 64 rows per workgroup; every lane issues the loads
// of its four rows before using any, so a workgroup costs one memory round
// trip.
constexpr int kDeltaRows = 64;
template <typename T>
__global__ __launch_bounds__(256) void delta_kernel(const BwdParams p) {
  const int tid = threadIdx.x;
  const int rsub = tid >> 4, c16 = tid & 15;
  const int64_t total = (int64_t)p.B * p.Hq * p.Sq;
  constexpr int RPT = kDeltaRows / 16;  // rows per 16-lane group
  u32x4 a[RPT], g[RPT];
  int64_t rows[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int64_t row = (int64_t)blockIdx.x * kDeltaRows + j * 16 + rsub;
    rows[j] = row;
    const int64_t rr = row < total ? row : 0;
    const int64_t bh = rr / p.Sq;
    const int i = (int)(rr - bh * p.Sq);
    const int b = (int)(bh / p.Hq), h = (int)(bh % p.Hq);
    const auto orr = make_rsrc(p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss, (uint32_t)p.D * 2u);
    const auto drr = make_rsrc(p.dout + b * p.do_sb + h * p.do_sh + i * p.do_ss, (uint32_t)p.D * 2u);
    // D <= 128: 16 lanes cover a row's 16-byte chunks.
    const uint32_t off = row < total && c16 * 8 < p.D ? (uint32_t)c16 * 16u : kOOB;
    a[j] = buf_load16(orr, off);
    g[j] = buf_load16(drr, off);
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      acc += Elem<T>::to_f32((uint16_t)(a[j][w] & 0xffff)) * Elem<T>::to_f32((uint16_t)(g[j][w] & 0xffff));
      acc += Elem<T>::to_f32((uint16_t)(a[j][w] >> 16)) * Elem<T>::to_f32((uint16_t)(g[j][w] >> 16));
    }
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 4);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 1);
    if (c16 == 0 && rows[j] < total) {
      p.delta[rows[j]] = -acc;
      p.lse2[rows[j]] = p.lse[rows[j]] * kLog2e;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. dQ, query-stationary: 4 waves x 32 rows, 64-key tiles, two workgroups
// per CU. Each 32-key block is finished (S, dP, dS, dQ update) before the next
// starts so the live registers fit two waves per SIMD. K/V tiles stream into
// a two-stage LDS ring by direct-to-LDS loads (no register staging), stored
// unpadded with the swizzle of SwizzledTile so that every LDS read of the
// tile body is a per-lane base register plus an immediate offset.
// KS: 16-column k-steps of the contractions over head_dim (S, dP and the row
// deltas): DT / 16, or 5 for head dims up to 80 in a 96-wide tile, whose
// last 16 columns are zero padding.
//
// SPLIT (short problems, the forward's split form): the workgroup owns 32
// query rows and its four waves split the key range, wave w taking tiles w,
// w + 4, ... through a ring of its own (two stages up to head dim 64, one
// above, where the next tile's V loads after the S/dP product and its K after
// the dQ product). The four fp32 dQ are summed through LDS; P already uses
// the global LSE, so no weights are needed. Wave 0 writes the row deltas.
template <typename T, int DT, int KS, bool CAUSAL, bool SPLIT>
__global__ __launch_bounds__(256, SPLIT ? 1 : 2) void dq_kernel(const BwdParams p) {
  constexpr int BM = SPLIT ? 32 : 128;
  constexpr int BN = 64;
  constexpr int CPR = DT / 8;
  constexpr int NKS = KS;
  static_assert(KS * 16 <= DT && KS * 16 > DT - 32, "KS covers the tile's head_dim");
  // Head dims up to 80 in the 96-wide tile (TAIL, tiled form only): dQ^T
  // columns 0-63 in two 32-wide blocks and 64-79 as a 16-wide tail of
  // v_mfma_f32_16x16x32 products, as in the forward, so the dQ product runs
  // 80 columns instead of 96.
  constexpr bool TAIL = DT == 96 && KS == 5 && !SPLIT;
  constexpr int NDB = TAIL ? 2 : DT / 32;
  constexpr int TB = BN * DT * 2;       // bytes of one K (or V) tile
  constexpr int STAGE_B = 2 * TB;       // K | V
  constexpr int NST = (SPLIT && DT > 64) ? 1 : 2;  // ring stages
  // 1 KB loads per wave per tile and matrix: a quarter of the tile, or all of
  // it in the split form.
  constexpr int NKI = BN * CPR / (SPLIT ? 64 : 256);
  static_assert(BN * CPR == (SPLIT ? 64 : 256) * NKI, "tile chunks must split into whole loads");
  constexpr int RING_B = (SPLIT ? 4 : 1) * NST * STAGE_B;
  constexpr int OSTR = DT + 1;  // split form: per-wave dQ^T rows in LDS
  constexpr int MERGE_B = SPLIT ? 4 * 32 * OSTR * 4 : 0;
  constexpr int SMEM_B = RING_B > MERGE_B ? RING_B : MERGE_B;
  using Tile = SwizzledTile<CPR>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM_B / 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int l32 = lane & 31, h32 = lane >> 5;

  // Longest query tiles first; KV groups kept on one XCD as in the forward.
  int qt, b, h;
  {
    const int bid = blockIdx.x;
    if ((p.ngroups & 7) == 0) {
      const int x = bid & 7, j = bid >> 3, gpx = p.ngroups >> 3, per_tile = p.G * gpx;
      const int t = j / per_tile, r = j - t * per_tile;
      qt = p.nqt - 1 - t;
      const int grp = x + 8 * (r / p.G);
      b = grp / p.Hkv;
      h = (grp % p.Hkv) * p.G + r % p.G;
    } else {
      const int bh = p.B * p.Hq, t = bid / bh, r = bid - t * bh;
      qt = p.nqt - 1 - t;
      b = r / p.Hq;
      h = r % p.Hq;
    }
  }
  const int kvh = h / p.G;
  const int q0 = qt * BM;
  const int qrow = q0 + (SPLIT ? 0 : wave * 32) + l32;
  const bool row_ok = qrow < p.Sq;

  const auto qr = make_rsrc(p.q + b * p.q_sb + h * p.q_sh, rows_extent(p.Sq, p.q_ss, p.D));
  const auto dor = make_rsrc(p.dout + b * p.do_sb + h * p.do_sh, rows_extent(p.Sq, p.do_ss, p.D));
  const auto kr = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, rows_extent(p.Sk, p.k_ss, p.D));
  const auto vr = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, rows_extent(p.Sk, p.v_ss, p.D));

  u32x4 qf[NKS], dof[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = 16 * ks + 8 * h32;
    const bool ok = row_ok && d < p.D;
    qf[ks] = buf_load16(qr, ok ? (uint32_t)(qrow * p.q_ss + d) * 2u : kOOB);
    dof[ks] = buf_load16(dor, ok ? (uint32_t)(qrow * p.do_ss + d) * 2u : kOOB);
  }
  const int64_t rowlin = ((int64_t)b * p.Hq + h) * p.Sq + qrow;
  const float lse2 = row_ok ? p.lse[rowlin] * kLog2e : 0.f;
  // Row delta = rowsum(O * dO) from the stored O (reference
  // triton_backward.py:45): this lane holds 8 head_dim slots per k-step of
  // its row for dO; the same slots of O give the lane's share, and the other
  // half of the row is in lane ^ 32. The dK/dV kernel reads -delta and
  // LSE * log2(e) from the workspace, written here by one lane per row.
  float dlt = 0.f;
  {
    const auto orr = make_rsrc(p.o + b * p.o_sb + h * p.o_sh, rows_extent(p.Sq, p.o_ss, p.D));
    u32x4 of[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = 16 * ks + 8 * h32;
      of[ks] = buf_load16(orr, row_ok && d < p.D ? (uint32_t)(qrow * p.o_ss + d) * 2u : kOOB);
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        dlt += Elem<T>::to_f32((uint16_t)(of[ks][w] & 0xffff)) * Elem<T>::to_f32((uint16_t)(dof[ks][w] & 0xffff));
        dlt += Elem<T>::to_f32((uint16_t)(of[ks][w] >> 16)) * Elem<T>::to_f32((uint16_t)(dof[ks][w] >> 16));
      }
    dlt = wave_xor32_sum(dlt);
    if (row_ok && h32 == 0 && (!SPLIT || wave == 0)) {
      p.delta[rowlin] = -dlt;
      p.lse2[rowlin] = lse2;
    }
  }

  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = zero16();
  // TAIL: dQ^T head dims 64-79 of rows 16 hf + l % 16 (lane l, register r:
  // head dim 64 + 4 (l / 16) + r).
  f32x4 dqt[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};

  const int nkeys = CAUSAL ? min(p.Sk, q0 + BM) : p.Sk;
  const int ntiles = cdiv(nkeys, BN);
  // This wave's tiles: all of them, or every fourth from tile `wave`.
  const int nl = SPLIT ? (ntiles > wave ? (ntiles - wave + 3) / 4 : 0) : ntiles;
  auto tile_of = [&](int li) { return SPLIT ? wave + 4 * li : li; };

  // Per-lane load plan: for each of this wave's NKI 1 KB blocks of a tile,
  // the byte offset of this lane's 16-byte chunk within the tile's rows
  // (kOOB for head-dim padding). The tile's first key enters as soffset;
  // keys past Sk fall beyond the resource extent and load as zeros.
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
  // The split form's one-stage ring loads a tile's K and V separately, each
  // once the previous tile's reads of it are done.
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
  // LDS read bases (bytes, stage 0, K tile, key block 0). S^T / dP^T rows:
  // lane row l32, logical chunk 2 ks + h32. dQ^T transposed reads: the
  // lo / hi rows 4 h + p / 4 (+ 8) of each 16-key half at head-dim block db.
  // Other stages, the V tile, key blocks and key halves are whole multiples
  // of 16 rows away, which keep the swizzle key, so they are immediates.
  uint32_t rd[NKS], tr[NDB][2], trt = 0;
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
        tr[db][hi] = lds0 + (uint32_t)Tile::elem(r, col) * 2u;
      }
    // TAIL: the A operand K^T[64 + i][keys] of a 32-key block for lane
    // (i = l % 16, g4 = l / 16), keys c4 + t and c4 + 16 + t - 4 with
    // c4 = 8 (g4 & 1) + 4 (g4 >> 1): the forward's tail operand, on K.
    if constexpr (TAIL) {
      const int g4 = lane >> 4;
      const int r = 8 * (g4 & 1) + 4 * (g4 >> 1) + (pl >> 2);
      trt = lds0 + (uint32_t)Tile::elem(r, 64 + 4 * (pl & 3)) * 2u;
    }
  }

  if (nl > 0) tile_load(tile_of(0), 0);
  wait_all_memory();
  if constexpr (!SPLIT) __syncthreads();

  const int wq0 = q0 + (SPLIT ? 0 : wave * 32);
  // This wave's li-th tile on ring stage ST (a compile-time constant, so
  // every LDS offset below is an immediate).
  auto tile_body = [&](int li, auto stc) {
    constexpr int ST = decltype(stc)::value;
    if constexpr (NST == 2) {
      if (li + 1 < nl) tile_load(tile_of(li + 1), ST ^ 1);
    }
    const int kbase = tile_of(li) * BN;
    const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && kbase + BN - 1 > wq0);
    bool v_next = false;  // one-stage ring: the next tile's V already issued
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kb0 = kbase + 32 * kb;
      if (CAUSAL && kb0 > wq0 + 31) continue;  // block entirely above the wave's rows
      // S^T and dP^T as one stream of 2 NKS MFMA slots (slot m: k-step m / 2,
      // S for even m, dP for odd), then dQ^T as NDQ slots (head-dim block
      // j / 2, key half j % 2). Each slot issues the LDS read of the operand
      // LA slots ahead (the last S/dP slots read the first dQ operands);
      // fences keep that order, otherwise the reads trail by one slot and
      // every MFMA waits for its operand.
      constexpr int NSD = 2 * NKS;
      // dQ slots: 2 NDB 32x32x16 products, then with TAIL two 16x16x32
      // products (row halves) over the whole 32-key block.
      constexpr int NDQ = 2 * NDB + (TAIL ? 2 : 0);
      // Operand read-ahead in slots: 5 for the 128-wide tile, the measured
      // optimum at config 3 (A/B in one process, fp16 -3.9%, bf16 -4.1%
      // against 4; 3 is level, 6 slower by 5%, 8 by 17%). At 5 the register
      // allocator spills 12 bytes to scratch (vector scratch_store/load): the
      // one reload inside the tile loop restores a DMA offset right after the
      // tile-end vmcnt(0) and barrier, so it drains nothing that was not
      // drained already. Narrower tiles stay at 4.
      constexpr int LA = DT == 128 ? 5 : 4;
      u32x4 op[NSD + NDQ];
      auto read_op = [&](int m) {
        if (m < NSD) {
          const uint32_t off = ST * STAGE_B + ((m & 1) ? TB : 0) + kb * 32 * CPR * 16;
          op[m] = *(const KF_LDS u32x4*)(uintptr_t)(rd[m >> 1] + off);
        } else if (m - NSD < 2 * NDB) {
          const int j = m - NSD;
          const uint32_t off = ST * STAGE_B + (32 * kb + 16 * (j & 1)) * CPR * 16;
          const u32x2 lo = lds_read_tr16_at(tr[j >> 1][0] + off);
          const u32x2 hi = lds_read_tr16_at(tr[j >> 1][1] + off);
          op[m] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else if (m - NSD == 2 * NDB) {
          const uint32_t off = ST * STAGE_B + 32 * kb * CPR * 16;
          const u32x2 lo = lds_read_tr16_at(trt + off);
          const u32x2 hi = lds_read_tr16_at(trt + off + 16 * CPR * 16);
          op[m] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      };
      // dP^T starts at -delta of the lane's row, so dS = P (dP - delta) is
      // one multiply per element.
      f32x16 s = zero16(), dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = -dlt;
      static_for<0, LA>([&](auto mc) { read_op(decltype(mc)::value); });
      __builtin_amdgcn_sched_barrier(0);
      // Raised priority while this wave issues MFMAs, so that the other wave
      // on the SIMD runs its softmax in the gaps instead of competing for them.
      __builtin_amdgcn_s_setprio(1);
      static_for<0, NSD>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        if constexpr (m & 1)
          dp = Elem<T>::mfma(op[m], dof[m >> 1], dp);
        else
          s = Elem<T>::mfma(op[m], qf[m >> 1], s);
        if constexpr (m + LA < NSD + NDQ) read_op(m + LA);
        __builtin_amdgcn_sched_barrier(0);
      });
      __builtin_amdgcn_s_setprio(0);
      if constexpr (NST == 1) {
        // Every V read of this tile fed a dP product (the last key block's):
        // the next V can land during the dQ product and the next S.
        if (kb == 1 && li + 1 < nl) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          tile_load_v(tile_of(li + 1));
          v_next = true;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = fmaf(s[r], p.scale_log2, -lse2);
      if (need_mask) {
        // Key kb0 + c is visible iff c < lim.
        const int lim = CAUSAL ? min(p.Sk - kb0, qrow - kb0 + 1) : p.Sk - kb0;
        if constexpr (CAUSAL || DT != 128) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int c = 8 * (r >> 2) + 4 * h32 + (r & 3);
            s[r] = c < lim ? s[r] : kNegInf;
          }
        } else {
          // Written as (c - 4 h32) < (lim - 4 h32), every comparison is a
          // compile-time constant against one per-lane value; comparing the
          // per-register key offsets themselves, the compiler keeps all 16
          // in registers across the tile loop, and the non-causal 128-wide
          // kernel then spilled inside it (this form: dQ -15% at B=4 H=12
          // S=2048 D=128; the causal kernels ran 0.7% and the non-causal
          // 96-wide ones 0.4-1% slower with it, so they keep the direct form).
          const int lh = lim - 4 * h32;
#pragma unroll
          for (int r = 0; r < 16; ++r) s[r] = 8 * (r >> 2) + (r & 3) < lh ? s[r] : kNegInf;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = fast_exp2(s[r]) * dp[r];
      u32x4 ds0 = pack8<T>(dp, 0), ds1 = pack8<T>(dp, 8);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      static_for<0, NDQ>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if constexpr (j < 2 * NDB) {
          dq[j >> 1] = Elem<T>::mfma(op[NSD + j], (j & 1) ? ds1 : ds0, dq[j >> 1]);
        } else {
          constexpr int hf = j - 2 * NDB;
          if constexpr (hf == 0) {
            // dS^T in the 16x16x32 B layout, by the forward's lane swap:
            // rows 0-15 in {ds0[0], ds0[1], ds1[0], ds1[1]}, rows 16-31 in
            // the other halves (the 32-wide dQ products have consumed them).
#pragma unroll
            for (int w = 0; w < 2; ++w) {
              const auto a = __builtin_amdgcn_permlane16_swap(ds0[w], ds0[w + 2], false, false);
              const auto c = __builtin_amdgcn_permlane16_swap(ds1[w], ds1[w + 2], false, false);
              ds0[w] = a[0]; ds0[w + 2] = a[1];
              ds1[w] = c[0]; ds1[w + 2] = c[1];
            }
          }
          const u32x4 bop = hf == 0 ? u32x4{ds0[0], ds0[1], ds1[0], ds1[1]}
                                    : u32x4{ds0[2], ds0[3], ds1[2], ds1[3]};
          dqt[hf] = Elem<T>::mfma16(op[NSD + 2 * NDB], bop, dqt[hf]);
        }
        if constexpr (NSD + j + LA < NSD + NDQ) read_op(NSD + j + LA);
        __builtin_amdgcn_sched_barrier(0);
      });
      __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (NST == 1) {
      // Every K read of this tile fed an S or dQ product (and every V read a
      // dP product, if the second key block was skipped).
      if (li + 1 < nl) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (!v_next) tile_load_v(tile_of(li + 1));
        tile_load_k(tile_of(li + 1));
      }
    }
    KF_WAIT_VMCNT(0);  // this wave's loads of the next tile
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
    // Sum the four waves' dQ^T of the same 32 rows. The buffer overlays the
    // other waves' rings, hence the barrier first.
    __syncthreads();
    float* ob = reinterpret_cast<float*>(smem);  // [wave][row][OSTR]
    {
      float* orow = ob + (wave * 32 + l32) * OSTR;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) orow[32 * db + 8 * (r >> 2) + 4 * h32 + (r & 3)] = dq[db][r];
    }
    __syncthreads();
    // Wave w stores head-dim columns [w DT/4, (w + 1) DT/4) of the 32 rows;
    // a lane takes row l32 and half h32 of those columns.
    constexpr int CW = DT / 4, CH = CW / 2;
    static_assert(CH % 4 == 0, "stores are 4 columns wide");
    if (row_ok) {
      uint16_t* Dq = p.dq + b * p.dq_sb + h * p.dq_sh + qrow * p.dq_ss;
      const int c0 = wave * CW + h32 * CH;
#pragma unroll
      for (int j = 0; j < CH; j += 4) {
        const int d = c0 + j;
        if (d < p.D) {
          float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float* src = ob + (w * 32 + l32) * OSTR + d;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] += src[e];
          }
          u32x2 wv;
          wv[0] = pack2<T>(o[0] * p.scale, o[1] * p.scale);
          wv[1] = pack2<T>(o[2] * p.scale, o[3] * p.scale);
          *reinterpret_cast<u32x2*>(Dq + d) = wv;
        }
      }
    }
    return;
  }

  if (row_ok) {
    uint16_t* Dq = p.dq + b * p.dq_sb + h * p.dq_sh + qrow * p.dq_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * db + 8 * g4 + 4 * h32;
        if (d < p.D) {
          u32x2 w;
          w[0] = pack2<T>(dq[db][4 * g4 + 0] * p.scale, dq[db][4 * g4 + 1] * p.scale);
          w[1] = pack2<T>(dq[db][4 * g4 + 2] * p.scale, dq[db][4 * g4 + 3] * p.scale);
          *reinterpret_cast<u32x2*>(Dq + d) = w;
        }
      }
    }
  }
  if constexpr (TAIL) {
    // Tail half hf: lane l holds head dims 64 + 4 (l / 16) .. + 3 of row
    // wq0 + 16 hf + l % 16.
    const int d = 64 + 4 * (lane >> 4);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = wq0 + 16 * hf + (lane & 15);
      if (row < p.Sq && d < p.D) {
        u32x2 w;
        w[0] = pack2<T>(dqt[hf][0] * p.scale, dqt[hf][1] * p.scale);
        w[1] = pack2<T>(dqt[hf][2] * p.scale, dqt[hf][3] * p.scale);
        *reinterpret_cast<u32x2*>(p.dq + b * p.dq_sb + h * p.dq_sh + row * p.dq_ss + d) = w;
      }
    }
  }
}

// Softmax plan of a dK/dV unit. Its 32 softmax elements, k = 16 qb + r for
// block qb and S/dP register r, each take three stages (exponent argument,
// exp2, dS and packing) in three consecutive MFMA slots; stage a of element
// k runs in slot a(k). The elements are spread evenly from the first slot
// after block 0's S/dP MFMAs (slot NSD) to the last slot from which block
// 1's high half still reaches its first dV/dK MFMA. A block's low (high)
// half is packed at the third stage of its element 7 (15) and consumed from
// slot 2 NSD + qb NVK (+ 2 NDB) on; block 1 cannot start before its S/dP
// MFMAs end (slot 2 NSD). Where the even spread breaks one of these, each
// block takes one phase: block 0 the S/dP slots of block 1, block 1 the
// dV/dK slots of block 0.
template <int NSD, int NVK, int NDB>
struct DkdvSoftPlan {
  static constexpr int kFirst = NSD;
  static constexpr int kLast = 2 * NSD + NVK + 2 * NDB - 3;
  static constexpr int even(int k) { return kFirst + k * (kLast - kFirst) / 31; }
  static constexpr int phased(int k) {
    return k < 16 ? NSD + k / ((16 + NSD - 1) / NSD) : 2 * NSD + (k - 16) / ((16 + NVK - 1) / NVK);
  }
  static constexpr bool even_ok() {
    for (int qb = 0; qb < 2; ++qb) {
      const int lo = 2 * NSD + qb * NVK, hi = lo + 2 * NDB;
      if (even(16 * qb + 7) + 2 >= lo || even(16 * qb + 15) + 2 >= hi) return false;
    }
    return even(16) >= 2 * NSD;
  }
  static constexpr int a(int k) { return even_ok() ? even(k) : phased(k); }
  // First element whose stage a runs at slot m or later (a is
  // non-decreasing): the elements starting in slot m are [at(m), at(m + 1)).
  static constexpr int at(int m) {
    int k = 0;
    while (k < 32 && a(k) < m) ++k;
    return k;
  }
};

// ---------------------------------------------------------------------------
// 3. dK/dV, key-stationary, stream-K over (KV group, key tile, head, query
// tile) units.
// Four waves, one per SIMD (the 512-register budget lets the dK/dV
// accumulators live in accumulation registers). Wave w owns keys
// 32 w .. 32 w + 31 of the 128-key tile and keeps their K and V rows in
// registers as MFMA B operands for the whole tile; per unit it covers all 64
// query rows. The unit's Q and dO tiles and its LSE / delta rows are loaded
// straight into LDS (no register staging) in a ring of NST stages, issued two
// units ahead. Per unit and 32-row query block:
//   S  = Q K^T,  dP = dO V^T            (A = Q / dO rows from LDS, B = K / V)
//   P  = exp2(scale log2e S - LSE log2e),  dS = P (dP - delta)
//   dV^T += dO^T P,  dK^T += Q^T dS      (A = transposed LDS reads, B = P / dS
//                                         straight from the S / dP registers)
// dV^T / dK^T accumulation, acc += a b on v_mfma_f32_32x32x16, written as
// inline assembly with the accumulator in accumulation registers ("+a") and
// the operands in VGPRs. This file is compiled with the VGPR form of the MFMA
// builtins (-amdgpu-mfma-vgpr-form, set in build.py), so the S and dP
// products land in VGPRs, where the softmax reads them, instead of in
// accumulation registers that cost 64 v_accvgpr_read per dK/dV unit; only
// these products keep the accumulation-register form, which the 128 dK/dV
// accumulator registers of the 128-wide tile need. The compiler's hazard tracking does not see
// inside inline assembly, so its wait states are written out: s_nop 1 gives
// the 2 wait states an MFMA needs after a VALU write of a VGPR it reads (the
// packed P / dS operands, and the zeroed accumulators at a segment's start,
// which are hundreds of cycles older still), and the segment flush waits 24
// wait states before VALU reads the accumulators. Back-to-back products into
// the same accumulator need none.
template <typename T>
__device__ inline void dkdv_mfma_acc(f32x16& acc, u32x4 a, u32x4 b) {
  if constexpr (std::is_same_v<T, _Float16>)
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

template <typename T, int DT, int KS, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void dkdv_kernel(const BwdParams p, const DkdvSplit sp) {
  constexpr int CPR = DT / 8;
  constexpr int QT = kBMQ * DT;        // elements of one Q (or dO) tile
  constexpr int NQI = CPR / 4;         // 1 KB DMA instructions per wave per tile
  constexpr int NST = 3;               // LDS ring stages
  constexpr int NKS = KS;              // k-steps of S and dP (as in dq_kernel)
  static_assert(KS * 16 <= DT && KS * 16 > DT - 32, "KS covers the tile's head_dim");
  constexpr int NDB = DT / 32;
  using Tile = SwizzledTile<CPR>;
  static_assert(kBMQ * CPR == 4 * 64 * NQI, "tile chunks must split into whole DMA instructions");
  __shared__ __attribute__((aligned(16))) uint16_t stage[NST][2][QT];   // [stage][Q | dO]
  // [stage][lse2, delta, (unused x2)][row]: waves 2 and 3 also issue a
  // (zero-filling) statistics load into the unused rows, so that every wave
  // runs the same instruction stream and vmcnt count.
  __shared__ __attribute__((aligned(16))) float rowstat[NST][4][kBMQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int l32 = lane & 31, h32 = lane >> 5;

  const int share = dkdv_share_of_block(blockIdx.x, p.nwg);
  int64_t u = sp.start[share];
  const int64_t uend = sp.start[share + 1];
  if (u >= uend) return;

  f32x16 dk[NDB], dv[NDB];

  // LDS read bases (bytes): stage 0 and, because a ds_read immediate is only
  // 16 bits, stage 2. Row reads of the Q / dO A operands: lane row l32,
  // logical chunk 2 ks + h32. Transposed reads: the lo / hi rows
  // 4 h + p / 4 (+ 8) of a 16-row block at head-dim block db. The other
  // stage, the dO tile and other row blocks are whole multiples of 16 rows
  // away, which keep the swizzle key, so they are immediate offsets.
  constexpr uint32_t kStageBytes = 2u * QT * 2u;
  uint32_t rdq[NKS], rdq2[NKS], trb[NDB][2], trb2[NDB][2];
  {
    const uint32_t s0 = lds_addr(&stage[0][0][0]);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      rdq[ks] = s0 + (uint32_t)Tile::chunk(l32, 2 * ks + h32) * 16u;
      rdq2[ks] = rdq[ks] + 2u * kStageBytes;
    }
    const int pl = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int r = 4 * h32 + (pl >> 2) + 8 * hi;
        const int col = 32 * db + 16 * g + 4 * (pl & 3);
        trb[db][hi] = s0 + (uint32_t)Tile::elem(r, col) * 2u;
        trb2[db][hi] = trb[db][hi] + 2u * kStageBytes;
      }
    // The stage-2 bases are opaque to the optimizer: seeing them as base +
    // 65536 it drops them and recomputes every stage-2 read address with a
    // v_add_u32 (the offset exceeds the 16-bit ds_read immediate), 64 extra
    // VALU instructions in every third unit.
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) asm volatile("" : "+v"(rdq2[ks]));
#pragma unroll
    for (int db = 0; db < NDB; ++db) asm volatile("" : "+v"(trb2[db][0]), "+v"(trb2[db][1]));
  }

  // Per-lane DMA plan, the same for every unit: for each of this wave's NQI
  // 1 KB blocks of a tile, the byte offset of this lane's 16-byte chunk
  // within the tile's rows (kOOB when the chunk is head-dim padding). A unit
  // adds its first row's offset as the (scalar) soffset; rows past Sq then
  // fall beyond the resource extent and load as zeros.
  uint32_t dma_qoff[NQI], dma_doff[NQI];
#pragma unroll
  for (int k = 0; k < NQI; ++k) {
    const int pc = (wave * NQI + k) * 64 + lane;  // physical chunk this lane fills
    const int r = pc / CPR;
    const int c = (pc % CPR) ^ Tile::key(r);
    const bool ok = c * 8 < p.D;
    dma_qoff[k] = ok ? (uint32_t)(r * p.q_ss + c * 8) * 2u : kOOB;
    dma_doff[k] = ok ? (uint32_t)(r * p.do_ss + c * 8) * 2u : kOOB;
  }
  // Statistics rows: wave 0 loads LSE * log2(e), wave 1 -delta; waves 2 and
  // 3 load zeros into the unused rows.
  const uint32_t dma_soff = wave < 2 ? (uint32_t)lane * 4u : kOOB;
  // LDS byte addresses (M0) of stage 0's blocks for this wave.
  const uint32_t lds_q0 = lds_addr(&stage[0][0][0]) + (uint32_t)(wave * NQI) * 1024u;
  const uint32_t lds_s0 = lds_addr(&rowstat[0][0][0]) + (uint32_t)wave * (kBMQ * 4u);
  constexpr uint32_t kStatBytes = 4u * kBMQ * 4u;
  const uint32_t q_ext = rows_extent(p.Sq, p.q_ss, p.D);
  const uint32_t do_ext = rows_extent(p.Sq, p.do_ss, p.D);
  // Units of a segment are walked in order (query head g, query tile qt
  // descending): workgroups that start a tile row together read the same
  // Q/dO tiles at the same time. `Walk` advances one unit without divisions,
  // and carries the row pointers of head kvh G + g, stepped when g changes,
  // so that a unit's DMA set-up needs no 64-bit products.
  struct Walk {
    int g, qt;
    int qs, nq;          // the segment's first query tile and query-tile count
    const uint16_t* qp;  // Q rows of the head
    const uint16_t* dp;  // dO rows
    const float* sp;     // statistics rows: LSE log2(e) (wave 0), -delta (wave 1)
  };
  auto walk_init = [&](int b, int kvh, int qs, int nq, int it) {
    Walk w;
    const int h0 = kvh * p.G;
    w.g = it / nq;
    w.qt = qs + nq - 1 - (it - w.g * nq);
    w.qs = qs;
    w.nq = nq;
    w.qp = p.q + b * p.q_sb + (int64_t)(h0 + w.g) * p.q_sh;
    w.dp = p.dout + b * p.do_sb + (int64_t)(h0 + w.g) * p.do_sh;
    w.sp = (wave == 0 ? p.lse2 : p.delta) + ((int64_t)b * p.Hq + h0 + w.g) * p.Sq;
    return w;
  };
  auto walk_next = [&](Walk& w) {
    if (--w.qt < w.qs) {
      w.qt = w.qs + w.nq - 1;
      ++w.g;
      w.qp += p.q_sh;
      w.dp += p.do_sh;
      w.sp += p.Sq;
    }
  };
  constexpr int NDMA = 2 * NQI + 1;  // DMA instructions per unit (the last: LSE or delta rows)
  struct Dma {
    __amdgpu_buffer_rsrc_t qr, dor, sr;
    uint32_t qso, dso, sso;  // soffsets: the unit's first row
    uint32_t lq, ls;         // M0 of this wave's first Q block and of its statistics row
  };
  // A unit past the segment's end gets empty resources (no load reaches
  // memory, whatever the base): its loads then only deposit zeros into the
  // (free) stage, which keeps the issue unconditional.
  auto dma_setup = [&](const Walk& w, int st, bool real) {
    Dma d;
    const int q0 = real ? w.qt * kBMQ : 0;
    d.qr = make_rsrc(w.qp, real ? q_ext : 0u);
    d.dor = make_rsrc(w.dp, real ? do_ext : 0u);
    d.sr = make_rsrc(w.sp, real ? (uint32_t)p.Sq * 4u : 0u);
    d.qso = (uint32_t)(q0 * p.q_ss) * 2u;
    d.dso = (uint32_t)(q0 * p.do_ss) * 2u;
    d.sso = (uint32_t)q0 * 4u;
    d.lq = lds_q0 + (uint32_t)st * kStageBytes;
    d.ls = lds_s0 + (uint32_t)st * kStatBytes;
    return d;
  };
  // DMA instruction j of a unit: Q / dO blocks, then the row statistics.
  auto dma_issue = [&](const Dma& d, int j) {
    if (j < 2 * NQI) {
      const int k = j >> 1;
      if ((j & 1) == 0)
        dma16_s(d.qr, d.lq + (uint32_t)k * 1024u, dma_qoff[k], d.qso);
      else
        dma16_s(d.dor, d.lq + (uint32_t)(QT * 2) + (uint32_t)k * 1024u, dma_doff[k], d.dso);
    } else {
      dma4_s(d.sr, d.ls, dma_soff, d.sso);
    }
  };

  // Segments: the tile row (grp, kt) holding unit u, of which this share
  // covers units [ua, ub) (row-relative). Rows are walked by their position
  // in the group's tile order.
  const int64_t group_units = p.units / p.ngroups;
  const int mseen = dkdv_seen_tiles(p.nqt, p.nkt, CAUSAL);
  int grp = (int)(u / group_units);
  int pos = 0;
  int kt = dkdv_tile_at(0, mseen);
  int64_t row_base = grp * group_units;  // first unit of tile row (grp, kt)
  auto seek = [&]() {
    for (;;) {
      const int64_t row_units = (int64_t)p.G * dkdv_nq(kt, p.nqt, CAUSAL);
      if (u < row_base + row_units) break;
      row_base += row_units;
      if (++pos == p.nkt) {
        pos = 0;
        ++grp;
      }
      kt = dkdv_tile_at(pos, mseen);
    }
  };
  // A segment's set-up loads: this wave's K and V rows as B operands (lane =
  // key, slots = head_dim) and the ring's first two units. Both go out
  // together, and for every segment after the first they go out before the
  // previous segment's flush, so that their latency overlaps its stores.
  u32x4 kf[NKS], vf[NKS];
  Walk wcur, wdma;
  auto segment_loads = [&]() {
    const int nq = dkdv_nq(kt, p.nqt, CAUSAL);
    const int qs = dkdv_qstart(kt, CAUSAL);
    const int per_tile = p.G * nq;
    const int ua = (int)(u - row_base);
    const int ub = (int)min((int64_t)per_tile, ua + (uend - u));
    const int b = grp / p.Hkv, kvh = grp % p.Hkv;
    const int key = kt * kBNK + wave * 32 + l32;
    const bool key_ok = key < p.Sk;
    const auto kr = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, rows_extent(p.Sk, p.k_ss, p.D));
    const auto vr = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, rows_extent(p.Sk, p.v_ss, p.D));
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d = 16 * ks + 8 * h32;
      const bool ok = key_ok && d < p.D;
      kf[ks] = buf_load16(kr, ok ? (uint32_t)(key * p.k_ss + d) * 2u : kOOB);
      vf[ks] = buf_load16(vr, ok ? (uint32_t)(key * p.v_ss + d) * 2u : kOOB);
    }
    // The K/V operands live in accumulation registers for the segment (the
    // S / dP products read their B operand from there): that leaves the
    // VGPRs to the S and dP accumulators.
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) asm volatile("" : "+a"(kf[ks]), "+a"(vf[ks]));
    wcur = walk_init(b, kvh, qs, nq, ua);
    wdma = wcur;
    const Dma d0 = dma_setup(wdma, 0, true);
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dma_issue(d0, j);
    walk_next(wdma);
    const Dma d1 = dma_setup(wdma, 1, ua + 1 < ub);
#pragma unroll
    for (int j = 0; j < NDMA; ++j) dma_issue(d1, j);
    walk_next(wdma);
  };
  seek();
  segment_loads();
  bool first_seg = true;
  for (;;) {
    const int nq = dkdv_nq(kt, p.nqt, CAUSAL);
    const int qs = dkdv_qstart(kt, CAUSAL);
    const int per_tile = p.G * nq;
    const int ua = (int)(u - row_base);
    const int ub = (int)min((int64_t)per_tile, ua + (uend - u));
    const int b = grp / p.Hkv, kvh = grp % p.Hkv;
    const int k0 = kt * kBNK;
    const int kw0 = k0 + wave * 32;  // first key of this wave
    const int key = kw0 + l32;
    const bool key_ok = key < p.Sk;
    (void)nq;
    (void)qs;

    // This segment's K/V rows and first two units have landed, and every
    // wave is done with the previous segment's stages and flush.
    wait_all_memory();
    __syncthreads();
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      dk[db] = zero16();
      dv[db] = zero16();
    }

    // One unit: both 32-row query blocks (qb) of the staged tile against this
    // wave's 32 keys, with the causal mask (key <= row) on blocks that cross
    // the diagonal for this wave's keys.
    //
    // With one wave per SIMD nothing else hides latency, so the unit is
    // software-pipelined by hand as one stream of MFMA slots, the order pinned
    // with scheduling fences:
    //   slots [0, NSD)          S/dP MFMAs of qb 0      + the DMA of unit + 2
    //   slots [NSD, 2 NSD)      S/dP MFMAs of qb 1
    //   slots [2 NSD, +NVK)     dV/dK MFMAs of qb 0
    //   slots [.., +NVK)        dV/dK MFMAs of qb 1
    // (NSD = NVK = 16 at head_dim 128), with the softmax of both blocks
    // spread over slots NSD .. (DkdvSoftPlan). Each slot also issues the LDS
    // read of the operand LA slots ahead (a short window keeps few operand
    // registers live). The DMA goes into the stage that unit - 1 used, free
    // since the barrier at the top of this unit; issued in the first slots,
    // which carry no softmax, it also has the longest time to land. The
    // MFMAs run on the matrix core while the interleaved VALU, LDS and memory
    // instructions issue. (Per-wave timestamps showed the slots that carried
    // the whole softmax of a block running 60-70% over their MFMA time and
    // the last phase at the MFMA rate; spreading the softmax and moving the
    // DMA to the first slots took 2.4% off the kernel at config 3.)
    auto unit = [&](auto stc, int qrow0, const Dma& nd) {
      constexpr int st = decltype(stc)::value;
      constexpr int NSD = 2 * NKS;  // S/dP MFMAs per block
      constexpr int NVK = 4 * NDB;  // dV/dK MFMAs per block
      constexpr int NSLOT = 2 * NSD + 2 * NVK;
      constexpr int LA = 4;         // operand read-ahead, in slots
      u32x4 op[NSLOT];              // A operand of every slot (short live ranges)
      f32x16 s[2], dp[2];
      f32x4 l4[2][4], d4[2][4];
      u32x4 pk[2][4];               // P lo/hi, dS lo/hi

      // Slot m -> (kind, block, index): kind 0 = S/dP, 1 = dV/dK. Every read
      // is a per-lane base register plus an immediate (stage, tile, row block).
      auto read_op = [&](int m) {
        constexpr uint32_t kStage = (st == 2 ? 0u : (uint32_t)st * kStageBytes);
        if (m < 2 * NSD) {
          const int qb = m / NSD, i = m % NSD, ks = i >> 1;
          const uint32_t off = kStage + ((i & 1) ? QT * 2u : 0u) + (uint32_t)(qb * 32 * CPR * 16);
          op[m] = *(const KF_LDS u32x4*)(uintptr_t)((st == 2 ? rdq2[ks] : rdq[ks]) + off);
        } else {
          const int qb = (m - 2 * NSD) / NVK, j = (m - 2 * NSD) % NVK;
          const int db = j % NDB, w = j / NDB;  // w: dV lo, dK lo, dV hi, dK hi
          const bool isv = (w & 1) == 0;
          const uint32_t off = kStage + (isv ? QT * 2u : 0u) + (uint32_t)((qb * 32 + 16 * (w >> 1)) * CPR * 16);
          const u32x2 lo = lds_read_tr16_at((st == 2 ? trb2[db][0] : trb[db][0]) + off);
          const u32x2 hi = lds_read_tr16_at((st == 2 ? trb2[db][1] : trb[db][1]) + off);
          op[m] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      };
      auto mfma_slot = [&](int m) {
        if (m < 2 * NSD) {
          const int qb = m / NSD, i = m % NSD, ks = i >> 1;
          if (i & 1)
            dp[qb] = Elem<T>::mfma(op[m], vf[ks], dp[qb]);
          else
            s[qb] = Elem<T>::mfma(op[m], kf[ks], s[qb]);
        } else {
          const int qb = (m - 2 * NSD) / NVK, j = (m - 2 * NSD) % NVK;
          const int db = j % NDB, w = j / NDB;
          // pk layout: [0] P lo, [1] P hi, [2] dS lo, [3] dS hi
          const int src = (w & 1) ? 2 + (w >> 1) : (w >> 1);
          if ((w & 1) == 0)
            dkdv_mfma_acc<T>(dv[db], op[m], pk[qb][src]);
          else
            dkdv_mfma_acc<T>(dk[db], op[m], pk[qb][src]);
        }
      };
      auto read_stats = [&](int qb) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int rl = qb * 32 + 8 * g4 + 4 * h32;
          l4[qb][g4] = *reinterpret_cast<const f32x4*>(&rowstat[st][0][rl]);
          d4[qb][g4] = *reinterpret_cast<const f32x4*>(&rowstat[st][1][rl]);
        }
      };
      // S layout: lane = key, register r = query row 8 (r/4) + 4 h + r % 4.
      // Causal mask of block qb: key <= row  <=>  t <= 8 (r/4) + r % 4 with
      // t = key - (block row 0) - 4 h. It is folded into the row statistics:
      // a masked (row, key) element gets LSE = +inf in this lane's copy, so
      // exp2(scale S - LSE) = 0 there and the softmax itself has no mask
      // instructions. Only blocks that cross this wave's diagonal take the
      // (wave-uniform) branch that does it; one unit body serves all units
      // (two specialised bodies exceed the register budget).
      // The softmax of an element runs in three stages spread over three
      // consecutive slots (exponent argument, exp2, then dS = P dP and the
      // packing of every eighth element), so the VALU instructions of a slot
      // belong to different elements and do not wait on each other: with one
      // wave per SIMD, a dependent chain inside a slot holds back the next
      // slot's MFMA.
      float xs[2][16], pv[2][16], dsv[2][16];
      auto soft_a = [&](int qb, int r) {
        const int g4 = r >> 2, e = r & 3;
        xs[qb][r] = fmaf(s[qb][r], p.scale_log2, -l4[qb][g4][e]);
      };
      auto soft_b = [&](int qb, int r) { pv[qb][r] = fast_exp2(xs[qb][r]); };
      auto soft_c = [&](int qb, int r) {
        dsv[qb][r] = pv[qb][r] * dp[qb][r];  // dP accumulated from -delta: dS = P (dP - delta)
        if ((r & 7) == 7) {
          const int h = r >> 3, r0 = r - 7;
          u32x4 a, d;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a[i] = pack2<T>(pv[qb][r0 + 2 * i], pv[qb][r0 + 2 * i + 1]);
            d[i] = pack2<T>(dsv[qb][r0 + 2 * i], dsv[qb][r0 + 2 * i + 1]);
          }
          pk[qb][h] = a;
          pk[qb][2 + h] = d;
        }
      };

      // dP accumulators start at -delta of their rows (register r <-> row
      // 8 (r/4) + 4 h + r % 4, the layout of d4), so dS = P * dP needs no
      // subtraction. Block 1's statistics are read a few slots before its
      // first MFMA.
      auto init_block = [&](int qb) {
        read_stats(qb);
        if (CAUSAL && qrow0 + 32 * qb < kw0 + 31) {
          const int t = key - (qrow0 + 32 * qb) - 4 * h32;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              l4[qb][g4][e] = t <= 8 * g4 + e ? l4[qb][g4][e] : __builtin_inff();
        }
        s[qb] = zero16();
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[qb][r] = d4[qb][r >> 2][r & 3];
      };
      // The dK/dV accumulators are pinned to accumulation registers at the
      // top of the unit (an empty asm with "+a" operands): left to itself,
      // the register allocator parks some of them in VGPRs while the S/dP
      // accumulators take their place, which costs 96 accumulator copies per
      // unit.
#pragma unroll
      for (int db = 0; db < NDB; ++db) asm volatile("" : "+a"(dk[db]), "+a"(dv[db]));
      init_block(0);
      static_for<0, LA>([&](auto mc) { read_op(decltype(mc)::value); });
      __builtin_amdgcn_sched_barrier(0);
      // Softmax elements per DkdvSoftPlan; each finishes before the first
      // MFMA that consumes its P/dS.
      using Plan = DkdvSoftPlan<NSD, NVK, NDB>;
      constexpr int DMA0 = 1;                                        // first slot carrying a DMA
      constexpr int DMAS = (NSD - 1) / NDMA > 0 ? (NSD - 1) / NDMA : 1;  // slot spacing
      static_assert(DMA0 + (NDMA - 1) * DMAS < NSLOT, "every DMA instruction gets a slot");
      static_assert(Plan::a(31) + 2 < NSLOT, "the softmax ends inside the unit");
      static_for<0, NSLOT>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        mfma_slot(m);
        if constexpr (m + LA < NSLOT) read_op(m + LA);
        if constexpr (m == NSD - 3) init_block(1);
        // Slot m runs stage c of the elements that started two slots ago,
        // stage b of those of the previous slot and stage a of its own, each
        // in element order (a block half is packed after its last element).
        static_for<Plan::at(m - 2), Plan::at(m - 1)>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          soft_c(k / 16, k % 16);
        });
        static_for<Plan::at(m - 1), Plan::at(m)>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          soft_b(k / 16, k % 16);
        });
        static_for<Plan::at(m), Plan::at(m + 1)>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          soft_a(k / 16, k % 16);
        });
        if constexpr (m >= DMA0 && (m - DMA0) % DMAS == 0 && (m - DMA0) / DMAS < NDMA)
          dma_issue(nd, (m - DMA0) / DMAS);
        __builtin_amdgcn_sched_barrier(0);
      });
    };

    // Ring: at the top of unit `it` the loads of units it and it + 1 are in
    // flight; wait for those of `it` (this wave's), then the barrier makes
    // every wave's loads visible and frees the stage of unit it - 1, which
    // receives unit it + 2 (issued from inside the unit's first phase).
    // The loop is unrolled by the ring's NST stages, so that every LDS offset
    // inside a unit is a compile-time constant.
    for (int it0 = ua; it0 < ub; it0 += NST) {
      static_for<0, NST>([&](auto stc) {
        constexpr int st = decltype(stc)::value;
        const int it = it0 + st;
        if (it < ub) {
          KF_WAIT_VMCNT(NDMA);  // unit it + 1's loads may still be in flight
          __syncthreads();
          const Dma nd = dma_setup(wdma, st == 0 ? NST - 1 : st - 1, it + 2 < ub);
          // Rows >= Sq and keys >= Sk need no mask: their Q/dO (K/V) rows load
          // as zeros and their LSE/delta as 0, so they add nothing to any valid
          // dK/dV row. A unit entirely above the causal diagonal for this wave
          // is computed fully masked rather than branched around.
          unit(stc, wcur.qt * kBMQ, nd);
          walk_next(wcur);
          walk_next(wdma);
        }
      });
    }
    // Every wave is done reading the ring's stages: the next segment's loads
    // can go out now, ahead of this segment's flush. This wave may still have
    // the zero-filling loads of the two units past the segment's end in
    // flight (they target its own rows of the ring, as the next segment's
    // first loads do). That is safe without a wait because one wave's
    // direct-to-LDS loads return, and write LDS, in issue order (the vmcnt
    // counter decrements in order), so the older zero fills land before the
    // next segment's data; the next segment's first vmcnt wait covers both.
    __syncthreads();
    const bool more = u + (ub - ua) < uend;
    if (more) {
      u += ub - ua;
      seek();
      segment_loads();
    }

    // The accumulators were last written by dkdv_mfma_acc, whose results
    // VALU may read only after the MFMA's passes: 24 wait states cover the
    // 8-pass 32x32x16 product with margin. The empty operands order the
    // accumulator reads below after them.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(dk[0]), "+a"(dv[0]));
#pragma unroll
    for (int db = 1; db < NDB; ++db) asm volatile("" : "+a"(dk[db]), "+a"(dv[db]));
    // Flush: dK^T / dV^T layout is lane = key, register r = head_dim
    // 32 db + 8 (r/4) + 4 h + r % 4. A tile this workgroup covered alone is
    // final; a shared one goes to this workgroup's partial slot.
    const bool full = ua == 0 && ub == per_tile;
    float* slot = p.part + (int64_t)(2 * share + (first_seg ? 0 : 1)) * 2 * kBNK * DT;
    uint16_t* Dk = p.dk + b * p.dk_sb + kvh * p.dk_sh + key * p.dk_ss;
    uint16_t* Dv = p.dv + b * p.dv_sb + kvh * p.dv_sh + key * p.dv_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * db + 8 * g4 + 4 * h32;
        const int r = 4 * g4;
        if (full) {
          if (key_ok && d < p.D) {
            u32x2 w;
            w[0] = pack2<T>(dk[db][r] * p.scale, dk[db][r + 1] * p.scale);
            w[1] = pack2<T>(dk[db][r + 2] * p.scale, dk[db][r + 3] * p.scale);
            *reinterpret_cast<u32x2*>(Dk + d) = w;
            w[0] = pack2<T>(dv[db][r], dv[db][r + 1]);
            w[1] = pack2<T>(dv[db][r + 2], dv[db][r + 3]);
            *reinterpret_cast<u32x2*>(Dv + d) = w;
          }
        } else {
          float* sk = slot + (wave * 32 + l32) * DT + d;
          *reinterpret_cast<float4*>(sk) =
              make_float4(dk[db][r] * p.scale, dk[db][r + 1] * p.scale, dk[db][r + 2] * p.scale,
                          dk[db][r + 3] * p.scale);
          *reinterpret_cast<float4*>(sk + kBNK * DT) =
              make_float4(dv[db][r], dv[db][r + 1], dv[db][r + 2], dv[db][r + 3]);
        }
      }
    }
    first_seg = false;
    if (!more) break;
  }
}

// ---------------------------------------------------------------------------
// 4. Fixup: kFixSub workgroups per key tile, kFixKeys keys each. Sums the partials
// of tiles shared by several dkdv workgroups, zero-fills tiles that no query
// can see, and leaves tiles one workgroup finished alone untouched. The host
// skips the launch when no share boundary cuts a tile row and every tile is
// seen (non-causal shapes whose shares end on tile rows, such as config 4):
// its thousands of workgroups would all return at once, which still costs
// about 15 us of dispatch.
constexpr int kFixKeys = 16;  // keys per fixup workgroup
constexpr int kFixSub = kBNK / kFixKeys;
template <typename T, int DT, bool CAUSAL>
__global__ __launch_bounds__(256) void dkdv_fixup_kernel(const BwdParams p, const DkdvSplit sp) {
  const int t = blockIdx.x / kFixSub, sub = blockIdx.x % kFixSub;
  const int kt = t / p.ngroups, grp = t % p.ngroups;
  const int b = grp / p.Hkv, kvh = grp % p.Hkv;
  const int k0 = kt * kBNK + sub * kFixKeys;
  const int nq = dkdv_nq(kt, p.nqt, CAUSAL);
  const int nkeys = min(kFixKeys, p.Sk - k0);
  if (nkeys <= 0) return;
  constexpr int QPR = DT / 4;
  if (nq == 0) {
    for (int e = threadIdx.x; e < nkeys * QPR; e += 256) {
      const int kr = e / QPR, d = (e % QPR) * 4;
      if (d >= p.D) continue;
      const u32x2 z = {0u, 0u};
      *reinterpret_cast<u32x2*>(p.dk + b * p.dk_sb + kvh * p.dk_sh + (k0 + kr) * p.dk_ss + d) = z;
      *reinterpret_cast<u32x2*>(p.dv + b * p.dv_sb + kvh * p.dv_sh + (k0 + kr) * p.dv_ss + d) = z;
    }
    return;
  }
  // First unit of the tile row: the rows at earlier positions of the group's
  // tile order come before it.
  const int mseen = dkdv_seen_tiles(p.nqt, p.nkt, CAUSAL);
  int64_t first = (int64_t)grp * (p.units / p.ngroups);
  const int kpos = dkdv_pos_of(kt, mseen);
  for (int q = 0; q < kpos; ++q) first += (int64_t)p.G * dkdv_nq(dkdv_tile_at(q, mseen), p.nqt, CAUSAL);
  const int64_t last = first + (int64_t)p.G * nq - 1;
  const int w0 = dkdv_owner(sp, p.nwg, first), w1 = dkdv_owner(sp, p.nwg, last);
  if (w0 == w1) return;
  for (int e = threadIdx.x; e < nkeys * QPR; e += 256) {
    const int kr = sub * kFixKeys + e / QPR, d = (e % QPR) * 4;
    if (d >= p.D) continue;
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f), sv = sk;
    for (int w = w0; w <= w1; ++w) {
      const int64_t wu0 = sp.start[w];
      if (sp.start[w + 1] == wu0) continue;  // empty share: wrote nothing
      const int side = wu0 >= first ? 0 : 1;
      const float* slot = p.part + (2 * w + side) * 2 * kBNK * DT + (int64_t)kr * DT + d;
      const float4 a = *reinterpret_cast<const float4*>(slot);
      const float4 c = *reinterpret_cast<const float4*>(slot + kBNK * DT);
      sk.x += a.x; sk.y += a.y; sk.z += a.z; sk.w += a.w;
      sv.x += c.x; sv.y += c.y; sv.z += c.z; sv.w += c.w;
    }
    u32x2 w2;
    w2[0] = pack2<T>(sk.x, sk.y);
    w2[1] = pack2<T>(sk.z, sk.w);
    *reinterpret_cast<u32x2*>(p.dk + b * p.dk_sb + kvh * p.dk_sh + (kt * kBNK + kr) * p.dk_ss + d) = w2;
    w2[0] = pack2<T>(sv.x, sv.y);
    w2[1] = pack2<T>(sv.z, sv.w);
    *reinterpret_cast<u32x2*>(p.dv + b * p.dv_sb + kvh * p.dv_sh + (kt * kBNK + kr) * p.dv_ss + d) = w2;
  }
}

// Stream-K bookkeeping from the host: total units and the workgroup count.
static int64_t dkdv_total_units(int ngroups, int G, int nqt, int nkt, bool causal) {
  int64_t U = 0;
  for (int kt = 0; kt < nkt; ++kt) U += (int64_t)ngroups * G * dkdv_nq(kt, nqt, causal);
  return U;
}

static int device_cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

// One dK/dV workgroup per CU (each takes a whole CU's LDS).
static int dkdv_workgroups() {
  const int n = device_cu_count();
  return n < kMaxDkdvWG ? n : kMaxDkdvWG;
}

static size_t delta_bytes(int64_t B, int64_t Hq, int64_t Sq) {
  return ((size_t)B * Hq * Sq * sizeof(float) + 255) / 256 * 256;
}

// Cost-weighted stream-K boundaries (see DkdvSplit). A segment start costs
// kSegmentCost8 / 8 units: on the MI355X at config 3 a sweep of the weight
// put the shortest launch at 4.5 to 6 units, and after a segment's loads
// came to overlap the previous segment's flush, 3 and 4 units were still
// 1-2% slower than 5. With the long-short tile order and cuts charged to the
// share that makes them, 3, 7 and 10 units were 0.4-1.2% slower than 5.
constexpr int kSegmentCost8 = 40;
// Returns the number of tile rows that a share boundary cuts (shared tiles).
static int dkdv_split(DkdvSplit& sp, int ngroups, int G, int nqt, int nkt, bool causal, int nwg) {
  struct Key {
    int ngroups, G, nqt, nkt, causal, nwg;
  };
  thread_local Key last{-1, 0, 0, 0, 0, 0};
  thread_local DkdvSplit cached;
  thread_local int cached_shared = 0;
  const Key k{ngroups, G, nqt, nkt, causal ? 1 : 0, nwg};
  if (memcmp(&k, &last, sizeof k) != 0) {
    int64_t rows_cost = 0, all_units = 0;
    for (int kt = 0; kt < nkt; ++kt) {
      const int64_t units = (int64_t)G * dkdv_nq(kt, nqt, causal);
      if (units) rows_cost += (int64_t)ngroups * (8 * units + kSegmentCost8);
      all_units += (int64_t)ngroups * units;
    }
    const int mseen = dkdv_seen_tiles(nqt, nkt, causal);
    // Boundaries at equal cost over the rows in unit order (KV group outer,
    // key tiles in dkdv_tile_at order inner). A boundary inside a tile row
    // starts one more segment (the next share enters the row part-way); with
    // cut_cost = kSegmentCost8 that segment start is charged to the share
    // that makes it, and `total` must then include the cuts. Returns the
    // number of cuts; `shared` counts the rows cut at least once.
    auto place = [&](DkdvSplit& out, int64_t total, int64_t cut_cost, int& shared_rows) {
      int w = 1, cuts = 0;
      int64_t base = 0, cost = 0;
      shared_rows = 0;
      out.start[0] = 0;
      for (int g = 0; g < ngroups && w < nwg; ++g) {
        for (int pos = 0; pos < nkt && w < nwg; ++pos) {
          const int64_t units = (int64_t)G * dkdv_nq(dkdv_tile_at(pos, mseen), nqt, causal);
          if (!units) continue;
          const int64_t row_cost = 8 * units + kSegmentCost8;
          int row_cuts = 0;
          int64_t prev = 0;  // boundaries never move backwards
          while (w < nwg) {
            const int64_t target = (total * w + nwg - 1) / nwg;
            if (target > cost + row_cost + row_cuts * cut_cost) break;
            int64_t into = (target - cost - kSegmentCost8 - row_cuts * cut_cost + 7) / 8;
            into = into < prev ? prev : (into > units ? units : into);
            prev = into;
            out.start[w++] = (int)(base + into);
            if (into > 0 && into < units) ++row_cuts;
          }
          shared_rows += row_cuts > 0 ? 1 : 0;
          cuts += row_cuts;
          cost += row_cost + row_cuts * cut_cost;
          base += units;
        }
      }
      while (w < nwg) out.start[w++] = (int)all_units;
      out.start[nwg] = (int)all_units;
      return cuts;
    };
    // The plain placement first; then the cut-charged one, started from the
    // plain cut count and kept when it reaches a fixed point (at config 3
    // at once: the long tile of each pair is cut once, half a segment later).
    int shared = 0;
    int cuts = place(cached, rows_cost, 0, shared);
    DkdvSplit refined;
    for (int pass = 0; pass < 3; ++pass) {
      int rshared = 0;
      const int rcuts = place(refined, rows_cost + (int64_t)cuts * kSegmentCost8, kSegmentCost8, rshared);
      if (rcuts == cuts) {
        cached = refined;
        shared = rshared;
        break;
      }
      cuts = rcuts;
    }
    cached_shared = shared;
    last = k;
  }
  sp = cached;
  return cached_shared;
}

static size_t partial_bytes(int nwg, int64_t D) {
  return (size_t)2 * nwg * 2 * kBNK * head_tile(D) * sizeof(float);
}

template <typename T, int DT, int KS>
static int launch_bwd(BwdParams p, bool causal, int stages, hipStream_t stream) {
  // dq_kernel computes the row deltas itself: the delta launch is only needed
  // when the dK/dV stage runs without it.
  if ((stages & KF_BWD_DELTA) && !(stages & KF_BWD_DQ)) {
    const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
    hipLaunchKernelGGL((delta_kernel<T>), dim3((unsigned)((rows + kDeltaRows - 1) / kDeltaRows)), dim3(256), 0, stream, p);
    int rc = check_launch("kf_attn_bwd(delta)");
    if (rc) return rc;
  }
  if (stages & KF_BWD_DQ) {
    // The forward's rule for its split form: grids of 128-row tiles that
    // leave most CUs idle take 32-row workgroups whose waves split the key
    // range.
    const bool split = attn_use_split(p.B, p.Hq, p.Sq, p.Sk, causal);
    p.nqt = cdiv(p.Sq, split ? 32 : 128);
    const int64_t gq = (int64_t)p.nqt * p.B * p.Hq;
    if (split) {
      if (causal)
        hipLaunchKernelGGL((dq_kernel<T, DT, KS, true, true>), dim3((unsigned)gq), dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL((dq_kernel<T, DT, KS, false, true>), dim3((unsigned)gq), dim3(256), 0, stream, p);
    } else if (causal) {
      hipLaunchKernelGGL((dq_kernel<T, DT, KS, true, false>), dim3((unsigned)gq), dim3(256), 0, stream, p);
    } else {
      hipLaunchKernelGGL((dq_kernel<T, DT, KS, false, false>), dim3((unsigned)gq), dim3(256), 0, stream, p);
    }
    int rc = check_launch("kf_attn_bwd(dq)");
    if (rc) return rc;
  }
  if (stages & KF_BWD_DKDV) {
    p.nqt = cdiv(p.Sq, kBMQ);
    p.nkt = cdiv(p.Sk, kBNK);
    p.units = dkdv_total_units(p.ngroups, p.G, p.nqt, p.nkt, causal);
    if (p.units > 0x7fffffff) return set_error(KF_EINVAL, "kf_attn_bwd: problem too large for one dK/dV launch");
    DkdvSplit sp;
    dkdv_split(sp, p.ngroups, p.G, p.nqt, p.nkt, causal, p.nwg);
    if (causal)
      hipLaunchKernelGGL((dkdv_kernel<T, DT, KS, true>), dim3((unsigned)p.nwg), dim3(256), 0, stream, p, sp);
    else
      hipLaunchKernelGGL((dkdv_kernel<T, DT, KS, false>), dim3((unsigned)p.nwg), dim3(256), 0, stream, p, sp);
    int rc = check_launch("kf_attn_bwd(dkdv)");
    if (rc) return rc;
  }
  if (stages & KF_BWD_DKDV_FIXUP) {
    p.nqt = cdiv(p.Sq, kBMQ);
    p.nkt = cdiv(p.Sk, kBNK);
    p.units = dkdv_total_units(p.ngroups, p.G, p.nqt, p.nkt, causal);
    DkdvSplit sp;
    const int shared = dkdv_split(sp, p.ngroups, p.G, p.nqt, p.nkt, causal, p.nwg);
    const int64_t unseen = (int64_t)p.ngroups * (p.nkt - dkdv_seen_tiles(p.nqt, p.nkt, causal));
    if (shared > 0 || unseen > 0) {
      const int64_t grid = (int64_t)p.nkt * p.ngroups * kFixSub;
      if (grid > 0x7fffffff) return set_error(KF_EINVAL, "kf_attn_bwd: problem too large for one fixup launch");
      if (causal)
        hipLaunchKernelGGL((dkdv_fixup_kernel<T, DT, true>), dim3((unsigned)grid), dim3(256), 0, stream, p, sp);
      else
        hipLaunchKernelGGL((dkdv_fixup_kernel<T, DT, false>), dim3((unsigned)grid), dim3(256), 0, stream, p, sp);
      int rc = check_launch("kf_attn_bwd(dkdv fixup)");
      if (rc) return rc;
    }
  }
  return KF_OK;
}

template <typename T>
static int dispatch_bwd(const BwdParams& p, bool causal, int stages, hipStream_t stream) {
  switch (head_tile(p.D)) {
    case 32: return launch_bwd<T, 32, 2>(p, causal, stages, stream);
    case 64: return launch_bwd<T, 64, 4>(p, causal, stages, stream);
    case 96:
      // Head dims 72 and 80 end 16 columns before the tile does.
      return p.D <= 80 ? launch_bwd<T, 96, 5>(p, causal, stages, stream)
                       : launch_bwd<T, 96, 6>(p, causal, stages, stream);
    default: return launch_bwd<T, 128, 8>(p, causal, stages, stream);
  }
}

}  // namespace kf

using namespace kf;

extern "C" size_t kf_attn_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                              int64_t Sk, int64_t D, int causal) {
  (void)Hkv; (void)Sk; (void)causal;
  if (B <= 0 || Hq <= 0 || Sq <= 0 || D <= 0) return 0;
  return 2 * delta_bytes(B, Hq, Sq) + partial_bytes(dkdv_workgroups(), D);
}

extern "C" int kf_attn_bwd_stages(int stages, const void* q, const void* k, const void* v,
                                  const void* o, const float* lse, const void* dout, void* dq,
                                  void* dk, void* dv, int64_t B, int64_t Hq, int64_t Hkv,
                                  int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides,
                                  const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* o_strides, const int64_t* do_strides,
                                  const int64_t* dq_strides, const int64_t* dk_strides,
                                  const int64_t* dv_strides, float scale, int causal, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kf_attn_bwd";
  if (stages <= 0 || stages > KF_BWD_ALL)
    return set_error(KF_EINVAL, "%s: stages must be a non-empty KF_BWD_* mask", what);
  int rc = check_attn_common(what, B, Hq, Hkv, Sq, Sk, D, dtype);
  if (rc) return rc;
  if ((rc = check_tensor(what, "q", q, q_strides)) || (rc = check_tensor(what, "k", k, k_strides)) ||
      (rc = check_tensor(what, "v", v, v_strides)) || (rc = check_tensor(what, "o", o, o_strides)) ||
      (rc = check_tensor(what, "dout", dout, do_strides)) ||
      (rc = check_tensor(what, "dq", dq, dq_strides)) ||
      (rc = check_tensor(what, "dk", dk, dk_strides)) ||
      (rc = check_tensor(what, "dv", dv, dv_strides)))
    return rc;
  if (lse == nullptr) return set_error(KF_EINVAL, "%s: lse is null", what);
  if (!(scale == scale) || scale - scale != 0.f) return set_error(KF_EINVAL, "%s: scale must be finite", what);
  if ((rc = check_extent(what, "q", Sq, q_strides[2], D)) || (rc = check_extent(what, "k", Sk, k_strides[2], D)) ||
      (rc = check_extent(what, "v", Sk, v_strides[2], D)) || (rc = check_extent(what, "dout", Sq, do_strides[2], D)))
    return rc;
  const size_t need = kf_attn_bwd_workspace_bytes(B, Hq, Hkv, Sq, Sk, D, causal);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(KF_EINVAL, "%s: workspace of %zu bytes required, got %zu", what, need,
                     workspace == nullptr ? (size_t)0 : workspace_bytes);
  BwdParams p{};
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k; p.v = (const uint16_t*)v;
  p.o = (const uint16_t*)o; p.dout = (const uint16_t*)dout; p.lse = lse;
  p.delta = (float*)workspace;
  p.nwg = dkdv_workgroups();
  p.lse2 = (float*)((char*)workspace + delta_bytes(B, Hq, Sq));
  p.part = (float*)((char*)workspace + 2 * delta_bytes(B, Hq, Sq));
  p.dq = (uint16_t*)dq; p.dk = (uint16_t*)dk; p.dv = (uint16_t*)dv;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.do_sb = do_strides[0]; p.do_sh = do_strides[1]; p.do_ss = do_strides[2];
  p.dq_sb = dq_strides[0]; p.dq_sh = dq_strides[1]; p.dq_ss = dq_strides[2];
  p.dk_sb = dk_strides[0]; p.dk_sh = dk_strides[1]; p.dk_ss = dk_strides[2];
  p.dv_sb = dv_strides[0]; p.dv_sh = dv_strides[1]; p.dv_ss = dv_strides[2];
  p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Sq = (int)Sq; p.Sk = (int)Sk; p.D = (int)D;
  p.G = (int)(Hq / Hkv);
  p.ngroups = (int)(B * Hkv);
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  return dtype == KF_F16 ? dispatch_bwd<_Float16>(p, causal != 0, stages, s)
                         : dispatch_bwd<__bf16>(p, causal != 0, stages, s);
}

extern "C" int kf_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                           const float* lse, const void* dout, void* dq, void* dk, void* dv,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                           const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* o_strides,
                           const int64_t* do_strides, const int64_t* dq_strides,
                           const int64_t* dk_strides, const int64_t* dv_strides, float scale,
                           int causal, int dtype, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return kf_attn_bwd_stages(KF_BWD_ALL, q, k, v, o, lse, dout, dq, dk,
                            dv, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides,
                            do_strides, dq_strides, dk_strides, dv_strides, scale, causal, dtype,
                            workspace, workspace_bytes, stream);
}
