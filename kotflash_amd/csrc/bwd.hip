// Attention backward for gfx950.
//
// Three launches on one stream, no atomics, deterministic:
//   1. delta_kernel: delta[i] = sum_d O[i,d] * dO[i,d] from the stored
//      low-precision O (reference triton_backward.py:45).
//   2. dq_kernel (query-stationary, same layout as the forward): per key tile it
//      recomputes S^T = K Q^T and dP^T = V dO^T, forms
//      dS^T = P^T (dP^T - delta) with P = exp(scale S - LSE), and accumulates
//      dQ^T += K^T dS^T; dQ = scale * dQ^T^T  (reference :17-91).
//   3. dkdv_kernel (key-stationary): a workgroup owns 128 keys of one
//      (batch, kv_head); K and V stay in registers as MFMA B operands, and for
//      every query head of the GQA group and every query tile it recomputes
//      S = Q K^T and dP = dO V^T, then accumulates dV^T += dO^T P and
//      dK^T += Q^T dS in registers. The group sum over query heads therefore
//      happens in registers, without partial buffers (reference :94-195, where
//      the group loop is :136-137 and the products :183-184).
// P and dS are rounded to the input dtype before the products that consume
// them, as in the reference (:85, :183-184).
#include "kf_common.hpp"
#include "kf_host.hpp"

namespace kf {

int check_attn_common(const char* what, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                      int64_t D, int dtype);
int check_tensor(const char* what, const char* name, const void* ptr, const int64_t* strides);

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  float* delta;
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
  int nqt, nkt;
  float scale, scale_log2;
};

// ---------------------------------------------------------------------------
// 1. delta = rowsum(O * dO): 16 lanes per row, 16 rows per workgroup.
template <typename T>
__global__ __launch_bounds__(256) void delta_kernel(const BwdParams p) {
  const int tid = threadIdx.x;
  const int rsub = tid >> 4, c16 = tid & 15;
  const int64_t total = (int64_t)p.B * p.Hq * p.Sq;
  const int64_t row = (int64_t)blockIdx.x * 16 + rsub;
  float acc = 0.f;
  if (row < total) {
    const int64_t bh = row / p.Sq;
    const int i = (int)(row - bh * p.Sq);
    const int b = (int)(bh / p.Hq), h = (int)(bh % p.Hq);
    const uint16_t* Op = p.o + b * p.o_sb + h * p.o_sh + i * p.o_ss;
    const uint16_t* Dp = p.dout + b * p.do_sb + h * p.do_sh + i * p.do_ss;
    for (int c = c16; c * 8 < p.D; c += 16) {
      const u32x4 a = ldg16(Op + c * 8), g = ldg16(Dp + c * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        acc += Elem<T>::to_f32((uint16_t)(a[w] & 0xffff)) * Elem<T>::to_f32((uint16_t)(g[w] & 0xffff));
        acc += Elem<T>::to_f32((uint16_t)(a[w] >> 16)) * Elem<T>::to_f32((uint16_t)(g[w] >> 16));
      }
    }
  }
  acc += __shfl_xor(acc, 8);
  acc += __shfl_xor(acc, 4);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 1);
  if (c16 == 0 && row < total) p.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// 2. dQ, query-stationary. QB = 1 block of 32 rows per wave, BM = 128.
template <typename T, int DT, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void dq_kernel(const BwdParams p) {
  constexpr int BM = 128;
  constexpr int BN = 64;
  constexpr int KSTR = DT + 16;  // K: b128 reads for S^T and transposed reads for dQ^T
  constexpr int VSTR = DT + 8;   // V: b128 reads for dP^T
  constexpr int KT = BN * KSTR;
  constexpr int STAGE = KT + BN * VSTR;
  constexpr int CPR = DT / 8;
  constexpr int CPT = BN * CPR / 256;
  constexpr int NKS = DT / 16;
  constexpr int NDB = DT / 32;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h32 = lane >> 5;

  // Longest query tiles first; same XCD grouping as the forward.
  int qt, b, h;
  {
    const int G = p.Hq / p.Hkv, ngroups = p.B * p.Hkv;
    const int bid = blockIdx.x;
    if ((ngroups & 7) == 0) {
      const int x = bid & 7, j = bid >> 3, gpx = ngroups >> 3, per_tile = G * gpx;
      const int t = j / per_tile, r = j - t * per_tile;
      qt = p.nqt - 1 - t;
      const int grp = x + 8 * (r / G);
      b = grp / p.Hkv;
      h = (grp % p.Hkv) * G + r % G;
    } else {
      const int bh = p.B * p.Hq, t = bid / bh, r = bid - t * bh;
      qt = p.nqt - 1 - t;
      b = r / p.Hq;
      h = r % p.Hq;
    }
  }
  const int kvh = h / (p.Hq / p.Hkv);
  const int q0 = qt * BM;
  const int qrow = q0 + wave * 32 + l32;
  const bool row_ok = qrow < p.Sq;

  const uint16_t* Qp = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* DOp = p.dout + b * p.do_sb + h * p.do_sh;
  const uint16_t* Kp = p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t* Vp = p.v + b * p.v_sb + kvh * p.v_sh;

  u32x4 qf[NKS], dof[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = 16 * ks + 8 * h32;
    const bool ok = row_ok && d < p.D;
    qf[ks] = ok ? ldg16(Qp + qrow * p.q_ss + d) : zero_u4();
    dof[ks] = ok ? ldg16(DOp + qrow * p.do_ss + d) : zero_u4();
  }
  const int64_t rowlin = ((int64_t)b * p.Hq + h) * p.Sq + qrow;
  const float lse2 = row_ok ? p.lse[rowlin] * kLog2e : 0.f;
  const float dlt = row_ok ? p.delta[rowlin] : 0.f;

  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = zero16();

  const int nkeys = CAUSAL ? min(p.Sk, q0 + BM) : p.Sk;
  const int ntiles = cdiv(nkeys, BN);

  u32x4 kreg[CPT], vreg[CPT];
  auto gload = [&](int tile) {
    const int kbase = tile * BN;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + 256 * c;
      const int row = e / CPR, col = e % CPR;
      const int key = kbase + row;
      const bool ok = key < p.Sk && col * 8 < p.D;
      kreg[c] = ok ? ldg16(Kp + key * p.k_ss + col * 8) : zero_u4();
      vreg[c] = ok ? ldg16(Vp + key * p.v_ss + col * 8) : zero_u4();
    }
  };
  auto sstore = [&](int buf) {
    uint16_t* Ks = smem + buf * STAGE;
    uint16_t* Vs = Ks + KT;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + 256 * c;
      const int row = e / CPR, col = e % CPR;
      lds_write16(Ks + row * KSTR + col * 8, kreg[c]);
      lds_write16(Vs + row * VSTR + col * 8, vreg[c]);
    }
  };

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  const int wq0 = q0 + wave * 32;
  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    if (it + 1 < ntiles) gload(it + 1);
    const uint16_t* Ks = smem + buf * STAGE;
    const uint16_t* Vs = Ks + KT;
    const int kbase = it * BN;
    const bool active = !CAUSAL || kbase <= wq0 + 31;
    if (active) {
      f32x16 s[2], dp[2];
      s[0] = zero16(); s[1] = zero16(); dp[0] = zero16(); dp[1] = zero16();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const u32x4 a = lds_read16(Ks + (kb * 32 + l32) * KSTR + 16 * ks + 8 * h32);
          s[kb] = Elem<T>::mfma(a, qf[ks], s[kb]);
          const u32x4 a2 = lds_read16(Vs + (kb * 32 + l32) * VSTR + 16 * ks + 8 * h32);
          dp[kb] = Elem<T>::mfma(a2, dof[ks], dp[kb]);
        }
      }
      const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && kbase + BN - 1 > wq0);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          bool valid = true;
          if (need_mask) {
            const int key = kbase + 32 * kb + 8 * (r >> 2) + 4 * h32 + (r & 3);
            valid = key < p.Sk && (!CAUSAL || key <= qrow);
          }
          const float pv = valid ? fast_exp2(s[kb][r] * p.scale_log2 - lse2) : 0.f;
          dp[kb][r] = pv * (dp[kb][r] - dlt);
        }
      }
      u32x4 dsk[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) dsk[st] = pack8<T>(dp[st >> 1], 8 * (st & 1));
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4 a = lds_read_tr_operand(Ks, KSTR, 16 * st, 32 * db, lane);
          dq[db] = Elem<T>::mfma(a, dsk[st], dq[db]);
        }
      }
    }
    if (it + 1 < ntiles) sstore(buf ^ 1);
    __syncthreads();
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
}

// ---------------------------------------------------------------------------
// 3. dK/dV, key-stationary. 4 waves x 32 keys = 128 keys per workgroup, query
// tiles of 64 rows.
template <typename T, int DT, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void dkdv_kernel(const BwdParams p) {
  constexpr int BNK = 128;
  constexpr int BMQ = 64;
  constexpr int QSTR = DT + 16;  // b128 row reads and transposed reads
  constexpr int QT = BMQ * QSTR;
  constexpr int STAGE = 2 * QT;  // Q tile, dO tile
  constexpr int CPR = DT / 8;
  constexpr int CPT = BMQ * CPR / 256;
  constexpr int NKS = DT / 16;
  constexpr int NDB = DT / 32;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];
  __shared__ __attribute__((aligned(16))) float rowstat[2][2][BMQ];  // [buf][lse2, delta][row]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h32 = lane >> 5;
  const int G = p.Hq / p.Hkv;

  // Key tile 0 has the most causal work: issue key tiles in ascending order,
  // KV groups on XCDs as in the forward.
  int kt, b, kvh;
  {
    const int ngroups = p.B * p.Hkv, bid = blockIdx.x;
    int grp;
    if ((ngroups & 7) == 0) {
      const int x = bid & 7, j = bid >> 3, gpx = ngroups >> 3;
      kt = j / gpx;
      grp = x + 8 * (j % gpx);
    } else {
      kt = bid / ngroups;
      grp = bid % ngroups;
    }
    b = grp / p.Hkv;
    kvh = grp % p.Hkv;
  }
  const int k0 = kt * BNK;
  const int kw0 = k0 + wave * 32;
  const int key = kw0 + l32;
  const bool key_ok = key < p.Sk;

  const uint16_t* Kp = p.k + b * p.k_sb + kvh * p.k_sh;
  const uint16_t* Vp = p.v + b * p.v_sb + kvh * p.v_sh;
  u32x4 kf[NKS], vf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = 16 * ks + 8 * h32;
    const bool ok = key_ok && d < p.D;
    kf[ks] = ok ? ldg16(Kp + key * p.k_ss + d) : zero_u4();
    vf[ks] = ok ? ldg16(Vp + key * p.v_ss + d) : zero_u4();
  }
  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = zero16();
    dv[db] = zero16();
  }

  // Query tiles that can see any key of this workgroup.
  const int qt_start = CAUSAL ? (k0 / BMQ) : 0;
  const int nq = max(0, p.nqt - qt_start);
  const int niter = G * nq;

  u32x4 qreg[CPT], dreg[CPT];
  float st_l = 0.f, st_d = 0.f;
  auto gload = [&](int it) {
    const int g = it / nq;
    const int qt = qt_start + (it - g * nq);
    const int h = kvh * G + g;
    const int qbase = qt * BMQ;
    const uint16_t* Qp = p.q + b * p.q_sb + h * p.q_sh;
    const uint16_t* DOp = p.dout + b * p.do_sb + h * p.do_sh;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + 256 * c;
      const int row = e / CPR, col = e % CPR;
      const int qi = qbase + row;
      const bool ok = qi < p.Sq && col * 8 < p.D;
      qreg[c] = ok ? ldg16(Qp + qi * p.q_ss + col * 8) : zero_u4();
      dreg[c] = ok ? ldg16(DOp + qi * p.do_ss + col * 8) : zero_u4();
    }
    if (tid < BMQ) {
      const int qi = qbase + tid;
      const int64_t rl = ((int64_t)b * p.Hq + h) * p.Sq + qi;
      st_l = qi < p.Sq ? p.lse[rl] * kLog2e : 0.f;
      st_d = qi < p.Sq ? p.delta[rl] : 0.f;
    }
  };
  auto sstore = [&](int buf) {
    uint16_t* Qs = smem + buf * STAGE;
    uint16_t* Ds = Qs + QT;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + 256 * c;
      const int row = e / CPR, col = e % CPR;
      lds_write16(Qs + row * QSTR + col * 8, qreg[c]);
      lds_write16(Ds + row * QSTR + col * 8, dreg[c]);
    }
    if (tid < BMQ) {
      rowstat[buf][0][tid] = st_l;
      rowstat[buf][1][tid] = st_d;
    }
  };

  if (niter > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int it = 0; it < niter; ++it) {
    const int buf = it & 1;
    if (it + 1 < niter) gload(it + 1);
    const int g = it / nq;
    const int qt = qt_start + (it - g * nq);
    const int qbase = qt * BMQ;
    const uint16_t* Qs = smem + buf * STAGE;
    const uint16_t* Ds = Qs + QT;
    const bool active = !CAUSAL || qbase + BMQ - 1 >= kw0;
    if (active) {
      f32x16 s[2], dp[2];
      s[0] = zero16(); s[1] = zero16(); dp[0] = zero16(); dp[1] = zero16();
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const u32x4 a = lds_read16(Qs + (qq * 32 + l32) * QSTR + 16 * ks + 8 * h32);
          s[qq] = Elem<T>::mfma(a, kf[ks], s[qq]);
          const u32x4 a2 = lds_read16(Ds + (qq * 32 + l32) * QSTR + 16 * ks + 8 * h32);
          dp[qq] = Elem<T>::mfma(a2, vf[ks], dp[qq]);
        }
      }
      const bool need_mask = (qbase + BMQ > p.Sq) || !key_ok || (CAUSAL && qbase < kw0 + 31);
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int rl = qq * 32 + 8 * g4 + 4 * h32;
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(&rowstat[buf][0][rl]);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(&rowstat[buf][1][rl]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            bool valid = true;
            if (need_mask) {
              const int qi = qbase + rl + e;
              valid = qi < p.Sq && key_ok && (!CAUSAL || key <= qi);
            }
            const float pv = valid ? fast_exp2(s[qq][r] * p.scale_log2 - l4[e]) : 0.f;
            s[qq][r] = pv;
            dp[qq][r] = pv * (dp[qq][r] - d4[e]);
          }
        }
      }
      u32x4 pk[4], dsk[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        pk[st] = pack8<T>(s[st >> 1], 8 * (st & 1));
        dsk[st] = pack8<T>(dp[st >> 1], 8 * (st & 1));
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4 a = lds_read_tr_operand(Ds, QSTR, 16 * st, 32 * db, lane);
          dv[db] = Elem<T>::mfma(a, pk[st], dv[db]);
          const u32x4 a2 = lds_read_tr_operand(Qs, QSTR, 16 * st, 32 * db, lane);
          dk[db] = Elem<T>::mfma(a2, dsk[st], dk[db]);
        }
      }
    }
    if (it + 1 < niter) sstore(buf ^ 1);
    __syncthreads();
  }

  if (key_ok) {
    uint16_t* Dk = p.dk + b * p.dk_sb + kvh * p.dk_sh + key * p.dk_ss;
    uint16_t* Dv = p.dv + b * p.dv_sb + kvh * p.dv_sh + key * p.dv_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * db + 8 * g4 + 4 * h32;
        if (d < p.D) {
          u32x2 w;
          w[0] = pack2<T>(dk[db][4 * g4 + 0] * p.scale, dk[db][4 * g4 + 1] * p.scale);
          w[1] = pack2<T>(dk[db][4 * g4 + 2] * p.scale, dk[db][4 * g4 + 3] * p.scale);
          *reinterpret_cast<u32x2*>(Dk + d) = w;
          u32x2 w2;
          w2[0] = pack2<T>(dv[db][4 * g4 + 0], dv[db][4 * g4 + 1]);
          w2[1] = pack2<T>(dv[db][4 * g4 + 2], dv[db][4 * g4 + 3]);
          *reinterpret_cast<u32x2*>(Dv + d) = w2;
        }
      }
    }
  }
}

template <typename T, int DT>
static int launch_bwd(BwdParams p, bool causal, int stages, hipStream_t stream) {
  if (stages & KF_BWD_DELTA) {
    const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
    hipLaunchKernelGGL((delta_kernel<T>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, stream, p);
    int rc = check_launch("kf_attn_bwd(delta)");
    if (rc) return rc;
  }
  if (stages & KF_BWD_DQ) {
    p.nqt = cdiv(p.Sq, 128);
    const int64_t gq = (int64_t)p.nqt * p.B * p.Hq;
    if (causal)
      hipLaunchKernelGGL((dq_kernel<T, DT, true>), dim3((unsigned)gq), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((dq_kernel<T, DT, false>), dim3((unsigned)gq), dim3(256), 0, stream, p);
    int rc = check_launch("kf_attn_bwd(dq)");
    if (rc) return rc;
  }
  if (stages & KF_BWD_DKDV) {
    p.nqt = cdiv(p.Sq, 64);
    p.nkt = cdiv(p.Sk, 128);
    const int64_t gk = (int64_t)p.nkt * p.B * p.Hkv;
    if (causal)
      hipLaunchKernelGGL((dkdv_kernel<T, DT, true>), dim3((unsigned)gk), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((dkdv_kernel<T, DT, false>), dim3((unsigned)gk), dim3(256), 0, stream, p);
    int rc = check_launch("kf_attn_bwd(dkdv)");
    if (rc) return rc;
  }
  return KF_OK;
}

template <typename T>
static int dispatch_bwd(const BwdParams& p, bool causal, int stages, hipStream_t stream) {
  switch (head_tile(p.D)) {
    case 32: return launch_bwd<T, 32>(p, causal, stages, stream);
    case 64: return launch_bwd<T, 64>(p, causal, stages, stream);
    case 96: return launch_bwd<T, 96>(p, causal, stages, stream);
    default: return launch_bwd<T, 128>(p, causal, stages, stream);
  }
}

}  // namespace kf

using namespace kf;

extern "C" size_t kf_attn_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                              int64_t Sk, int64_t D, int causal) {
  (void)Hkv; (void)Sk; (void)D; (void)causal;
  const size_t rows = (size_t)(B > 0 ? B : 0) * (size_t)(Hq > 0 ? Hq : 0) * (size_t)(Sq > 0 ? Sq : 0);
  return ((rows * sizeof(float) + 255) / 256) * 256;
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
  if (stages <= 0 || stages > (KF_BWD_DELTA | KF_BWD_DQ | KF_BWD_DKDV))
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
  const size_t need = kf_attn_bwd_workspace_bytes(B, Hq, Hkv, Sq, Sk, D, causal);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(KF_EINVAL, "%s: workspace of %zu bytes required, got %zu", what, need,
                     workspace == nullptr ? (size_t)0 : workspace_bytes);
  BwdParams p{};
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k; p.v = (const uint16_t*)v;
  p.o = (const uint16_t*)o; p.dout = (const uint16_t*)dout; p.lse = lse;
  p.delta = (float*)workspace;
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
  return kf_attn_bwd_stages(KF_BWD_DELTA | KF_BWD_DQ | KF_BWD_DKDV, q, k, v, o, lse, dout, dq, dk,
                            dv, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides,
                            do_strides, dq_strides, dk_strides, dv_strides, scale, causal, dtype,
                            workspace, workspace_bytes, stream);
}
