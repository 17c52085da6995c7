// K/V cache append for gfx950: cache[b, h, start_b + t, :] = new[b, h, t, :]
// for K and V in one launch (reference kotflash/csrc/kv_append_cuda.cu:12-40,
// index map :29-36), bit-exact.
//
// Differences from the reference kernel, by design:
//  * start_b may differ per batch entry (read from a device array), so ragged
//    caches append every sequence at its own position in one launch;
//  * when every row is 16-byte aligned each thread moves 16 bytes (8 elements)
//    of K and of V; otherwise one element per thread, like the reference;
//  * with per-sequence starts the host passes their maximum as a bound and the
//    launch is rejected unless bound + S fits the capacity (the reference's
//    capacity check, kv_append_cuda.cu:72-73, applied to that bound); a
//    device start outside [0, bound] breaks the caller's contract: its rows
//    are not written, so nothing lands outside [0, capacity).
#include "kf_common.hpp"
#include "kf_host.hpp"

namespace kf {

struct AppendParams {
  uint16_t* kc;
  uint16_t* vc;
  const uint16_t* nk;
  const uint16_t* nv;
  const int64_t* start_dev;
  int64_t start;
  int64_t kc_sb, kc_sh, kc_ss;
  int64_t vc_sb, vc_sh, vc_ss;
  int64_t nk_sb, nk_sh, nk_ss, nk_sd;
  int64_t nv_sb, nv_sh, nv_ss, nv_sd;
  int64_t total;  // work items
  int B, H, S, D;
};

template <bool VEC>
__global__ __launch_bounds__(256) void append_kernel(const AppendParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= p.total) return;
  const int per_row = VEC ? p.D / 8 : p.D;
  const int c = (int)(idx % per_row);
  int64_t rest = idx / per_row;
  const int t = (int)(rest % p.S);
  rest /= p.S;
  const int h = (int)(rest % p.H);
  const int b = (int)(rest / p.H);
  const int64_t s0 = p.start_dev ? p.start_dev[b] : p.start;
  // With start_dev, p.start is the host's bound on it (checked to fit).
  if (s0 < 0 || s0 > p.start) return;
  const int64_t pos = s0 + t;
  if (VEC) {
    const int d = c * 8;
    const u32x4 kk = ldg16(p.nk + b * p.nk_sb + h * p.nk_sh + t * p.nk_ss + d);
    const u32x4 vv = ldg16(p.nv + b * p.nv_sb + h * p.nv_sh + t * p.nv_ss + d);
    stg16(p.kc + b * p.kc_sb + h * p.kc_sh + pos * p.kc_ss + d, kk);
    stg16(p.vc + b * p.vc_sb + h * p.vc_sh + pos * p.vc_ss + d, vv);
  } else {
    const int d = c;
    p.kc[b * p.kc_sb + h * p.kc_sh + pos * p.kc_ss + d] =
        p.nk[b * p.nk_sb + h * p.nk_sh + t * p.nk_ss + d * p.nk_sd];
    p.vc[b * p.vc_sb + h * p.vc_sh + pos * p.vc_ss + d] =
        p.nv[b * p.nv_sb + h * p.nv_sh + t * p.nv_ss + d * p.nv_sd];
  }
}

}  // namespace kf

using namespace kf;

extern "C" int kf_kv_append(void* k_cache, void* v_cache, const void* new_k, const void* new_v,
                            const int64_t* start_dev, int64_t start, int64_t B, int64_t H,
                            int64_t Snew, int64_t D, int64_t capacity,
                            const int64_t* k_cache_strides, const int64_t* v_cache_strides,
                            const int64_t* new_k_strides4, const int64_t* new_v_strides4, int dtype,
                            void* stream) {
  const char* what = "kf_kv_append";
  if (!k_cache || !v_cache || !new_k || !new_v)
    return set_error(KF_EINVAL, "%s: null tensor pointer", what);
  if (!k_cache_strides || !v_cache_strides || !new_k_strides4 || !new_v_strides4)
    return set_error(KF_EINVAL, "%s: null strides", what);
  if (B <= 0 || H <= 0 || Snew <= 0 || D <= 0 || capacity <= 0)
    return set_error(KF_EINVAL, "%s: new K/V dimensions must be non-empty", what);
  if (dtype != KF_F16 && dtype != KF_BF16)
    return set_error(KF_EINVAL, "%s: dtype must be KF_F16 or KF_BF16", what);
  // The scalar start, or with start_dev the host-side bound on every
  // start_dev[b]: either way the whole range must fit before anything launches.
  if (start < 0 || start + Snew > capacity)
    return set_error(KF_EINVAL, "%s: append range exceeds cache capacity (%s %lld + %lld new "
                     "tokens > capacity %lld)", what, start_dev ? "max start" : "start",
                     (long long)start, (long long)Snew, (long long)capacity);
  if (B > 0x7fffffff || H > 0x7fffffff || Snew > 0x7fffffff || D > 0x7fffffff)
    return set_error(KF_EUNSUPPORTED, "%s: dimension too large", what);
  AppendParams p{};
  p.kc = (uint16_t*)k_cache; p.vc = (uint16_t*)v_cache;
  p.nk = (const uint16_t*)new_k; p.nv = (const uint16_t*)new_v;
  p.start_dev = start_dev; p.start = start;
  p.kc_sb = k_cache_strides[0]; p.kc_sh = k_cache_strides[1]; p.kc_ss = k_cache_strides[2];
  p.vc_sb = v_cache_strides[0]; p.vc_sh = v_cache_strides[1]; p.vc_ss = v_cache_strides[2];
  p.nk_sb = new_k_strides4[0]; p.nk_sh = new_k_strides4[1]; p.nk_ss = new_k_strides4[2]; p.nk_sd = new_k_strides4[3];
  p.nv_sb = new_v_strides4[0]; p.nv_sh = new_v_strides4[1]; p.nv_ss = new_v_strides4[2]; p.nv_sd = new_v_strides4[3];
  p.B = (int)B; p.H = (int)H; p.S = (int)Snew; p.D = (int)D;
  bool vec = D % 8 == 0 && p.nk_sd == 1 && p.nv_sd == 1 && aligned16(k_cache) && aligned16(v_cache) &&
             aligned16(new_k) && aligned16(new_v);
  const int64_t s8[] = {p.kc_sb, p.kc_sh, p.kc_ss, p.vc_sb, p.vc_sh, p.vc_ss,
                        p.nk_sb, p.nk_sh, p.nk_ss, p.nv_sb, p.nv_sh, p.nv_ss};
  for (int64_t s : s8) vec = vec && (s % 8 == 0);
  p.total = B * H * Snew * (vec ? D / 8 : D);
  const int64_t blocks = (p.total + 255) / 256;
  if (blocks > 0x7fffffff) return set_error(KF_EUNSUPPORTED, "%s: grid too large", what);
  hipStream_t s = (hipStream_t)stream;
  if (vec)
    hipLaunchKernelGGL((append_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((append_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, s, p);
  return check_launch(what);
}
