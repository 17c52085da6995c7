/*
 * kotflash_amd C ABI: the drop-in boundary of the attention hot path.
 *
 * One shared library (kotflash_amd/libkotflash_amd.so, gfx950 code objects)
 * exports these entry points. They replace the reference's host launcher layer
 * (the Python functions that allocate outputs and launch Triton kernels) and its
 * pybind11 K/V append op. Conventions, kept from the reference launchers:
 *
 *  - every tensor pointer is a device pointer owned by the caller (torch);
 *    inputs are borrowed, outputs and workspaces are caller-allocated;
 *  - tensors are [batch, heads, sequence, head_dim] with a unit head_dim
 *    stride; the other three strides are given in elements, as int64_t[3]
 *    {batch, head, sequence}; 16-byte aligned base pointers and strides that are
 *    multiples of 8 elements are required (KF_EINVAL otherwise);
 *  - head_dim D is a multiple of 8 in [8, 128]; the GQA map is
 *    kv_head = q_head / (Hq / Hkv) (contiguous groups, repeat_interleave);
 *  - causal masking is upper-left: key j is visible to query i iff j <= i;
 *  - LSE is the natural-log row log-sum-exp in fp32, contiguous [B, Hq, Sq];
 *  - launches are asynchronous on the given HIP stream of the current device;
 *    nothing here allocates device memory, synchronizes or is thread-safe
 *    with respect to concurrent use of the same output buffers;
 *  - the return value is KF_OK (0) or a KF_E* code; kf_last_error() then
 *    holds a message for the calling thread.
 */
#ifndef KOTFLASH_AMD_H_
#define KOTFLASH_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_ABI_VERSION 6

enum kf_status {
  KF_OK = 0,
  KF_EINVAL = 1,       /* invalid argument (shape, stride, alignment, pointer) */
  KF_EUNSUPPORTED = 2, /* valid but outside what the kernels implement */
  KF_ELAUNCH = 3       /* HIP reported a launch failure */
};

enum kf_dtype { KF_F16 = 0, KF_BF16 = 1 };

/* Message for the last failing call on this thread. */
const char* kf_last_error(void);
/* KF_ABI_VERSION of the loaded library. */
int kf_abi_version(void);

/*
 * Attention forward: O = softmax(scale * Q K^T + mask) V and its LSE.
 * Replaces attention_forward + _attention_fwd_kernel
 * (reference kotflash/kernels/triton_forward.py:372-456 and :20-165).
 * o has q's shape; lse is fp32 contiguous [B, Hq, Sq].
 */
int kf_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                const int64_t* o_strides, float scale, int causal, int dtype, void* stream);

/*
 * Workspace for kf_attn_bwd in bytes (fp32 row deltas and partial sums).
 */
size_t kf_attn_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                                   int64_t D, int causal);

/*
 * Attention backward: dQ, dK, dV from Q, K, V, O, LSE and dO. dK/dV are summed
 * over the Hq/Hkv query heads of each KV group. The row delta
 * rowsum(O * dO) is computed from the stored low-precision O.
 * Replaces attention_backward + _attention_bwd_dq/_dkv/_dkv_split/_dkv_reduce
 * (reference kotflash/kernels/triton_backward.py:335-421, :17-332).
 * dq/dk/dv have q/k/v's shapes; strides are int64_t[3] like the inputs.
 */
int kf_attn_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
                const void* dout, void* dq, void* dk, void* dv, int64_t B, int64_t Hq,
                int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides,
                const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                const int64_t* do_strides, const int64_t* dq_strides, const int64_t* dk_strides,
                const int64_t* dv_strides, float scale, int causal, int dtype, void* workspace,
                size_t workspace_bytes, void* stream);

/*
 * The launches of kf_attn_bwd, selectable by a mask of KF_BWD_* bits and run
 * in the order delta, dq, dkdv, dkdv fixup: the delta stage writes the fp32 row
 * deltas into the workspace (dq and dkdv read them); dkdv writes dK/dV of
 * tiles it finishes alone and fp32 partials of shared tiles into the
 * workspace; the fixup completes dK/dV from those partials. kf_attn_bwd is
 * this call with KF_BWD_ALL. Same launch split as the reference backward,
 * whose dQ and dK/dV kernels are separate launches
 * (triton_backward.py:374-419); used to time each kernel on its own.
 */
enum kf_bwd_stage {
  KF_BWD_DELTA = 1,
  KF_BWD_DQ = 2,
  KF_BWD_DKDV = 4,
  KF_BWD_DKDV_FIXUP = 8,
  KF_BWD_ALL = 15
};
int kf_attn_bwd_stages(int stages, const void* q, const void* k, const void* v, const void* o,
                       const float* lse, const void* dout, void* dq, void* dk, void* dv,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                       const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides,
                       const int64_t* do_strides, const int64_t* dq_strides,
                       const int64_t* dk_strides, const int64_t* dv_strides, float scale,
                       int causal, int dtype, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * Number of KV splits the gfx950 decode planner picks for a short-query,
 * long-cache problem: about one workgroup per CU, each split a whole number of
 * 128-key granules. kf_attn_decode accepts any count whose chunk (rounded up
 * to whole granules) partitions Sk into exactly that many splits.
 */
int kf_decode_num_splits(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D);

/*
 * The same for a ragged batch whose visible lengths are known on the host
 * (lengths: B entries; Sk of the kf_attn_decode call is max(lengths)). The
 * chunk is sized from the total visible keys, so that the non-empty splits of
 * short and long sequences fill the GPU evenly; splits beyond a sequence's
 * length are empty and cheap. No reference counterpart: the reference's cache
 * has one scalar length (kotflash/cache.py:122) and its planner one Sk
 * (kotflash/_planning.py:25-34).
 */
int kf_decode_num_splits_ragged(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                const int32_t* lengths, int64_t D);

/* Workspace for kf_attn_decode in bytes (fp32 partial O and LSE per split);
 * 0 when num_splits == 1. */
size_t kf_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                                 int num_splits);

/*
 * Split-KV decode, non-causal: every query row sees keys [0, L_b) of its
 * batch entry, L_b = seqlens_k[b] (device int32, nullable: L_b = Sk for all b).
 * K/V may be strided prefix views of a larger cache (sequence stride >= D).
 * Each workgroup reads one KV chunk of one (batch, kv_head) once for all
 * Hq/Hkv * Sq query rows and writes an fp32 (O, LSE) partial into the
 * workspace; a second launch merges the partials with LSE weights (one launch
 * when num_splits == 1). lse is nullable.
 * Replaces attention_forward_strided_decode + _strided_decode_split /
 * _strided_decode_reduce (reference kotflash/kernels/triton_decode.py:412-468,
 * :16-104, :241-297) and the split-KV branch of attention_forward
 * (triton_forward.py:410-445, kernels :169-349).
 */
int kf_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse,
                   const int32_t* seqlens_k, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                   int64_t Sk, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides, float scale,
                   int num_splits, int dtype, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * LSE-weighted merge of split-KV partials computed elsewhere, e.g. by the
 * GPUs of a sequence-sharded decode or by a caller's own split kernel:
 *   O[b,h,i,:] = sum_s w_s part_o[s,b,h,i,:],  w_s = exp(LSE_s - M) / sum_t exp(LSE_t - M),
 *   LSE[b,h,i] = M + ln(sum_t exp(LSE_t - M)),  M = max_s LSE_s,
 * with a row whose splits are all empty (LSE_s = -inf) giving O = 0 and
 * LSE = -inf. part_o is fp32 contiguous [num_splits, B, H, S, D] (16-byte
 * aligned), part_lse fp32 contiguous [num_splits, B, H, S] (natural log); o
 * is [B, H, S, D] in `dtype` with a unit head_dim stride, strides in
 * elements (multiples of 4, 8-byte aligned base); lse (nullable) fp32
 * contiguous [B, H, S]. D is a multiple of 4 up to 128. One launch, one wave
 * per output row. Replaces _attention_fwd_split_kv_reduce (reference
 * kotflash/kernels/triton_forward.py:269-349), the merge the reference runs
 * after its split kernel (:430-444); kf_attn_decode runs the same merge on
 * its own partials.
 */
int kf_lse_merge(const float* part_o, const float* part_lse, void* o, float* lse,
                 int64_t num_splits, int64_t B, int64_t H, int64_t S, int64_t D,
                 const int64_t* o_strides, int dtype, void* stream);

/*
 * kf_attn_decode without a workspace argument: it allocates nothing and
 * takes no caller memory beyond its inputs and outputs. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The split partials go to a static device array of
 * KF_DECODE_NOALLOC_SCRATCH_BYTES (32 MiB) that every GPU the library runs on
 * holds until the process ends; a problem whose partials need more
 * (kf_decode_workspace_bytes) is rejected with KF_EINVAL before any launch.
 * Every call on a GPU shares that GPU's array: calls that overlap in time on
 * one GPU (concurrent streams or threads) race. Same arguments, results and
 * errors as kf_attn_decode otherwise (bit-identical outputs for the same
 * num_splits).
 */
#define KF_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int kf_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, float* lse,
                           const int32_t* seqlens_k, int64_t B, int64_t Hq, int64_t Hkv,
                           int64_t Sq, int64_t Sk, int64_t D, const int64_t* q_strides,
                           const int64_t* k_strides, const int64_t* v_strides,
                           const int64_t* o_strides, float scale, int num_splits, int dtype,
                           void* stream);

/*
 * K/V cache append: cache[b, h, start_b + t, :] = new[b, h, t, :] for K and V
 * in one launch, bit-exact. start_b = start_dev[b] when start_dev (device
 * int64 [B]) is non-null, else the scalar start. With start_dev, `start` is
 * the host-side bound max_b start_dev[b]. Either way the call is rejected with
 * KF_EINVAL before any launch unless 0 <= start and start + Snew <= capacity,
 * as the reference rejects an out-of-range append (kv_append_cuda.cu:72-73);
 * a device start outside [0, start] breaks the caller's bound and its rows
 * are not written. new_k/new_v may have any strides
 * (int64_t[4], element units, including head_dim); the caches need a unit
 * head_dim stride.
 * Replaces append_kv_cuda / append_kv_ (reference
 * kotflash/csrc/kv_append_cuda.cu:12-96, kotflash/csrc/kv_append.cpp:11-14),
 * extended from one scalar start to per-sequence positions.
 */
int kf_kv_append(void* k_cache, void* v_cache, const void* new_k, const void* new_v,
                 const int64_t* start_dev, int64_t start, int64_t B, int64_t H, int64_t Snew,
                 int64_t D, int64_t capacity, const int64_t* k_cache_strides,
                 const int64_t* v_cache_strides, const int64_t* new_k_strides4,
                 const int64_t* new_v_strides4, int dtype, void* stream);

/*
 * Fused append + split-KV decode in one decode launch (plus the merge):
 * new tokens new_k/new_v [B, Hkv, Snew, D] are stored at cache positions
 * start_b .. start_b + Snew - 1, and query rows of batch entry b attend,
 * non-causally, to cache keys [0, start_b) followed by the Snew new keys,
 * i.e. to the first start_b + Snew positions of the cache after the append.
 * start_b = lengths[b] (device int32 [B], nullable: then start_b =
 * past_length for every b, and past_length must equal max_length).
 * max_length >= max_b start_b (host-side) sizes the splits over the old keys
 * (num_splits from kf_decode_num_splits / _ragged over those lengths; 0 keys
 * allowed); one more split reads the new tokens from their own buffer and a
 * single workgroup per (b, kv_head) writes them into the cache (bit-exact).
 * Workspace: kf_decode_workspace_bytes(..., num_splits + 1). The call is
 * rejected with KF_EINVAL before any launch unless max_length + Snew <=
 * capacity (the reference's capacity check, kv_append_cuda.cu:72-73, applied
 * to the host-side bound); a device length outside [0, max_length] breaks
 * that bound: it attends to max_length keys and its new tokens are not
 * written. Caches, q, new_k/new_v and o need a unit head_dim stride.
 * Replaces attention_forward_strided_append + _strided_decode_append_split
 * (reference kotflash/kernels/triton_decode.py:302-386, :108-238), which
 * folds one token's slot write into its split kernel; here Snew >= 1 tokens
 * and per-sequence positions.
 */
int kf_attn_append_decode(const void* q, void* k_cache, void* v_cache, const void* new_k,
                          const void* new_v, void* o, float* lse, const int32_t* lengths,
                          int64_t past_length, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                          int64_t Snew, int64_t max_length, int64_t capacity, int64_t D,
                          const int64_t* q_strides, const int64_t* k_cache_strides,
                          const int64_t* v_cache_strides, const int64_t* new_k_strides,
                          const int64_t* new_v_strides, const int64_t* o_strides, float scale,
                          int num_splits, int dtype, void* workspace, size_t workspace_bytes,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KOTFLASH_AMD_H_ */
