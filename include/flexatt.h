/*
 * flexatt.h — C ABI of the MI355X (gfx950) flash-attention library
 * (libflexatt.so).
 *
 * The reference (dropletzhu/npu-flex-att) has no C ABI: its host wrappers in
 * npu_flash_attention.py launch Triton kernels directly.  Each entry point
 * below replaces one such launch (or one torch op of the wrapper) and is what
 * a foreign-function binding of that wrapper calls; the Python host layer of
 * this repository binds them with ctypes.
 *
 * Conventions
 *  - Tensors are 4-D [B, H, S, D] views: a device pointer plus element
 *    strides.  The innermost stride must be 1 and every row must start on a
 *    16-byte boundary (data pointer and the b/h/s strides times the element
 *    size are multiples of 16 bytes).  Batch and head strides may be 0
 *    (broadcast).
 *  - q, o, dout and dq have shape [B, Hq, Sq, D]; k, v, dk and dv have shape
 *    [B, Hkv, Skv, D]; Hq is a multiple of Hkv and query head h reads KV head
 *    h / (Hq / Hkv).
 *  - lse and delta are contiguous fp32 [B, Hq, Sq]; lse is the natural-log
 *    log-sum-exp of the masked, scaled (and soft-capped, ALiBi-biased) scores.
 *  - All work is enqueued on `stream` (a hipStream_t; NULL = the null
 *    stream) and is asynchronous.  Nothing is allocated or freed: the caller
 *    owns every buffer (flexatt_fwd_decode_noalloc alone uses a fixed
 *    library-owned device buffer instead of a workspace argument).  Results
 *    are bitwise deterministic.
 *  - Return value: FLEXATT_OK, a negative FLEXATT_E* code for a rejected
 *    argument (nothing is launched), or a positive hipError_t from a launch.
 */
#ifndef FLEXATT_H_
#define FLEXATT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of q/k/v/o/dout/dq/dk/dv. */
enum flexatt_dtype { FLEXATT_F32 = 0, FLEXATT_F16 = 1, FLEXATT_BF16 = 2 };

/* Status codes (negative: argument rejected before any launch). */
enum flexatt_status {
  FLEXATT_OK = 0,
  FLEXATT_EINVAL = -1,     /* null pointer, non-positive size, bad flag */
  FLEXATT_EDTYPE = -2,     /* unknown dtype */
  FLEXATT_EHEADDIM = -3,   /* head_dim not in {32, 64, 128, 256} */
  FLEXATT_ESHAPE = -4,     /* heads_q % heads_kv != 0, or sizes overflow */
  FLEXATT_ELAYOUT = -5,    /* innermost stride != 1 or a row not 16-byte aligned */
  FLEXATT_ERANGE = -6,     /* problem outside an entry point's range (see its comment) */
  FLEXATT_ESCRATCH = -7    /* problem needs more than the fixed scratch buffer of a no-alloc entry point */
};

/* One [B, H, S, D] tensor: device pointer and element strides. */
typedef struct flexatt_tensor {
  void* data;
  int64_t stride_b, stride_h, stride_s, stride_d;
} flexatt_tensor;

/* The attention problem: sizes and the mask primitives.
 * npu_flash_attention.py:606-616 (forward signature) and :659-668 (backward)
 * carry the same fields as Python arguments; block_m / block_n are tiling
 * hints there and have no counterpart here. */
typedef struct flexatt_problem {
  int32_t dtype;          /* enum flexatt_dtype */
  int32_t batch;          /* B */
  int32_t heads_q;        /* Hq */
  int32_t heads_kv;       /* Hkv */
  int32_t seqlen_q;       /* Sq */
  int32_t seqlen_kv;      /* Skv (any value >= 1; no tile-multiple requirement) */
  int32_t head_dim;       /* D in {32, 64, 128, 256} */
  float scale;            /* softmax scale (the caller applies the 1/sqrt(D) default) */
  int32_t causal;         /* 1: keep j <= i (top-left aligned) */
  int32_t sliding_window; /* W > 0: keep i - j <= W; 0: off */
  float soft_cap;         /* c > 0: x -> c * tanh(x / c); 0: off */
  const float* alibi_slopes; /* device fp32 [Hq]: x += slope[h] * (i - j); NULL: off */
  /* Interval masks (no counterpart in the reference, which lists document
   * masking and PrefixLM as future work, README.md:219, DESIGN.md:374):
   * device int32 [B, Sq, 2] holding, for query row i of batch b, the range
   * [lo, hi) of keys it may attend, on top of the other primitives.  Both
   * bounds must be non-decreasing in i.  A document mask is symmetric: the
   * range of positions of i's document (then col_bounds may stay NULL and
   * seqlen_q == seqlen_kv).  NULL: off. */
  const int32_t* doc_bounds;
  /* The transpose of doc_bounds for a mask that is not symmetric (PrefixLM):
   * device int32 [B, Skv, 2], for key j the range [lo, hi) of query rows
   * that may attend it, both non-decreasing in j; it must describe the same
   * mask as doc_bounds.  NULL: doc_bounds is symmetric and read as both. */
  const int32_t* col_bounds;
  /* Block-sparse mask (the reference lists the block-sparse BlockMask index
   * format as unsupported, README.md:198): device uint8 [B, block_heads,
   * ceil(Sq / 128), ceil(Skv / 128)]; a zero entry removes the 128 x 128
   * block of (query rows, keys) from the attention of those heads, on top of
   * the other primitives.  block_heads is 1 (one map for every head) or
   * heads_q; ceil(Skv / 128) <= 2048.  NULL: off. */
  const uint8_t* block_map;
  int32_t block_heads;
  int32_t reserved; /* 0 */
} flexatt_problem;

/* Forward: o = softmax(mask(score(q k^T))) v and lse.
 * Replaces the flash_attn_fwd_kernel launch of npu_flash_attention_forward,
 * npu_flash_attention.py:634-652. */
int flexatt_fwd(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* stream);

/* Split-KV decode forward (flash-decoding): the results of flexatt_fwd for
 * problems with few query rows per KV head, computed by splitting the KV
 * range over many workgroups.  Range: fp16/bf16, head_dim <= 128 and
 * (heads_q / heads_kv) * seqlen_q <= 32; otherwise FLEXATT_ERANGE.
 * `workspace` is caller-owned device memory of at least
 * flexatt_fwd_decode_workspace(p) bytes, 16-byte aligned; it holds partial
 * results between the two kernels of this call and may be reused once the
 * call's work on `stream` is done.  Same o / lse as flexatt_fwd up to the
 * rounding of a different summation order; bitwise deterministic.
 * Replaces the unused split-KV pair flash_attn_fwd_split_kv_kernel /
 * flash_attn_fwd_reduce_kernel, npu_flash_attention.py:169-293. */
size_t flexatt_fwd_decode_workspace(const flexatt_problem* p); /* 0: outside the range */
int flexatt_fwd_decode(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                       const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Split-KV decode forward that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory or pass a
 * workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same kernels, split plan and results as
 * flexatt_fwd_decode (bitwise equal), with the partial results in a
 * library-owned device buffer of FLEXATT_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends; nothing is allocated or freed per call.
 * Range: that of flexatt_fwd_decode (else FLEXATT_ERANGE), and
 * flexatt_fwd_decode_workspace(p) <= FLEXATT_NOALLOC_SCRATCH_BYTES (else
 * FLEXATT_ESCRATCH, checked before any GPU work).  `stream` must belong to
 * the current device.  Every call on one GPU shares that GPU's buffer:
 * calls that overlap on one GPU (on different streams or host threads)
 * race, so the caller serialises them; calls in order on one stream are
 * safe (each one overwrites every partial it reads). */
#define FLEXATT_NOALLOC_SCRATCH_BYTES (16u << 20)
int flexatt_fwd_decode_noalloc(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                               const flexatt_tensor* v, const flexatt_tensor* o, float* lse, void* stream);

/* Backward pre-pass: delta[b,h,i] = sum_d o * dout in fp32.
 * Replaces the torch op at npu_flash_attention.py:681-685. */
int flexatt_bwd_delta(const flexatt_problem* p, const flexatt_tensor* o, const flexatt_tensor* dout,
                      float* delta, void* stream);

/* Backward dQ (needs lse and delta).
 * Replaces the flash_attn_bwd_dq_kernel launch, npu_flash_attention.py:695-712. */
int flexatt_bwd_dq(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                   const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse,
                   const float* delta, const flexatt_tensor* dq, void* stream);

/* Backward Delta and dQ in one pass where the dQ kernel can form Delta itself
 * (fp16/bf16, head_dim 64 or 128, no interval or block mask; otherwise the Delta
 * pass then dQ): delta (the caller's fp32 [B,Hq,Sq] buffer) receives sum_d o * dout,
 * for flexatt_bwd_dkdv after it.  Replaces the Delta op and the
 * flash_attn_bwd_dq_kernel launch of npu_flash_attention_backward,
 * npu_flash_attention.py:681-712. */
int flexatt_bwd_dq_delta(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                         const flexatt_tensor* v, const flexatt_tensor* o, const flexatt_tensor* dout,
                         const float* lse, float* delta, const flexatt_tensor* dq, void* stream);

/* Backward dK/dV with the GQA group sum folded in: dk/dv are [B, Hkv, Skv, D].
 * Replaces the flash_attn_bwd_dkdv_kernel launch plus the group sum,
 * npu_flash_attention.py:714-737. */
int flexatt_bwd_dkdv(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                     const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse,
                     const float* delta, const flexatt_tensor* dk, const flexatt_tensor* dv,
                     void* stream);

/* Whole backward: delta (into the caller's fp32 [B,Hq,Sq] `delta` buffer)
 * and dQ (flexatt_bwd_dq_delta), then dK/dV.  Replaces the kernel launches and torch ops of
 * npu_flash_attention_backward, npu_flash_attention.py:659-739. */
int flexatt_bwd(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                const flexatt_tensor* v, const flexatt_tensor* o, const flexatt_tensor* dout,
                const float* lse, float* delta, const flexatt_tensor* dq, const flexatt_tensor* dk,
                const flexatt_tensor* dv, void* stream);

/* Bytes of work-queue counters at the end of the staged-dS workspace. */
#define FLEXATT_BWD_QUEUE_BYTES 256

/* Backward with dS staged through HBM (fp16/bf16 at head_dim 64, 128 or
 * 256; fp32 at every head_dim).  The dK/dV kernel already forms dS
 * for every attended pair; it writes those values (rounded to the input
 * dtype, as its own dK MFMAs consume them) to a caller-owned workspace, and
 * the dQ kernel forms dQ = scale * dS K from them instead of recomputing S
 * and dP.  The workspace holds 2 bytes (fp32: 4 bytes) per attended (query
 * row, KV row) pair of each query head, in 32 x 128 units over the causal /
 * window band (interval and block masks keep that band; masked pairs hold
 * zeros, and the units of removed 128 x 128 blocks are neither written nor
 * read), followed by FLEXATT_BWD_QUEUE_BYTES of
 * work-queue counters:
 * flexatt_bwd_workspace(p) bytes in all (0: the problem is outside this
 * range), 16-byte aligned, not zeroed, reusable once the call's work on
 * `stream` is done.  Same results as flexatt_bwd up to fp32 summation
 * order; bitwise deterministic.
 *
 * flexatt_bwd_ws: the whole backward (replaces the Delta op, both kernel
 * launches and the group sum of npu_flash_attention_backward,
 * npu_flash_attention.py:681-737): the Delta pass into `delta`, dK/dV
 * writing dS, then dQ.  Past the first workgroup per CU, the dK/dV and dQ
 * workgroups take the longest remaining work items from the queue counters
 * (which the Delta pass clears), so that faster XCDs take more work (fp16/
 * bf16); with a workspace of only the dS band's size the static order is
 * kept.  Outside
 * the range it runs flexatt_bwd and the workspace may be NULL.
 *
 * Bounded memory.  The band grows as Sq * Skv (about 1 byte per (query row,
 * KV row) pair of each query head for causal fp16/bf16, 1.1 GB at B=2 Hq=32
 * S=4096), while the reference's backward needs O(S) memory
 * (npu_flash_attention.py:675-685).  flexatt_bwd_ws therefore also accepts:
 *  - a workspace smaller than the whole band but holding the band of at
 *    least one (batch, KV head) group (G = heads_q / heads_kv query heads):
 *    the staged backward then runs in passes over chunks of whole groups
 *    (whole batches when one fits, else KV heads of one batch), reusing the
 *    workspace pass after pass on `stream`; smaller: FLEXATT_EINVAL;
 *  - workspace == NULL with workspace_bytes == 0: the recomputing backward
 *    (flexatt_bwd), O(S) memory.
 * flexatt_bwd_workspace_limited(p, limit) is the size to allocate under a
 * byte budget: the whole band (plus the queue counters) when it fits, else
 * the most whole groups that fit, else 0 (no staging: pass NULL, 0).  Passes
 * give the same results as one pass up to fp32 summation order. */
size_t flexatt_bwd_workspace(const flexatt_problem* p);
size_t flexatt_bwd_workspace_limited(const flexatt_problem* p, size_t limit_bytes);
/* Whether staging pays for p: 1 when p is in the staged range and the staged
 * backward measured faster than the recomputing one on MI355X, 0 otherwise
 * (out of range, or fp16/bf16 at head_dim 64 without soft-cap and without
 * document, prefix or block-map masks, where the recomputing backward is
 * 2-15% faster).  Advisory: flexatt_bwd_ws stages whenever it is given a
 * workspace.  No counterpart in the reference, which has one backward. */
int flexatt_bwd_prefers_staging(const flexatt_problem* p);
int flexatt_bwd_ws(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                   const flexatt_tensor* v, const flexatt_tensor* o, const flexatt_tensor* dout,
                   const float* lse, float* delta, const flexatt_tensor* dq, const flexatt_tensor* dk,
                   const flexatt_tensor* dv, void* workspace, size_t workspace_bytes, void* stream);

/* The two kernels of flexatt_bwd_ws on their own (FLEXATT_ERANGE outside
 * its range).  flexatt_bwd_dkdv_ds replaces the flash_attn_bwd_dkdv_kernel
 * launch and the group sum (npu_flash_attention.py:714-737) and also fills
 * the workspace; flexatt_bwd_dq_ds replaces the flash_attn_bwd_dq_kernel
 * launch (:695-712) and reads the workspace a flexatt_bwd_dkdv_ds call on
 * the same problem wrote before it on the stream.  Both keep the static work
 * order (the queue counters are not used). */
int flexatt_bwd_dkdv_ds(const flexatt_problem* p, const flexatt_tensor* q, const flexatt_tensor* k,
                        const flexatt_tensor* v, const flexatt_tensor* dout, const float* lse,
                        const float* delta, const flexatt_tensor* dk, const flexatt_tensor* dv,
                        void* workspace, size_t workspace_bytes, void* stream);
int flexatt_bwd_dq_ds(const flexatt_problem* p, const flexatt_tensor* k, const void* workspace,
                      size_t workspace_bytes, const flexatt_tensor* dq, void* stream);

/* Human-readable text for a status code (static storage). */
const char* flexatt_status_string(int status);

/* ABI version of this header (bumped on any signature change). */
int flexatt_abi_version(void);

#define FLEXATT_ABI_VERSION 8

#ifdef __cplusplus
}
#endif

#endif /* FLEXATT_H_ */
