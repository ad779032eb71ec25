/*
 * flashattn_hip.h — C ABI of the MI355X (gfx950) FlashAttention library
 * (libflashattn_hip.so).
 *
 * The ABI carries plain device pointers, sizes and a HIP stream handle. It
 * has no torch types, so ctypes, cgo, JNI or a C++ host can bind it directly.
 * The Python package `flashattn_cuda` wraps it with the reference's
 * pybind11 surface (`prefill`, `decode`, `_decode_with_split`,
 * `choose_decode_split`, `occupancy_report`, `head_dim`, `legacy_naive`,
 * `legacy_tiled`, `legacy_fused`).
 *
 * Reference interface that each entry point replaces
 * (paths relative to shrvan30/flash-attention-cuda):
 *   fa_head_dim              <- kHeadDim          csrc/flash_common.h:11,
 *                                                 bindings.cpp:112 (m.attr)
 *   fa_choose_decode_split   <- choose_decode_split  csrc/decode.cu:183-192,
 *                                                 bindings.cpp:122-125
 *   fa_decode_min_blocks     <- min_blocks = 2 * multiProcessorCount
 *                                                 csrc/decode.cu:205-206
 *   fa_prefill_workspace_bytes, fa_prefill
 *                            <- launch_prefill    csrc/prefill.cu:347-373
 *                               (called by prefill, bindings.cpp:10-27)
 *   fa_decode_workspace_bytes, fa_decode
 *                            <- launch_decode     csrc/decode.cu:194-240
 *                               (called by decode_impl, bindings.cpp:36-76)
 *   fa_occupancy_report      <- prefill_occupancy / decode_occupancy
 *                               csrc/prefill.cu:375-394, csrc/decode.cu:242-261
 *   fa_prefill_gqa, fa_decode_gqa_workspace_bytes, fa_decode_gqa
 *                            <- no counterpart: kernel-side grouped-query
 *                               attention is future work in the reference
 *                               (README.md:398); its callers repeat K/V per
 *                               query head and call prefill / decode.
 *   fa_kv_append             <- no counterpart: the cache write its caller
 *                               (the FlashStack engine, README.md:9-13) does
 *                               before each decode step.
 *   fa_prefill_hd, fa_decode_hd_workspace_bytes, fa_decode_hd, fa_kv_append_hd
 *                            <- no counterpart: head_dim 128 is named future
 *                               work in the reference (README.md:230, :397);
 *                               with head_dim 64 they are fa_prefill_gqa /
 *                               fa_decode_gqa / fa_kv_append.
 *   fa_decode_hd_noalloc     <- no counterpart: fa_decode_hd without a workspace
 *                               argument, for callers that cannot allocate.
 *   fa_prefill_plan_units    <- no counterpart: reads this build's prefill work-unit
 *                               plan (tests, tools); launches nothing.
 *   fa_legacy_attention      <- launch_naive_attention / launch_tiled_attention /
 *                               launch_fused_attention,
 *                               src/legacy/{naive,tiled,fused}_attention.cu
 *                               (called by legacy_naive / legacy_tiled /
 *                               legacy_fused, csrc/legacy/legacy_ops.cu:38-51)
 *
 * Tensor layout (same as the reference): q, k, v, o are [B, H, S, 64]
 * contiguous fp16 (IEEE binary16); a decode cache is [B, H, Lmax, 64]; the
 * decode query and output are [B, H, 1, 64]; seq_lens is [B] int32 in device
 * memory. The *_hd entry points take the head size (64 or 128) as an
 * argument and the same layouts with that last dimension; the legacy entry
 * point takes (n, 64) fp32 rows. Every pointer must be a device pointer
 * aligned to 16 bytes.
 *
 * Launches are asynchronous on `stream` (a hipStream_t; NULL is the default
 * stream) and never synchronise the host. A non-zero return value is an
 * fa_status; fa_last_error() then returns a message for the calling thread.
 */
#ifndef FLASHATTN_HIP_H_
#define FLASHATTN_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_HEAD_DIM 64
#define FA_DECODE_SPLIT_MIN 128  /* csrc/flash_common.h:21 */
#define FA_DECODE_SPLIT_MAX 1024 /* csrc/flash_common.h:22 */

typedef enum fa_status {
  FA_OK = 0,
  FA_ERR_INVALID_ARGUMENT = 1, /* bad size, pointer, alignment or scale */
  FA_ERR_WORKSPACE = 2,        /* workspace missing or too small */
  FA_ERR_HIP = 3               /* a HIP runtime call or launch failed */
} fa_status;

/* Output element type. FA_OUT_F16 is the public contract; FA_OUT_F32 writes
 * the same kernels' fp32 result before the final rounding (a parity hook). */
typedef enum fa_out_dtype { FA_OUT_F16 = 0, FA_OUT_F32 = 1 } fa_out_dtype;

/* One row of the occupancy report (bindings.cpp:80-97 dict keys). */
typedef struct fa_occupancy_entry {
  char kernel[64];
  int threads_per_block;
  int registers_per_thread;
  int shared_bytes_per_block;
  int max_active_blocks_per_sm;
  double theoretical_occupancy;
} fa_occupancy_entry;

/* Library version string, e.g. "2.0.0-gfx950". */
const char *fa_version(void);

/* The reference's head size, 64 (the entry points without a head_dim
 * argument use it; the *_hd ones also take 128). */
int fa_head_dim(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char *fa_last_error(void);

/* Largest power-of-two chunk C in [128, 1024] with
 * batch * heads * ceil(max_seq / C) >= min_blocks, else 128. Pure integer
 * function of its arguments. */
int fa_choose_decode_split(int max_seq, int batch, int heads, int min_blocks);

/* Split-K unit target the automatic chunk choice uses on `device`:
 * 2 * (compute units), as the reference. Returns an fa_status. */
int fa_decode_min_blocks(int device, int *min_blocks);

/* Bytes of device workspace that let fa_prefill (and the _gqa / _hd entry
 * points, sized for head_dim 128) split the heaviest query tiles' key ranges
 * over two CUs for this shape on the current device; 0 when the shape gains
 * nothing. Every prefill entry point also runs with no workspace. */
size_t fa_prefill_workspace_bytes(int batch, int heads, int seq, int causal);

/* No counterpart in the reference (it inspects this build's host planner,
 * for tests and tools): the work units a prefill of batch_heads = B * H
 * query heads, K/V grouping `group` (H / H_kv), would run on a device of `cu`
 * compute units when given its workspace. *n_blocks = 0 means no plan (every
 * item runs whole). Otherwise block b runs units[2 b] and then units[2 b + 1]
 * (0xffffffff: none), each pos | code << 20 | split << 22: item pos (query
 * tile n_qtiles - 1 - pos / batch_heads), code 0 for all its keys, 1 / 2 for
 * the first / second key chunk, split < *n_splits its partial slot. Writes at
 * most `cap` entries. Needs no GPU. */
int fa_prefill_plan_units(int batch_heads, int seq, int causal, int head_dim, int group, int cu,
                          unsigned *units, int cap, int *n_blocks, int *n_splits);

/* o = softmax(q k^T * scale [+ causal mask]) v for every (b, h).
 * causal: query row i attends keys 0..i. fp32 accumulation throughout.
 * workspace may be NULL when fa_prefill_workspace_bytes(...) is 0. */
int fa_prefill(const void *q, const void *k, const void *v, void *o,
               int out_dtype, int batch, int heads, int seq, int causal,
               float scale, void *workspace, size_t workspace_bytes,
               void *stream);

/* Bytes of device workspace fa_decode needs. split_size 0 selects the chunk
 * the same way fa_decode does (it queries the current device). Returns 0
 * with fa_last_error() empty when the call needs no workspace (the
 * whole-sequence kernel, which merges in LDS: B * H at least the device's
 * compute-unit count, or Lmax <= 512; fa_decode then accepts NULL), and 0
 * with fa_last_error() set on invalid arguments. */
size_t fa_decode_workspace_bytes(int batch, int heads, int max_seq,
                                 int split_size);

/* Single-query attention against a KV cache: sequence b attends cache rows
 * [0, min(seq_lens[b], max_seq)); a sequence with seq_lens[b] <= 0 gets a
 * zero output. split_size 0 chooses the split-K chunk automatically; a
 * positive value forces it and must be a multiple of 4. */
int fa_decode(const void *q, const void *k_cache, const void *v_cache,
              const int32_t *seq_lens, void *o, int out_dtype, int batch,
              int heads, int max_seq, float scale, int split_size,
              void *workspace, size_t workspace_bytes, void *stream);

/* Grouped-query attention: k and v (or the caches) are [B, H_kv, S, 64]
 * (or [B, H_kv, Lmax, 64]) with 0 < H_kv <= H and H % H_kv == 0; query head
 * h reads K/V head h / (H / H_kv), the pairing of
 * k.repeat_interleave(H / H_kv, dim=1). q and o keep H heads. With
 * kv_heads == heads these are fa_prefill / fa_decode; otherwise the result
 * equals theirs on the repeated K/V, which is never materialised (a K/V head
 * is read once for all of its query heads). Same rules for workspace,
 * split_size, streams and errors as the non-grouped entry points. */
int fa_prefill_gqa(const void *q, const void *k, const void *v, void *o,
                   int out_dtype, int batch, int heads, int kv_heads, int seq,
                   int causal, float scale, void *workspace,
                   size_t workspace_bytes, void *stream);

size_t fa_decode_gqa_workspace_bytes(int batch, int heads, int kv_heads,
                                     int max_seq, int split_size);

int fa_decode_gqa(const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, int out_dtype, int batch,
                  int heads, int kv_heads, int max_seq, float scale,
                  int split_size, void *workspace, size_t workspace_bytes,
                  void *stream);

/* KV-cache append, the caller step before a decode: for every batch row b
 * with 0 <= seq_lens[b] < max_seq, write k_new[b, h] / v_new[b, h]
 * ([B, H_kv, 1, 64]) into row seq_lens[b] of k_cache / v_cache
 * ([B, H_kv, max_seq, 64]) for every K/V head h, then set
 * seq_lens[b] += 1, all on the device (seq_lens is never read on the host).
 * Rows with seq_lens[b] < 0 or >= max_seq are left alone, lengths included.
 * The lengths live only in device memory, so an append + decode step has
 * the same arguments for every token and can be captured in a HIP graph. */
int fa_kv_append(void *k_cache, void *v_cache, const void *k_new,
                 const void *v_new, int32_t *seq_lens, int batch, int kv_heads,
                 int max_seq, void *stream);

/* head_dim 64 or 128: the entry points above with the head size as an
 * argument. Tensors are [B, H, S, head_dim] (prefill), [B, H_kv, Lmax,
 * head_dim] caches and [B, H, 1, head_dim] decode queries / outputs, with
 * kv_heads dividing heads. Same rules for workspace, split_size, streams and
 * errors; any other head_dim fails with FA_ERR_INVALID_ARGUMENT. */
int fa_prefill_hd(const void *q, const void *k, const void *v, void *o,
                  int out_dtype, int batch, int heads, int kv_heads, int seq,
                  int head_dim, int causal, float scale, void *workspace,
                  size_t workspace_bytes, void *stream);

size_t fa_decode_hd_workspace_bytes(int batch, int heads, int kv_heads,
                                    int max_seq, int head_dim, int split_size);

int fa_decode_hd(const void *q, const void *k_cache, const void *v_cache,
                 const int32_t *seq_lens, void *o, int out_dtype, int batch,
                 int heads, int kv_heads, int max_seq, int head_dim, float scale,
                 int split_size, void *workspace, size_t workspace_bytes,
                 void *stream);

int fa_kv_append_hd(void *k_cache, void *v_cache, const void *k_new,
                    const void *v_new, int32_t *seq_lens, int batch,
                    int kv_heads, int max_seq, int head_dim, void *stream);

/* No counterpart in the reference: fa_decode_hd for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * hosts that forbid allocation). It takes no workspace and calls no
 * hipMalloc / hipFree: the split-K partials go to a scratch array of
 * FA_NOALLOC_SCRATCH_BYTES that the library holds on every device it runs on
 * until the process ends. A shape whose partials need more fails with
 * FA_ERR_WORKSPACE before anything is launched (fa_decode_hd_workspace_bytes
 * gives the need). Every call on one device shares that device's array and
 * leaves its contents behind: calls that overlap in time on one device
 * (several streams or threads) race, so the caller must serialise them.
 * Same arguments, rules and results as fa_decode_hd otherwise. */
#define FA_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)

int fa_decode_hd_noalloc(const void *q, const void *k_cache,
                         const void *v_cache, const int32_t *seq_lens, void *o,
                         int out_dtype, int batch, int heads, int kv_heads,
                         int max_seq, int head_dim, float scale, int split_size,
                         void *stream);

/* The reference's v1 single-head kernels: o = softmax(q k^T / sqrt(64)) v
 * for q, k, v, o of shape (n, 64) fp32, row-major, no mask. The three
 * variants compute the same function (results agree to fp32 rounding):
 * FA_LEGACY_NAIVE takes the exact row max in a first pass, FA_LEGACY_TILED
 * and FA_LEGACY_FUSED an online softmax (O renormalised per tile, resp.
 * divided once at the end). n == 0 launches nothing. Asynchronous on
 * `stream` like every other entry point (the v1 launchers synchronised). */
typedef enum fa_legacy_variant {
  FA_LEGACY_NAIVE = 0,
  FA_LEGACY_TILED = 1,
  FA_LEGACY_FUSED = 2
} fa_legacy_variant;

int fa_legacy_attention(const float *q, const float *k, const float *v,
                        float *o, int n, int variant, void *stream);

/* Fill up to `capacity` entries (one per kernel) for the current device;
 * *count receives the number of kernels. Returns an fa_status. */
int fa_occupancy_report(fa_occupancy_entry *out, int capacity, int *count);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FLASHATTN_HIP_H_ */
