// Internal declarations shared by the gfx950 HIP sources of libflashattn_hip.
//
// Everything here is CDNA4-specific: wave64, 32x32x16 fp16 MFMA fragments,
// DPP lane exchanges. Nothing is shared with, or adapted from, a CUDA path.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "flashattn_hip.h"

namespace fa {

constexpr int kHeadDim = FA_HEAD_DIM;
constexpr int kMaxDevices = 64;  // per-device host caches
// Split-K scratch that fa_decode_hd_noalloc keeps per device (8 MiB).
constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;
constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// MFMA fragment types for v_mfma_f32_32x32x16_f16: 8 halves in (A or B),
// 16 fp32 accumulators out (a 32x32 tile over the 64 lanes).
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---- host-side status plumbing (runtime.hip) -------------------------------
// Record `msg` as the calling thread's last error and return `code`.
int set_error(int code, const char *fmt, ...);
void clear_error();
// Check a HIP runtime result; on failure record it and return FA_ERR_HIP.
int check_hip(hipError_t err, const char *what);
// Compute-unit count of `device`, cached per device (0 on failure).
int device_cu_count(int device);

// ---- kernel launchers (prefill.hip / decode.hip) ---------------------------
// kv_heads divides heads; query head h reads K/V head h / (heads / kv_heads).
// head_dim is 64 or 128.
// workspace (may be NULL): prefill_workspace_bytes(...) bytes let the launch
// split the heaviest items' key ranges over more CUs (with less, it does not).
int launch_prefill(const void *q, const void *k, const void *v, void *o,
                   bool out_f32, int batch, int heads, int kv_heads, int seq,
                   int head_dim, bool causal, float scale, void *workspace,
                   size_t workspace_bytes, hipStream_t stream);
// Workspace that lets launch_prefill split items for this shape on the
// current device (either head size), 0 when it would not split.
size_t prefill_workspace_bytes(int batch, int heads, int seq, bool causal);
// The host's unit plan for a prefill shape on a `cu`-CU device (fa_prefill_plan_units).
int prefill_plan_units(int bh, int seq, int causal, int head_dim, int group, int cu,
                       unsigned *units, int cap, int *n_blocks, int *n_splits);
// head_dim is 64 or 128; grouped queries take the matrix-core grouped pass
// and the merge, the others the VALU split-K / whole-sequence kernels.
int launch_decode(const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, bool out_f32, int batch,
                  int heads, int kv_heads, int max_seq, int head_dim, float scale,
                  int split_size, bool auto_split, float *workspace, hipStream_t stream);
// Whether launch_decode writes split-K partials to its workspace for this
// shape on the current device: the whole-sequence kernel (no grouped queries,
// B * H >= CUs or a short cache) merges in LDS and needs none.
bool decode_needs_workspace(int batch, int heads, int kv_heads, int max_seq);
// Counter slot (kMergeCountersPerSlot zeroed counters) of the current device
// for kernels launched on `stream` (and, under graph capture, that capture),
// claimed on first use and kept; nullptr when `n` counters exceed a slot,
// every slot is taken, or `stream` is hipStreamPerThread / hipStreamLegacy.
// Kernels that count arrivals in it set each counter back to zero before
// they end (decode.hip).
constexpr size_t kMergeCountersPerSlot = 4096;
unsigned *merge_counters(hipStream_t stream, size_t n);
// Decode work units per batch row: one per head without grouped queries,
// else one per (K/V head, chunk of up to 32 of its query heads).
int decode_units_per_row(int heads, int kv_heads);
// Automatic chunk (cache rows per split) of the grouped-query decode pass:
// the batch's max_seq-row work over the waves the GPU runs at once, in
// multiples of 32 rows, at least 64.
int decode_group_chunk(int batch, int units_per_row, int max_seq, int head_dim);

// Writes k_new / v_new ([B, H_kv, 1, 64]) at row seq_lens[b] of the caches
// and advances seq_lens[b] (kv_cache.hip).
int launch_kv_append(void *k_cache, void *v_cache, const void *k_new, const void *v_new,
                     int32_t *seq_lens, int batch, int kv_heads, int max_seq, int head_dim,
                     hipStream_t stream);

// o = softmax(q k^T / 8) v for one (n, 64) fp32 head, no mask; variant is an
// fa_legacy_variant (legacy.hip).
int launch_legacy_attention(const float *q, const float *k, const float *v, float *o, int n,
                            int variant, hipStream_t stream);

// Occupancy rows for each kernel (appended to `out`, at most `cap` rows).
int prefill_occupancy(fa_occupancy_entry *out, int cap, int *n);
int decode_occupancy(fa_occupancy_entry *out, int cap, int *n);
int fill_occupancy_row(fa_occupancy_entry *row, const char *name,
                       const void *func, int threads, int dyn_smem);

// ---- device helpers --------------------------------------------------------
// DPP lane permutations (gfx9 dpp_ctrl encodings). `bound_ctrl` is set so an
// invalid source lane reads 0; every pattern used here stays inside its row.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                         0xF, 0xF, true));
}
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i inside 8 lanes
constexpr int kDppRowMirror = 0x140;  // lane i <-> 15 - i inside 16 lanes

// Sum over each aligned group of 8 lanes; every lane gets the group total.
__device__ __forceinline__ float sum_lanes8(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppHalfMirror>(x);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

}  // namespace fa
