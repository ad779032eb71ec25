// C ABI of libflashattn_hip: argument checks, status codes, the split-K chunk
// chooser, device queries and the occupancy report. The kernels themselves
// live in prefill.hip and decode.hip.
//
// Argument checks mirror the pointer-level part of the reference's
// validation (csrc/bindings.cpp:12-22, :39-64; csrc/decode.cu:209-211). The
// tensor-level checks (device, dtype, contiguity, rank) belong to whoever
// holds tensors: the pybind11 layer in bindings.cpp for Python callers.

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "fa_internal.h"

// Split-K partials of fa_decode_hd_noalloc: one copy of this array per
// device, part of the library's code object, held until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host it names
// a stand-in, not device memory); it uses the address that
// hipGetSymbolAddress returns for the current device (device_scratch below).
static __device__ __align__(256) float scratch[fa::kNoAllocScratchBytes / sizeof(float)];

namespace fa {

static_assert(kNoAllocScratchBytes == FA_NOALLOC_SCRATCH_BYTES,
              "scratch size and its public constant agree");

namespace {
thread_local char g_last_error[512] = "";

// Longest KV cache decode accepts: row indices up to 8x this stay in int.
constexpr int kMaxCacheRows = 1 << 27;
std::once_flag g_cu_once[kMaxDevices];
int g_cu_count[kMaxDevices];

bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

std::once_flag g_scratch_once[kMaxDevices];
void *g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int device_scratch(void **ptr) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != FA_OK) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(FA_ERR_HIP, "device %d is beyond the %d devices the library tracks", dev,
                     kMaxDevices);
  std::call_once(g_scratch_once[dev], [dev] {
    void *p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = p;
  });
  rc = check_hip(g_scratch_err[dev], "hipGetSymbolAddress(scratch)");
  if (rc != FA_OK) return rc;
  if (g_scratch_ptr[dev] == nullptr)
    return set_error(FA_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
  *ptr = g_scratch_ptr[dev];
  return FA_OK;
}
}  // namespace

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_hip(hipError_t err, const char *what) {
  if (err == hipSuccess) return FA_OK;
  return set_error(FA_ERR_HIP, "%s failed: %s (%s)", what,
                   hipGetErrorString(err), hipGetErrorName(err));
}

int device_cu_count(int device) {
  if (device < 0 || device >= kMaxDevices) return 0;
  std::call_once(g_cu_once[device], [device] {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount,
                              device) != hipSuccess)
      cu = 0;
    g_cu_count[device] = cu;
  });
  return g_cu_count[device];
}

int fill_occupancy_row(fa_occupancy_entry *row, const char *name,
                       const void *func, int threads, int dyn_smem) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != FA_OK) return rc;
  hipFuncAttributes attr{};
  rc = check_hip(hipFuncGetAttributes(&attr, func), "hipFuncGetAttributes");
  if (rc != FA_OK) return rc;
  int blocks = 0;
  rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, func,
                                                              threads, dyn_smem),
                 "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  if (rc != FA_OK) return rc;
  int max_threads = 0;
  rc = check_hip(hipDeviceGetAttribute(
                     &max_threads,
                     hipDeviceAttributeMaxThreadsPerMultiProcessor, dev),
                 "hipDeviceGetAttribute");
  if (rc != FA_OK) return rc;
  std::memset(row, 0, sizeof(*row));
  std::snprintf(row->kernel, sizeof(row->kernel), "%s", name);
  row->threads_per_block = threads;
  row->registers_per_thread = attr.numRegs;
  row->shared_bytes_per_block = static_cast<int>(attr.sharedSizeBytes) + dyn_smem;
  row->max_active_blocks_per_sm = blocks;
  row->theoretical_occupancy =
      max_threads > 0 ? static_cast<double>(blocks) * threads / max_threads : 0.0;
  return FA_OK;
}

}  // namespace fa

using namespace fa;

extern "C" {

const char *fa_version(void) { return "2.0.0-gfx950"; }

int fa_head_dim(void) { return FA_HEAD_DIM; }

const char *fa_last_error(void) { return g_last_error; }

// csrc/decode.cu:183-192: the largest power-of-two chunk in [128, 1024] that
// still yields min_blocks split blocks; otherwise the smallest chunk.
int fa_choose_decode_split(int max_seq, int batch, int heads, int min_blocks) {
  const int64_t per_split = static_cast<int64_t>(batch) * heads;
  for (int split = FA_DECODE_SPLIT_MAX; split > FA_DECODE_SPLIT_MIN;
       split >>= 1) {
    const int64_t splits = (static_cast<int64_t>(max_seq) + split - 1) / split;
    if (per_split * splits >= min_blocks) return split;
  }
  return FA_DECODE_SPLIT_MIN;
}

// csrc/decode.cu:205-206: two split units per compute unit. The split-K path
// only serves B * H below the compute-unit count, where the longer chunks this
// target gives measured best (B1 H12 L32768: 25.0 us at 512-row chunks
// against 39.9 us at 128; short caches pick 128 either way).
constexpr int kDecodeUnitsPerCu = 2;

int fa_decode_min_blocks(int device, int *min_blocks) {
  clear_error();
  if (min_blocks == nullptr)
    return set_error(FA_ERR_INVALID_ARGUMENT, "min_blocks must not be NULL");
  const int cu = device_cu_count(device);
  if (cu <= 0)
    return set_error(FA_ERR_HIP, "could not query the compute-unit count of device %d",
                     device);
  *min_blocks = kDecodeUnitsPerCu * cu;
  return FA_OK;
}

size_t fa_prefill_workspace_bytes(int batch, int heads, int seq, int causal) {
  return prefill_workspace_bytes(batch, heads, seq, causal != 0);
}

int fa_prefill_plan_units(int batch_heads, int seq, int causal, int head_dim, int group, int cu,
                          unsigned *units, int cap, int *n_blocks, int *n_splits) {
  clear_error();
  return prefill_plan_units(batch_heads, seq, causal, head_dim, group, cu, units, cap, n_blocks,
                            n_splits);
}

namespace {
int check_groups(int heads, int kv_heads) {
  if (kv_heads <= 0 || kv_heads > heads || heads % kv_heads != 0)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "kv_heads must divide heads, got H=%d H_kv=%d", heads, kv_heads);
  return FA_OK;
}

int prefill_impl(const void *q, const void *k, const void *v, void *o, int out_dtype,
                 int batch, int heads, int kv_heads, int seq, int head_dim, int causal,
                 float scale, void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  if (head_dim != 64 && head_dim != 128)
    return set_error(FA_ERR_INVALID_ARGUMENT, "head_dim must be 64 or 128, got %d", head_dim);
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr)
    return set_error(FA_ERR_INVALID_ARGUMENT, "q, k, v and o must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "q, k, v and o must be 16-byte aligned device pointers");
  // The split units store their partials with coherent (atomic) stores; the
  // workspace takes the decode workspace's 16-byte rule.
  if (workspace != nullptr && !aligned16(workspace))
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "workspace must be a 16-byte aligned device pointer (or NULL)");
  if (out_dtype != FA_OUT_F16 && out_dtype != FA_OUT_F32)
    return set_error(FA_ERR_INVALID_ARGUMENT, "unknown out_dtype %d", out_dtype);
  if (batch <= 0 || heads <= 0)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "batch and heads must be > 0, got B=%d H=%d", batch, heads);
  int rc = check_groups(heads, kv_heads);
  if (rc != FA_OK) return rc;
  if (seq <= 0)
    return set_error(FA_ERR_INVALID_ARGUMENT, "sequence length must be > 0");
  if (static_cast<int64_t>(batch) * heads * ((static_cast<int64_t>(seq) + 127) / 128) >
      0x7fffffffll)
    return set_error(FA_ERR_INVALID_ARGUMENT, "batch * heads * seq too large");
  if (!std::isfinite(scale) || !std::isfinite(scale * 1.4426950408889634f))
    return set_error(FA_ERR_INVALID_ARGUMENT, "scale must be finite");
  return launch_prefill(q, k, v, o, out_dtype == FA_OUT_F32, batch, heads, kv_heads, seq,
                        head_dim, causal != 0, scale, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream));
}

// Resolves split_size 0 to the automatic choice; returns an fa_status.
// Without grouped queries that is the reference's chooser; with them, the
// grouped pass's own chunk (it has no reference counterpart).
int resolve_split(int batch, int heads, int kv_heads, int max_seq, int head_dim,
                  int *split_size) {
  if (*split_size < 0)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "decode split size must be >= 0, got %d", *split_size);
  if (*split_size == 0) {
    // The matrix-core grouped pass has its own chunk policy.
    if (kv_heads != heads) {
      *split_size = decode_group_chunk(batch, decode_units_per_row(heads, kv_heads), max_seq,
                                       head_dim);
      return FA_OK;
    }
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != FA_OK) return rc;
    int min_blocks = 0;
    rc = fa_decode_min_blocks(dev, &min_blocks);
    if (rc != FA_OK) return rc;
    *split_size = fa_choose_decode_split(max_seq, batch, heads, min_blocks);
  }
  // csrc/decode.cu:209-211.
  if (*split_size % 4 != 0)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "decode split size must be a multiple of the warp count, got %d",
                     *split_size);
  return FA_OK;
}

size_t decode_ws_bytes(int batch, int heads, int max_seq, int head_dim, int split) {
  const size_t n_splits = (static_cast<size_t>(max_seq) + split - 1) / split;
  return static_cast<size_t>(batch) * heads * n_splits * (head_dim + 2) * sizeof(float);
}

int check_head_dim(int head_dim) {
  if (head_dim != 64 && head_dim != 128)
    return set_error(FA_ERR_INVALID_ARGUMENT, "head_dim must be 64 or 128, got %d", head_dim);
  return FA_OK;
}

size_t decode_workspace_impl(int batch, int heads, int kv_heads, int max_seq, int head_dim,
                             int split_size) {
  clear_error();
  if (batch <= 0 || heads <= 0 || max_seq <= 0) {
    set_error(FA_ERR_INVALID_ARGUMENT, "batch, heads and max_seq must be > 0");
    return 0;
  }
  if (check_head_dim(head_dim) != FA_OK) return 0;
  if (check_groups(heads, kv_heads) != FA_OK) return 0;
  if (resolve_split(batch, heads, kv_heads, max_seq, head_dim, &split_size) != FA_OK) return 0;
  if (!decode_needs_workspace(batch, heads, kv_heads, max_seq)) return 0;
  return decode_ws_bytes(batch, heads, max_seq, head_dim, split_size);
}

// scratch_ws: the workspace is the library's own per-device scratch
// (fa_decode_hd_noalloc), which only changes the message of a size failure.
int decode_impl(const void *q, const void *k_cache, const void *v_cache,
                const int32_t *seq_lens, void *o, int out_dtype, int batch, int heads,
                int kv_heads, int max_seq, int head_dim, float scale, int split_size,
                void *workspace, size_t workspace_bytes, void *stream,
                bool scratch_ws = false) {
  clear_error();
  if (check_head_dim(head_dim) != FA_OK) return FA_ERR_INVALID_ARGUMENT;
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      seq_lens == nullptr || o == nullptr)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "q, k_cache, v_cache, seq_lens and o must be non-NULL");
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(o))
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "q, k_cache, v_cache and o must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(seq_lens) & 3u) != 0)
    return set_error(FA_ERR_INVALID_ARGUMENT, "seq_lens must be 4-byte aligned");
  if (out_dtype != FA_OUT_F16 && out_dtype != FA_OUT_F32)
    return set_error(FA_ERR_INVALID_ARGUMENT, "unknown out_dtype %d", out_dtype);
  if (batch <= 0 || heads <= 0)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "batch and heads must be > 0, got B=%d H=%d", batch, heads);
  int rc = check_groups(heads, kv_heads);
  if (rc != FA_OK) return rc;
  if (max_seq <= 0 || max_seq > kMaxCacheRows)
    return set_error(FA_ERR_INVALID_ARGUMENT, "cache length must be in [1, %d], got %d",
                     kMaxCacheRows, max_seq);
  if (!std::isfinite(scale) || !std::isfinite(scale * 1.4426950408889634f))
    return set_error(FA_ERR_INVALID_ARGUMENT, "scale must be finite");
  const bool auto_split = split_size == 0;
  rc = resolve_split(batch, heads, kv_heads, max_seq, head_dim, &split_size);
  if (rc != FA_OK) return rc;
  const size_t n_splits = (static_cast<size_t>(max_seq) + split_size - 1) / split_size;
  if (static_cast<size_t>(batch) * heads * n_splits > 0x7fffffffull)
    return set_error(FA_ERR_INVALID_ARGUMENT, "too many split blocks");
  const size_t need = decode_needs_workspace(batch, heads, kv_heads, max_seq)
                          ? decode_ws_bytes(batch, heads, max_seq, head_dim, split_size)
                          : 0;
  if (scratch_ws && need > workspace_bytes)
    return set_error(FA_ERR_WORKSPACE,
                     "fa_decode_hd_noalloc: this shape needs %zu bytes of split-K scratch, "
                     "above the library's fixed %zu bytes; call fa_decode_hd with a workspace",
                     need, workspace_bytes);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return set_error(FA_ERR_WORKSPACE,
                     "decode workspace too small: need %zu bytes, got %zu", need,
                     workspace == nullptr ? size_t{0} : workspace_bytes);
  if (need > 0 && !aligned16(workspace))
    return set_error(FA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  return launch_decode(q, k_cache, v_cache, seq_lens, o, out_dtype == FA_OUT_F32,
                       batch, heads, kv_heads, max_seq, head_dim, scale, split_size, auto_split,
                       static_cast<float *>(workspace),
                       static_cast<hipStream_t>(stream));
}
}  // namespace

int fa_prefill(const void *q, const void *k, const void *v, void *o,
               int out_dtype, int batch, int heads, int seq, int causal,
               float scale, void *workspace, size_t workspace_bytes,
               void *stream) {
  return prefill_impl(q, k, v, o, out_dtype, batch, heads, heads, seq, 64, causal, scale,
                      workspace, workspace_bytes, stream);
}

int fa_prefill_gqa(const void *q, const void *k, const void *v, void *o, int out_dtype,
                   int batch, int heads, int kv_heads, int seq, int causal, float scale,
                   void *workspace, size_t workspace_bytes, void *stream) {
  return prefill_impl(q, k, v, o, out_dtype, batch, heads, kv_heads, seq, 64, causal, scale,
                      workspace, workspace_bytes, stream);
}

int fa_prefill_hd(const void *q, const void *k, const void *v, void *o, int out_dtype,
                  int batch, int heads, int kv_heads, int seq, int head_dim, int causal,
                  float scale, void *workspace, size_t workspace_bytes, void *stream) {
  return prefill_impl(q, k, v, o, out_dtype, batch, heads, kv_heads, seq, head_dim, causal,
                      scale, workspace, workspace_bytes, stream);
}

size_t fa_decode_workspace_bytes(int batch, int heads, int max_seq,
                                 int split_size) {
  return decode_workspace_impl(batch, heads, heads, max_seq, 64, split_size);
}

size_t fa_decode_gqa_workspace_bytes(int batch, int heads, int kv_heads, int max_seq,
                                     int split_size) {
  return decode_workspace_impl(batch, heads, kv_heads, max_seq, 64, split_size);
}

size_t fa_decode_hd_workspace_bytes(int batch, int heads, int kv_heads, int max_seq,
                                    int head_dim, int split_size) {
  return decode_workspace_impl(batch, heads, kv_heads, max_seq, head_dim, split_size);
}

int fa_decode(const void *q, const void *k_cache, const void *v_cache,
              const int32_t *seq_lens, void *o, int out_dtype, int batch,
              int heads, int max_seq, float scale, int split_size,
              void *workspace, size_t workspace_bytes, void *stream) {
  return decode_impl(q, k_cache, v_cache, seq_lens, o, out_dtype, batch, heads, heads,
                     max_seq, 64, scale, split_size, workspace, workspace_bytes, stream);
}

int fa_decode_gqa(const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, int out_dtype, int batch, int heads,
                  int kv_heads, int max_seq, float scale, int split_size, void *workspace,
                  size_t workspace_bytes, void *stream) {
  return decode_impl(q, k_cache, v_cache, seq_lens, o, out_dtype, batch, heads, kv_heads,
                     max_seq, 64, scale, split_size, workspace, workspace_bytes, stream);
}

int fa_decode_hd(const void *q, const void *k_cache, const void *v_cache,
                 const int32_t *seq_lens, void *o, int out_dtype, int batch, int heads,
                 int kv_heads, int max_seq, int head_dim, float scale, int split_size,
                 void *workspace, size_t workspace_bytes, void *stream) {
  return decode_impl(q, k_cache, v_cache, seq_lens, o, out_dtype, batch, heads, kv_heads,
                     max_seq, head_dim, scale, split_size, workspace, workspace_bytes, stream);
}

// No reference counterpart: fa_decode_hd for callers that cannot allocate.
// Its split-K partials go to the library's per-device scratch array.
int fa_decode_hd_noalloc(const void *q, const void *k_cache, const void *v_cache,
                         const int32_t *seq_lens, void *o, int out_dtype, int batch, int heads,
                         int kv_heads, int max_seq, int head_dim, float scale, int split_size,
                         void *stream) {
  clear_error();
  void *ws = nullptr;
  const int rc = device_scratch(&ws);
  if (rc != FA_OK) return rc;
  return decode_impl(q, k_cache, v_cache, seq_lens, o, out_dtype, batch, heads, kv_heads,
                     max_seq, head_dim, scale, split_size, ws, kNoAllocScratchBytes, stream,
                     true);
}

namespace {
int kv_append_impl(void *k_cache, void *v_cache, const void *k_new, const void *v_new,
                   int32_t *seq_lens, int batch, int kv_heads, int max_seq, int head_dim,
                   void *stream) {
  clear_error();
  if (check_head_dim(head_dim) != FA_OK) return FA_ERR_INVALID_ARGUMENT;
  if (k_cache == nullptr || v_cache == nullptr || k_new == nullptr || v_new == nullptr ||
      seq_lens == nullptr)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "k_cache, v_cache, k_new, v_new and seq_lens must be non-NULL");
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(k_new) || !aligned16(v_new))
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "k_cache, v_cache, k_new and v_new must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(seq_lens) & 3u) != 0)
    return set_error(FA_ERR_INVALID_ARGUMENT, "seq_lens must be 4-byte aligned");
  if (batch <= 0 || kv_heads <= 0)
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "batch and kv_heads must be > 0, got B=%d H_kv=%d", batch, kv_heads);
  if (max_seq <= 0 || max_seq > kMaxCacheRows)
    return set_error(FA_ERR_INVALID_ARGUMENT, "cache length must be in [1, %d], got %d",
                     kMaxCacheRows, max_seq);
  return launch_kv_append(k_cache, v_cache, k_new, v_new, seq_lens, batch, kv_heads, max_seq,
                          head_dim, static_cast<hipStream_t>(stream));
}
}  // namespace

int fa_kv_append(void *k_cache, void *v_cache, const void *k_new, const void *v_new,
                 int32_t *seq_lens, int batch, int kv_heads, int max_seq, void *stream) {
  return kv_append_impl(k_cache, v_cache, k_new, v_new, seq_lens, batch, kv_heads, max_seq,
                        64, stream);
}

int fa_kv_append_hd(void *k_cache, void *v_cache, const void *k_new, const void *v_new,
                    int32_t *seq_lens, int batch, int kv_heads, int max_seq, int head_dim,
                    void *stream) {
  return kv_append_impl(k_cache, v_cache, k_new, v_new, seq_lens, batch, kv_heads, max_seq,
                        head_dim, stream);
}

int fa_legacy_attention(const float *q, const float *k, const float *v, float *o, int n,
                        int variant, void *stream) {
  clear_error();
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr)
    return set_error(FA_ERR_INVALID_ARGUMENT, "q, k, v and o must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return set_error(FA_ERR_INVALID_ARGUMENT,
                     "q, k, v and o must be 16-byte aligned device pointers");
  if (variant != FA_LEGACY_NAIVE && variant != FA_LEGACY_TILED && variant != FA_LEGACY_FUSED)
    return set_error(FA_ERR_INVALID_ARGUMENT, "unknown legacy variant %d", variant);
  if (n < 0 || static_cast<int64_t>(n) * kHeadDim > 0x7fffffffll)
    return set_error(FA_ERR_INVALID_ARGUMENT, "row count must be in [0, 2^31 / 64), got %d", n);
  if (n == 0) return FA_OK;  // nothing to compute, nothing launched
  return launch_legacy_attention(q, k, v, o, n, variant, static_cast<hipStream_t>(stream));
}

int fa_occupancy_report(fa_occupancy_entry *out, int capacity, int *count) {
  clear_error();
  if (count == nullptr || (capacity > 0 && out == nullptr))
    return set_error(FA_ERR_INVALID_ARGUMENT, "bad occupancy report buffer");
  int n = 0;
  int rc = prefill_occupancy(out, capacity, &n);
  if (rc == FA_OK) rc = decode_occupancy(out, capacity, &n);
  *count = n;
  return rc;
}

}  // extern "C"
