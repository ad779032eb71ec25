// KV-cache append: the caller step before each decode. It writes one new
// token's K and V rows into the caches at row seq_lens[b] and advances
// seq_lens[b] by one, on the device.
//
// Reference behaviour: the reference leaves this step to its caller (the
// FlashStack engine writes token t into the cache at seq_lens[b] before
// calling decode; README.md:9-13 of shrvan30/flash-attention-cuda), with the
// cache layout decode reads: [B, H_kv, Lmax, 64] fp16, sequence b's tokens in
// rows [0, seq_lens[b]).
//
// Because the only state is seq_lens in device memory, an append + decode
// step has launch arguments that do not change from token to token: a caller
// can capture one step in a HIP graph and replay it once per generated token.
//
// Layout: one block per batch row b. Its threads copy the 2 * H_kv rows of
// 2 * head_dim bytes (16 bytes per thread per row) and then, after a
// barrier, one thread advances seq_lens[b]. A row is written only when
// 0 <= seq_lens[b] < Lmax; otherwise the block writes nothing and leaves
// seq_lens[b] unchanged (a full cache is the caller's to handle).

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kAppendThreads = 256;

__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(
    _Float16 *__restrict__ k_cache, _Float16 *__restrict__ v_cache,
    const _Float16 *__restrict__ k_new, const _Float16 *__restrict__ v_new,
    int32_t *__restrict__ seq_lens, int kv_heads, int max_seq, int head_dim) {
  const int b = static_cast<int>(blockIdx.x);
  const int len = seq_lens[b];
  // Every thread has read seq_lens[b] before it can change.
  __syncthreads();
  if (len < 0 || len >= max_seq) return;
  const int row_pieces = head_dim / 8;   // 16-byte pieces per row (8 or 16)
  const int pieces = kv_heads * 2 * row_pieces;  // (head, K|V, piece)
  for (int i = static_cast<int>(threadIdx.x); i < pieces; i += kAppendThreads) {
    const int h = i / (2 * row_pieces);
    const int is_v = (i / row_pieces) & 1;
    const int piece = i % row_pieces;
    const size_t bh = static_cast<size_t>(b) * kv_heads + h;
    const _Float16 *src = (is_v ? v_new : k_new) + bh * head_dim + piece * 8;
    _Float16 *dst = (is_v ? v_cache : k_cache) +
                    (bh * max_seq + static_cast<size_t>(len)) * head_dim + piece * 8;
    *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
  }
  if (threadIdx.x == 0) seq_lens[b] = len + 1;
}

}  // namespace

int launch_kv_append(void *k_cache, void *v_cache, const void *k_new, const void *v_new,
                     int32_t *seq_lens, int batch, int kv_heads, int max_seq, int head_dim,
                     hipStream_t stream) {
  hipLaunchKernelGGL(kv_append_kernel, dim3(static_cast<unsigned>(batch)),
                     dim3(kAppendThreads), 0, stream, static_cast<_Float16 *>(k_cache),
                     static_cast<_Float16 *>(v_cache), static_cast<const _Float16 *>(k_new),
                     static_cast<const _Float16 *>(v_new), seq_lens, kv_heads, max_seq,
                     head_dim);
  return check_hip(hipGetLastError(), "kv_append_kernel launch");
}

}  // namespace fa
