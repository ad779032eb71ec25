// Single-query attention over a ragged KV cache (the decode step) for gfx950.
//
// Reference behaviour: csrc/decode.cu:50-240 of shrvan30/flash-attention-cuda
// (split pass :50-138, log-sum-exp merge :143-175, chunk chooser :183-192,
// launcher :194-240). The work split is the same (grid over (split, head,
// batch), partial (m, l, acc[64]) per split, then a merge); everything below
// the work split is laid out for CDNA4 instead:
//
//  * A wave reads 8 cache rows per load instruction: lane = 8 * row + slice,
//    each lane owns 8 head dims (16 B), so one wave64 load moves 1 KiB of
//    contiguous cache and every row is one 128 B segment.
//  * Each wave keeps two groups of 4 row-slots (8 KiB per wave) of K and V in
//    flight: the next group's loads are issued before the current group's
//    arithmetic, so HBM latency is hidden by load-level parallelism rather
//    than by occupancy alone.
//  * q.k is an 8-FMA partial dot per lane followed by a 3-step DPP sum inside
//    each 8-lane row group (no LDS, no ds_bpermute).
//  * The softmax runs in the log2 domain: q is pre-multiplied by
//    scale * log2(e), so p = exp2(s - m) maps to one v_exp_f32.
//  * The per-lane online-softmax states are merged across the 8 row groups
//    of a wave with shuffles, across the 4 waves through LDS, and across
//    splits by the merge kernel.
//
// Partial results are stored with m in the log2 domain; only this file
// produces and consumes them.

#include <hip/hip_fp16.h>

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kSplitThreads = 256;  // 4 waves
constexpr int kSplitWaves = kSplitThreads / kWave;
constexpr int kRowsPerGroup = 8;    // rows covered by one wave load
constexpr int kGroupsPerStep = 4;   // row groups loaded together per wave
constexpr int kRowsPerWaveStep = kRowsPerGroup * kGroupsPerStep;  // 32
constexpr int kRowsPerBlockStep = kRowsPerWaveStep * kSplitWaves; // 128
constexpr int kMergeThreads = kHeadDim;
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for m

struct RowSlots {
  uint4 k[kGroupsPerStep];
  uint4 v[kGroupsPerStep];
};

__device__ __forceinline__ void load_slots(RowSlots &r, const _Float16 *kp,
                                           const _Float16 *vp, int row0,
                                           int end, int sub, int slice) {
#pragma unroll
  for (int u = 0; u < kGroupsPerStep; ++u) {
    const int row = row0 + u * kRowsPerGroup + sub;
    if (row < end) {
      const size_t off = static_cast<size_t>(row) * kHeadDim + slice * 8;
      r.k[u] = *reinterpret_cast<const uint4 *>(kp + off);
      r.v[u] = *reinterpret_cast<const uint4 *>(vp + off);
    } else {
      r.k[u] = make_uint4(0, 0, 0, 0);
      r.v[u] = make_uint4(0, 0, 0, 0);
    }
  }
}

__device__ __forceinline__ void unpack8(const uint4 &raw, float f[8]) {
  const half2 *h = reinterpret_cast<const half2 *>(&raw);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    f[2 * t] = static_cast<float>(h[t][0]);
    f[2 * t + 1] = static_cast<float>(h[t][1]);
  }
}

// Fold one group of rows (already loaded) into the running state.
__device__ __forceinline__ void consume_slots(const RowSlots &r,
                                              const float qf[8], int row0,
                                              int end, int sub, float &m,
                                              float &l, float acc[8]) {
  float s[kGroupsPerStep];
#pragma unroll
  for (int u = 0; u < kGroupsPerStep; ++u) {
    float kf[8];
    unpack8(r.k[u], kf);
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part = fmaf(qf[e], kf[e], part);
    part = sum_lanes8(part);
    const int row = row0 + u * kRowsPerGroup + sub;
    s[u] = (row < end) ? part : -INFINITY;
  }
  const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  const float m_new = fmaxf(m, mx);
  const float alpha = fast_exp2(m - m_new);
  float p[kGroupsPerStep];
  float psum = 0.f;
#pragma unroll
  for (int u = 0; u < kGroupsPerStep; ++u) {
    p[u] = fast_exp2(s[u] - m_new);  // masked rows: exp2(-inf) = 0
    psum += p[u];
  }
  l = fmaf(l, alpha, psum);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < kGroupsPerStep; ++u) {
    float vf[8];
    unpack8(r.v[u], vf);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(p[u], vf[e], acc[e]);
  }
  m = m_new;
}

// Merge state (mb, lb, accb) into (m, l, acc); both in the log2 domain.
__device__ __forceinline__ void merge_state(float &m, float &l, float acc[8],
                                            float mb, float lb,
                                            const float accb[8]) {
  const float m_new = fmaxf(m, mb);
  const float fa_ = fast_exp2(m - m_new);
  const float fb = fast_exp2(mb - m_new);
  l = l * fa_ + lb * fb;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = acc[e] * fa_ + accb[e] * fb;
  m = m_new;
}

// Pass 1 (decode.cu:50-138): one block folds cache rows
// [split * chunk, min(len, (split + 1) * chunk)) of one (b, h) into a partial
// (m, l, acc[64]). Grid: 1-D, block id = (b * H + h) * n_splits + split.
__global__ __launch_bounds__(kSplitThreads) void decode_split_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    float *__restrict__ part_acc, float *__restrict__ part_ml, int heads,
    int max_seq, int n_splits, int chunk, float qscale) {
  const int split = blockIdx.x % n_splits;
  const int bh = blockIdx.x / n_splits;
  const int b = bh / heads;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int sub = lane >> 3;   // row inside an 8-row group
  const int slice = lane & 7;  // head dims [8 * slice, 8 * slice + 8)

  // decode.cu:69-71: clamp to the cache capacity; empty chunks write l = 0.
  const int len = min(seq_lens[b], max_seq);
  const int begin = split * chunk;
  const int end = min(len, begin + chunk);

  float qf[8];
  {
    const uint4 raw = *reinterpret_cast<const uint4 *>(
        q + static_cast<size_t>(bh) * kHeadDim + slice * 8);
    unpack8(raw, qf);
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[e] *= qscale;
  }

  float m = kNegBig, l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;

  const size_t head_off = static_cast<size_t>(bh) * max_seq * kHeadDim;
  const _Float16 *kp = k_cache + head_off;
  const _Float16 *vp = v_cache + head_off;

  // Double-buffered row slots: the loads of step i+1 are in flight while
  // step i is consumed.
  int row0 = begin + wave * kRowsPerWaveStep;
  if (row0 < end) {
    RowSlots cur, nxt;
    load_slots(cur, kp, vp, row0, end, sub, slice);
    for (;;) {
      const int next0 = row0 + kRowsPerBlockStep;
      const bool more = next0 < end;
      if (more) load_slots(nxt, kp, vp, next0, end, sub, slice);
      consume_slots(cur, qf, row0, end, sub, m, l, acc);
      if (!more) break;
      cur = nxt;
      row0 = next0;
    }
  }

  // Merge the 8 row groups of the wave (lanes that share `slice`).
#pragma unroll
  for (int off = 8; off < kWave; off <<= 1) {
    const float mb = __shfl_xor(m, off);
    const float lb = __shfl_xor(l, off);
    float accb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) accb[e] = __shfl_xor(acc[e], off);
    merge_state(m, l, acc, mb, lb, accb);
  }

  __shared__ float s_acc[kSplitWaves][kHeadDim];
  __shared__ float s_m[kSplitWaves];
  __shared__ float s_l[kSplitWaves];
  if (sub == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave][slice * 8 + e] = acc[e];
    if (slice == 0) {
      s_m[wave] = m;
      s_l[wave] = l;
    }
  }
  __syncthreads();

  if (threadIdx.x < kHeadDim) {
    const int d = threadIdx.x;
    float mb = s_m[0];
#pragma unroll
    for (int w = 1; w < kSplitWaves; ++w) mb = fmaxf(mb, s_m[w]);
    float lb = 0.f, ab = 0.f;
#pragma unroll
    for (int w = 0; w < kSplitWaves; ++w) {
      const float f = fast_exp2(s_m[w] - mb);
      lb = fmaf(s_l[w], f, lb);
      ab = fmaf(s_acc[w][d], f, ab);
    }
    const size_t slot = static_cast<size_t>(bh) * n_splits + split;
    part_acc[slot * kHeadDim + d] = ab;
    if (d == 0) {
      part_ml[slot * 2] = mb;
      part_ml[slot * 2 + 1] = lb;
    }
  }
}

// Pass 2 (decode.cu:143-175): log-sum-exp merge of the partials of one
// (b, h); splits with l <= 0 (past the sequence end) are skipped, and a
// sequence with no rows produces zeros. Grid: B * H blocks of 64 threads.
template <bool OUT_F32>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(
    const float *__restrict__ part_acc, const float *__restrict__ part_ml,
    void *__restrict__ o, int n_splits) {
  const int bh = blockIdx.x;
  const int d = threadIdx.x;
  const size_t base = static_cast<size_t>(bh) * n_splits;

  float m_all = kNegBig;
  for (int s = 0; s < n_splits; ++s) {
    const float l_s = part_ml[(base + s) * 2 + 1];
    if (l_s > 0.f) m_all = fmaxf(m_all, part_ml[(base + s) * 2]);
  }
  float l_all = 0.f, acc = 0.f;
  for (int s = 0; s < n_splits; ++s) {
    const float l_s = part_ml[(base + s) * 2 + 1];
    if (!(l_s > 0.f)) continue;
    const float f = fast_exp2(part_ml[(base + s) * 2] - m_all);
    l_all = fmaf(l_s, f, l_all);
    acc = fmaf(part_acc[(base + s) * kHeadDim + d], f, acc);
  }
  const float out = (l_all > 0.f) ? acc / l_all : 0.f;
  const size_t idx = static_cast<size_t>(bh) * kHeadDim + d;
  if (OUT_F32) {
    static_cast<float *>(o)[idx] = out;
  } else {
    static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(out);
  }
}

}  // namespace

int launch_decode(const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, bool out_f32, int batch,
                  int heads, int max_seq, float scale, int split_size,
                  float *workspace, hipStream_t stream) {
  const int n_splits = (max_seq + split_size - 1) / split_size;
  const size_t bh = static_cast<size_t>(batch) * heads;
  float *part_acc = workspace;
  float *part_ml = workspace + bh * n_splits * kHeadDim;
  const unsigned split_blocks = static_cast<unsigned>(bh * n_splits);

  hipLaunchKernelGGL(decode_split_kernel, dim3(split_blocks),
                     dim3(kSplitThreads), 0, stream,
                     static_cast<const _Float16 *>(q),
                     static_cast<const _Float16 *>(k_cache),
                     static_cast<const _Float16 *>(v_cache), seq_lens,
                     part_acc, part_ml, heads, max_seq, n_splits, split_size,
                     scale * kLog2e);
  int rc = check_hip(hipGetLastError(), "decode_split_kernel launch");
  if (rc != FA_OK) return rc;

  if (out_f32) {
    hipLaunchKernelGGL(decode_merge_kernel<true>, dim3(static_cast<unsigned>(bh)),
                       dim3(kMergeThreads), 0, stream, part_acc, part_ml, o,
                       n_splits);
  } else {
    hipLaunchKernelGGL(decode_merge_kernel<false>, dim3(static_cast<unsigned>(bh)),
                       dim3(kMergeThreads), 0, stream, part_acc, part_ml, o,
                       n_splits);
  }
  return check_hip(hipGetLastError(), "decode_merge_kernel launch");
}

int decode_occupancy(fa_occupancy_entry *out, int cap, int *n) {
  struct K { const char *name; const void *fn; int threads; };
  const K ks[] = {
      {"decode_split_kernel", reinterpret_cast<const void *>(decode_split_kernel),
       kSplitThreads},
      {"decode_merge_kernel",
       reinterpret_cast<const void *>(decode_merge_kernel<false>), kMergeThreads},
  };
  for (const K &k : ks) {
    if (*n < cap) {
      const int rc = fill_occupancy_row(&out[*n], k.name, k.fn, k.threads, 0);
      if (rc != FA_OK) return rc;
    }
    ++*n;
  }
  return FA_OK;
}

}  // namespace fa
