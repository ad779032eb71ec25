// Single-query attention over a ragged KV cache (the decode step) for gfx950.
//
// Reference behaviour: csrc/decode.cu:50-240 of shrvan30/flash-attention-cuda
// (split pass :50-138, log-sum-exp merge :143-175, chunk chooser :183-192,
// launcher :194-240). The result is the same softmax(q K^T * scale) V over the
// first seq_lens[b] cache rows; the work split depends on the grid:
//
//  * B * H < compute units (too few (b, h) pairs to fill the chip): the
//    reference's split-K scheme. The cache rows of each (b, h) are cut into
//    chunks of `chunk` rows, each chunk yields a partial (m, l, acc[64]) in
//    the workspace, and a merge kernel combines them.
//  * B * H >= compute units: one 8-wave block per (b, h) folds the whole
//    sequence (decode_bh_kernel below), merging its waves through LDS, so no
//    partials reach HBM and there is no second kernel.
//
// Split path details, laid out for CDNA4:
//
//  * One WAVE owns one (b, h, chunk) unit; a block is four independent waves
//    (no LDS, no barrier). Chunks past a sequence's end exit at once.
//  * A wave reads 8 cache rows per load instruction: lane = 8 * row + slice,
//    each lane owns 8 head dims (16 B), so one wave64 load moves 1 KiB of
//    contiguous cache and every row is one 128 B segment. The loads are
//    non-temporal (each row is read once per call).
//  * Rows are consumed in sub-steps of 64 (8 row groups, 16 loads per lane);
//    the next sub-step's loads are in flight while the current one is
//    consumed, so each wave keeps 16-32 KiB of cache reads outstanding.
//  * q.k is four v_dot2_f32_f16 per lane on the raw fp16 pairs (exact
//    products, fp32 sums) followed by a 3-step DPP sum inside each 8-lane
//    row group (no LDS, no ds_bpermute).
//  * The softmax runs in the log2 domain: each score is multiplied by
//    scale * log2(e), so p = exp2(s - m) maps to one v_exp_f32.
//  * Grouped-query attention (H_kv < H K/V heads): a unit holds NQ query
//    heads of one K/V head (NQ the largest divisor of H / H_kv up to 8), so
//    each cache row is loaded once for all of them.
//  * The per-lane online-softmax states are merged across the 8 row groups
//    of the wave with shuffles, and across chunks by the merge kernel.
//
// Partial results are stored with m in the log2 domain; only this file
// produces and consumes them.

#include <hip/hip_fp16.h>

#include <mutex>
#include <type_traits>

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kSplitThreads = 256;  // 4 independent waves
constexpr int kSplitWaves = kSplitThreads / kWave;
constexpr int kRowsPerGroup = 8;    // rows covered by one wave load
constexpr int kGroupsPerStep = 8;   // row groups loaded together per wave
constexpr int kMergeThreads = kHeadDim;
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for m

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte non-temporal load: every cache row is read exactly once per call,
// so the loads bypass the normal cache-allocation policy (measured on
// gfx950: ~7.1 TB/s streaming reads versus ~6.0 TB/s with plain loads).
__device__ __forceinline__ uint4 load_stream(const _Float16 *p) {
  const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}

template <int G>
struct RowSlotsT {
  uint4 k[G];
  uint4 v[G];
};

template <int G>
__device__ __forceinline__ void load_slots(RowSlotsT<G> &r, const _Float16 *kp,
                                           const _Float16 *vp, int row0,
                                           int end, int sub, int slice) {
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int row = row0 + u * kRowsPerGroup + sub;
    if (row < end) {
      const size_t off = static_cast<size_t>(row) * kHeadDim + slice * 8;
      r.k[u] = load_stream(kp + off);
      r.v[u] = load_stream(vp + off);
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

// Fold one sub-step of rows (already loaded) into the running states of the
// NQ queries that share this K/V head (NQ = 1 without grouped queries). The
// q.k partial of a lane is four v_dot2_f32_f16 on the raw fp16 pairs (exact
// fp16 products, fp32 sums), scaled once by qscale = scale * log2(e); each V
// row is unpacked once and feeds every query's accumulator.
template <int G, int NQ>
__device__ __forceinline__ void consume_slots(const RowSlotsT<G> &r,
                                              const half2 (&qh)[NQ][4], float qscale,
                                              int row0, int end, int sub, float (&m)[NQ],
                                              float (&l)[NQ], float (&acc)[NQ][8]) {
  float s[NQ][G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const half2 *kh = reinterpret_cast<const half2 *>(&r.k[u]);
    const int row = row0 + u * kRowsPerGroup + sub;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      float part = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t) part = __builtin_amdgcn_fdot2(qh[j][t], kh[t], part, false);
      part = sum_lanes8(part);
      s[j][u] = (row < end) ? part * qscale : -INFINITY;
    }
  }
  float p[NQ][G];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float mx = s[j][0];
#pragma unroll
    for (int u = 1; u < G; ++u) mx = fmaxf(mx, s[j][u]);
    const float m_new = fmaxf(m[j], mx);
    const float alpha = fast_exp2(m[j] - m_new);
    float psum = 0.f;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      p[j][u] = fast_exp2(s[j][u] - m_new);  // masked rows: exp2(-inf) = 0
      psum += p[j][u];
    }
    l[j] = fmaf(l[j], alpha, psum);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] *= alpha;
    m[j] = m_new;
  }
#pragma unroll
  for (int u = 0; u < G; ++u) {
    float vf[8];
    unpack8(r.v[u], vf);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(p[j][u], vf[e], acc[j][e]);
  }
}

// Query j of a query unit: the NQ query heads that read one K/V head.
// The unit index u runs over (b, kv head, query chunk); query j is head
// kv * group + chunk * NQ + j of batch row b.
struct QueryUnit {
  int b, kv, h0;
};
__device__ __forceinline__ QueryUnit query_unit(int u, int kv_heads, int q_chunks, int group,
                                                int nq) {
  QueryUnit r;
  const int per_b = kv_heads * q_chunks;
  r.b = u / per_b;
  const int rest = u - r.b * per_b;
  r.kv = rest / q_chunks;
  r.h0 = r.kv * group + (rest - r.kv * q_chunks) * nq;
  return r;
}

// The 8 head dims [8 * slice, +8) of each of the NQ queries, as fp16 pairs.
template <int NQ>
__device__ __forceinline__ void load_queries(const _Float16 *q, size_t bh0, int slice,
                                             half2 (&qh)[NQ][4]) {
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const uint4 raw = *reinterpret_cast<const uint4 *>(q + (bh0 + j) * kHeadDim + slice * 8);
    const half2 *h = reinterpret_cast<const half2 *>(&raw);
#pragma unroll
    for (int t = 0; t < 4; ++t) qh[j][t] = h[t];
  }
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

// Pass 1 (decode.cu:50-138): one wave folds cache rows
// [chunk_i * chunk, min(len, (chunk_i + 1) * chunk)) of one K/V head into a
// partial (m, l, acc[64]) for each of the NQ query heads that read it. Unit
// w = chunk_i * n_qu + u (u over (b, kv head, query chunk)) is handled by
// wave w % 4 of block w / 4. G row groups (8 rows each) are loaded per
// sub-step.
template <int G, int NQ>
__global__ __launch_bounds__(kSplitThreads) void decode_split_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    float *__restrict__ part_acc, float *__restrict__ part_ml, int heads,
    int kv_heads, int group, int max_seq, int n_splits, int n_units, int chunk,
    float qscale) {
  const int lane = threadIdx.x & (kWave - 1);
  const int unit = static_cast<int>(blockIdx.x) * kSplitWaves +
                   __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  if (unit >= n_units) return;
  // Chunk-major order: every unit's first chunk is dispatched first, its
  // last chunks (empty for short sequences) last, so the hardware dispatcher
  // hands out the heaviest units first (a longest-first list schedule).
  const int n_qu = n_units / n_splits;
  const int split = unit / n_qu;
  const QueryUnit qu = query_unit(unit - split * n_qu, kv_heads, group / NQ, group, NQ);

  const int sub = lane >> 3;   // row inside an 8-row group
  const int slice = lane & 7;  // head dims [8 * slice, 8 * slice + 8)

  // decode.cu:69-71: clamp to the cache capacity. A chunk past the sequence
  // end has no rows: it writes nothing, and the merge pass only reads the
  // partials of the ceil(len / chunk) chunks that have rows.
  const int len = min(seq_lens[qu.b], max_seq);
  const int begin = split * chunk;
  if (begin >= len) return;
  const int end = min(len, begin + chunk);

  const size_t kv_off =
      (static_cast<size_t>(qu.b) * kv_heads + qu.kv) * max_seq * kHeadDim;
  const _Float16 *kp = k_cache + kv_off;
  const _Float16 *vp = v_cache + kv_off;
  const size_t bh0 = static_cast<size_t>(qu.b) * heads + qu.h0;

  // Double-buffered row slots: the loads of sub-step i+1 are in flight while
  // sub-step i is consumed.
  constexpr int kStepRows = kRowsPerGroup * G;
  RowSlotsT<G> cur, nxt;
  int row0 = begin;
  load_slots(cur, kp, vp, row0, end, sub, slice);

  half2 qh[NQ][4];
  load_queries<NQ>(q, bh0, slice, qh);

  float m[NQ], l[NQ], acc[NQ][8];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    m[j] = kNegBig;
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
  }

  for (;;) {
    const int next0 = row0 + kStepRows;
    const bool more = next0 < end;
    if (more) load_slots(nxt, kp, vp, next0, end, sub, slice);
    consume_slots(cur, qh, qscale, row0, end, sub, m, l, acc);
    if (!more) break;
    cur = nxt;
    row0 = next0;
  }

#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    // Merge the 8 row groups of the wave (lanes that share `slice`).
#pragma unroll
    for (int off = 8; off < kWave; off <<= 1) {
      const float mb = __shfl_xor(m[j], off);
      const float lb = __shfl_xor(l[j], off);
      float accb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) accb[e] = __shfl_xor(acc[j][e], off);
      merge_state(m[j], l[j], acc[j], mb, lb, accb);
    }
    if (sub == 0) {
      const size_t slot = (bh0 + j) * n_splits + split;
      float4 *dst = reinterpret_cast<float4 *>(part_acc + slot * kHeadDim + slice * 8);
      dst[0] = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
      dst[1] = make_float4(acc[j][4], acc[j][5], acc[j][6], acc[j][7]);
      if (slice == 0) *reinterpret_cast<float2 *>(part_ml + slot * 2) = make_float2(m[j], l[j]);
    }
  }
}

// Pass 2 (decode.cu:143-175): log-sum-exp merge of the partials of one
// (b, h). Only the ceil(len / chunk) chunks that hold rows are read (the
// reference skips the others through l <= 0); a sequence with no rows
// produces zeros. One wave per (b, h): lane s takes partials s, s + 64, ...
// for the max and the row sum, then lane d accumulates head dim d over the
// chunks, with the per-chunk weights broadcast from the lane that computed
// them. The loads of the common case (seq_len, the first 64 (m, l) pairs
// and the first 8 partial rows) are all issued before any of them is used,
// so the pass costs about one memory round trip.
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

template <bool OUT_F32>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(
    const float *__restrict__ part_acc, const float *__restrict__ part_ml,
    const int32_t *__restrict__ seq_lens, void *__restrict__ o, int heads,
    int max_seq, int n_splits, int chunk) {
  constexpr int kBatch = 8;  // chunks whose partial rows are loaded together
  const int bh = blockIdx.x;
  const int lane = threadIdx.x;
  const size_t base = static_cast<size_t>(bh) * n_splits;
  // Issued together, before the number of live chunks is known: seq_len, the
  // (m, l) of chunk `lane` and head dim `lane` of the first kBatch partials
  // (slots past the live ones are read, all inside the workspace, and then
  // discarded by a select).
  const int raw_len = seq_lens[bh / heads];
  float2 ml = make_float2(kNegBig, 0.f);
  if (lane < n_splits) ml = *reinterpret_cast<const float2 *>(part_ml + (base + lane) * 2);
  float x[kBatch];
  const float *col = part_acc + base * kHeadDim + lane;
#pragma unroll
  for (int u = 0; u < kBatch; ++u) x[u] = (u < n_splits) ? col[u * kHeadDim] : 0.f;

  const int len = min(raw_len, max_seq);
  const int n_act = len > 0 ? (len + chunk - 1) / chunk : 0;
  float m_all = lane < n_act ? ml.x : kNegBig;
  for (int s = lane + kWave; s < n_act; s += kWave) m_all = fmaxf(m_all, part_ml[(base + s) * 2]);
  m_all = wave_max(m_all);
  float l_all = lane < n_act ? ml.y * fast_exp2(ml.x - m_all) : 0.f;
  for (int s = lane + kWave; s < n_act; s += kWave) {
    const float2 mls = *reinterpret_cast<const float2 *>(part_ml + (base + s) * 2);
    l_all = fmaf(mls.y, fast_exp2(mls.x - m_all), l_all);
  }
  l_all = wave_sum(l_all);

  float acc = 0.f;
  for (int s0 = 0; s0 < n_act; s0 += kWave) {
    const int s = s0 + lane;
    const float w = (s < n_act) ? fast_exp2((s0 == 0 ? ml.x : part_ml[(base + s) * 2]) - m_all) : 0.f;
    const int cnt = min(kWave, n_act - s0);
    int t = 0;
    if (s0 == 0) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        // Slots past n_act were never written for this call (their chunks
        // hold no rows) and may hold any bits, NaN included: select them
        // out rather than multiplying them by a zero weight.
        const float xu = u < n_act ? x[u] : 0.f;
        acc = fmaf(xu, __shfl(w, u), acc);
      }
      t = kBatch;
    }
    for (; t + kBatch <= cnt; t += kBatch) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) x[u] = col[(s0 + t + u) * kHeadDim];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) acc = fmaf(x[u], __shfl(w, t + u), acc);
    }
    for (; t < cnt; ++t) acc = fmaf(col[(s0 + t) * kHeadDim], __shfl(w, t), acc);
  }
  const float out = (l_all > 0.f) ? acc / l_all : 0.f;
  const size_t idx = static_cast<size_t>(bh) * kHeadDim + lane;
  if (OUT_F32) {
    static_cast<float *>(o)[idx] = out;
  } else {
    static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(out);
  }
}

// Whole-sequence variant for batches with at least one unit per compute
// unit: one block of 8 waves owns one unit (a (b, h), or with grouped queries
// NQ query heads of one (b, K/V head)), and wave w folds the chunks
// w, w + 8, w + 16, ... of `chunk` rows each. Rows go in sub-steps of 32 (16
// for NQ >= 7), the next one in flight while the current one is consumed; the
// 8 wave states merge through LDS and the block writes the NQ outputs, so
// there is no partial workspace and no merge pass.
// With chunk == 0 (the automatic choice) the chunk follows the grid:
//  * every block resident at once (target_waves > 0): the batch's cache rows
//    times the blocks per batch row, over target_waves, so about target_waves waves stream rows, each a long
//    contiguous range (measured on ragged batches: fewer, longer streams beat
//    more, shorter ones);
//  * more blocks than fit (target_waves == 0): 1/8 of the block's own
//    sequence, so all 8 waves of each resident block stream.
// Chunks are multiples of 64 rows. Blocks take the sequences in decreasing
// length order (every block ranks the batch's lengths itself, for batches of
// up to kRankMax), so the dispatcher runs a longest-first list schedule.
constexpr int kBhWaves = 8;
constexpr int kBhThreads = kBhWaves * kWave;
// Row groups per sub-step: 4 (32 rows), 2 for 7-8 queries per block, whose
// per-query state would otherwise not fit in 256 VGPRs.
template <int NQ>
constexpr int bh_groups() {
  return NQ <= 6 ? 4 : 2;
}
constexpr int kRankMax = 256;   // ranking costs batch^2 / 512 LDS reads per thread
constexpr int kBhWavesPerCu = 5;  // streaming waves per CU when the grid is resident

template <int NQ, bool OUT_F32>
__global__ __launch_bounds__(kBhThreads) void decode_bh_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    void *__restrict__ o, int batch, int heads, int kv_heads, int group, int max_seq,
    int chunk, int target_waves, float qscale) {
  __shared__ int s_len[kRankMax];
  __shared__ int s_order[kRankMax];
  __shared__ float s_acc[kBhWaves][NQ][kHeadDim];
  __shared__ float s_m[kBhWaves][NQ];
  __shared__ float s_l[kBhWaves][NQ];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  // Blocks per batch row: one per (kv head, query chunk).
  const int q_chunks = group / NQ;
  const int per_b = kv_heads * q_chunks;
  QueryUnit qu = query_unit(static_cast<int>(blockIdx.x), kv_heads, q_chunks, group, NQ);
  if (batch <= kRankMax) {
    // rank(t) = #{u : len_u > len_t or (len_u == len_t and u < t)}: the
    // blocks of batch slot i take the i-th longest sequence.
    for (int t = tid; t < batch; t += kBhThreads) s_len[t] = max(0, min(seq_lens[t], max_seq));
    __syncthreads();
    for (int t = tid; t < batch; t += kBhThreads) {
      const int lt = s_len[t];
      int rank = 0;
      for (int u = 0; u < batch; ++u) {
        const int lu = s_len[u];
        rank += (lu > lt || (lu == lt && u < t)) ? 1 : 0;
      }
      s_order[rank] = t;
    }
    __syncthreads();
    qu.b = s_order[qu.b];
  }
  const int b = qu.b;
  const int len = max(0, min(seq_lens[b], max_seq));
  if (chunk == 0) {
    int rows_per_wave;
    if (target_waves > 0) {
      int part = 0;
      for (int t = lane; t < batch; t += kWave)
        part += batch <= kRankMax ? s_len[t] : max(0, min(seq_lens[t], max_seq));
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
      const float total = static_cast<float>(__builtin_amdgcn_readfirstlane(part));
      rows_per_wave = static_cast<int>(
          fminf(ceilf(total * static_cast<float>(per_b) / static_cast<float>(target_waves)),
                static_cast<float>(max_seq)));
    } else {
      rows_per_wave = (len + kBhWaves - 1) / kBhWaves;
    }
    chunk = max(64, (rows_per_wave + 63) & ~63);
  }
  chunk = min(chunk, max_seq);  // max_seq <= 2^27 (host check): 8 * chunk fits in int

  const int sub = lane >> 3;   // row inside an 8-row group
  const int slice = lane & 7;  // head dims [8 * slice, 8 * slice + 8)
  const size_t kv_off = (static_cast<size_t>(b) * kv_heads + qu.kv) * max_seq * kHeadDim;
  const _Float16 *kp = k_cache + kv_off;
  const _Float16 *vp = v_cache + kv_off;
  const size_t bh0 = static_cast<size_t>(b) * heads + qu.h0;

  float m[NQ], l[NQ], acc[NQ][8];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    m[j] = kNegBig;
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
  }

  constexpr int kGroups = bh_groups<NQ>();
  constexpr int kStepRows = kRowsPerGroup * kGroups;
  const int stride = kBhWaves * chunk;  // distance between a wave's chunks
  int c0 = wave * chunk;                // this wave's current chunk
  if (c0 < len) {
    half2 qh[NQ][4];
    load_queries<NQ>(q, bh0, slice, qh);
    int end = min(len, c0 + chunk);
    int row0 = c0;
    RowSlotsT<kGroups> cur, nxt;
    load_slots(cur, kp, vp, row0, end, sub, slice);
    for (;;) {
      // Next sub-step: the rest of this chunk, else this wave's next chunk.
      int n_row0 = row0 + kStepRows, n_end = end, n_c0 = c0;
      if (n_row0 >= end) {
        n_c0 = c0 + stride;
        n_row0 = n_c0;
        n_end = min(len, n_c0 + chunk);
      }
      const bool more = n_row0 < n_end;
      if (more) load_slots(nxt, kp, vp, n_row0, n_end, sub, slice);
      consume_slots(cur, qh, qscale, row0, end, sub, m, l, acc);
      if (!more) break;
      cur = nxt;
      row0 = n_row0;
      end = n_end;
      c0 = n_c0;
    }
  }

#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    // Merge the 8 row groups of the wave (lanes that share `slice`).
#pragma unroll
    for (int off = 8; off < kWave; off <<= 1) {
      const float mb = __shfl_xor(m[j], off);
      const float lb = __shfl_xor(l[j], off);
      float accb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) accb[e] = __shfl_xor(acc[j][e], off);
      merge_state(m[j], l[j], acc[j], mb, lb, accb);
    }
    if (sub == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[wave][j][slice * 8 + e] = acc[j][e];
      if (slice == 0) {
        s_m[wave][j] = m[j];
        s_l[wave][j] = l[j];
      }
    }
  }
  __syncthreads();
  if (tid < NQ * kHeadDim) {  // NQ <= 8: one thread per (query, head dim)
    const int j = tid / kHeadDim;
    const int d = tid % kHeadDim;
    float mb = s_m[0][j];
#pragma unroll
    for (int w = 1; w < kBhWaves; ++w) mb = fmaxf(mb, s_m[w][j]);
    float lb = 0.f, ab = 0.f;
#pragma unroll
    for (int w = 0; w < kBhWaves; ++w) {
      const float f = fast_exp2(s_m[w][j] - mb);  // empty waves: l = 0, acc = 0
      lb = fmaf(s_l[w][j], f, lb);
      ab = fmaf(s_acc[w][j][d], f, ab);
    }
    // decode.cu:172: a sequence with no rows gets a zero output.
    const float out = (lb > 0.f) ? ab / lb : 0.f;
    const size_t idx = (bh0 + j) * kHeadDim + d;
    if (OUT_F32)
      static_cast<float *>(o)[idx] = out;
    else
      static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(out);
  }
}

// Queries per unit for a query group of `group` heads per K/V head: the
// largest divisor of the group up to kMaxGroupQueries, so every unit holds
// the same number of queries and a group of up to 8 reads its K/V head once.
constexpr int kMaxGroupQueries = 8;
int queries_per_unit(int group) {
  for (int nq = kMaxGroupQueries; nq > 1; --nq)
    if (group % nq == 0) return nq;
  return 1;
}

// Calls f(std::integral_constant<int, NQ>) for the runtime nq in [1, 8].
template <typename F>
void with_nq(int nq, F &&f) {
  switch (nq) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 5: f(std::integral_constant<int, 5>{}); break;
    case 6: f(std::integral_constant<int, 6>{}); break;
    case 7: f(std::integral_constant<int, 7>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
  }
}

// Row groups per sub-step of the split kernel: 8 for one query per unit,
// 4 for grouped queries (their per-query state takes the registers).
template <int NQ>
constexpr int split_groups() {
  return NQ == 1 ? kGroupsPerStep : kGroupsPerStep / 2;
}

// Blocks of decode_bh_kernel<nq> resident on one CU at once, per device.
int bh_blocks_per_cu(int device, int nq) {
  static std::once_flag once[kMaxDevices][kMaxGroupQueries];
  static int blocks[kMaxDevices][kMaxGroupQueries];
  if (device < 0 || device >= kMaxDevices || nq < 1 || nq > kMaxGroupQueries) return 1;
  std::call_once(once[device][nq - 1], [device, nq] {
    int n = 0;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return;
    const void *fn = nullptr;
    with_nq(nq, [&fn](auto c) {
      fn = reinterpret_cast<const void *>(decode_bh_kernel<decltype(c)::value, false>);
    });
    if (hipSetDevice(device) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kBhThreads, 0) != hipSuccess)
      n = 0;
    (void)hipSetDevice(prev);
    blocks[device][nq - 1] = n;
  });
  return blocks[device][nq - 1] > 0 ? blocks[device][nq - 1] : 1;
}

// Whole-sequence blocks need at least one unit per compute unit to fill the
// chip; below that, the split-K grid spreads each sequence over CUs.
bool use_bh_path(int batch, int units_per_row) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const int cu = device_cu_count(dev);
  return cu > 0 && static_cast<long long>(batch) * units_per_row >= cu;
}

}  // namespace

int decode_units_per_row(int heads, int kv_heads) {
  const int group = heads / kv_heads;
  return kv_heads * (group / queries_per_unit(group));
}

int launch_decode(const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, bool out_f32, int batch,
                  int heads, int kv_heads, int max_seq, float scale, int split_size,
                  bool auto_split, float *workspace, hipStream_t stream) {
  const int group = heads / kv_heads;
  const int nq = queries_per_unit(group);
  const int units_per_row = kv_heads * (group / nq);
  const size_t n_qu = static_cast<size_t>(batch) * units_per_row;
  const size_t bh = static_cast<size_t>(batch) * heads;
  const float qscale = scale * kLog2e;
  const auto *qh = static_cast<const _Float16 *>(q);
  const auto *kh = static_cast<const _Float16 *>(k_cache);
  const auto *vh = static_cast<const _Float16 *>(v_cache);
  if (use_bh_path(batch, units_per_row)) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != FA_OK) return rc;
    const int cu = device_cu_count(dev);
    const bool resident = n_qu <= static_cast<size_t>(bh_blocks_per_cu(dev, nq)) * cu;
    const int target_waves = resident ? kBhWavesPerCu * cu : 0;
    const int chunk = auto_split ? 0 : split_size;
    with_nq(nq, [&](auto c) {
      constexpr int NQ = decltype(c)::value;
      if (out_f32)
        hipLaunchKernelGGL((decode_bh_kernel<NQ, true>), dim3(static_cast<unsigned>(n_qu)),
                           dim3(kBhThreads), 0, stream, qh, kh, vh, seq_lens, o, batch, heads,
                           kv_heads, group, max_seq, chunk, target_waves, qscale);
      else
        hipLaunchKernelGGL((decode_bh_kernel<NQ, false>), dim3(static_cast<unsigned>(n_qu)),
                           dim3(kBhThreads), 0, stream, qh, kh, vh, seq_lens, o, batch, heads,
                           kv_heads, group, max_seq, chunk, target_waves, qscale);
    });
    return check_hip(hipGetLastError(), "decode_bh_kernel launch");
  }
  const int n_splits = (max_seq + split_size - 1) / split_size;
  float *part_acc = workspace;
  float *part_ml = workspace + bh * n_splits * kHeadDim;
  const size_t n_units = n_qu * n_splits;
  const unsigned split_blocks =
      static_cast<unsigned>((n_units + kSplitWaves - 1) / kSplitWaves);

  with_nq(nq, [&](auto c) {
    constexpr int NQ = decltype(c)::value;
    hipLaunchKernelGGL((decode_split_kernel<split_groups<NQ>(), NQ>), dim3(split_blocks),
                       dim3(kSplitThreads), 0, stream, qh, kh, vh, seq_lens, part_acc, part_ml,
                       heads, kv_heads, group, max_seq, n_splits, static_cast<int>(n_units),
                       split_size, qscale);
  });
  int rc = check_hip(hipGetLastError(), "decode_split_kernel launch");
  if (rc != FA_OK) return rc;

  if (out_f32) {
    hipLaunchKernelGGL(decode_merge_kernel<true>, dim3(static_cast<unsigned>(bh)),
                       dim3(kMergeThreads), 0, stream, part_acc, part_ml, seq_lens,
                       o, heads, max_seq, n_splits, split_size);
  } else {
    hipLaunchKernelGGL(decode_merge_kernel<false>, dim3(static_cast<unsigned>(bh)),
                       dim3(kMergeThreads), 0, stream, part_acc, part_ml, seq_lens,
                       o, heads, max_seq, n_splits, split_size);
  }
  return check_hip(hipGetLastError(), "decode_merge_kernel launch");
}

int decode_occupancy(fa_occupancy_entry *out, int cap, int *n) {
  struct K { const char *name; const void *fn; int threads; };
  const K ks[] = {
      {"decode_split_kernel",
       reinterpret_cast<const void *>(decode_split_kernel<kGroupsPerStep, 1>), kSplitThreads},
      {"decode_merge_kernel",
       reinterpret_cast<const void *>(decode_merge_kernel<false>), kMergeThreads},
      {"decode_bh_kernel", reinterpret_cast<const void *>(decode_bh_kernel<1, false>),
       kBhThreads},
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
