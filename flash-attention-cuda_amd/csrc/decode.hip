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
//    the workspace, and the partials are combined in the same launch
//    (decode_split_fused_kernel): groups of W waves pre-merge in LDS, publish
//    one partial per group, and bump a per-(b, h) counter; the group that
//    arrives last merges the rest and resets the counter. Counters live in a
//    zero-initialised device array, one slot per (device, stream); a call
//    that finds no free slot takes the two-launch path (split kernel, then
//    merge kernel).
//  * B * H >= compute units, or a cache of at most 512 rows: one 8-wave
//    block per (b, h) folds the whole sequence (decode_bh_kernel below),
//    merging its waves through LDS, so no partials reach HBM and there is no
//    second kernel.
//
// Split path details, laid out for CDNA4:
//
//  * One WAVE owns one (b, h, chunk) unit; a block is one wave (grids of up
//    to 2 x CUs units) or four independent waves (no LDS, no barrier).
//    Chunks past a sequence's end exit at once.
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
//  * head_dim 128 keeps the lane -> 16 B mapping: 16 lanes per row, 4 rows
//    per load instruction, a 4-step DPP sum (RowGeo<D>).
//  * The per-lane online-softmax states are merged across the row groups of
//    the wave with shuffles, and across chunks as described above.
//  * Grouped-query attention (H_kv < H K/V heads) does not use these VALU
//    passes: decode_group_kernel (below) runs the split pass on the matrix
//    cores with up to 32 query heads of one K/V head per wave, so each cache
//    row is loaded once for all of them, and shares the merge kernel.
//
// Partial results are stored with m in the log2 domain; only this file
// produces and consumes them.

#include <hip/hip_fp16.h>

#include <algorithm>
#include <mutex>

#include "fa_internal.h"
#include "mfma_tile.h"

namespace fa {
namespace {

constexpr int kSplitThreads = 256;  // 4 independent waves
constexpr int kSplitWaves = kSplitThreads / kWave;
constexpr int kGroupsPerStep = 8;   // row groups loaded together per wave
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for m

// Row geometry of the VALU kernels for head_dim D (64 or 128): a lane owns 8
// head dims (16 B), D / 8 lanes cover one cache row, so one wave load moves
// 512 / D rows (8 rows of 128 B, or 4 rows of 256 B).
template <int D>
struct RowGeo {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static constexpr int kLanesPerRow = D / 8;
  static constexpr int kRowsPerGroup = kWave / kLanesPerRow;
};

// Sum over each aligned group of D / 8 lanes (8 or 16); every lane gets the
// group total.
template <int D>
__device__ __forceinline__ float sum_row_lanes(float x) {
  x = sum_lanes8(x);
  if constexpr (D == 128) x += dpp<kDppRowMirror>(x);
  return x;
}

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

template <int D, int G>
__device__ __forceinline__ void load_slots(RowSlotsT<G> &r, const _Float16 *kp,
                                           const _Float16 *vp, int row0,
                                           int end, int sub, int slice) {
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int row = row0 + u * RowGeo<D>::kRowsPerGroup + sub;
    if (row < end) {
      const size_t off = static_cast<size_t>(row) * D + slice * 8;
      r.k[u] = load_stream(kp + off);
      r.v[u] = load_stream(vp + off);
    } else {
      r.k[u] = make_uint4(0, 0, 0, 0);
      r.v[u] = make_uint4(0, 0, 0, 0);
    }
  }
}

// Keeps a load that only later code uses from being sunk below a branch
// between the two: each early exit "uses" the loaded value (it waits for the
// load there), so the load stays where it was written, ahead of the branch.
template <typename T, int N>
__device__ __forceinline__ void hold(const T (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" ::"v"(x[i]));
}

// Rows at or past `end` of slots loaded from row0 with a larger bound (they
// may hold any bits, NaN included, which a zero weight would not cancel).
template <int D, int G>
__device__ __forceinline__ void zero_rows_from(RowSlotsT<G> &r, int row0, int end, int sub) {
#pragma unroll
  for (int u = 0; u < G; ++u) {
    if (row0 + u * RowGeo<D>::kRowsPerGroup + sub >= end) {
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

// Fold one sub-step of rows (already loaded) into the running state. The
// q.k partial of a lane is four v_dot2_f32_f16 on the raw fp16 pairs (exact
// fp16 products, fp32 sums), scaled once by qscale = scale * log2(e).
template <int D, int G>
__device__ __forceinline__ void consume_slots(const RowSlotsT<G> &r, const half2 (&qh)[4],
                                              float qscale, int row0, int end, int sub,
                                              float &m, float &l, float (&acc)[8]) {
  float s[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const half2 *kh = reinterpret_cast<const half2 *>(&r.k[u]);
    float part = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) part = __builtin_amdgcn_fdot2(qh[t], kh[t], part, false);
    part = sum_row_lanes<D>(part);
    const int row = row0 + u * RowGeo<D>::kRowsPerGroup + sub;
    s[u] = (row < end) ? part * qscale : -INFINITY;
  }
  float mx = s[0];
#pragma unroll
  for (int u = 1; u < G; ++u) mx = fmaxf(mx, s[u]);
  const float m_new = fmaxf(m, mx);
  const float alpha = fast_exp2(m - m_new);
  float p[G];
  float psum = 0.f;
#pragma unroll
  for (int u = 0; u < G; ++u) {
    p[u] = fast_exp2(s[u] - m_new);  // masked rows: exp2(-inf) = 0
    psum += p[u];
  }
  l = fmaf(l, alpha, psum);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < G; ++u) {
    float vf[8];
    unpack8(r.v[u], vf);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(p[u], vf[e], acc[e]);
  }
  m = m_new;
}

// Head dims [8 * slice, +8) of query row bh, as fp16 pairs.
template <int D>
__device__ __forceinline__ void load_query(const _Float16 *q, size_t bh, int slice,
                                           half2 (&qh)[4]) {
  const uint4 raw = *reinterpret_cast<const uint4 *>(q + bh * D + slice * 8);
  const half2 *h = reinterpret_cast<const half2 *>(&raw);
#pragma unroll
  for (int t = 0; t < 4; ++t) qh[t] = h[t];
}

// A grouped-query unit: nq query heads that read one K/V head. The unit index
// u runs over (b, K/V head, query chunk); its queries are heads
// kv * group + chunk * nq + j (j < nq) of batch row b.
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

// Single-launch merge: the wave that finishes a (b, h)'s last live group of
// chunks merges all of its partials itself, so the split pass needs no
// second kernel. It is found with one counter per (b, h): each group
// publishes its partial, then counts itself; the wave that sees the count
// reach the number of live groups merges and sets the counter back to zero,
// so a finished call leaves every counter at zero. The counters are zero when
// the code object loads and are split into slots, one per (device, stream)
// in use, so calls that may overlap in time (other streams) never share one.
constexpr int kCounterSlots = 64;
constexpr int kCountersPerSlot = static_cast<int>(kMergeCountersPerSlot);
__device__ unsigned g_merge_counters[kCounterSlots * kCountersPerSlot];

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

// One wave merges the n_act partials of one (b, h) (slots base .. base +
// n_act - 1) with the log-sum-exp rule of the merge pass below and writes
// the output row; lane j owns head dims j and j + 64.
template <int D, bool OUT_F32>
__device__ __forceinline__ void merge_partials_wave(const float *__restrict__ part_acc,
                                                    const float *__restrict__ part_ml,
                                                    size_t base, int n_act, void *o,
                                                    size_t bh, int lane) {
  constexpr int kDims = D / kWave;  // head dims per lane (1 or 2)
  constexpr int kRound = 32;        // partial rows loaded in one round
  // One round of loads for up to kRound chunks: every (m, l) and this lane's
  // head dims of every partial row are issued before any is used.
  float m_all = kNegBig, l_part = 0.f, ms = kNegBig, ls = 0.f;
  float acc[kDims];
#pragma unroll
  for (int j = 0; j < kDims; ++j) acc[j] = 0.f;
  for (int s0 = 0; s0 < n_act; s0 += kRound) {
    const int cnt = min(kRound, n_act - s0);
    const int sl = s0 + (lane & (kRound - 1));
    const bool own = lane < kRound && sl < n_act;  // lane holds chunk sl's (m, l)
    if (own) {
      ms = load_coherent(part_ml + (base + sl) * 2);
      ls = load_coherent(part_ml + (base + sl) * 2 + 1);
    } else {
      ms = kNegBig;
      ls = 0.f;
    }
    float x[kRound][kDims];
#pragma unroll
    for (int u = 0; u < kRound; ++u)
#pragma unroll
      for (int j = 0; j < kDims; ++j)
        x[u][j] = u < cnt ? load_coherent(part_acc + (base + s0 + u) * D + lane + kWave * j) : 0.f;
    // Running log-sum-exp over the rounds (one round for <= kRound chunks).
    const float m_new = fmaxf(m_all, wave_max(ms));
    const float f = fast_exp2(m_all - m_new);
    const float w = own ? fast_exp2(ms - m_new) : 0.f;
    l_part = l_part * f + ls * w;
#pragma unroll
    for (int j = 0; j < kDims; ++j) acc[j] *= f;
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      const float wu = __shfl(w, u);
#pragma unroll
      for (int j = 0; j < kDims; ++j) acc[j] = fmaf(x[u][j], wu, acc[j]);
    }
    m_all = m_new;
  }
  const float l_all = wave_sum(l_part);
#pragma unroll
  for (int j = 0; j < kDims; ++j) {
    const float out = l_all > 0.f ? acc[j] / l_all : 0.f;
    const size_t idx = bh * D + lane + kWave * j;
    if (OUT_F32)
      static_cast<float *>(o)[idx] = out;
    else
      static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(out);
  }
}

// Pass 1 (decode.cu:50-138): one wave folds cache rows
// [chunk_i * chunk, min(len, (chunk_i + 1) * chunk)) of one (b, h) into a
// partial (m, l, acc[D]). Unit u = chunk_i * (B * H) + (b * H + h) is
// handled by wave u % W of block u / W, W = blockDim.x / 64 (1 or 4).
template <int D>
__global__ __launch_bounds__(kSplitThreads) void decode_split_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    float *__restrict__ part_acc, float *__restrict__ part_ml, int heads,
    int max_seq, int n_splits, int n_units, int chunk, float qscale) {
  const int lane = threadIdx.x & (kWave - 1);
  const int unit = static_cast<int>(blockIdx.x * (blockDim.x / kWave)) +
                   __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  if (unit >= n_units) return;
  // Chunk-major order: every (b, h)'s first chunk is dispatched first, its
  // last chunks (empty for short sequences) last, so the hardware dispatcher
  // hands out the heaviest units first (a longest-first list schedule).
  const int n_bh = n_units / n_splits;
  const int split = unit / n_bh;
  const int bh = unit % n_bh;
  const int b = bh / heads;

  const int sub = lane / RowGeo<D>::kLanesPerRow;    // row inside a row group
  const int slice = lane % RowGeo<D>::kLanesPerRow;  // head dims [8 * slice, +8)

  // decode.cu:69-71: clamp to the cache capacity. A chunk past the sequence
  // end has no rows: it writes nothing, and the merge pass only reads the
  // partials of the ceil(len / chunk) chunks that have rows.
  const int len = min(seq_lens[b], max_seq);
  const int begin = split * chunk;
  if (begin >= len) return;
  const int end = min(len, begin + chunk);

  const size_t head_off = static_cast<size_t>(bh) * max_seq * D;
  const _Float16 *kp = k_cache + head_off;
  const _Float16 *vp = v_cache + head_off;

  // Double-buffered row slots: the loads of sub-step i+1 are in flight while
  // sub-step i is consumed.
  constexpr int kStepRows = RowGeo<D>::kRowsPerGroup * kGroupsPerStep;
  RowSlotsT<kGroupsPerStep> cur, nxt;
  int row0 = begin;
  load_slots<D>(cur, kp, vp, row0, end, sub, slice);

  half2 qh[4];
  load_query<D>(q, bh, slice, qh);

  float m = kNegBig, l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;

  for (;;) {
    const int next0 = row0 + kStepRows;
    const bool more = next0 < end;
    if (more) load_slots<D>(nxt, kp, vp, next0, end, sub, slice);
    consume_slots<D>(cur, qh, qscale, row0, end, sub, m, l, acc);
    if (!more) break;
    cur = nxt;
    row0 = next0;
  }

  // Merge the row groups of the wave (lanes that share `slice`).
#pragma unroll
  for (int off = RowGeo<D>::kLanesPerRow; off < kWave; off <<= 1) {
    const float mb = __shfl_xor(m, off);
    const float lb = __shfl_xor(l, off);
    float accb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) accb[e] = __shfl_xor(acc[e], off);
    merge_state(m, l, acc, mb, lb, accb);
  }

  if (sub == 0) {
    const size_t slot = static_cast<size_t>(bh) * n_splits + split;
    float4 *dst = reinterpret_cast<float4 *>(part_acc + slot * D + slice * 8);
    dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    if (slice == 0) *reinterpret_cast<float2 *>(part_ml + slot * 2) = make_float2(m, l);
  }
}

// Single-launch split-K: a block of W waves takes W consecutive chunks
// (group g) of one (b, h). The waves merge through LDS, wave 0 publishes the
// group's partial and counts it, and the wave that counts the (b, h)'s last
// live group merges the group partials and writes o. Grouping cuts the
// partials, and the counter increments that contend on one (b, h), by W.
template <int D, bool OUT_F32, int W>
__global__ __launch_bounds__(W * kWave) void decode_split_fused_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    float *__restrict__ part_acc, float *__restrict__ part_ml, int heads, int max_seq,
    int n_groups, int chunk, float qscale, unsigned *__restrict__ counters,
    void *__restrict__ o) {
  __shared__ float s_acc[W][D];
  __shared__ float s_ml[W][2];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int bh = static_cast<int>(blockIdx.x) / n_groups;
  const int g = static_cast<int>(blockIdx.x) % n_groups;
  const int b = bh / heads;
  const int sub = lane / RowGeo<D>::kLanesPerRow;
  const int slice = lane % RowGeo<D>::kLanesPerRow;
  const int begin = (g * W + wave) * chunk;
  const size_t head_off = static_cast<size_t>(bh) * max_seq * D;
  const _Float16 *kp = k_cache + head_off;
  const _Float16 *vp = v_cache + head_off;
  // The query and the chunk's first sub-step are requested together with
  // seq_lens (one memory round trip before the rows arrive, not two): the
  // chunk start does not depend on the length, and rows below max_seq lie
  // in the cache. Rows at or past the length are zeroed once it is known.
  constexpr int kStepRows = RowGeo<D>::kRowsPerGroup * kGroupsPerStep;
  // (The row loads are predicated per lane, which keeps the compiler from
  // sinking them below the length tests; the query load is held there.)
  RowSlotsT<kGroupsPerStep> cur, nxt;
  load_slots<D>(cur, kp, vp, begin, min(max_seq, begin + chunk), sub, slice);
  half2 qh[4];
  load_query<D>(q, bh, slice, qh);
  const int len = min(seq_lens[b], max_seq);
  if (len <= 0) {
    hold(qh);
    // decode.cu:172: a sequence with no rows gets a zero output.
    if (g == 0 && wave == 0) {
#pragma unroll
      for (int j = 0; j < D / kWave; ++j) {
        const size_t idx = static_cast<size_t>(bh) * D + lane + kWave * j;
        if (OUT_F32)
          static_cast<float *>(o)[idx] = 0.f;
        else
          static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(0.f);
      }
    }
    return;
  }
  const int group_rows = W * chunk;
  const int n_live = (len + group_rows - 1) / group_rows;  // groups with rows
  if (g >= n_live) {
    hold(qh);
    return;
  }

  float m = kNegBig, l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  if (begin < len) {
    const int end = min(len, begin + chunk);
    if (begin + kStepRows > end) zero_rows_from<D>(cur, begin, end, sub);
    int row0 = begin;
    for (;;) {
      const int next0 = row0 + kStepRows;
      const bool more = next0 < end;
      if (more) load_slots<D>(nxt, kp, vp, next0, end, sub, slice);
      consume_slots<D>(cur, qh, qscale, row0, end, sub, m, l, acc);
      if (!more) break;
      cur = nxt;
      row0 = next0;
    }
  }
  // Merge the row groups of the wave, then the W waves through LDS.
#pragma unroll
  for (int off = RowGeo<D>::kLanesPerRow; off < kWave; off <<= 1) {
    const float mb = __shfl_xor(m, off);
    const float lb = __shfl_xor(l, off);
    float accb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) accb[e] = __shfl_xor(acc[e], off);
    merge_state(m, l, acc, mb, lb, accb);
  }
  if (sub == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave][slice * 8 + e] = acc[e];
    if (slice == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float mg = s_ml[0][0];
#pragma unroll
  for (int w = 1; w < W; ++w) mg = fmaxf(mg, s_ml[w][0]);
  float lg = 0.f, ag[D / kWave];
#pragma unroll
  for (int j = 0; j < D / kWave; ++j) ag[j] = 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float f = fast_exp2(s_ml[w][0] - mg);  // empty waves: l = 0, acc = 0
    lg = fmaf(s_ml[w][1], f, lg);
#pragma unroll
    for (int j = 0; j < D / kWave; ++j) ag[j] = fmaf(s_acc[w][lane + kWave * j], f, ag[j]);
  }
  // Publish the group partial, wait until it is stored, then count it.
  const size_t slot = static_cast<size_t>(bh) * n_groups + g;
#pragma unroll
  for (int j = 0; j < D / kWave; ++j) store_coherent(part_acc + slot * D + lane + kWave * j, ag[j]);
  if (lane == 0) {
    store_coherent(part_ml + slot * 2, mg);
    store_coherent(part_ml + slot * 2 + 1, lg);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  unsigned ticket = 0;
  if (lane == 0)
    ticket = __hip_atomic_fetch_add(counters + bh, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0);
  if (static_cast<int>(ticket) != n_live - 1) return;
  merge_partials_wave<D, OUT_F32>(part_acc, part_ml, static_cast<size_t>(bh) * n_groups, n_live,
                                  o, static_cast<size_t>(bh), lane);
  if (lane == 0)
    __hip_atomic_store(counters + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// D threads: lane = threadIdx.x % 64 runs the per-chunk statistics (each wave
// of a 128-thread block computes them for itself), dim = threadIdx.x is the
// head dim it accumulates.
template <int D, bool OUT_F32>
__global__ __launch_bounds__(D) void decode_merge_kernel(
    const float *__restrict__ part_acc, const float *__restrict__ part_ml,
    const int32_t *__restrict__ seq_lens, void *__restrict__ o, int heads,
    int max_seq, int n_splits, int chunk) {
  constexpr int kBatch = 16;  // chunks whose partial rows are loaded together
  const int bh = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int dim = threadIdx.x;
  const size_t base = static_cast<size_t>(bh) * n_splits;
  // Issued together, before the number of live chunks is known: seq_len, the
  // (m, l) of chunk `lane` and head dim `dim` of the first kBatch partials
  // (slots past the live ones are read, all inside the workspace, and then
  // discarded by a select).
  const int raw_len = seq_lens[bh / heads];
  float2 ml = make_float2(kNegBig, 0.f);
  if (lane < n_splits) ml = *reinterpret_cast<const float2 *>(part_ml + (base + lane) * 2);
  float x[kBatch];
  const float *col = part_acc + base * D + dim;
#pragma unroll
  for (int u = 0; u < kBatch; ++u) x[u] = (u < n_splits) ? col[u * D] : 0.f;

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
      for (int u = 0; u < kBatch; ++u) x[u] = col[(s0 + t + u) * D];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) acc = fmaf(x[u], __shfl(w, t + u), acc);
    }
    for (; t < cnt; ++t) acc = fmaf(col[(s0 + t) * D], __shfl(w, t), acc);
  }
  const float out = (l_all > 0.f) ? acc / l_all : 0.f;
  const size_t idx = static_cast<size_t>(bh) * D + dim;
  if (OUT_F32) {
    static_cast<float *>(o)[idx] = out;
  } else {
    static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(out);
  }
}

// Grouped-query split pass on the matrix cores (H_kv < H): one wave owns the
// cache rows [chunk_i * chunk, min(len, (chunk_i + 1) * chunk)) of one
// (b, K/V head) and up to 32 of the query heads that read it, and writes one
// partial (m, l, acc[64]) per query head in the layout of the VALU split pass
// above, so the same merge pass combines them. Per 32-row tile:
//   S^T = K Q^T   4 x v_mfma_f32_32x32x16_f16, the group's queries as the 32
//                 columns (columns past the group compute zeros, unused);
//   softmax       per lane: one query column, 16 of the 32 rows (the other 16
//                 in lane l ^ 32), log2 domain, rows past the chunk -> -inf;
//   O^T += V^T P^T with P split into fp16 hi + lo parts (4 + 4 MFMAs), so
//                 the weights are P to ~2^-22 at any logit width. (Rounding P
//                 once to fp16 and computing a chunk again with split P when
//                 its rounded mass was too large was 3 % faster on N(0,1)
//                 inputs but 50 % slower once q and k were 1.5x wider: a
//                 chunk's weights are normalised over its own rows, so most
//                 chunks failed the check and ran twice. C5 shape with 2 K/V
//                 heads: 13.6 -> 14.0 us per call at N(0,1), 20.8 -> 14.0 us
//                 with q and k x1.5.)
// K and V tiles stream through a per-wave LDS ring filled by direct
// global->LDS loads kGroupAhead tiles ahead (row-major, 16-byte chunks
// XOR-swizzled, as the prefill kernel's tiles), with the non-temporal hint:
// each cache row is read once per call (B8 H32/8 L4096 17.7 -> 16.1 us per
// call, the ragged C5 shape with 2 K/V heads within noise). A block is one wave, so
// nothing is shared and there is no barrier; the ring sets 5 waves per CU.
// The MFMA work per row is the same for 1 to 32 queries, so a K/V head is
// read once for its whole group at HBM speed, where the VALU path above pays
// the dot products and the P V update once per query.
constexpr int kGroupTile = 32;                           // cache rows per tile
constexpr int kGroupCols = 32;                           // queries per wave

// Ring geometry of the grouped pass for head_dim D. A tile is 32 rows of
// 2 D bytes (4 KiB at D = 64, 8 KiB at D = 128); the ring depth keeps the
// per-wave LDS at 32 KiB (5 waves per CU) for D = 64 and 48 KiB (3 waves per
// CU) for D = 128.
template <int D>
struct GroupGeo {
  static constexpr int kStages = D == 64 ? 4 : 3;        // ring depth per wave (2..4)
  static constexpr int kAhead = kStages - 1;             // tiles in flight
  static constexpr int kTileHalves = kGroupTile * D;
  static constexpr int kChunks = D / 8;                  // 16-byte chunks per row
  static constexpr int kRowsPerLoad = kWave / kChunks;   // 8 or 4
  static constexpr int kRowBlocks = kGroupTile / kRowsPerLoad;  // 4 or 8
  static constexpr int kLoads = 2 * kRowBlocks;          // K + V loads per lane per tile
  static constexpr int kWavesPerCu = (160 * 1024) / (2 * kStages * kTileHalves * 2);
};

// Wait until a ring tile is resident while the `later` (<= K) tiles issued
// after it, L loads each, may still fly (vmcnt counts at most 63).
template <int K, int L>
__device__ __forceinline__ void wait_ring(int later) {
  static_assert(K * L <= 63, "vmcnt holds at most 63 loads");
  if constexpr (K == 0) {
    wait_loads<0>();
  } else {
    if (later >= K)
      wait_loads<K * L>();
    else
      wait_ring<K - 1, L>(later);
  }
}

// Online softmax and O^T += V^T P^T for one tile whose S^T (raw q.k) is in
// `sacc`: m is the running max in the log2 domain (scores times c), l this
// lane's share of the row sum. MASK: rows >= lim of this lane's half are past
// the chunk end. P goes to the matrix cores as fp16 hi + lo parts (two PV
// products), so the weights that multiply V are P to ~2^-22 whatever the
// logit width; l sums the same fp16 values the products consume.
template <int D, bool MASK>
__device__ __forceinline__ void group_softmax_pv(floatx16 &sacc, const half8 (&vf)[2][D / 32],
                                                 int lim, float c, float &m, float &l,
                                                 floatx16 (&o)[D / 32]) {
  float mx = -INFINITY;
#pragma unroll
  for (int a = 0; a < 16; ++a) {
    if (MASK && 8 * (a >> 2) + (a & 3) >= lim) sacc[a] = -INFINITY;
    mx = fmaxf(mx, sacc[a]);
  }
  mx = max_lane_pair(mx);  // the tile has a row in range: finite
  const float m_new = fmaxf(m, mx * c);
  const float alpha = fast_exp2(m - m_new);
  m = m_new;
  const half2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  half8 p_hi[2], p_lo[2];
  float lsum = 0.f;
#pragma unroll
  for (int hs = 0; hs < 2; ++hs)
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float s0 = sacc[8 * hs + e], s1 = sacc[8 * hs + e + 1];
      float p0 = fast_exp2(fmaf(s0, c, -m_new));
      float p1 = fast_exp2(fmaf(s1, c, -m_new));
      if (MASK) {  // -inf * c is NaN when c = 0
        p0 = (s0 == -INFINITY) ? 0.f : p0;
        p1 = (s1 == -INFINITY) ? 0.f : p1;
      }
      const half2 hi2 = {static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
      p_hi[hs][e] = hi2[0];
      p_hi[hs][e + 1] = hi2[1];
      lsum = __builtin_amdgcn_fdot2(hi2, ones, lsum, false);
      const half2 lo2 = {static_cast<_Float16>(p0 - static_cast<float>(hi2[0])),
                         static_cast<_Float16>(p1 - static_cast<float>(hi2[1]))};
      p_lo[hs][e] = lo2[0];
      p_lo[hs][e + 1] = lo2[1];
      lsum = __builtin_amdgcn_fdot2(lo2, ones, lsum, false);
    }
  l = fmaf(l, alpha, lsum);
  // Rescaled on every tile (alpha is 1 where the max did not rise): behind a
  // wave-uniform branch the accumulators were copied to other registers and
  // back around it on every tile, which cost as much as the multiplies.
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) o[db][a] *= alpha;
#pragma unroll
  for (int hs = 0; hs < 2; ++hs)
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      o[db] = mfma(vf[hs][db], p_hi[hs], o[db]);
      o[db] = mfma(vf[hs][db], p_lo[hs], o[db]);
    }
}

template <int D>
__global__ __launch_bounds__(kWave) void decode_group_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    float *__restrict__ part_acc, float *__restrict__ part_ml, int heads, int kv_heads,
    int group, int nq, int max_seq, int n_splits, int n_units, int chunk, float qscale) {
  using G = GroupGeo<D>;
  constexpr int kGroupStages = G::kStages;
  constexpr int kGroupAhead = G::kAhead;
  constexpr int kGroupTileHalves = G::kTileHalves;
  constexpr int kGroupLoads = G::kLoads;
  constexpr int kDS = D / 16;  // k-steps of S^T = K Q^T
  constexpr int kDB = D / 32;  // d-blocks of O^T
  __shared__ __attribute__((aligned(1024))) _Float16 lds[2 * kGroupStages * kGroupTileHalves];
  const int unit = static_cast<int>(blockIdx.x);
  if (unit >= n_units) return;
  const int lane = threadIdx.x;
  const int col = lane & 31;
  const int g = lane >> 5;
  // Chunk-major unit order, as the VALU split pass (longest-first dispatch).
  // Within a chunk index the query units rotate by that index: block i runs
  // on XCD i % 8, and with a unit count per chunk that is a multiple of 8
  // every XCD would otherwise stream all chunks of the same sequences, so
  // ragged lengths would load the XCDs unevenly (C5 shape with 2 K/V heads:
  // rows per XCD up to 1.14x the mean, 1.02x rotated; 14.1 -> 13.7 us per
  // call, B8 H32/8 L4096 19.3 -> 17.7).
  const int n_qu = n_units / n_splits;
  const int split = unit / n_qu;
  const QueryUnit qu =
      query_unit((unit - split * n_qu + split) % n_qu, kv_heads, group / nq, group, nq);
  const int begin = split * chunk;

  const size_t kv_off = (static_cast<size_t>(qu.b) * kv_heads + qu.kv) * max_seq * D;
  const _Float16 *const kp = k_cache + kv_off;
  const _Float16 *const vp = v_cache + kv_off;
  _Float16 *const kring = lds;
  _Float16 *const vring = lds + kGroupStages * kGroupTileHalves;

  // Loads of tile t: lane = (D / 8) * (row in a row block) + 16-byte chunk;
  // 32 / (512 / D) row blocks each of K and V. Rows past the chunk end are
  // clamped to its last row (they are masked out of the softmax).
  const int rr = lane / G::kChunks;
  const int c16 = lane % G::kChunks;
  int src_k[G::kRowBlocks], src_v[G::kRowBlocks];
#pragma unroll
  for (int rb = 0; rb < G::kRowBlocks; ++rb) {
    const int r = rb * G::kRowsPerLoad + rr;  // row inside the tile (tiles start at a multiple of 32)
    src_k[rb] = (c16 ^ k_swz_d<D>(r)) << 3;
    src_v[rb] = (c16 ^ v_swz_d<D>(r)) << 3;
  }
  // The Q^T fragments are requested together with seq_lens (two memory
  // round trips before the rows arrive, not three): column `col` is query
  // head h0 + col of the unit (zeros past nq), head dims [(D / 2) g + 8 s,
  // +8) for k-step s. They are waited for before the ring's first loads: a
  // Q load still pending inside the loop would make the compiler wait for
  // every load (ring included) there. (Requesting the chunk's first tile
  // before the length as well cost more than it saved on ragged batches,
  // whose units past a sequence's end would read a tile for nothing: C5
  // shape with 2 K/V heads 15.0 -> 15.7 us.)
  const size_t bh0 = static_cast<size_t>(qu.b) * heads + qu.h0;
  const int qcol = min(col, nq - 1);  // columns past nq load a valid row, then zero it
  half8 qf[kDS];
#pragma unroll
  for (int st = 0; st < kDS; ++st)
    qf[st] = *reinterpret_cast<const half8 *>(q + (bh0 + qcol) * D + (D / 2) * g + 8 * st);
  const int len = min(seq_lens[qu.b], max_seq);
  if (begin >= len) {  // no rows: no partial (the merge skips this chunk)
    hold(qf);
    return;
  }
  const int end = min(len, begin + chunk);
  const int n_tiles = (end - begin + kGroupTile - 1) / kGroupTile;
  auto issue = [&](int t) {
    const int row0 = begin + t * kGroupTile;
    _Float16 *const ks = kring + (t % kGroupStages) * kGroupTileHalves;
    _Float16 *const vs = vring + (t % kGroupStages) * kGroupTileHalves;
#pragma unroll
    for (int rb = 0; rb < G::kRowBlocks; ++rb) {
      const size_t row =
          static_cast<size_t>(min(row0 + rb * G::kRowsPerLoad + rr, end - 1)) * D;
      global_to_lds16_nt(kp + row + src_k[rb], ks + rb * G::kRowsPerLoad * D);
      global_to_lds16_nt(vp + row + src_v[rb], vs + rb * G::kRowsPerLoad * D);
    }
  };
  // A negative scale is folded into Q (an exact fp16 negation), so the
  // softmax works with c = |scale| log2(e) > 0 and takes its max on the raw
  // scores.
  const float c_scale = fabsf(qscale);
#pragma unroll
  for (int st = 0; st < kDS; ++st) {
    if (col >= nq) qf[st] = half8{};
    if (qscale < 0.f) qf[st] = -qf[st];
    asm volatile("" ::"v"(qf[st]));
  }
#pragma unroll
  for (int t = 0; t < kGroupAhead; ++t)
    if (t < n_tiles) issue(t);

  const FragOffsetsD<D> fo = frag_offsets_d<D>(lane);
  float m = kNegBig, l = 0.f;
  floatx16 o[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) o[db][a] = 0.f;

  // The last tile is partial when the chunk's row count is not a multiple of
  // 32: only that tile is masked.
  const bool partial_tail = ((end - begin) & (kGroupTile - 1)) != 0;
  for (int t = 0; t < n_tiles; ++t) {
    // Tile t resident: the loads of the tiles issued after it (up to
    // kGroupAhead - 1 of them) may still fly.
    wait_ring<kGroupAhead - 1, kGroupLoads>(min(kGroupAhead - 1, n_tiles - 1 - t));
    const _Float16 *const ks = kring + (t % kGroupStages) * kGroupTileHalves;
    const _Float16 *const vs = vring + (t % kGroupStages) * kGroupTileHalves;
    half8 kf[kDS];
#pragma unroll
    for (int st = 0; st < kDS; ++st) kf[st] = *reinterpret_cast<const half8 *>(ks + fo.k[st]);
    half8 vf[2][kDB];  // [16-row step][d-block]
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      lds_half *pv = opaque_lds(vs + fo.v[db]);
#pragma unroll
      for (int hs = 0; hs < 2; ++hs)
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) short4v *)(pv + (16 * hs + 8 * part) * D));
          const half4 v4 = __builtin_bit_cast(half4, r);
#pragma unroll
          for (int e = 0; e < 4; ++e) vf[hs][db][4 * part + e] = v4[e];
        }
    }
    // The stage of tile t - 1 is free (its fragments were consumed): refill
    // it with tile t + kGroupAhead.
    if (t + kGroupAhead < n_tiles) issue(t + kGroupAhead);

    floatx16 sacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) sacc[a] = 0.f;
#pragma unroll
    for (int st = 0; st < kDS; ++st) sacc = mfma(kf[st], qf[st], sacc);
    if (partial_tail && t == n_tiles - 1) {
      // Element a: row 8 (a / 4) + 4 g + a % 4 of the tile.
      const int lim = end - (begin + t * kGroupTile) - 4 * g;
      group_softmax_pv<D, true>(sacc, vf, lim, c_scale, m, l, o);
    } else {
      group_softmax_pv<D, false>(sacc, vf, 0, c_scale, m, l, o);
    }
  }

  // Lanes l and l ^ 32 hold the two row halves of column col: m is shared,
  // l adds up; each lane writes its half of the D head dims.
  l += __shfl_xor(l, 32);
  if (col < nq) {
    const size_t slot = (bh0 + col) * n_splits + split;
    float *const dst = part_acc + slot * D;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
        *reinterpret_cast<float4 *>(dst + db * 32 + 8 * rb + 4 * g) =
            make_float4(o[db][4 * rb], o[db][4 * rb + 1], o[db][4 * rb + 2], o[db][4 * rb + 3]);
    if (g == 0) *reinterpret_cast<float2 *>(part_ml + slot * 2) = make_float2(m, l);
  }
}

// Whole-sequence variant for batches with at least one (b, h) per compute
// unit: one block of 8 waves owns one (b, h), and wave w folds the chunks
// w, w + 8, w + 16, ... of `chunk` rows each. Rows go in sub-steps of 32, the
// next one in flight while the current one is consumed; the 8 wave states
// merge through LDS and the block writes the output, so there is no partial
// workspace and no merge pass.
// With chunk == 0 (the automatic choice) the chunk follows the grid:
//  * every block resident at once (target_waves > 0): the batch's cache rows
//    over target_waves, so about target_waves waves stream rows, each a long
//    contiguous range (measured on ragged batches: fewer, longer streams beat
//    more, shorter ones);
//  * more blocks than fit (target_waves == 0): 1/8 of the block's own
//    sequence, so all 8 waves of each resident block stream.
// Chunks are multiples of 64 rows. Blocks take the sequences in decreasing
// length order (every block ranks the batch's lengths itself, for batches of
// up to kRankMax), so the dispatcher runs a longest-first list schedule.
constexpr int kBhWaves = 8;
constexpr int kBhThreads = kBhWaves * kWave;
constexpr int kBhGroups = 4;  // 32-row sub-steps
constexpr int kRankMax = 256;   // ranking costs batch^2 / 512 LDS reads per thread
constexpr int kBhWavesPerCu = 5;  // streaming waves per CU when the grid is resident

template <int D, bool OUT_F32>
__global__ __launch_bounds__(kBhThreads) void decode_bh_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k_cache,
    const _Float16 *__restrict__ v_cache, const int32_t *__restrict__ seq_lens,
    void *__restrict__ o, int batch, int heads, int max_seq, int chunk,
    int target_waves, float qscale) {
  __shared__ int s_len[kRankMax];
  __shared__ int s_order[kRankMax];
  __shared__ float s_acc[kBhWaves][D];
  __shared__ float s_m[kBhWaves];
  __shared__ float s_l[kBhWaves];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  // Block -> position in the longest-first order. With the whole grid
  // resident (target_waves = kBhWavesPerCu x CUs), blocks [0, CUs) take one
  // CU each and block CUs + j lands on the CU of block j. Of the n blocks,
  // the 2 CUs - n longest positions run alone (on the CUs that get no second
  // block) and the rest pair heaviest with lightest: CU j < n - CUs takes
  // position 2 CUs - n + j, then position n - 1 - j. (Config 5: the busiest
  // CU streams 4,541 rows against a 4,013 mean, 4,919 when every CU paired
  // its first-round position with the reversed second round; the launch
  // gains ~0.6 %, since the chip's HBM rate, not one CU's, sets its pace.)
  int pos = static_cast<int>(blockIdx.x);
  const int n_blocks = static_cast<int>(gridDim.x);
  const int cus = target_waves / kBhWavesPerCu;
  if (target_waves > 0 && n_blocks > cus) {
    if (n_blocks <= 2 * cus) {
      const int pairs = n_blocks - cus;  // CUs that take two blocks
      const int singles = cus - pairs;
      if (pos >= cus)
        pos = n_blocks - 1 - (pos - cus);
      else
        pos = pos < pairs ? singles + pos : pos - pairs;
    } else if (pos >= cus) {
      pos = cus + (n_blocks - 1 - pos);  // three or more per CU: later rounds reversed
    }
  }
  int b = pos / heads;
  const int h = pos % heads;
  const bool ranked = batch <= kRankMax;
  if (ranked) {
    // rank(t) = #{u : len_u > len_t or (len_u == len_t and u < t)}: block i
    // takes the (i / H)-th longest sequence.
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
    b = s_order[b];
  }
  const int bh = b * heads + h;
  const int sub = lane / RowGeo<D>::kLanesPerRow;    // row inside a row group
  const int slice = lane % RowGeo<D>::kLanesPerRow;  // head dims [8 * slice, +8)
  // The query load is issued first; after a ranking the lengths come from
  // LDS, so the first cache loads wait for no other memory round trip.
  half2 qh[4];
  load_query<D>(q, bh, slice, qh);
  const int len = ranked ? s_len[b] : max(0, min(seq_lens[b], max_seq));
  if (chunk == 0) {
    int rows_per_wave;
    if (target_waves > 0) {
      int part = 0;
      for (int t = lane; t < batch; t += kWave)
        part += ranked ? s_len[t] : max(0, min(seq_lens[t], max_seq));
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
      const float total = static_cast<float>(__builtin_amdgcn_readfirstlane(part));
      rows_per_wave = static_cast<int>(
          fminf(ceilf(total * static_cast<float>(heads) / static_cast<float>(target_waves)),
                static_cast<float>(max_seq)));
      // No wave takes a second chunk: that would double its time, and the
      // whole block waits for it.
      rows_per_wave = max(rows_per_wave, (len + kBhWaves - 1) / kBhWaves);
    } else {
      rows_per_wave = (len + kBhWaves - 1) / kBhWaves;
    }
    chunk = max(64, (rows_per_wave + 63) & ~63);
  }
  chunk = min(chunk, max_seq);  // max_seq <= 2^27 (host check): 8 * chunk fits in int

  const size_t head_off = static_cast<size_t>(bh) * max_seq * D;
  const _Float16 *kp = k_cache + head_off;
  const _Float16 *vp = v_cache + head_off;

  float m = kNegBig, l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;

  constexpr int kStepRows = RowGeo<D>::kRowsPerGroup * kBhGroups;  // 32 (D 64) / 16
  const int stride = kBhWaves * chunk;  // distance between a wave's chunks
  int c0 = wave * chunk;                // this wave's current chunk
  if (c0 < len) {
    int end = min(len, c0 + chunk);
    int row0 = c0;
    RowSlotsT<kBhGroups> cur, nxt;
    load_slots<D>(cur, kp, vp, row0, end, sub, slice);
    for (;;) {
      // Next sub-step: the rest of this chunk, else this wave's next chunk.
      int n_row0 = row0 + kStepRows, n_end = end, n_c0 = c0;
      if (n_row0 >= end) {
        n_c0 = c0 + stride;
        n_row0 = n_c0;
        n_end = min(len, n_c0 + chunk);
      }
      const bool more = n_row0 < n_end;
      if (more) load_slots<D>(nxt, kp, vp, n_row0, n_end, sub, slice);
      consume_slots<D>(cur, qh, qscale, row0, end, sub, m, l, acc);
      if (!more) break;
      cur = nxt;
      row0 = n_row0;
      end = n_end;
      c0 = n_c0;
    }
  }

  // Merge the row groups of the wave (lanes that share `slice`).
#pragma unroll
  for (int off = RowGeo<D>::kLanesPerRow; off < kWave; off <<= 1) {
    const float mb = __shfl_xor(m, off);
    const float lb = __shfl_xor(l, off);
    float accb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) accb[e] = __shfl_xor(acc[e], off);
    merge_state(m, l, acc, mb, lb, accb);
  }
  if (sub == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave][slice * 8 + e] = acc[e];
    if (slice == 0) {
      s_m[wave] = m;
      s_l[wave] = l;
    }
  }
  __syncthreads();
  if (tid < D) {
    float mb = s_m[0];
#pragma unroll
    for (int w = 1; w < kBhWaves; ++w) mb = fmaxf(mb, s_m[w]);
    float lb = 0.f, ab = 0.f;
#pragma unroll
    for (int w = 0; w < kBhWaves; ++w) {
      const float f = fast_exp2(s_m[w] - mb);  // empty waves: l = 0, acc = 0
      lb = fmaf(s_l[w], f, lb);
      ab = fmaf(s_acc[w][tid], f, ab);
    }
    // decode.cu:172: a sequence with no rows gets a zero output.
    const float out = (lb > 0.f) ? ab / lb : 0.f;
    const size_t idx = static_cast<size_t>(bh) * D + tid;
    if (OUT_F32)
      static_cast<float *>(o)[idx] = out;
    else
      static_cast<_Float16 *>(o)[idx] = static_cast<_Float16>(out);
  }
}

// Blocks of decode_bh_kernel<D> resident on one CU at once, per device.
template <int D>
int bh_blocks_per_cu(int device) {
  static std::once_flag once[kMaxDevices];
  static int blocks[kMaxDevices];
  if (device < 0 || device >= kMaxDevices) return 1;
  std::call_once(once[device], [device] {
    int n = 0;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return;
    if (hipSetDevice(device) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void *>(decode_bh_kernel<D, false>), kBhThreads, 0) !=
            hipSuccess)
      n = 0;
    (void)hipSetDevice(prev);
    blocks[device] = n;
  });
  return blocks[device] > 0 ? blocks[device] : 1;
}

// Whole-sequence blocks need at least one (b, h) per compute unit to fill
// the chip; below that, the split-K grid spreads each sequence over CUs.
// Short caches are the exception: with at most kBhShortCache rows, the
// whole-sequence block finishes in one or two 64-row chunks per wave, and
// its single launch beats the split + merge pair (GPU time at B1 H12:
// 4.2 vs 6.7 us at 128 rows, 5.1 vs 6.9 us at 512; even at 1024, and
// split-K ahead from 2048 rows).
constexpr int kBhShortCache = 512;
bool use_bh_path(int batch, int heads, int max_seq) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const int cu = device_cu_count(dev);
  return cu > 0 && (static_cast<long long>(batch) * heads >= cu || max_seq <= kBhShortCache);
}

// Queries per wave of the grouped pass: the largest divisor of the group
// that fits the 32 columns of one MFMA tile.
int group_queries(int group) {
  for (int nq = min(group, kGroupCols); nq > 1; --nq)
    if (group % nq == 0) return nq;
  return 1;
}



}  // namespace

// Counter slot of g_merge_counters for the current device and `stream`,
// claimed on first use and kept; nullptr (decode: the two-launch path;
// prefill: whole items) when n_bh counters exceed a slot or every slot is
// taken. The split-K decode and the split prefill units share a stream's
// slot: kernels on one stream run one at a time, and each leaves its
// counters at zero.
//  * hipStreamPerThread names a different stream in every thread and
//    hipStreamLegacy the legacy default stream: one handle, several streams,
//    so neither gets a slot.
//  * A stream under graph capture gets a slot of that capture's own (keyed by
//    its capture id): graphs captured one after another on one stream (as
//    torch.cuda.graph does) hold different slots and may replay concurrently.
//    Replays of one graph share its slot and must not overlap each other.
unsigned *merge_counters(hipStream_t stream, size_t n_bh) {
  if (n_bh > static_cast<size_t>(kCountersPerSlot)) return nullptr;
  if (stream == hipStreamPerThread || stream == hipStreamLegacy) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  unsigned long long capture = 0;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamGetCaptureInfo(stream, &status, &capture) != hipSuccess) {
    (void)hipGetLastError();  // the query's error is not the caller's
    return nullptr;
  }
  if (status != hipStreamCaptureStatusActive) capture = 0;
  struct Owner {
    int dev;
    hipStream_t stream;
    unsigned long long capture;
  };
  static std::mutex mu;
  static unsigned *base[kMaxDevices];
  static bool looked_up[kMaxDevices];
  static Owner owner[kCounterSlots];
  static int n_used = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (!looked_up[dev]) {
    looked_up[dev] = true;
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_merge_counters)) == hipSuccess)
      base[dev] = static_cast<unsigned *>(p);
  }
  if (base[dev] == nullptr) return nullptr;
  for (int i = 0; i < n_used; ++i)
    if (owner[i].dev == dev && owner[i].stream == stream && owner[i].capture == capture)
      return base[dev] + static_cast<size_t>(i) * kCountersPerSlot;
  if (n_used == kCounterSlots) return nullptr;
  owner[n_used] = {dev, stream, capture};
  return base[dev] + static_cast<size_t>(n_used++) * kCountersPerSlot;
}

bool decode_needs_workspace(int batch, int heads, int kv_heads, int max_seq) {
  return heads != kv_heads || !use_bh_path(batch, heads, max_seq);
}

int decode_units_per_row(int heads, int kv_heads) {
  const int group = heads / kv_heads;
  if (group == 1) return heads;
  return kv_heads * (group / group_queries(group));
}

int decode_group_chunk(int batch, int units_per_row, int max_seq, int head_dim) {
  int dev = 0;
  int cu = 0;
  if (hipGetDevice(&dev) == hipSuccess) cu = device_cu_count(dev);
  // The waves of decode_group_kernel its LDS ring lets run at once per CU.
  const int per_cu =
      head_dim == 128 ? GroupGeo<128>::kWavesPerCu : GroupGeo<64>::kWavesPerCu;
  const long long waves = static_cast<long long>(per_cu) * (cu > 0 ? cu : 256);
  const long long work = static_cast<long long>(max_seq) * batch * units_per_row;
  // head_dim 64: chunks 1.25x the one-round share, and at least 5 tiles: a
  // wave's first tile arrives ~2 us after it starts and every chunk adds a
  // partial to merge, so fewer, longer chunks win (measured per call: B32
  // H14/2 L4096 ragged 15.8 -> 14.5 us, B8 H32/8 L4096 22.2 -> 19.4, B16
  // H14/2 L2048 13.0 -> 10.1, B1 H32/8 L8192 12.1 -> 11.6, B4 H28/4 L16384
  // 15.4 -> 15.6). head_dim 128 keeps the one-round share.
  const bool d64 = head_dim != 128;
  long long rows = d64 ? (5 * work + 4 * waves - 1) / (4 * waves) : (work + waves - 1) / waves;
  rows = ((rows + kGroupTile - 1) / kGroupTile) * kGroupTile;
  const long long cap = ((static_cast<long long>(max_seq) + kGroupTile - 1) / kGroupTile) * kGroupTile;
  rows = std::max<long long>(rows, (d64 ? 5 : 2) * kGroupTile);
  return static_cast<int>(std::min(rows, std::max<long long>(cap, 2 * kGroupTile)));
}

namespace {

// The VALU kernels for head_dim D (no grouped queries): the whole-sequence
// kernel when B * H fills the chip (or the cache is short), else split-K and
// the merge.
template <int D>
int launch_valu_decode(const void *q, const void *k_cache, const void *v_cache,
                       const int32_t *seq_lens, void *o, bool out_f32, int batch, int heads,
                       int max_seq, float scale, int split_size, bool auto_split,
                       float *workspace, hipStream_t stream) {
  const int n_splits = (max_seq + split_size - 1) / split_size;
  const size_t bh = static_cast<size_t>(batch) * heads;
  if (use_bh_path(batch, heads, max_seq)) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != FA_OK) return rc;
    const int cu = device_cu_count(dev);
    const bool resident = bh <= static_cast<size_t>(bh_blocks_per_cu<D>(dev)) * cu;
    const int target_waves = resident ? kBhWavesPerCu * cu : 0;
    if (out_f32)
      hipLaunchKernelGGL((decode_bh_kernel<D, true>), dim3(static_cast<unsigned>(bh)),
                         dim3(kBhThreads), 0, stream, static_cast<const _Float16 *>(q),
                         static_cast<const _Float16 *>(k_cache),
                         static_cast<const _Float16 *>(v_cache), seq_lens, o, batch,
                         heads, max_seq, auto_split ? 0 : split_size,
                         target_waves, scale * kLog2e);
    else
      hipLaunchKernelGGL((decode_bh_kernel<D, false>), dim3(static_cast<unsigned>(bh)),
                         dim3(kBhThreads), 0, stream, static_cast<const _Float16 *>(q),
                         static_cast<const _Float16 *>(k_cache),
                         static_cast<const _Float16 *>(v_cache), seq_lens, o, batch,
                         heads, max_seq, auto_split ? 0 : split_size,
                         target_waves, scale * kLog2e);
    return check_hip(hipGetLastError(), "decode_bh_kernel launch");
  }
  float *part_acc = workspace;
  float *part_ml = workspace + bh * n_splits * D;
  const size_t n_units = bh * n_splits;
  // Up to 2 x CUs units (the chunk chooser's own target), one-wave blocks
  // put the units on every CU instead of a quarter of them (measured per
  // call: B1 H12 L4096 8.2 against 8.5 us, B2 H8 L16384 18.7 against 21.5);
  // above that, four-wave blocks (B4 H12 L4096: 13.3 against 14.9 us).
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != FA_OK) return rc;
  const int waves_per_block =
      n_units <= 2 * static_cast<size_t>(device_cu_count(dev)) ? 1 : kSplitWaves;
  const unsigned split_blocks =
      static_cast<unsigned>((n_units + waves_per_block - 1) / waves_per_block);

  // One launch when a counter slot is free: each group of W waves merges
  // in LDS and the last group of a (b, h) merges the groups (W = 4 for
  // chunks of up to 256 rows, where the per-chunk merge traffic and counter
  // contention dominate; 2 for longer chunks, where more blocks stream).
  // Else the split pass, then the merge pass.
  unsigned *const counters = merge_counters(stream, bh);
  if (counters != nullptr) {
    const int w = split_size <= 256 ? 4 : 2;
    const int n_groups = (n_splits + w - 1) / w;
    const unsigned blocks = static_cast<unsigned>(bh * n_groups);
    const float qs = scale * kLog2e;
    const auto *qp = static_cast<const _Float16 *>(q);
    const auto *kp = static_cast<const _Float16 *>(k_cache);
    const auto *vp = static_cast<const _Float16 *>(v_cache);
    if (w == 4) {
      if (out_f32)
        hipLaunchKernelGGL((decode_split_fused_kernel<D, true, 4>), dim3(blocks), dim3(4 * kWave),
                           0, stream, qp, kp, vp, seq_lens, part_acc, part_ml, heads, max_seq,
                           n_groups, split_size, qs, counters, o);
      else
        hipLaunchKernelGGL((decode_split_fused_kernel<D, false, 4>), dim3(blocks), dim3(4 * kWave),
                           0, stream, qp, kp, vp, seq_lens, part_acc, part_ml, heads, max_seq,
                           n_groups, split_size, qs, counters, o);
    } else {
      if (out_f32)
        hipLaunchKernelGGL((decode_split_fused_kernel<D, true, 2>), dim3(blocks), dim3(2 * kWave),
                           0, stream, qp, kp, vp, seq_lens, part_acc, part_ml, heads, max_seq,
                           n_groups, split_size, qs, counters, o);
      else
        hipLaunchKernelGGL((decode_split_fused_kernel<D, false, 2>), dim3(blocks), dim3(2 * kWave),
                           0, stream, qp, kp, vp, seq_lens, part_acc, part_ml, heads, max_seq,
                           n_groups, split_size, qs, counters, o);
    }
    return check_hip(hipGetLastError(), "decode_split_fused_kernel launch");
  }
  hipLaunchKernelGGL((decode_split_kernel<D>), dim3(split_blocks),
                     dim3(waves_per_block * kWave), 0, stream,
                     static_cast<const _Float16 *>(q),
                     static_cast<const _Float16 *>(k_cache),
                     static_cast<const _Float16 *>(v_cache), seq_lens,
                     part_acc, part_ml, heads, max_seq, n_splits,
                     static_cast<int>(n_units), split_size, scale * kLog2e);
  rc = check_hip(hipGetLastError(), "decode_split_kernel launch");
  if (rc != FA_OK) return rc;

  if (out_f32) {
    hipLaunchKernelGGL((decode_merge_kernel<D, true>), dim3(static_cast<unsigned>(bh)),
                       dim3(D), 0, stream, part_acc, part_ml, seq_lens,
                       o, heads, max_seq, n_splits, split_size);
  } else {
    hipLaunchKernelGGL((decode_merge_kernel<D, false>), dim3(static_cast<unsigned>(bh)),
                       dim3(D), 0, stream, part_acc, part_ml, seq_lens,
                       o, heads, max_seq, n_splits, split_size);
  }
  return check_hip(hipGetLastError(), "decode_merge_kernel launch");
}

// Grouped queries: the matrix-core split pass, then the common merge.
template <int D>
int launch_group_decode(const void *q, const void *k_cache, const void *v_cache,
                        const int32_t *seq_lens, void *o, bool out_f32, int batch, int heads,
                        int kv_heads, int max_seq, float scale, int split_size,
                        float *workspace, hipStream_t stream) {
  const int group = heads / kv_heads;
  const int nqg = group_queries(group);
  const size_t n_qg = static_cast<size_t>(batch) * kv_heads * (group / nqg);
  const int n_sp = (max_seq + split_size - 1) / split_size;
  const size_t n_gu = n_qg * n_sp;
  float *part_acc = workspace;
  float *part_ml = workspace + static_cast<size_t>(batch) * heads * n_sp * D;
  hipLaunchKernelGGL((decode_group_kernel<D>), dim3(static_cast<unsigned>(n_gu)), dim3(kWave),
                     0, stream, static_cast<const _Float16 *>(q),
                     static_cast<const _Float16 *>(k_cache),
                     static_cast<const _Float16 *>(v_cache), seq_lens, part_acc, part_ml,
                     heads, kv_heads, group, nqg, max_seq, n_sp, static_cast<int>(n_gu),
                     split_size, scale * kLog2e);
  int rc = check_hip(hipGetLastError(), "decode_group_kernel launch");
  if (rc != FA_OK) return rc;
  const unsigned n_bh = static_cast<unsigned>(static_cast<size_t>(batch) * heads);
  if (out_f32)
    hipLaunchKernelGGL((decode_merge_kernel<D, true>), dim3(n_bh), dim3(D), 0, stream,
                       part_acc, part_ml, seq_lens, o, heads, max_seq, n_sp, split_size);
  else
    hipLaunchKernelGGL((decode_merge_kernel<D, false>), dim3(n_bh), dim3(D), 0, stream,
                       part_acc, part_ml, seq_lens, o, heads, max_seq, n_sp, split_size);
  return check_hip(hipGetLastError(), "decode_merge_kernel launch");
}

}  // namespace

int launch_decode(const void *q, const void *k_cache, const void *v_cache,
                  const int32_t *seq_lens, void *o, bool out_f32, int batch,
                  int heads, int kv_heads, int max_seq, int head_dim, float scale,
                  int split_size, bool auto_split, float *workspace, hipStream_t stream) {
  if (heads != kv_heads) {
    if (head_dim == 128)
      return launch_group_decode<128>(q, k_cache, v_cache, seq_lens, o, out_f32, batch, heads,
                                      kv_heads, max_seq, scale, split_size, workspace, stream);
    return launch_group_decode<64>(q, k_cache, v_cache, seq_lens, o, out_f32, batch, heads,
                                   kv_heads, max_seq, scale, split_size, workspace, stream);
  }
  if (head_dim == 128)
    return launch_valu_decode<128>(q, k_cache, v_cache, seq_lens, o, out_f32, batch, heads,
                                   max_seq, scale, split_size, auto_split, workspace, stream);
  return launch_valu_decode<64>(q, k_cache, v_cache, seq_lens, o, out_f32, batch, heads,
                                max_seq, scale, split_size, auto_split, workspace, stream);
}

int decode_occupancy(fa_occupancy_entry *out, int cap, int *n) {
  struct K { const char *name; const void *fn; int threads; };
  // The split-K path runs decode_split_fused_kernel (4 waves per block for
  // chunks of <= 256 rows, else 2); decode_split_kernel + decode_merge_kernel
  // serve it when no counter slot is free.
  const K ks[] = {
      {"decode_split_fused_kernel<waves=4>",
       reinterpret_cast<const void *>(decode_split_fused_kernel<64, false, 4>), 4 * kWave},
      {"decode_split_fused_kernel<waves=2>",
       reinterpret_cast<const void *>(decode_split_fused_kernel<64, false, 2>), 2 * kWave},
      {"decode_split_kernel", reinterpret_cast<const void *>(decode_split_kernel<64>),
       kSplitThreads},
      {"decode_merge_kernel",
       reinterpret_cast<const void *>(decode_merge_kernel<64, false>), kHeadDim},
      {"decode_bh_kernel", reinterpret_cast<const void *>(decode_bh_kernel<64, false>),
       kBhThreads},
      {"decode_group_kernel", reinterpret_cast<const void *>(decode_group_kernel<64>), kWave},
      {"decode_split_fused_kernel<head_dim=128, waves=4>",
       reinterpret_cast<const void *>(decode_split_fused_kernel<128, false, 4>), 4 * kWave},
      {"decode_split_fused_kernel<head_dim=128, waves=2>",
       reinterpret_cast<const void *>(decode_split_fused_kernel<128, false, 2>), 2 * kWave},
      {"decode_split_kernel<head_dim=128>",
       reinterpret_cast<const void *>(decode_split_kernel<128>), kSplitThreads},
      {"decode_merge_kernel<head_dim=128>",
       reinterpret_cast<const void *>(decode_merge_kernel<128, false>), 128},
      {"decode_bh_kernel<head_dim=128>",
       reinterpret_cast<const void *>(decode_bh_kernel<128, false>), kBhThreads},
      {"decode_group_kernel<head_dim=128>",
       reinterpret_cast<const void *>(decode_group_kernel<128>), kWave},
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
