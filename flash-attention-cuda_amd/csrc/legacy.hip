// The reference's v1 single-head fp32 kernels (legacy_naive / legacy_tiled /
// legacy_fused), rebuilt for gfx950.
//
// Reference behaviour (csrc/legacy/legacy_ops.cu:10-51 and
// src/legacy/{naive,tiled,fused}_attention.cu of shrvan30/flash-attention-cuda):
// q, k, v and o are (N, 64) fp32, one head, no mask, and
// o = softmax(q k^T / sqrt(64)) v in fp32. The three v1 kernels compute the
// same function with different algorithms:
//   naive  an exact row max over every key first, then the exponentials and
//          the weighted sum (naive_attention.cu:45-110, three passes there);
//   tiled  an online softmax over 32-key tiles with O renormalised at every
//          tile, O = (l_old * e^(m_old - m_new) O + e^(m_tile - m_new) PV) / l_new
//          (tiled_attention.cu:170-205);
//   fused  the same online softmax with the two factors computed once per
//          tile (fused_attention.cu:160-183).
// The v1 warp reductions return each thread's own value
// (softmax_stable.cu / fused_attention.cu:26-52), so every row is independent.
//
// This build keeps the three entry points and their arithmetic contract
// (fp32 in, fp32 products and sums, fp32 out); the kernels are its own:
//   block   = 4 waves over 64 query rows; lane = row, wave w = key quarter:
//             of every 64-key tile staged in LDS, wave w takes rows
//             [16 w, +16), so all lanes of a wave read the same K / V row
//             (an LDS broadcast) while each keeps its own query in registers.
//   merge   the four quarter states (m, l, o[64]) of each row meet in LDS; wave
//             w then finishes head dims [16 w, +16) of all 64 rows.
//   naive   pass 1 folds only the row max (the quarters' maxima merged in
//             LDS), pass 2 accumulates e^(s - m) and e^(s - m) v with that
//             exact max, one division at the end.
//   tiled   online softmax, O kept normalised after every tile.
//   fused   online softmax, O unnormalised, one division at the end.
// The launch is asynchronous on the caller's stream (the v1 launchers
// synchronised the device after every call, naive_attention.cu:150).

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kLegacyRows = 64;          // query rows per block (one per lane)
constexpr int kLegacyQuarters = 4;       // waves per block
constexpr int kLegacyThreads = kLegacyRows * kLegacyQuarters;
constexpr int kLegacyTile = 64;          // keys staged per tile
constexpr int kLegacyKeysPerWave = kLegacyTile / kLegacyQuarters;  // 16
constexpr int kLegacyState = kHeadDim + 2;  // o[64], m, l

enum LegacyMode { kNaive = 0, kTiled = 1, kFused = 2 };

// Stage keys [key0, key0 + 64) of k and v (fp32 rows of 64) into LDS; rows
// past n are zero (their scores are masked).
__device__ __forceinline__ void stage_tile(const float *__restrict__ k,
                                           const float *__restrict__ v, int n, int key0,
                                           float *ks, float *vs, bool with_v) {
  // 64 rows x 16 float4 per tile: 4 float4 of K (and of V) per thread.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = static_cast<int>(threadIdx.x) + i * kLegacyThreads;  // [0, 1024)
    const int row = idx >> 4, c4 = idx & 15;
    const int key = key0 + row;
    float4 kv4 = make_float4(0.f, 0.f, 0.f, 0.f), vv4 = kv4;
    if (key < n) {
      const size_t off = static_cast<size_t>(key) * kHeadDim + c4 * 4;
      kv4 = *reinterpret_cast<const float4 *>(k + off);
      if (with_v) vv4 = *reinterpret_cast<const float4 *>(v + off);
    }
    reinterpret_cast<float4 *>(ks)[idx] = kv4;
    if (with_v) reinterpret_cast<float4 *>(vs)[idx] = vv4;
  }
}

// Scores of this lane's query against the wave's 16 keys of the staged tile.
__device__ __forceinline__ void tile_scores(const float (&qr)[kHeadDim], const float *ks,
                                            int wave, int key0, int n, float scale,
                                            float (&s)[kLegacyKeysPerWave]) {
#pragma unroll
  for (int j = 0; j < kLegacyKeysPerWave; ++j) {
    const float4 *krow =
        reinterpret_cast<const float4 *>(ks + (wave * kLegacyKeysPerWave + j) * kHeadDim);
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < kHeadDim / 4; ++c) {
      const float4 kk = krow[c];
      acc = fmaf(qr[4 * c], kk.x, acc);
      acc = fmaf(qr[4 * c + 1], kk.y, acc);
      acc = fmaf(qr[4 * c + 2], kk.z, acc);
      acc = fmaf(qr[4 * c + 3], kk.w, acc);
    }
    const bool valid = key0 + wave * kLegacyKeysPerWave + j < n;
    s[j] = valid ? acc * scale : -INFINITY;
  }
}

// o += sum_j p_j v_j over the wave's 16 keys of the staged tile.
__device__ __forceinline__ void tile_pv(const float (&p)[kLegacyKeysPerWave], const float *vs,
                                        int wave, float (&o)[kHeadDim]) {
#pragma unroll
  for (int j = 0; j < kLegacyKeysPerWave; ++j) {
    const float4 *vrow =
        reinterpret_cast<const float4 *>(vs + (wave * kLegacyKeysPerWave + j) * kHeadDim);
#pragma unroll
    for (int c = 0; c < kHeadDim / 4; ++c) {
      const float4 vv = vrow[c];
      o[4 * c] = fmaf(p[j], vv.x, o[4 * c]);
      o[4 * c + 1] = fmaf(p[j], vv.y, o[4 * c + 1]);
      o[4 * c + 2] = fmaf(p[j], vv.z, o[4 * c + 2]);
      o[4 * c + 3] = fmaf(p[j], vv.w, o[4 * c + 3]);
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(kLegacyThreads) void legacy_attention_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ o, int n, float scale) {
  // [K tile | V tile] while streaming, [quarter][66][64 lanes] for the merge.
  __shared__ __attribute__((aligned(16))) float lds[kLegacyQuarters * kLegacyState * kLegacyRows];
  float *const ks = lds;
  float *const vs = lds + kLegacyTile * kHeadDim;

  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int row = static_cast<int>(blockIdx.x) * kLegacyRows + lane;
  const bool row_ok = row < n;

  float qr[kHeadDim];
  {
    const float4 *qrow = reinterpret_cast<const float4 *>(q + static_cast<size_t>(row_ok ? row : 0) * kHeadDim);
#pragma unroll
    for (int c = 0; c < kHeadDim / 4; ++c) {
      const float4 x = row_ok ? qrow[c] : make_float4(0.f, 0.f, 0.f, 0.f);
      qr[4 * c] = x.x; qr[4 * c + 1] = x.y; qr[4 * c + 2] = x.z; qr[4 * c + 3] = x.w;
    }
  }
  float acc[kHeadDim];
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) acc[d] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int n_tiles = (n + kLegacyTile - 1) / kLegacyTile;
  float s[kLegacyKeysPerWave];

  if (MODE == kNaive) {
    // Pass 1: the exact row max over every key.
    for (int t = 0; t < n_tiles; ++t) {
      __syncthreads();
      stage_tile(k, v, n, t * kLegacyTile, ks, vs, false);
      __syncthreads();
      tile_scores(qr, ks, wave, t * kLegacyTile, n, scale, s);
#pragma unroll
      for (int j = 0; j < kLegacyKeysPerWave; ++j) m = fmaxf(m, s[j]);
    }
    __syncthreads();
    float *mx = lds + kLegacyTile * kHeadDim * 2;  // after the K / V tiles
    mx[wave * kLegacyRows + lane] = m;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kLegacyQuarters; ++w) m = fmaxf(m, mx[w * kLegacyRows + lane]);
  }

  // Pass 2 (naive) or the only pass (tiled, fused).
  for (int t = 0; t < n_tiles; ++t) {
    __syncthreads();
    stage_tile(k, v, n, t * kLegacyTile, ks, vs, true);
    __syncthreads();
    tile_scores(qr, ks, wave, t * kLegacyTile, n, scale, s);
    if (MODE == kNaive) {
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < kLegacyKeysPerWave; ++j) {
        s[j] = (s[j] == -INFINITY) ? 0.f : expf(s[j] - m);
        ls += s[j];
      }
      l += ls;
      tile_pv(s, vs, wave, acc);
    } else {
      float mt = -INFINITY;
#pragma unroll
      for (int j = 0; j < kLegacyKeysPerWave; ++j) mt = fmaxf(mt, s[j]);
      if (mt == -INFINITY) continue;  // the wave's 16 keys are all past n
      const float m_new = fmaxf(m, mt);
      const float a_old = expf(m - m_new);  // 0 on the first tile (m = -inf)
      float lt = 0.f;
#pragma unroll
      for (int j = 0; j < kLegacyKeysPerWave; ++j) {
        s[j] = (s[j] == -INFINITY) ? 0.f : expf(s[j] - m_new);
        lt += s[j];
      }
      const float l_new = l * a_old + lt;
      if (MODE == kTiled) {
        // O stays normalised: O = O * (l a_old / l_new) + sum_j (p_j / l_new) v_j.
        const float c_old = l * a_old / l_new, inv = 1.0f / l_new;
#pragma unroll
        for (int d = 0; d < kHeadDim; ++d) acc[d] *= c_old;
#pragma unroll
        for (int j = 0; j < kLegacyKeysPerWave; ++j) s[j] *= inv;
      } else {
#pragma unroll
        for (int d = 0; d < kHeadDim; ++d) acc[d] *= a_old;
      }
      tile_pv(s, vs, wave, acc);
      m = m_new;
      l = l_new;
    }
  }

  // Merge the four quarter states of each row.
  __syncthreads();
  float *mine = lds + wave * (kLegacyState * kLegacyRows) + lane;
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) mine[d * kLegacyRows] = acc[d];
  mine[kHeadDim * kLegacyRows] = m;
  mine[(kHeadDim + 1) * kLegacyRows] = l;
  __syncthreads();
  float mw[kLegacyQuarters], lw[kLegacyQuarters];
  float m_all = -INFINITY;
#pragma unroll
  for (int w = 0; w < kLegacyQuarters; ++w) {
    const float *st = lds + w * (kLegacyState * kLegacyRows) + lane;
    mw[w] = st[kHeadDim * kLegacyRows];
    lw[w] = st[(kHeadDim + 1) * kLegacyRows];
    m_all = fmaxf(m_all, mw[w]);
  }
  // Weight of quarter w's unnormalised sums: e^(m_w - m_all) (tiled states
  // are normalised, so their sums are o_w * l_w).
  float f[kLegacyQuarters], l_all = 0.f;
#pragma unroll
  for (int w = 0; w < kLegacyQuarters; ++w) {
    f[w] = (lw[w] > 0.f) ? expf(mw[w] - m_all) : 0.f;
    l_all += f[w] * lw[w];
    if (MODE == kTiled) f[w] *= lw[w];
  }
  const float inv_l = (l_all > 0.f) ? 1.0f / l_all : 0.f;
  if (row_ok) {
    float *orow = o + static_cast<size_t>(row) * kHeadDim + wave * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = wave * 16 + 4 * c + e;
        float x = 0.f;
#pragma unroll
        for (int w = 0; w < kLegacyQuarters; ++w)
          x = fmaf(f[w], lds[w * (kLegacyState * kLegacyRows) + d * kLegacyRows + lane], x);
        r[e] = x * inv_l;
      }
      reinterpret_cast<float4 *>(orow)[c] = make_float4(r[0], r[1], r[2], r[3]);
    }
  }
}

}  // namespace

int launch_legacy_attention(const float *q, const float *k, const float *v, float *o, int n,
                            int variant, hipStream_t stream) {
  const float scale = 1.0f / sqrtf(static_cast<float>(kHeadDim));
  const unsigned blocks = static_cast<unsigned>((n + kLegacyRows - 1) / kLegacyRows);
  switch (variant) {
    case kNaive:
      hipLaunchKernelGGL(legacy_attention_kernel<kNaive>, dim3(blocks), dim3(kLegacyThreads), 0,
                         stream, q, k, v, o, n, scale);
      break;
    case kTiled:
      hipLaunchKernelGGL(legacy_attention_kernel<kTiled>, dim3(blocks), dim3(kLegacyThreads), 0,
                         stream, q, k, v, o, n, scale);
      break;
    default:
      hipLaunchKernelGGL(legacy_attention_kernel<kFused>, dim3(blocks), dim3(kLegacyThreads), 0,
                         stream, q, k, v, o, n, scale);
      break;
  }
  return check_hip(hipGetLastError(), "legacy_attention_kernel launch");
}

}  // namespace fa
