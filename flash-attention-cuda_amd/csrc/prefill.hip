// Causal / full FlashAttention prefill for head_dim 64 on gfx950 MFMA.
//
// Reference behaviour: prefill_kernel<CAUSAL> and launch_prefill in
// csrc/prefill.cu:164-373 of shrvan30/flash-attention-cuda (online softmax
// over key tiles, causal tile skipping :208-212, mask `k < N && k <= q`
// :268, 1/l with an l > 0 guard :334). The reference runs both products on
// scalar FP32 FMAs; here both are dense fp16 contractions on the matrix
// cores with fp32 accumulation.
//
// Work decomposition
//   block  = 4 waves = 128 query rows of one (b, h); waves own 32 rows each.
//   tile   = 64 keys, staged in LDS (K row-major, V transposed), double
//            buffered, refilled from registers that were loaded one tile
//            ahead (the global loads overlap the MFMA work of a tile).
//
// Products (v_mfma_f32_32x32x16_f16, lane l: column l % 32, half g = l / 32)
//   S^T = K Q^T : A = K rows (32 keys x 16 dims), B = Q^T (16 dims x 32
//                 queries, resident in registers for the whole block). The
//                 accumulator gives each lane ONE query column and 16 keys, so
//                 the softmax statistics of a query live in a lane pair
//                 (l, l ^ 32) and the row max needs one cross-half exchange.
//   O^T += V^T P^T : B = P^T comes straight from the S^T accumulators
//                 (fp32 -> fp16 pack, no data movement), A = V^T read from
//                 the transposed LDS tile. The O^T accumulator again gives
//                 each lane one query column, so the online-softmax rescale
//                 is a per-lane scalar multiply.
//   The contraction index order inside an MFMA is free as long as A and B
//   agree; the head-dim order of Q/K and the key order of V^T are chosen so
//   that every fragment is one 16-byte load.
//
// Softmax: log2 domain, p = exp2(s * c - m * c) with c = |scale| * log2(e)
// (a negative scale is folded into Q by an exact fp16 negation). On tiles
// that carry a mask (causal diagonal, ragged tail) and whenever the key
// range is short, P is split into hi + lo fp16 parts and the PV product is
// issued twice: those rows have few, large weights, where a single fp16
// rounding of P would cost up to ~4e-4 of output accuracy.

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;  // 4
constexpr int kRowsPerWave = 32;
constexpr int kBr = kWaves * kRowsPerWave;  // 128 query rows per block
constexpr int kBc = 64;                     // keys per tile
constexpr int kTileHalves = kBc * kHeadDim; // 4096 halves = 8 KiB
constexpr int kSplitPAllTilesBelow = 512;   // short key ranges: split P everywhere

// LDS tile addressing. Both tiles are 64 rows of 128 B (8 chunks of 16 B);
// chunk c of row r is stored at chunk c ^ swz(r), so the 8 lanes of an LDS
// phase that read the same logical chunk from 8 consecutive rows hit 8
// different bank groups.
__device__ __forceinline__ int k_swz(int row) { return row & 7; }
__device__ __forceinline__ int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }

// Position of key `kk` (0..63) inside a transposed V row: keys are permuted
// inside every 16-key group (bits 2 and 3 swapped) so the 8 keys one lane
// feeds to a PV MFMA are contiguous.
__device__ __forceinline__ int vt_pos(int kk) {
  const int r = kk & 15;
  return (kk & ~15) | (((r >> 2) & 1) << 3) | ((r >> 3) << 2) | (r & 3);
}

struct TileRegs {
  uint4 k[2];   // two 16 B chunks of K
  uint4 v[2];   // rows 2p and 2p+1, same 8 dims
};

// Global -> registers for key tile starting at `key0`; rows >= seq are zero.
__device__ __forceinline__ void load_tile(TileRegs &t, const _Float16 *kp,
                                          const _Float16 *vp, int key0,
                                          int seq, int tid) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int c = tid + it * kThreads;
    const int row = c >> 3, ch = c & 7;
    const int key = key0 + row;
    t.k[it] = (key < seq) ? *reinterpret_cast<const uint4 *>(
                                kp + static_cast<size_t>(key) * kHeadDim + ch * 8)
                          : make_uint4(0, 0, 0, 0);
  }
  const int pair = tid >> 3, ch = tid & 7;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int key = key0 + 2 * pair + it;
    t.v[it] = (key < seq) ? *reinterpret_cast<const uint4 *>(
                                vp + static_cast<size_t>(key) * kHeadDim + ch * 8)
                          : make_uint4(0, 0, 0, 0);
  }
}

// Registers -> LDS: K row-major (swizzled chunks), V transposed to [d][pos].
__device__ __forceinline__ void store_tile(const TileRegs &t, _Float16 *k_lds,
                                           _Float16 *vt_lds, int tid) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int c = tid + it * kThreads;
    const int row = c >> 3, ch = c & 7;
    *reinterpret_cast<uint4 *>(k_lds + row * kHeadDim +
                               ((ch ^ k_swz(row)) << 3)) = t.k[it];
  }
  const int pair = tid >> 3, ch = tid & 7;
  const int pos = vt_pos(2 * pair);  // 2 * pair + 1 lands at pos + 1
  const uint32_t *r0 = reinterpret_cast<const uint32_t *>(&t.v[0]);
  const uint32_t *r1 = reinterpret_cast<const uint32_t *>(&t.v[1]);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    // dims 2w and 2w+1 of this chunk; pack (row 2p, row 2p+1) per dim.
    const uint32_t lo = __builtin_amdgcn_perm(r1[w], r0[w], 0x05040100u);
    const uint32_t hi = __builtin_amdgcn_perm(r1[w], r0[w], 0x07060302u);
    const int d0 = ch * 8 + 2 * w;
    const int d1 = d0 + 1;
    *reinterpret_cast<uint32_t *>(
        vt_lds + d0 * kBc + (((pos >> 3) ^ vt_swz(d0)) << 3) + (pos & 7)) = lo;
    *reinterpret_cast<uint32_t *>(
        vt_lds + d1 * kBc + (((pos >> 3) ^ vt_swz(d1)) << 3) + (pos & 7)) = hi;
  }
}

__device__ __forceinline__ half8 lds_frag(const _Float16 *p) {
  return *reinterpret_cast<const half8 *>(p);
}

// One key tile for one wave: S^T = K Q^T, mask, online softmax, O^T += V^T P^T.
// MASK: the tile holds keys past the sequence end or above the causal
// diagonal. SPLIT: P is fed to the PV product as hi + lo fp16 parts.
template <bool CAUSAL, bool MASK, bool SPLIT>
__device__ __forceinline__ void tile_step(const _Float16 *__restrict__ kl,
                                          const _Float16 *__restrict__ vl,
                                          const half8 qf[4], int key0, int seq,
                                          int my_q, int col, int g,
                                          float c_scale, floatx16 acc_o[2],
                                          float &m_raw, float &m_scaled,
                                          float &l_part) {
  // ---- S^T = K Q^T over two 32-key blocks ----------------------------------
  floatx16 s_acc[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int a = 0; a < 16; ++a) s_acc[kb][a] = 0.f;
    const int row = kb * 32 + col;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int ch = 4 * g + s;
      const half8 kf = lds_frag(kl + row * kHeadDim + ((ch ^ k_swz(row)) << 3));
      s_acc[kb] =
          __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], s_acc[kb], 0, 0, 0);
    }
  }

  // ---- mask, running max ---------------------------------------------------
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      if (MASK) {
        const int key = key0 + kb * 32 + 8 * (a >> 2) + 4 * g + (a & 3);
        const bool keep = key < seq && (!CAUSAL || key <= my_q);
        s_acc[kb][a] = keep ? s_acc[kb][a] : -INFINITY;
      }
      mx = fmaxf(mx, s_acc[kb][a]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_raw_new = fmaxf(m_raw, mx);
  const float m_scaled_new = fmaxf(m_raw_new * c_scale, -3.0e38f);
  const float alpha = fast_exp2(m_scaled - m_scaled_new);
  m_raw = m_raw_new;
  m_scaled = m_scaled_new;

  // ---- p = exp2(s c - m c), row-sum share, rescale O -----------------------
  float psum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      float p = fast_exp2(fmaf(s_acc[kb][a], c_scale, -m_scaled_new));
      if (MASK) p = (s_acc[kb][a] == -INFINITY) ? 0.f : p;
      s_acc[kb][a] = p;
      psum += p;
    }
  }
  l_part = fmaf(l_part, alpha, psum);
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) acc_o[db][a] *= alpha;

  // ---- O^T += V^T P^T --------------------------------------------------------
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int kb = ks >> 1, h = ks & 1;
    half8 p_hi, p_lo;
#pragma unroll
    for (int t8 = 0; t8 < 8; ++t8) {
      const float p = s_acc[kb][8 * h + t8];
      p_hi[t8] = static_cast<_Float16>(p);
      if (SPLIT) p_lo[t8] = static_cast<_Float16>(p - static_cast<float>(p_hi[t8]));
    }
    const int ch = 4 * kb + 2 * h + g;  // logical 16 B chunk of the V^T row
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int d = db * 32 + col;
      const half8 vf = lds_frag(vl + d * kBc + ((ch ^ vt_swz(d)) << 3));
      acc_o[db] =
          __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_hi, acc_o[db], 0, 0, 0);
      if (SPLIT)
        acc_o[db] =
            __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_lo, acc_o[db], 0, 0, 0);
    }
  }
}

template <bool CAUSAL, bool OUT_F32>
__global__ __launch_bounds__(kThreads) void prefill_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k,
    const _Float16 *__restrict__ v, void *__restrict__ o, int seq,
    int n_qtiles, float c_scale, bool negate_q) {
  __shared__ __attribute__((aligned(16))) _Float16 k_lds[2][kTileHalves];
  __shared__ __attribute__((aligned(16))) _Float16 vt_lds[2][kTileHalves];

  // Heaviest (last) query tiles first: with causal masking their key range
  // is the longest, so dispatching them early shortens the tail.
  const int bh_count = gridDim.x / n_qtiles;
  const int qtile = n_qtiles - 1 - static_cast<int>(blockIdx.x) / bh_count;
  const int bh = static_cast<int>(blockIdx.x) % bh_count;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int col = lane & 31;  // query column (and K row / V^T row) of lane
  const int g = lane >> 5;    // which half of the 64 lanes

  const size_t head_off = static_cast<size_t>(bh) * seq * kHeadDim;
  const _Float16 *qp = q + head_off;
  const _Float16 *kp = k + head_off;
  const _Float16 *vp = v + head_off;

  const int q0 = qtile * kBr;
  const int qw0 = q0 + wave * kRowsPerWave;  // first query row of this wave
  const int my_q = qw0 + col;

  // Q^T fragments (B operand of S^T = K Q^T): lane holds query `my_q`,
  // head dims [32 g + 8 s, 32 g + 8 s + 8) for d-step s.
  half8 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (my_q < seq) {
      qf[s] = *reinterpret_cast<const half8 *>(
          qp + static_cast<size_t>(my_q) * kHeadDim + 32 * g + 8 * s);
      if (negate_q) qf[s] = -qf[s];
    } else {
      qf[s] = half8{};
    }
  }

  const int key_end = CAUSAL ? min(seq, q0 + kBr) : seq;
  const int n_tiles = (key_end + kBc - 1) / kBc;
  // Keys this wave can see at all (causal); tiles past them are skipped.
  const int wave_key_end = CAUSAL ? min(seq, qw0 + kRowsPerWave) : seq;
  const bool short_range = seq < kSplitPAllTilesBelow;

  floatx16 acc_o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) acc_o[db][a] = 0.f;
  float m_raw = -1.0e30f;     // running max of raw scores for this lane's query
  float m_scaled = -3.0e38f;  // m_raw * c_scale, kept finite
  float l_part = 0.f;         // this lane's share of the row sum

  TileRegs regs;
  load_tile(regs, kp, vp, 0, seq, tid);
  store_tile(regs, k_lds[0], vt_lds[0], tid);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int key0 = t * kBc;
    const int buf = t & 1;
    const bool has_next = t + 1 < n_tiles;
    if (has_next) load_tile(regs, kp, vp, key0 + kBc, seq, tid);

    if (key0 < wave_key_end) {
      const bool masked = (CAUSAL && key0 + kBc - 1 > qw0) || (key0 + kBc > seq);
      if (masked)
        tile_step<CAUSAL, true, true>(k_lds[buf], vt_lds[buf], qf, key0, seq,
                                      my_q, col, g, c_scale, acc_o, m_raw,
                                      m_scaled, l_part);
      else if (short_range)
        tile_step<CAUSAL, false, true>(k_lds[buf], vt_lds[buf], qf, key0, seq,
                                       my_q, col, g, c_scale, acc_o, m_raw,
                                       m_scaled, l_part);
      else
        tile_step<CAUSAL, false, false>(k_lds[buf], vt_lds[buf], qf, key0, seq,
                                        my_q, col, g, c_scale, acc_o, m_raw,
                                        m_scaled, l_part);
    }

    if (has_next) store_tile(regs, k_lds[buf ^ 1], vt_lds[buf ^ 1], tid);
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, one query row per lane ------------------------
  const float l_tot = l_part + __shfl_xor(l_part, 32);
  const float inv_l = (l_tot > 0.f) ? 1.0f / l_tot : 0.f;
  if (my_q < seq) {
    const size_t row_off = head_off + static_cast<size_t>(my_q) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + 8 * j + 4 * g;  // 4 consecutive dims
        if (OUT_F32) {
          floatx4 r;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = acc_o[db][4 * j + e] * inv_l;
          *reinterpret_cast<floatx4 *>(static_cast<float *>(o) + row_off + d) = r;
        } else {
          half4 r;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            r[e] = static_cast<_Float16>(acc_o[db][4 * j + e] * inv_l);
          *reinterpret_cast<half4 *>(static_cast<_Float16 *>(o) + row_off + d) = r;
        }
      }
    }
  }
}

template <bool CAUSAL, bool OUT_F32>
void launch_one(const void *q, const void *k, const void *v, void *o, int bh,
                int seq, float c_scale, bool negate_q, hipStream_t stream) {
  const int n_qtiles = (seq + kBr - 1) / kBr;
  const unsigned blocks = static_cast<unsigned>(bh) * n_qtiles;
  hipLaunchKernelGGL((prefill_kernel<CAUSAL, OUT_F32>), dim3(blocks),
                     dim3(kThreads), 0, stream,
                     static_cast<const _Float16 *>(q),
                     static_cast<const _Float16 *>(k),
                     static_cast<const _Float16 *>(v), o, seq, n_qtiles,
                     c_scale, negate_q);
}

}  // namespace

int launch_prefill(const void *q, const void *k, const void *v, void *o,
                   bool out_f32, int batch, int heads, int seq, bool causal,
                   float scale, hipStream_t stream) {
  const int bh = batch * heads;
  const float c_scale = fabsf(scale) * kLog2e;
  const bool negate_q = scale < 0.f;
  if (causal) {
    if (out_f32)
      launch_one<true, true>(q, k, v, o, bh, seq, c_scale, negate_q, stream);
    else
      launch_one<true, false>(q, k, v, o, bh, seq, c_scale, negate_q, stream);
  } else {
    if (out_f32)
      launch_one<false, true>(q, k, v, o, bh, seq, c_scale, negate_q, stream);
    else
      launch_one<false, false>(q, k, v, o, bh, seq, c_scale, negate_q, stream);
  }
  return check_hip(hipGetLastError(), "prefill_kernel launch");
}

int prefill_occupancy(fa_occupancy_entry *out, int cap, int *n) {
  struct K { const char *name; const void *fn; };
  const K ks[] = {
      {"prefill_kernel<causal=true>",
       reinterpret_cast<const void *>(prefill_kernel<true, false>)},
      {"prefill_kernel<causal=false>",
       reinterpret_cast<const void *>(prefill_kernel<false, false>)},
  };
  for (const K &k : ks) {
    if (*n < cap) {
      const int rc = fill_occupancy_row(&out[*n], k.name, k.fn, kThreads, 0);
      if (rc != FA_OK) return rc;
    }
    ++*n;
  }
  return FA_OK;
}

}  // namespace fa
