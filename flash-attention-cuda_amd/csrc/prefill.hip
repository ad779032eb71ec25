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
//   block  = 4 waves over 128 query rows of one (b, h): wave w owns the 64
//            rows [64 (w % 2), +64) ("row group") and half w / 2 of the key
//            tiles (even or odd 64-key tiles). The two halves merge their
//            (m, l, O) states through LDS at the end. A wave covers 64 rows
//            so that every K / V fragment it reads from LDS feeds two MFMAs
//            (LDS bandwidth, not the matrix cores, bounds 32-row waves).
//   CU     = two blocks (64 KiB LDS and <= 256 VGPRs each), so each SIMD runs
//            two waves of independent blocks whose MFMA and softmax phases
//            interleave.
//   grid   = one block per (b, h, 128-row query tile). With causal masking
//            the work per block grows with the query tile; block b and block
//            b + (number of CUs) share a CU, so the first CU-count blocks take
//            the heaviest tiles in descending order and the rest the lightest
//            in ascending order, pairing heavy with light work on every CU.
//   tiles  = K and V stay row-major in LDS (16-byte chunks XOR-swizzled per
//            row), double buffered per half and filled by direct global->LDS
//            loads (global_load_lds_dwordx4) one tile pair ahead.
//
// Products (v_mfma_f32_32x32x16_f16, lane l: column l % 32, half g = l / 32)
//   S^T = K Q^T : A = K rows (ds_read_b128), B = Q^T fragments resident in
//                 registers (two 32-row column groups per wave). Each lane
//                 ends up with ONE query column per group and 16 of the 32
//                 keys, so a query's softmax state lives in the lane pair
//                 (l, l ^ 32).
//   O^T += V^T P^T : B = P^T straight from the S^T accumulators (fp32 -> fp16
//                 pack), A = V^T read with ds_read_b64_tr_b16: inside each
//                 16-lane group, lane j receives element e from source lane
//                 4 e + j / 4, item j % 4, so four lanes pointing at four key
//                 rows of the row-major tile deliver four keys of one head dim
//                 per lane. The O^T accumulator gives each lane one query
//                 column again, so rescaling is a per-lane multiply.
//   The contraction order inside an MFMA only has to agree between A and B;
//   head dims of Q/K are grouped [32 g + 8 s, +8) so each fragment is one
//   16-byte load, and the key order of P^T is the accumulator's own.
//
// Softmax: log2 domain, p = exp2(s * c - m) with c = |scale| * log2(e) (a
// negative scale is folded into Q by an exact fp16 negation). m is the exact
// running max, so the dominant key of a row always enters the PV product as
// P = 1 exactly; the O rescale is skipped (wave-uniform branch) whenever no
// row of the wave raised its max. The row sum l is accumulated from the same
// fp16 P values the PV product consumes (v_dot2_f32_f16), so the weights
// that multiply V sum to exactly the l they are divided by.
// On tiles that carry a mask (causal diagonal, ragged tail) and for query
// rows that see fewer than 512 keys, P is split into hi + lo fp16 parts and
// the PV product is issued twice: those rows have few, large weights, where
// one fp16 rounding of P would cost up to ~4e-4 of output accuracy (about
// 1.6 % extra MFMA work at causal S = 4096).

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;      // 256
constexpr int kRowsPerWave = 64;              // two 32-row column groups
constexpr int kBr = 2 * kRowsPerWave;         // 128 query rows per block
constexpr int kBc = 64;                       // keys per tile
constexpr int kTileHalves = kBc * kHeadDim;   // 4096 halves = 8 KiB
constexpr int kStages = 2;
constexpr int kSplitPRowsBelow = 512;  // rows with fewer keys than this: split P
constexpr float kNegHuge = -3.0e38f;

// LDS: [half][stage][K | V][64 rows x 64 halves] = 64 KiB
constexpr int kStageHalves = 2 * kTileHalves;
constexpr int kHalfHalves = kStages * kStageHalves;
constexpr int kLdsHalves = 2 * kHalfHalves;

typedef __attribute__((address_space(3))) void lds_void;
typedef short short4v __attribute__((ext_vector_type(4)));

// Chunk swizzles (16-byte chunk index within a 128-byte row).
//  K: a ds_read_b128 phase reads the same logical chunk of 8 (32 banks) or
//     16 (64 banks) consecutive rows; f(r) = ((r >> 1) & 7) ^ ((r & 1) << 2)
//     is a bijection on every 8 consecutive rows and keeps the 8 even and the
//     8 odd rows of any 16 apart, so both bank layouts are conflict free.
//  V: a 16-lane transpose-read phase reads chunks {c, c+1} (c even) of 4
//     consecutive rows: c ^ 2 (row & 3) puts them in 8 distinct bank groups.
__device__ __forceinline__ int k_swz(int row) {
  return ((row >> 1) & 7) ^ ((row & 1) << 2);
}
__device__ __forceinline__ int v_swz(int row) { return (row & 3) << 1; }

// Issue the direct global->LDS loads of one 64-key K tile and V tile for one
// half (128 threads, 8 x 16 B each). Rows past the sequence end are clamped
// to the last row: they are masked in the softmax (K) and weighted by 0 (V).
__device__ __forceinline__ void issue_tile_loads(const _Float16 *__restrict__ kp,
                                                 const _Float16 *__restrict__ vp,
                                                 _Float16 *stage_lds, int key0,
                                                 int seq, int htid) {
  const int lane = htid & 63;
  const int w = htid >> 6;  // wave within the half, 0..1
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int rblock = (w * 4 + it) * 8;  // 8 rows per wave instruction
    const int r = rblock + (lane >> 3);
    const int p = lane & 7;
    const int key = min(key0 + r, seq - 1);
    const size_t row_off = static_cast<size_t>(key) * kHeadDim;
    __builtin_amdgcn_global_load_lds(kp + row_off + ((p ^ k_swz(r)) << 3),
                                     (lds_void *)(stage_lds + rblock * kHeadDim),
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds(
        vp + row_off + ((p ^ v_swz(r)) << 3),
        (lds_void *)(stage_lds + kTileHalves + rblock * kHeadDim), 16, 0, 0);
  }
}

// Make this thread's global->LDS loads complete, then synchronise the block.
// A plain s_barrier: __syncthreads() would add a release fence, which drains
// every outstanding memory operation.
__device__ __forceinline__ void loads_done_barrier() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ half8 lds_b128(const _Float16 *p) {
  return *reinterpret_cast<const half8 *>(p);
}

__device__ __forceinline__ half4 lds_tr16(const _Float16 *p) {
  const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v *)(p));
  return __builtin_bit_cast(half4, r);
}

// Softmax state of the two 32-row column groups a wave owns.
struct SoftmaxState {
  float m[2];       // running max per group (log2 domain, scaled by c)
  float l[2];       // this lane's share of each row sum
  floatx16 o[2][2]; // O^T accumulators [group][d-block]
};

// Per-lane LDS offsets (in halves, relative to a stage) of every fragment a
// wave reads from a tile; loop invariant.
struct FragOffsets {
  int k[4];  // K fragment for d-step s (32-key block 0; block 1 is +32 rows)
  int v[2];  // V^T transpose-read base for d-block db (key sub-blocks add rows)
};

__device__ __forceinline__ FragOffsets frag_offsets(int lane) {
  FragOffsets f;
  const int col = lane & 31;
  const int g = lane >> 5;
#pragma unroll
  for (int s = 0; s < 4; ++s)
    f.k[s] = col * kHeadDim + (((4 * g + s) ^ k_swz(col)) << 3);
  // Lane l of a 16-lane group points at row 4 g + (l % 16) / 4 (plus the
  // 8-key sub-block), head dims [16 ((l / 16) % 2) + 4 (l % 4), +4).
  const int tr_row = 4 * g + ((lane & 15) >> 2);
  const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
  for (int db = 0; db < 2; ++db) {
    const int d = db * 32 + tr_dim;
    f.v[db] = kTileHalves + tr_row * kHeadDim + (((d >> 3) ^ v_swz(tr_row)) << 3) + (d & 7);
  }
  return f;
}

// max(x[l], x[l ^ 32]) for every lane: one v_permlane32_swap (VALU), no LDS.
// With both operands holding x, the swap leaves lanes 0-31 of the first
// register and lanes 32-63 of the second unchanged and exchanges the other
// halves, so the two registers hold x[l] and x[l ^ 32] in some order. It is
// written in asm: the compiler treats a swap of two equal values as a no-op
// and folds the max away.
__device__ __forceinline__ float max_lane_pair(float x) {
  float a = x, b = x;
  asm volatile(
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "s_nop 0\n\t"
      "v_max_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
}

// S^T = K Q^T for one 64-key tile and both row groups: every K fragment
// feeds two MFMAs.
__device__ __forceinline__ void qk_tile(const _Float16 *__restrict__ tile,
                                        const FragOffsets &f,
                                        const half8 (&qf)[2][4],
                                        floatx16 (&s_acc)[2][2]) {
#pragma unroll
  for (int gq = 0; gq < 2; ++gq)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int a = 0; a < 16; ++a) s_acc[gq][kb][a] = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const half8 kf = lds_b128(tile + f.k[s] + kb * 32 * kHeadDim);
#pragma unroll
      for (int gq = 0; gq < 2; ++gq)
        s_acc[gq][kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[gq][s],
                                                              s_acc[gq][kb], 0, 0, 0);
    }
  }
}

// S^T = K Q^T for one 64-key tile and one row group (slow path).
__device__ __forceinline__ void qk_group(const _Float16 *__restrict__ tile,
                                         const FragOffsets &f, const half8 (&qf)[4],
                                         floatx16 (&s_acc)[2]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int a = 0; a < 16; ++a) s_acc[kb][a] = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      s_acc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          lds_b128(tile + f.k[s] + kb * 32 * kHeadDim), qf[s], s_acc[kb], 0, 0, 0);
}

// Online softmax of one S^T tile for one row group, producing P^T fragments.
// MASK: keys past the end or above the causal diagonal;
// SPLIT: P feeds the PV product as hi + lo fp16 parts.
template <bool CAUSAL, bool MASK, bool SPLIT>
__device__ __forceinline__ void softmax_group(floatx16 (&s_acc)[2], int key0,
                                              int seq, int my_q, int lane,
                                              float c_scale, float &m, float &l,
                                              floatx16 (&o)[2], half8 (&p_hi)[4],
                                              half8 (&p_lo)[4]) {
  // Element a of key block kb holds key key0 + kb*32 + 8 (a/4) + 4 g + a%4;
  // it is visible iff that offset is <= lim (last visible key - key0 - 4 g).
  const int lim = (CAUSAL ? min(my_q, seq - 1) : seq - 1) - key0 - 4 * (lane >> 5);
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      if (MASK)
        s_acc[kb][a] = (kb * 32 + 8 * (a >> 2) + (a & 3) <= lim) ? s_acc[kb][a] : -INFINITY;
      mx = fmaxf(mx, s_acc[kb][a]);
    }
  }
  mx = max_lane_pair(mx);
  const float mx_scaled = mx * c_scale;
  const bool raise = mx_scaled > m;
  if (__builtin_amdgcn_ballot_w64(raise) != 0) {
    const float m_new = raise ? mx_scaled : m;
    const float alpha = fast_exp2(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) o[db][a] *= alpha;
  }
  const float m_use = m;

  const half2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  float lsum = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int kb = ks >> 1, h = ks & 1;
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
      float p0 = fast_exp2(fmaf(s_acc[kb][8 * h + t], c_scale, -m_use));
      float p1 = fast_exp2(fmaf(s_acc[kb][8 * h + t + 1], c_scale, -m_use));
      if (MASK) {
        p0 = (s_acc[kb][8 * h + t] == -INFINITY) ? 0.f : p0;
        p1 = (s_acc[kb][8 * h + t + 1] == -INFINITY) ? 0.f : p1;
      }
      const half2 hi2 = {static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
      p_hi[ks][t] = hi2[0];
      p_hi[ks][t + 1] = hi2[1];
      lsum = __builtin_amdgcn_fdot2(hi2, ones, lsum, false);
      if (SPLIT) {
        const half2 lo2 = {static_cast<_Float16>(p0 - static_cast<float>(hi2[0])),
                           static_cast<_Float16>(p1 - static_cast<float>(hi2[1]))};
        p_lo[ks][t] = lo2[0];
        p_lo[ks][t + 1] = lo2[1];
        lsum = __builtin_amdgcn_fdot2(lo2, ones, lsum, false);
      }
    }
  }
  l += lsum;
}

// O^T += V^T P^T for one 64-key tile and both row groups: every V^T
// fragment feeds two MFMAs.
template <bool SPLIT>
__device__ __forceinline__ void pv_tile(const _Float16 *__restrict__ tile,
                                        const FragOffsets &f,
                                        const half8 (&p_hi)[2][4],
                                        const half8 (&p_lo)[2][4],
                                        SoftmaxState &st) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int kb = ks >> 1, h = ks & 1;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      half8 vf;
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int row_off = (kb * 32 + 16 * h + 8 * part) * kHeadDim;
        const half4 v4 = lds_tr16(tile + f.v[db] + row_off);
#pragma unroll
        for (int e = 0; e < 4; ++e) vf[4 * part + e] = v4[e];
      }
#pragma unroll
      for (int gq = 0; gq < 2; ++gq) {
        st.o[gq][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_hi[gq][ks],
                                                             st.o[gq][db], 0, 0, 0);
        if (SPLIT)
          st.o[gq][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_lo[gq][ks],
                                                               st.o[gq][db], 0, 0, 0);
      }
    }
  }
}

// O^T += V^T P^T for one row group with P split into hi + lo parts (the
// rare masked / short-row path; V fragments are read once per group there to
// keep the live P registers of only one group).
__device__ __forceinline__ void pv_group_split(const _Float16 *__restrict__ tile,
                                               const FragOffsets &f,
                                               const half8 (&p_hi)[4],
                                               const half8 (&p_lo)[4],
                                               floatx16 (&o)[2]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int kb = ks >> 1, h = ks & 1;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      half8 vf;
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int row_off = (kb * 32 + 16 * h + 8 * part) * kHeadDim;
        const half4 v4 = lds_tr16(tile + f.v[db] + row_off);
#pragma unroll
        for (int e = 0; e < 4; ++e) vf[4 * part + e] = v4[e];
      }
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_hi[ks], o[db], 0, 0, 0);
      o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, p_lo[ks], o[db], 0, 0, 0);
    }
  }
}

// One 64-key tile for one wave. Fast path: QK, softmax of both row groups,
// PV with shared K / V fragments. Masked / short-row path: QK, softmax and
// split-P PV one row group at a time (fewer live registers).
template <bool CAUSAL, bool SLOW>
__device__ __forceinline__ void tile_step(const _Float16 *__restrict__ tile,
                                          const FragOffsets &f,
                                          const half8 (&qf)[2][4], int key0,
                                          int seq, int row0, int lane,
                                          float c_scale, SoftmaxState &st) {
  if (!SLOW) {
    floatx16 s_acc[2][2];
    qk_tile(tile, f, qf, s_acc);
    half8 p_hi[2][4], p_unused[2][4];
#pragma unroll
    for (int gq = 0; gq < 2; ++gq)
      softmax_group<CAUSAL, false, false>(s_acc[gq], key0, seq,
                                          row0 + 32 * gq + (lane & 31), lane,
                                          c_scale, st.m[gq], st.l[gq], st.o[gq],
                                          p_hi[gq], p_unused[gq]);
    pv_tile<false>(tile, f, p_hi, p_unused, st);
  } else {
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      floatx16 s_acc[2];
      half8 p_hi[4], p_lo[4];
      qk_group(tile, f, qf[gq], s_acc);
      softmax_group<CAUSAL, true, true>(s_acc, key0, seq,
                                        row0 + 32 * gq + (lane & 31), lane,
                                        c_scale, st.m[gq], st.l[gq], st.o[gq],
                                        p_hi, p_lo);
      pv_group_split(tile, f, p_hi, p_lo, st.o[gq]);
    }
  }
}

template <bool CAUSAL, bool OUT_F32>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k,
    const _Float16 *__restrict__ v, void *__restrict__ o, int seq,
    int n_qtiles, int n_cu, float c_scale, bool negate_q) {
  __shared__ __attribute__((aligned(1024))) _Float16 lds[kLdsHalves];

  // Block -> (query tile, head). Rank 0 is the heaviest tile. While the grid
  // fits in two blocks per CU, block b and block b + n_cu share a CU: ranks
  // ascend over the first n_cu blocks and descend over the rest.
  const int nb = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  const int rank = (CAUSAL && nb <= 2 * n_cu && b >= n_cu) ? nb - 1 - (b - n_cu) : b;
  const int bh_count = nb / n_qtiles;
  const int qtile = n_qtiles - 1 - rank / bh_count;
  const int bh = rank % bh_count;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int rg = wave & 1;    // row group of this wave
  const int half = wave >> 1; // 0: even key tiles, 1: odd key tiles
  const int htid = tid & 127;
  const int col = lane & 31;
  const int g = lane >> 5;

  const size_t head_off = static_cast<size_t>(bh) * seq * kHeadDim;
  const _Float16 *qp = q + head_off;
  const _Float16 *kp = k + head_off;
  const _Float16 *vp = v + head_off;

  const int q0 = qtile * kBr;
  const int row0 = q0 + rg * kRowsPerWave;  // first query row of this wave

  // Q^T fragments: group gq, lane holds query row0 + 32 gq + col, head dims
  // [32 g + 8 s, +8).
  half8 qf[2][4];
#pragma unroll
  for (int gq = 0; gq < 2; ++gq) {
    const int my_q = row0 + 32 * gq + col;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (my_q < seq) {
        qf[gq][s] = *reinterpret_cast<const half8 *>(
            qp + static_cast<size_t>(my_q) * kHeadDim + 32 * g + 8 * s);
        if (negate_q) qf[gq][s] = -qf[gq][s];
      } else {
        qf[gq][s] = half8{};
      }
    }
  }

  const int key_end = CAUSAL ? min(seq, q0 + kBr) : seq;
  const int n_tiles = (key_end + kBc - 1) / kBc;
  const int n_pairs = (n_tiles + 1) / 2;
  // Keys this wave can see; tiles past them are skipped.
  const int wave_key_end = CAUSAL ? min(seq, row0 + kRowsPerWave) : seq;
  // Tiles below main_end need no mask for any row of the block and all its
  // rows see >= kSplitPRowsBelow keys: plain fast path.
  const bool short_rows = CAUSAL ? q0 < kSplitPRowsBelow : seq < kSplitPRowsBelow;
  const int main_end = short_rows ? 0 : (CAUSAL ? q0 / kBc : seq / kBc);

  const FragOffsets fo = frag_offsets(lane);
  SoftmaxState st;
#pragma unroll
  for (int gq = 0; gq < 2; ++gq) {
    st.m[gq] = kNegHuge;
    st.l[gq] = 0.f;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) st.o[gq][db][a] = 0.f;
  }

  _Float16 *my_lds = lds + half * kHalfHalves;
  if (half * kBc < key_end)
    issue_tile_loads(kp, vp, my_lds, half * kBc, seq, htid);
  loads_done_barrier();

  for (int j = 0; j < n_pairs; ++j) {
    const int next_key0 = (2 * (j + 1) + half) * kBc;
    if (next_key0 < key_end)
      issue_tile_loads(kp, vp, my_lds + ((j + 1) & 1) * kStageHalves, next_key0,
                       seq, htid);
    const int t = 2 * j + half;
    const int key0 = t * kBc;
    if (key0 < wave_key_end) {
      const _Float16 *tile = my_lds + (j & 1) * kStageHalves;
      if (t < main_end)
        tile_step<CAUSAL, false>(tile, fo, qf, key0, seq, row0, lane, c_scale, st);
      else
        tile_step<CAUSAL, true>(tile, fo, qf, key0, seq, row0, lane, c_scale, st);
    }
    loads_done_barrier();
  }

  // ---- merge the two halves through LDS, normalise, store ------------------
  // Layout: [row group][68 values][64 lanes] fp32 (reuses the tile buffers;
  // the barrier above ended every read of them).
  float *xchg = reinterpret_cast<float *>(lds) + rg * (68 * kWave) + lane;
  if (half == 1) {
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int a = 0; a < 16; ++a)
          xchg[(32 * gq + 16 * db + a) * kWave] = st.o[gq][db][a];
      xchg[(64 + gq) * kWave] = st.m[gq];
      xchg[(66 + gq) * kWave] = st.l[gq];
    }
  }
  __syncthreads();
  if (half == 1) return;

#pragma unroll
  for (int gq = 0; gq < 2; ++gq) {
    const float m1 = xchg[(64 + gq) * kWave];
    const float l1 = xchg[(66 + gq) * kWave];
    const float m = fmaxf(st.m[gq], m1);
    const float f0 = fast_exp2(st.m[gq] - m);
    const float f1 = fast_exp2(m1 - m);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a)
        st.o[gq][db][a] =
            st.o[gq][db][a] * f0 + xchg[(32 * gq + 16 * db + a) * kWave] * f1;
    const float l_own = st.l[gq] * f0 + l1 * f1;
    const float l_tot = l_own + __shfl_xor(l_own, 32);
    const float inv_l = (l_tot > 0.f) ? 1.0f / l_tot : 0.f;
    const int my_q = row0 + 32 * gq + col;
    if (my_q < seq) {
      const size_t row_off = head_off + static_cast<size_t>(my_q) * kHeadDim;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int d = db * 32 + 8 * jj + 4 * g;  // 4 consecutive dims
          if (OUT_F32) {
            floatx4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = st.o[gq][db][4 * jj + e] * inv_l;
            *reinterpret_cast<floatx4 *>(static_cast<float *>(o) + row_off + d) = r;
          } else {
            half4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              r[e] = static_cast<_Float16>(st.o[gq][db][4 * jj + e] * inv_l);
            *reinterpret_cast<half4 *>(static_cast<_Float16 *>(o) + row_off + d) = r;
          }
        }
      }
    }
  }
}

template <bool CAUSAL, bool OUT_F32>
void launch_one(const void *q, const void *k, const void *v, void *o, int bh,
                int seq, int n_cu, float c_scale, bool negate_q,
                hipStream_t stream) {
  const int n_qtiles = (seq + kBr - 1) / kBr;
  const unsigned blocks = static_cast<unsigned>(bh) * n_qtiles;
  hipLaunchKernelGGL((prefill_kernel<CAUSAL, OUT_F32>), dim3(blocks),
                     dim3(kThreads), 0, stream,
                     static_cast<const _Float16 *>(q),
                     static_cast<const _Float16 *>(k),
                     static_cast<const _Float16 *>(v), o, seq, n_qtiles, n_cu,
                     c_scale, negate_q);
}

}  // namespace

int launch_prefill(const void *q, const void *k, const void *v, void *o,
                   bool out_f32, int batch, int heads, int seq, bool causal,
                   float scale, hipStream_t stream) {
  const int bh = batch * heads;
  const float c_scale = fabsf(scale) * kLog2e;
  const bool negate_q = scale < 0.f;
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != FA_OK) return rc;
  const int n_cu = device_cu_count(dev) > 0 ? device_cu_count(dev) : 1;
  if (causal) {
    if (out_f32)
      launch_one<true, true>(q, k, v, o, bh, seq, n_cu, c_scale, negate_q, stream);
    else
      launch_one<true, false>(q, k, v, o, bh, seq, n_cu, c_scale, negate_q, stream);
  } else {
    if (out_f32)
      launch_one<false, true>(q, k, v, o, bh, seq, n_cu, c_scale, negate_q, stream);
    else
      launch_one<false, false>(q, k, v, o, bh, seq, n_cu, c_scale, negate_q, stream);
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
