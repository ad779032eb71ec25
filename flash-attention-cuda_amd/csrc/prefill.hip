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
//   block  = 8 waves, 128 query rows of one (b, h): 4 row waves x 2 key
//            halves. Row wave r owns rows [32 r, +32); key half h streams the
//            64-key tiles 2 k + h its rows can see. The two halves keep
//            separate online-softmax states and merge them through LDS at the
//            end, so a block's critical path is half its key range.
//   CU     = one block (128 KiB LDS, <= 256 VGPRs per lane): each SIMD runs
//            the two waves of one row wave, one per key half.
//   grid   = one block per (b, h, 128-row query tile), heaviest (last) query
//            tiles first: with causal masking the work per block grows with
//            the query tile, and dispatching in decreasing work order is a
//            longest-first list schedule over the CUs.
//   tiles  = K and V stay row-major in LDS (16-byte chunks XOR-swizzled per
//            row), in one 4-stage ring per key half filled by direct
//            global->LDS loads (global_load_lds_dwordx4) three of that half's
//            tiles ahead of the MFMA work.
//
// Main-loop schedule (tiles that need no mask), per wave and step k:
//   barrier -> issue every LDS fragment read of V and of the next K tile ->
//   half 0: softmax of S_k, then the burst PV(k) + QK(k+1);
//   half 1: the burst PV(k) + QK(k+1), then the softmax of S_{k+1}.
//   The burst interleaves four independent MFMA accumulation chains and runs
//   at raised wave priority. The two waves that share a SIMD are therefore in
//   opposite phases: one issues MFMAs while the other runs its exp-heavy
//   softmax on the VALU. S dies as P is formed, so one S buffer serves both
//   tiles. Tiles that need a mask (causal diagonal, ragged tail) and query
//   rows that see fewer than 512 keys take a plain per-tile step.
//
// Products (v_mfma_f32_32x32x16_f16, lane l: column l % 32, half g = l / 32)
//   S^T = K Q^T : A = K rows (ds_read_b128), B = Q^T fragments resident in
//                 registers. Each lane ends up with ONE query column and 16 of
//                 the 32 keys, so a query's softmax state lives in the lane
//                 pair (l, l ^ 32).
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

constexpr int kQWaves = 4;                    // row waves per key half
constexpr int kThreads = 2 * kQWaves * kWave; // 512: two key halves
constexpr int kRowsPerWave = 32;
constexpr int kBr = kQWaves * kRowsPerWave;   // 128 query rows per block
constexpr int kBc = 64;                       // keys per tile
constexpr int kTileHalves = kBc * kHeadDim;   // 4096 halves = 8 KiB
constexpr int kStages = 4;
constexpr int kAhead = kStages - 1;           // tiles in flight ahead of use
constexpr int kLoadsPerTile = 4;              // global_load_lds per thread per tile
constexpr int kSplitPRowsBelow = 512;  // rows with fewer keys than this: split P
constexpr float kNegHuge = -3.0e38f;
// s_waitcnt immediate for vmcnt(0) with expcnt / lgkmcnt left unconstrained.
constexpr int kWaitVmcnt0 = 0x0F70;

// LDS: [key half][stage][K | V][64 rows x 64 halves] = 128 KiB
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

// One direct global->LDS load: 16 bytes per lane from `src` to LDS address
// m0 + 16 * lane. Written in asm so the compiler does not treat later LDS
// reads of other stages as possibly aliasing the in-flight write (it would
// otherwise wait for every outstanding load before each of them); the ring
// tracks completion itself with explicit vmcnt waits.
__device__ __forceinline__ void global_to_lds16(const void *src, const void *lds_dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(lds_dst))));
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "s"(m0)
      : "memory", "m0");
}

// Issue the direct global->LDS loads of one 64-key K tile and V tile
// (256 threads, 4 x 16 B each). Rows past the sequence end are clamped to the
// last row: they are masked in the softmax (K) and weighted by 0 (V).
__device__ __forceinline__ void issue_tile_loads(const _Float16 *__restrict__ kp,
                                                 const _Float16 *__restrict__ vp,
                                                 _Float16 *stage_lds, int key0,
                                                 int seq, int tid) {
  const int lane = tid & 63;
  const int w = tid >> 6;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int rblock = (w * 2 + it) * 8;  // 8 rows per wave instruction
    const int r = rblock + (lane >> 3);
    const int p = lane & 7;
    const int key = min(key0 + r, seq - 1);
    const size_t row_off = static_cast<size_t>(key) * kHeadDim;
    global_to_lds16(kp + row_off + ((p ^ k_swz(r)) << 3), stage_lds + rblock * kHeadDim);
    global_to_lds16(vp + row_off + ((p ^ v_swz(r)) << 3),
                    stage_lds + kTileHalves + rblock * kHeadDim);
  }
}

// Wait until at most N of this thread's global->LDS loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_loads() {
  if constexpr (N == 0)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ half8 lds_b128(const _Float16 *p) {
  return *reinterpret_cast<const half8 *>(p);
}

__device__ __forceinline__ half4 lds_tr16(const _Float16 *p) {
  const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v *)(p));
  return __builtin_bit_cast(half4, r);
}

struct SoftmaxState {
  float m;       // running max (log2 domain, already scaled by c)
  float l;       // this lane's share of the row sum
  floatx16 o[2]; // O^T accumulators: d-blocks 0 and 1
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

// Register copies of the LDS fragments one tile step consumes.
struct KFrags { half8 f[2][4]; };  // [32-key block][d-step]
struct VFrags { half8 f[4][2]; };  // [16-key step][d-block]

__device__ __forceinline__ void read_k(const _Float16 *__restrict__ tile,
                                       const FragOffsets &fo, KFrags &k) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int s = 0; s < 4; ++s) k.f[kb][s] = lds_b128(tile + fo.k[s] + kb * 32 * kHeadDim);
}

__device__ __forceinline__ void read_v(const _Float16 *__restrict__ tile,
                                       const FragOffsets &fo, VFrags &v) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int kb = ks >> 1, h = ks & 1;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int row_off = (kb * 32 + 16 * h + 8 * part) * kHeadDim;
        const half4 v4 = lds_tr16(tile + fo.v[db] + row_off);
#pragma unroll
        for (int e = 0; e < 4; ++e) v.f[ks][db][4 * part + e] = v4[e];
      }
    }
  }
}

__device__ __forceinline__ floatx16 mfma(const half8 &a, const half8 &b,
                                         const floatx16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
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

// Online softmax of one S^T tile, producing P^T fragments (hi [+ lo]).
// MASK: keys past the end or above the causal diagonal;
// SPLIT: P feeds the PV product as hi + lo fp16 parts.
template <bool CAUSAL, bool MASK, bool SPLIT>
__device__ __forceinline__ void softmax_tile(floatx16 (&s_acc)[2], int key0, int seq,
                                             int my_q, int lane, float c_scale,
                                             SoftmaxState &st, half8 (&p_hi)[4],
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
  const bool raise = mx_scaled > st.m;
  if (__builtin_amdgcn_ballot_w64(raise) != 0) {
    const float m_new = raise ? mx_scaled : st.m;
    const float alpha = fast_exp2(st.m - m_new);
    st.m = m_new;
    st.l *= alpha;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) st.o[db][a] *= alpha;
  }
  const float m_use = st.m;

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
  st.l += lsum;
}

// PV(t) and QK(t+1) as four independent accumulation chains (O d-blocks 0/1,
// S key-blocks 0/1), issued alternately.
template <bool WITH_QK>
__device__ __forceinline__ void pv_qk_mfma(const VFrags &v, const half8 (&p)[4],
                                           const KFrags &k, const half8 (&qf)[4],
                                           floatx16 (&o)[2], floatx16 (&s)[2]) {
  if (WITH_QK) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int a = 0; a < 16; ++a) s[kb][a] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      o[db] = mfma(v.f[i][db], p[i], o[db]);
      if (WITH_QK) s[db] = mfma(k.f[db][i], qf[i], s[db]);
    }
  }
}

// Plain (non-pipelined) step for masked / short-row tiles: QK, softmax with
// mask and split P, PV issued twice.
template <bool CAUSAL>
__device__ __forceinline__ void slow_step(const _Float16 *__restrict__ tile,
                                          const FragOffsets &fo, const half8 (&qf)[4],
                                          int key0, int seq, int my_q, int lane,
                                          float c_scale, SoftmaxState &st) {
  KFrags k;
  VFrags v;
  read_k(tile, fo, k);
  read_v(tile, fo, v);
  floatx16 s[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int a = 0; a < 16; ++a) s[kb][a] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kb] = mfma(k.f[kb][i], qf[i], s[kb]);
  }
  half8 p_hi[4], p_lo[4];
  softmax_tile<CAUSAL, true, true>(s, key0, seq, my_q, lane, c_scale, st, p_hi, p_lo);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      st.o[db] = mfma(v.f[i][db], p_hi[i], st.o[db]);
      st.o[db] = mfma(v.f[i][db], p_lo[i], st.o[db]);
    }
  }
}

// Tile ring of one key half: half h owns tiles 2k + h (k = 0, 1, ...), stage
// k % kStages of its LDS region.
struct HalfRing {
  _Float16 *lds;
  const _Float16 *kp, *vp;
  int seq, n_tiles, half, htid;

  __device__ __forceinline__ int tile(int k) const { return 2 * k + half; }
  __device__ __forceinline__ _Float16 *stage(int k) const {
    return lds + (k & (kStages - 1)) * kStageHalves;
  }
  __device__ __forceinline__ void issue(int k) const {
    if (tile(k) < n_tiles) issue_tile_loads(kp, vp, stage(k), tile(k) * kBc, seq, htid);
  }
  // Start of step k: this half's tiles k and k+1 are resident and visible to
  // the whole block, then the load of its tile k + kAhead is issued into the
  // stage tile k-1 used (every wave finished reading it before the barrier).
  // A plain s_barrier: __syncthreads() would add a release fence, which
  // drains every outstanding load of the ring.
  __device__ __forceinline__ void advance(int k) const {
    if (tile(k + 2) < n_tiles)
      wait_loads<kLoadsPerTile>();
    else
      wait_loads<0>();
    __builtin_amdgcn_s_barrier();
    issue(k + kAhead);
  }
};

template <bool CAUSAL, bool OUT_F32>
__global__ __launch_bounds__(kThreads, 1) void prefill_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k,
    const _Float16 *__restrict__ v, void *__restrict__ o, int seq,
    int n_qtiles, float c_scale, bool negate_q) {
  __shared__ __attribute__((aligned(1024))) _Float16 lds[kLdsHalves];

  // Heaviest (last) query tiles first: one block fills a CU, so dispatching
  // in decreasing work order is a longest-first list schedule.
  const int bh_count = static_cast<int>(gridDim.x) / n_qtiles;
  const int qtile = n_qtiles - 1 - static_cast<int>(blockIdx.x) / bh_count;
  const int bh = static_cast<int>(blockIdx.x) % bh_count;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int rw = wave & (kQWaves - 1);  // row wave: rows [32 rw, +32)
  const int half = wave / kQWaves;      // key half: tiles 2k + half
  const int htid = tid & (kQWaves * kWave - 1);
  const int col = lane & 31;
  const int g = lane >> 5;

  const size_t head_off = static_cast<size_t>(bh) * seq * kHeadDim;
  const _Float16 *qp = q + head_off;

  const int q0 = qtile * kBr;
  const int qw0 = q0 + rw * kRowsPerWave;
  const int my_q = qw0 + col;

  const int key_end = CAUSAL ? min(seq, q0 + kBr) : seq;
  const int n_tiles = (key_end + kBc - 1) / kBc;
  HalfRing ring{lds + half * kHalfHalves, k + head_off, v + head_off, seq, n_tiles,
                half, htid};
  const int wave_key_end = CAUSAL ? min(seq, qw0 + kRowsPerWave) : seq;
  // Tiles [0, 2 n_main) need no mask for any wave of the block and all its
  // rows see >= kSplitPRowsBelow keys: each half runs n_main pipelined steps
  // on them. The rest (causal diagonal, ragged tail, short rows) take the
  // plain masked step.
  const bool short_rows = CAUSAL ? q0 < kSplitPRowsBelow : seq < kSplitPRowsBelow;
  const int main_tiles = short_rows ? 0 : (CAUSAL ? q0 / kBc : seq / kBc);
  const int n_main = main_tiles / 2;
  const int n_steps = (n_tiles + 1) / 2;  // steps of the longer half

#pragma unroll
  for (int kk = 0; kk < kAhead; ++kk) ring.issue(kk);

  // Q^T fragments: lane holds query my_q, head dims [32 g + 8 s, +8).
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
  // One wait the compiler can see (it cannot see the ring's asm waits): Q and
  // the first kAhead tiles are resident, and no compiler-issued load is
  // pending inside the loops, so it adds no vmcnt waits there.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __builtin_amdgcn_s_barrier();
  ring.issue(kAhead);

  const FragOffsets fo = frag_offsets(lane);
  SoftmaxState st;
  st.m = kNegHuge;
  st.l = 0.f;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int a = 0; a < 16; ++a) st.o[db][a] = 0.f;

  // ---- pipelined main loop, ping-pong between the halves --------------------
  // Step kk, half 0: softmax S(kk) -> burst [PV(kk), QK(kk+1)].
  //          half 1: burst [PV(kk), QK(kk+1)] -> softmax S(kk+1).
  // The two waves sharing a SIMD (same row wave, different half) are thus in
  // opposite phases: one issues MFMAs while the other runs the exp-heavy
  // softmax. The burst runs at raised priority so its MFMAs issue first.
  floatx16 s_acc[2];
  KFrags kf;
  VFrags vf;
  half8 p_hi[4], p_lo[4];
  if (n_main > 0) {
    read_k(ring.stage(0), fo, kf);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int a = 0; a < 16; ++a) s_acc[kb][a] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) s_acc[kb] = mfma(kf.f[kb][i], qf[i], s_acc[kb]);
    }
    if (half == 1)
      softmax_tile<CAUSAL, false, false>(s_acc, ring.tile(0) * kBc, seq, my_q, lane,
                                         c_scale, st, p_hi, p_lo);
  }
  int kk = 0;
  for (; kk < n_main; ++kk) {
    if (kk > 0) ring.advance(kk);
    // QK(kk+1) is issued unconditionally: on the last main step it reads
    // whatever stage kk+1 holds (in bounds) and the result is discarded,
    // which keeps the accumulators in place (a branch makes the compiler
    // copy them every step).
    read_v(ring.stage(kk), fo, vf);
    read_k(ring.stage(kk + 1), fo, kf);
    if (half == 0)
      softmax_tile<CAUSAL, false, false>(s_acc, ring.tile(kk) * kBc, seq, my_q,
                                         lane, c_scale, st, p_hi, p_lo);
    __builtin_amdgcn_s_setprio(2);
    pv_qk_mfma<true>(vf, p_hi, kf, qf, st.o, s_acc);
    __builtin_amdgcn_s_setprio(0);
    if (half == 1 && kk + 1 < n_main)
      softmax_tile<CAUSAL, false, false>(s_acc, ring.tile(kk + 1) * kBc, seq, my_q,
                                         lane, c_scale, st, p_hi, p_lo);
  }

  // ---- masked / short-row tiles: one plain step per tile ---------------------
  for (; kk < n_steps; ++kk) {
    if (kk > 0) ring.advance(kk);
    const int key0 = ring.tile(kk) * kBc;
    if (key0 < wave_key_end)
      slow_step<CAUSAL>(ring.stage(kk), fo, qf, key0, seq, my_q, lane, c_scale, st);
  }

  // ---- merge the two halves through LDS, normalise, store ------------------
  // Layout: [row wave][34 values][64 lanes] fp32, reusing the tile buffers.
  // Every load the ring issued has completed (the last steps waited with
  // vmcnt(0)); the barrier ends every read of the tiles.
  wait_loads<0>();
  __builtin_amdgcn_s_barrier();
  float *xchg = reinterpret_cast<float *>(lds) + rw * (34 * kWave) + lane;
  if (half == 1) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) xchg[(16 * db + a) * kWave] = st.o[db][a];
    xchg[32 * kWave] = st.m;
    xchg[33 * kWave] = st.l;
  }
  __syncthreads();
  if (half == 1) return;
  {
    const float m1 = xchg[32 * kWave];
    const float l1 = xchg[33 * kWave];
    const float m = fmaxf(st.m, m1);
    const float f0 = fast_exp2(st.m - m);
    const float f1 = fast_exp2(m1 - m);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a)
        st.o[db][a] = st.o[db][a] * f0 + xchg[(16 * db + a) * kWave] * f1;
    st.l = st.l * f0 + l1 * f1;
  }

  // ---- epilogue: O = O^T / l, one query row per lane -------------------------
  const float l_tot = st.l + __shfl_xor(st.l, 32);
  const float inv_l = (l_tot > 0.f) ? 1.0f / l_tot : 0.f;
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
          for (int e = 0; e < 4; ++e) r[e] = st.o[db][4 * jj + e] * inv_l;
          *reinterpret_cast<floatx4 *>(static_cast<float *>(o) + row_off + d) = r;
        } else {
          half4 r;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            r[e] = static_cast<_Float16>(st.o[db][4 * jj + e] * inv_l);
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
