// Causal / full FlashAttention prefill for head_dim 64 (and 128) on gfx950 MFMA.
//
// Reference behaviour: prefill_kernel<CAUSAL> and launch_prefill in
// csrc/prefill.cu:164-373 of shrvan30/flash-attention-cuda (online softmax
// over key tiles, causal tile skipping :208-212, mask `k < N && k <= q`
// :268, 1/l with an l > 0 guard :334). The reference runs both products on
// scalar FP32 FMAs; here both are dense fp16 contractions on the matrix
// cores with fp32 accumulation.
//
// What bounds this kernel on gfx950 (measured):
//   * One v_mfma_f32_32x32x16_f16 occupies the matrix core of its SIMD for
//     ~16 ns. One wave issues VALU at half the SIMD's rate, two waves at the
//     full rate; VALU work of the other wave mostly runs while an MFMA does
//     (v_exp_f32 partly, v_dot2c_f32_f16 not at all). The softmax is more
//     VALU time than the two products are MFMA time, so each wave runs a
//     software pipeline: the MFMAs of its neighbouring tiles interleave with
//     the softmax of the current one, and the second wave on each SIMD fills
//     the VALU and covers the latencies (barrier, LDS reads, loads).
//   * LDS serves ~one 64-lane read instruction per 3 ns per CU.
//
// Work decomposition
//   block  = 8 waves, 128 query rows of one (b, h): 4 row waves x 2 key
//            halves. Row wave r owns rows [32 r, +32); key half h streams the
//            64-key tiles 2 k + h its rows can see. The halves keep separate
//            online-softmax states and merge them through LDS at the end, so a
//            block's critical path is half its key range.
//   CU     = one block (160 KiB LDS, <= 256 VGPRs per lane): each SIMD runs
//            the two waves of one row wave, one per key half.
//   grid   = persistent blocks of up to two units each. A unit is an item
//            (b, h, 128-row query tile) or one of the two key chunks of a
//            split item. Without a plan, block b takes item b, then item
//            G + mirror(b), items numbered heaviest (last) query tile first,
//            so a heavy first item pairs with a light second one and both
//            stay on the block's XCD; with a plan (the host's unit table,
//            when the items do not fill the chip evenly and a workspace is
//            given) block b takes the two units the table assigns it.
//   LDS    = the block's Q tile, plus per key half a 4-stage K ring and a
//            5-stage V ring of 64-key tiles, all row-major with 16-byte
//            chunks XOR-swizzled per row, filled by direct global->LDS loads
//            (global_load_lds_dwordx4) four tiles ahead of use.
//   head_dim 128: the same block, pipeline and rules with 32-key tiles of
//            256-byte rows (still 8 KiB, still 16 MFMAs per step), Q^T loaded
//            from HBM straight into registers instead of through LDS, and
//            two masked tiles per key half on the causal diagonal (the second
//            one takes the plain per-tile step). Constants in Geo<D>.
//
// Main loop (tiles that need no mask), per wave and step k of its half:
//   wait for tile k+2 and this wave's LDS reads -> barrier -> issue the loads
//   of tile k+4 ->
//   note the row sum (head_dim 64) -> O *= alpha_{k-1} (only when m moved) ->
//   row max of S_k ->
//   { QK(k+1), PV(k-1) and the row sums of P_{k-1} on the matrix cores }
//   interleaved with { exp / pack of S_k on the VALU } ->
//   LDS reads of the next step's fragments (K_{k+2}, V_k), which land while
//   the next barrier and row max run.
//   S and P are double-buffered (the loop is unrolled by two), so the MFMAs of
//   a step never wait for that step's softmax. The one tile per half that
//   needs a mask (causal diagonal, ragged tail) is the pipeline's last step,
//   with a masked softmax. Blocks whose query rows see fewer than 256 keys,
//   and every block when the scale alone makes the logits wide
//   (|scale| sqrt(D) > 1.5), take a plain per-tile step with split P instead;
//   so does a second pass over any other block whose rows turn out peaky
//   (softmax paragraph below).
//
// Products (v_mfma_f32_32x32x16_f16, lane l: column l % 32, half g = l / 32)
//   S^T = K Q^T : A = K rows (ds_read_b128), B = Q^T fragments resident in
//                 registers. Each lane ends up with ONE query column and 16 of
//                 each 32 keys, so a query's softmax state lives in the lane
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
// negative scale is folded into Q by an exact fp16 negation). The row sum l
// is accumulated from the same fp16 P values the PV product consumes, so the
// weights that multiply V sum to exactly the l they are divided by: at
// head_dim 64 on the matrix cores (one v_mfma_f32_16x16x32_f16 per 16-key
// step against a 0/1 selector, rowsum_mfma), at head_dim 128 per lane with
// v_dot2_f32_f16.
// The max m: rows that see >= 1024 keys take a lazy max. m moves, to the
// row's exact running max, only when a tile max exceeds it by more than 8
// (log2 units), so P <= 2^8, or when the new max carries more than 1/16 of
// the row sum so far; O is then rescaled on a few steps per item instead of
// on most of them. Shorter rows keep m at the exact running max (every step
// where some row's max rose rescales). Whenever a tile sets m, its dominant
// key enters the PV product as P = 1 exactly.
//
// Precision of P: one fp16 rounding of each weight w = p / l moves an output
// row by about 2^-11 sqrt(sum w^2) times the spread of V, summed over the
// rounded weights (a P = 1 key is exact and does not count). Rows carried by
// a few keys therefore need P split into hi + lo fp16 parts, with the PV
// product issued twice (relative error ~2^-22). Rows that see fewer than 256
// keys always take the split. Every other row sums its rounded mass
// r = sum P^2 over the fp16 weights it rounded (v_dot2_f32_f16 of the packed
// P with itself), less the exact 1 of a tile whose largest weight is exactly
// 1, rescaled with m like l. A block with a row whose r / l^2 ends above
// kRedoRoundedMassAbove is computed again with split P on every tile.
// Measured on N(0,1) q, k, v scaled to 1x-1.84x the standard logit width
// (head_dim 64 and 128, causal and full, 512-2048 keys): rows kept at
// r / l^2 <= 0.03 show fp32-output errors <= 2.17e-4 (error up to ~1.5e-3 x
// sqrt(r / l^2)); N(0,1) inputs at 1/sqrt(D) stay below 0.013 and take the
// single-rounding pass only.

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <vector>

#include "fa_internal.h"
#include "mfma_tile.h"

// This file is compiled once per head size: FA_PREFILL_D = 64 gives the
// head_dim 64 kernels and the shared host entry points, FA_PREFILL_D = 128
// the head_dim 128 kernels. The two builds take different instruction-
// scheduling options (the library's build script).
#if !defined(FA_PREFILL_D) || (FA_PREFILL_D != 64 && FA_PREFILL_D != 128)
#error "compile prefill.hip with -DFA_PREFILL_D=64 or -DFA_PREFILL_D=128"
#endif

namespace fa {
namespace {

constexpr int kRowWaves = 4;                  // row waves per key half
constexpr int kWaves = 2 * kRowWaves;         // x 2 key halves
constexpr int kThreads = kWaves * kWave;      // 512
constexpr int kRowsPerWave = 32;
constexpr int kBr = kRowWaves * kRowsPerWave; // 128 query rows per block
constexpr int kKStages = 4;
constexpr int kVStages = 5;
constexpr int kAhead = 4;                     // tiles in flight ahead of use
constexpr int kLoadsPerTile = 4;              // global_load_lds per thread per tile
constexpr int kSplitPRowsBelow = 256;  // rows with fewer keys than this: split P
// A block is recomputed with split P when, for one of its rows, the squared
// normalised weights that took a single fp16 rounding sum to more than this
// (see the precision note at the top of the file).
constexpr float kRedoRoundedMassAbove = 0.03f;
// |scale| * sqrt(D) above this (1 is the standard 1/sqrt(D)): rows are peaky
// from the scale alone, so the first (single-rounding) pass is skipped.
[[maybe_unused]] constexpr float kSplitAllWidth = 1.5f;  // used by the head_dim 64 build
constexpr float kNegHuge = -3.0e38f;
// The max that P is taken against moves only when a row's tile max exceeds it
// by more than this (log2 units), so P <= 2^8 and O is rescaled on few steps...
constexpr float kLazyMaxSlack = 8.0f;
// ...or when the tile max's weight exceeds this fraction of the row sum so
// far: a key that carries a large share of its row is then taken at the exact
// max, where its P = 1 is exact and leaves the rounded mass.
constexpr float kLazyMaxDominant = 1.0f / 16;
constexpr int kLazyMaxRowsFrom = 1024;  // keys a row sees (at least) to take the lazy max

// Tile geometry for head_dim D (64 or 128). A K or V tile is always 8 KiB:
// 64 keys of 128 B rows for D = 64, 32 keys of 256 B rows for D = 128, so a
// step is 16 MFMAs either way (D = 64: QK 2 key blocks x 4 d-steps, PV 4
// k-steps x 2 d-blocks; D = 128: QK 1 x 8, PV 2 x 4).
template <int D>
struct Geo {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static constexpr int kBc = D == 64 ? 64 : 32;    // keys per tile
  static constexpr int kKB = kBc / 32;             // 32-key blocks per tile (S^T tiles)
  static constexpr int kDS = D / 16;               // k-steps of S^T = K Q^T
  static constexpr int kDB = D / 32;               // d-blocks of O^T
  static constexpr int kKS = kBc / 16;             // k-steps of O^T += V^T P^T
  static constexpr int kChunks = D / 8;            // 16-byte chunks per row
  static constexpr int kRowsPerLoad = kWave / kChunks;  // rows per wave load
  static constexpr int kTileHalves = kBc * D;      // 4096 halves = 8 KiB
  // D = 64 stages the Q tile in LDS; D = 128 loads Q^T straight into
  // registers, which leaves the whole LDS to the two rings.
  static constexpr bool kQInLds = D == 64;
  // LDS (halves): [Q: 128 rows x 64 (D = 64 only)] [half 0: K ring | V ring] [half 1: ...]
  static constexpr int kQHalves = kQInLds ? kBr * D : 0;                  // 16 KiB / 0
  static constexpr int kHalfHalves = (kKStages + kVStages) * kTileHalves; // 72 KiB
  static constexpr int kLdsHalves = kQHalves + 2 * kHalfHalves;           // 160 / 144 KiB
  // Half-merge exchange at the end: [row wave][group][64 lanes][4] fp32, the
  // groups holding the O^T values, then (m, l, r, unused); 16 B per lane and
  // group, so each group is one conflict-free ds_write_b128 / ds_read_b128.
  static constexpr int kXchg = 16 * kDB + 4;  // floats per lane
  static constexpr int kXchgBytes = kRowWaves * kXchg * kWave * 4;
  // Output staging after the exchange: per row wave, its 32 rows of O,
  // row-major with 16-byte chunks XOR-swizzled by row, so that each lane can
  // store 16 contiguous bytes and a store instruction covers whole rows.
  template <bool F32>
  static constexpr int kOutRowBytes = D * (F32 ? 4 : 2);
  static_assert(kXchgBytes + kRowWaves * kRowsPerWave * kOutRowBytes<true> <= kLdsHalves * 2,
                "exchange and output staging fit in LDS");
};


[[maybe_unused]] __device__ __forceinline__ half8 lds_b128(const _Float16 *p) {
  return *reinterpret_cast<const half8 *>(p);
}

// The lane index read afresh from the hardware (v_mbcnt, in volatile asm so
// that the compiler cannot merge it with the kernel's first lane index). The
// code after the main loop (masked tail, verdict, epilogue) derives its
// per-lane values from this instead of from values computed before the loop,
// which the compiler otherwise keeps live across it: at 256 VGPRs they went
// to scratch (5 per lane at head_dim 64, 11-15 at 128), each item stored and
// reloaded them, and their write-backs were 2.5-3.4 MB of a C3 launch's HBM
// writes (C3 46.2 -> 45.8 us, C2 full 27.1 -> 26.4 us without them).
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// head_dim 64 sums P rows on the matrix cores (rowsum_mfma); head_dim 128,
// whose loop has no registers to spare, sums them with v_dot2_f32_f16 per
// lane.
template <int D>
constexpr bool kMfmaRowSum = D == 64;

// Per-lane softmax state of one query row. Both lanes of a pair hold the same
// m and mt; r is this lane's share of the row's rounded mass; head_dim 64:
// both lanes hold the row sum (lacc[0]); head_dim 128: l is this lane's share.
template <int D>
struct SoftmaxState {
  float m;                      // the max P is taken against (log2 domain, scaled by c)
  float mt;                     // the row's true running max (log2 domain)
  float r;                      // rounded mass: sum of P^2 of rounded weights, units of m
  float lprev;                  // row sum at the start of the step (head_dim 64)
  float l;                      // this lane's share of the row sum (head_dim 128)
  floatx4 lacc;                 // row sum on the matrix cores: element 0 (head_dim 64)
  floatx16 o[Geo<D>::kDB];      // O^T accumulators, one per 32-dim block
};

// Register copies of the LDS fragments one tile step consumes.
template <int D>
struct KFrags { half8 f[Geo<D>::kKB][Geo<D>::kDS]; };  // [32-key block][d-step]
template <int D>
struct VFrags { half8 f[Geo<D>::kKS][Geo<D>::kDB]; };  // [16-key step][d-block]


template <int D>
__device__ __forceinline__ void read_k(unsigned tile, const FragOffsetsD<D> &fo, KFrags<D> &k) {
  const unsigned base = uniform_lds_u(tile);
#pragma unroll
  for (int s = 0; s < Geo<D>::kDS; ++s) {
    lds_half *p = opaque_lds_at(base, fo.k[s]);
#pragma unroll
    for (int kb = 0; kb < Geo<D>::kKB; ++kb)
      k.f[kb][s] = *reinterpret_cast<__attribute__((address_space(3))) const half8 *>(
          p + kb * 32 * D);
  }
}

template <int D>
__device__ __forceinline__ void read_v(unsigned tile, const FragOffsetsD<D> &fo, VFrags<D> &v) {
  const unsigned base = uniform_lds_u(tile);
#pragma unroll
  for (int db = 0; db < Geo<D>::kDB; ++db) {
    lds_half *p = opaque_lds_at(base, fo.v[db]);
#pragma unroll
    for (int ks = 0; ks < Geo<D>::kKS; ++ks) {
      const int kb = ks >> 1, h = ks & 1;
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4v *)(p + (kb * 32 + 16 * h + 8 * part) * D));
        const half4 v4 = __builtin_bit_cast(half4, r);
#pragma unroll
        for (int e = 0; e < 4; ++e) v.f[ks][db][4 * part + e] = v4[e];
      }
    }
  }
}

// S^T[kb] = K_kb Q^T for every 32-key block of the tile (8 MFMAs).
template <int D>
__device__ __forceinline__ void qk_mfma(const KFrags<D> &k, const half8 (&qf)[Geo<D>::kDS],
                                        floatx16 (&s)[Geo<D>::kKB]) {
#pragma unroll
  for (int kb = 0; kb < Geo<D>::kKB; ++kb)
#pragma unroll
    for (int a = 0; a < 16; ++a) s[kb][a] = 0.f;
#pragma unroll
  for (int i = 0; i < Geo<D>::kDS; ++i)
#pragma unroll
    for (int kb = 0; kb < Geo<D>::kKB; ++kb) s[kb] = mfma(k.f[kb][i], qf[i], s[kb]);
}

// The same 8 MFMAs in two parts of four, part 0 first: head_dim 64, part p is
// 32-key block p (all four d-steps); head_dim 128, whose tile is one 32-key
// block, part p is its d-steps [4 p, 4 p + 4). A pipelined step issues part 0
// at the step boundary, before the block barrier: it reads only registers
// (the K fragments of the next tile, read at the end of the previous step,
// and Q^T), so the matrix cores work through it while the wave waits at the
// barrier and issues its tile loads, and the step's interleave keeps the
// other 12 (+ 4 row sums at head_dim 64) for the softmax. Output
// bit-identical; C3 46.8 -> 46.2 us, C2 full 27.9 -> 27.2 us, head_dim 128
// C3 shape 87.4 -> 86.1 us.
template <int D>
__device__ __forceinline__ void qk_mfma_part(const KFrags<D> &k, const half8 (&qf)[Geo<D>::kDS],
                                             floatx16 (&s)[Geo<D>::kKB], int part) {
  if constexpr (Geo<D>::kKB == 2) {
#pragma unroll
    for (int a = 0; a < 16; ++a) s[part][a] = 0.f;
#pragma unroll
    for (int i = 0; i < Geo<D>::kDS; ++i) s[part] = mfma(k.f[part][i], qf[i], s[part]);
  } else {
    if (part == 0) {
#pragma unroll
      for (int a = 0; a < 16; ++a) s[0][a] = 0.f;
    }
#pragma unroll
    for (int i = 4 * part; i < 4 * part + 4; ++i) s[0] = mfma(k.f[0][i], qf[i], s[0]);
  }
}

// O^T[db] += V^T_db P^T for every 32-dim block (8 MFMAs).
template <int D>
__device__ __forceinline__ void pv_mfma(const VFrags<D> &v, const half8 (&p)[Geo<D>::kKS],
                                        floatx16 (&o)[Geo<D>::kDB]) {
#pragma unroll
  for (int ks = 0; ks < Geo<D>::kKS; ++ks)
#pragma unroll
    for (int db = 0; db < Geo<D>::kDB; ++db) o[db] = mfma(v.f[ks][db], p[ks], o[db]);
}

// Row sums of a tile's P^T fragments, on the matrix cores (one
// v_mfma_f32_16x16x32_f16 per 16-key step, see rowsum_selector): element 0
// of lacc gathers the sum of the same fp16 P values that the PV product
// consumes, for the lane's own query.
template <int D>
__device__ __forceinline__ void rowsum_mfma(const half8 &sel, const half8 (&p)[Geo<D>::kKS],
                                            floatx4 &lacc) {
  if constexpr (!kMfmaRowSum<D>) return;
#pragma unroll
  for (int ks = 0; ks < Geo<D>::kKS; ++ks) lacc = mfma16(sel, p[ks], lacc);
}

// Row max of one tile and the lazy update of m. Returns whether the wave
// rescales (wave-uniform): m moves, to the row's exact running max, only when
// some row of the wave has a tile max more than kLazyMaxSlack above its m, or
// one whose weight exceeds kLazyMaxDominant times the row sum so far (head_dim
// 64: lprev, the sum at the start of the step; head_dim 128: the lane's share
// l); alpha (set then) rescales the previous O and row sum (head_dim 64: at
// the next step's rescale_o) and the rounded mass. pm is the tile's largest
// weight in units of the (new) m.
// MASK: keys past the end or above the causal diagonal become -inf.
template <bool CAUSAL, bool MASK, int D>
__device__ __forceinline__ bool tile_max(floatx16 (&s)[Geo<D>::kKB], int lim, float c_scale,
                                         float slack, SoftmaxState<D> &st, float &alpha,
                                         float &pm) {
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < Geo<D>::kKB; ++kb) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      if (MASK)
        s[kb][a] = (kb * 32 + 8 * (a >> 2) + (a & 3) <= lim) ? s[kb][a] : -INFINITY;
      mx = fmaxf(mx, s[kb][a]);
    }
  }
  mx = max_lane_pair(mx);
  float mx_c;
  {
    // No contraction: with mx_c rounded once, a tile that sets m gets
    // largest weight exp2(0) = 1 exactly.
#pragma clang fp contract(off)
    mx_c = mx * c_scale;
  }
  st.mt = fmaxf(st.mt, mx_c);
  pm = fast_exp2(mx_c - st.m);
  const float l_seen = kMfmaRowSum<D> ? st.lprev : st.l;
  const bool move = mx_c > st.m + slack || pm > fmaxf(1.0f, kLazyMaxDominant * l_seen);
  const bool rescale = __builtin_amdgcn_ballot_w64(move) != 0;
  alpha = 1.0f;
  if (rescale) {
    alpha = fast_exp2(st.m - st.mt);
    st.m = st.mt;
    if constexpr (!kMfmaRowSum<D>) st.l *= alpha;
    st.r *= alpha * alpha;
    pm = fast_exp2(mx_c - st.m);
  }
  return rescale;
}

// P^T fragments (hi [+ lo]) of one tile. head_dim 128 also adds the tile to
// its row-sum share. With one rounding of P, the lane adds the squares of its
// rounded weights to its share of the rounded mass, less the exact 1 of a
// tile whose largest weight is exactly 1 (the key at m: fp16 holds it
// exactly; half of it in each lane of the pair, since only their sum is used).
template <bool MASK, bool SPLIT, int D>
__device__ __forceinline__ void tile_exp(const floatx16 (&s)[Geo<D>::kKB], float c_scale,
                                         float pm, SoftmaxState<D> &st,
                                         half8 (&p_hi)[Geo<D>::kKS],
                                         half8 (&p_lo)[Geo<D>::kKS]) {
  const half2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  float lsum = 0.f, sq = 0.f;
  const float m_use = st.m;
#pragma unroll
  for (int ks = 0; ks < Geo<D>::kKS; ++ks) {
    const int kb = ks >> 1, h = ks & 1;
#pragma unroll
    for (int t = 0; t < 8; t += 2) {
      const float s0 = s[kb][8 * h + t], s1 = s[kb][8 * h + t + 1];
      float p0 = fast_exp2(fmaf(s0, c_scale, -m_use));
      float p1 = fast_exp2(fmaf(s1, c_scale, -m_use));
      if (MASK) {
        p0 = (s0 == -INFINITY) ? 0.f : p0;
        p1 = (s1 == -INFINITY) ? 0.f : p1;
      }
      const half2 hi2 = {static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
      p_hi[ks][t] = hi2[0];
      p_hi[ks][t + 1] = hi2[1];
      if constexpr (!kMfmaRowSum<D>) lsum = __builtin_amdgcn_fdot2(hi2, ones, lsum, false);
      if (!SPLIT) sq = __builtin_amdgcn_fdot2(hi2, hi2, sq, false);
      if (SPLIT) {
        const half2 lo2 = {static_cast<_Float16>(p0 - static_cast<float>(hi2[0])),
                           static_cast<_Float16>(p1 - static_cast<float>(hi2[1]))};
        p_lo[ks][t] = lo2[0];
        p_lo[ks][t + 1] = lo2[1];
        if constexpr (!kMfmaRowSum<D>) lsum = __builtin_amdgcn_fdot2(lo2, ones, lsum, false);
      }
    }
  }
  if constexpr (!kMfmaRowSum<D>) st.l += lsum;
  if (!SPLIT) st.r += sq - (pm == 1.0f ? 0.5f : 0.0f);
}

// O (and, head_dim 64, the row sum on the matrix cores) follow a move of m
// (wave-uniform branch).
template <int D>
__device__ __forceinline__ void rescale_o(SoftmaxState<D> &st, float alpha, bool rescale) {
  if (rescale) {
#pragma unroll
    for (int db = 0; db < Geo<D>::kDB; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) st.o[db][a] *= alpha;
    if constexpr (kMfmaRowSum<D>) {
      st.lacc[0] *= alpha;
      st.lprev *= alpha;
    }
  }
}

// head_dim 64: the row sum the next tile_max weighs a new max against (the
// accumulator as the step starts, which holds P up to two steps back).
template <int D>
__device__ __forceinline__ void note_row_sum(SoftmaxState<D> &st) {
  if constexpr (kMfmaRowSum<D>) st.lprev = st.lacc[0];
}

// Scheduling pipeline for one main step: each of its MFMAs followed by a
// group of VALU instructions (the softmax of the other tile), then a hard
// scheduling boundary so no compute sinks below the next step's barrier.
template <int D>
__device__ __forceinline__ void interleave_step() {
  // QK (less the part issued at the boundary) + PV + row sums
  constexpr int kMfmas = 16 + Geo<D>::kKS - 4;
#pragma unroll
  for (int i = 0; i < kMfmas; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Pins the P fragments of a step to that step: without a use there, the
// compiler sinks their computation into the next step (next to the PV MFMAs
// that consume them), which defeats the interleave.
// The rounded mass gets the same pin: its squares would otherwise sink to the
// next step's row max, outside the interleave.
template <int N, int D>
__device__ __forceinline__ void keep(const half8 (&p)[N], const SoftmaxState<D> &st) {
#pragma unroll
  for (int ks = 0; ks < N; ++ks) asm volatile("" ::"v"(p[ks]));
  asm volatile("" ::"v"(st.r));
}

// Plain (non-pipelined) step for masked / short-row tiles: QK, softmax with
// mask and split P, PV and the row sums issued for both parts.
template <bool CAUSAL, int D>
__device__ __forceinline__ void slow_step(const KFrags<D> &kf, const VFrags<D> &vf,
                                          const half8 (&qf)[Geo<D>::kDS], const half8 &sel,
                                          int key0, int seq, int my_q, int lane, float c_scale,
                                          float slack, SoftmaxState<D> &st) {
  floatx16 s[Geo<D>::kKB];
  qk_mfma<D>(kf, qf, s);
  // Element a of key block kb holds key key0 + kb*32 + 8 (a/4) + 4 g + a%4;
  // it is visible iff that offset is <= lim (last visible key - key0 - 4 g).
  const int lim = (CAUSAL ? min(my_q, seq - 1) : seq - 1) - key0 - 4 * (lane >> 5);
  float alpha, pm;
  const bool rescale = tile_max<CAUSAL, true, D>(s, lim, c_scale, slack, st, alpha, pm);
  rescale_o(st, alpha, rescale);
  half8 p_hi[Geo<D>::kKS], p_lo[Geo<D>::kKS];
  tile_exp<true, true, D>(s, c_scale, pm, st, p_hi, p_lo);
  pv_mfma<D>(vf, p_hi, st.o);
  pv_mfma<D>(vf, p_lo, st.o);
  rowsum_mfma<D>(sel, p_hi, st.lacc);
  rowsum_mfma<D>(sel, p_lo, st.lacc);
}

// The K and V rings of one key half: half h owns tiles 2 k + h (k = 0, 1,
// ...), in K stage k % kKStages and V stage k % kVStages.
template <int D>
struct HalfRing {
  using G = Geo<D>;
  unsigned kring, vring;  // LDS byte addresses of the two rings
  const _Float16 *kp, *vp;
  int seq, t0, n_tiles, half;  // this half streams tiles t0 + 2 k + half below n_tiles
  unsigned voff[2][2];  // [K|V][row block i]: byte offset of this lane's chunk in a tile
  int row_in_tile[2];
  int lds_off[2];       // row block i of this wave, in halves

  __device__ __forceinline__ int tile(int k) const { return t0 + 2 * k + half; }
  __device__ __forceinline__ bool exists(int k) const { return tile(k) < n_tiles; }
  __device__ __forceinline__ unsigned kstage(int k) const {
    return kring + (k % kKStages) * (2 * G::kTileHalves);
  }
  __device__ __forceinline__ unsigned vstage(int k) const {
    return vring + (k % kVStages) * (2 * G::kTileHalves);
  }
  // The half's four waves each load row blocks {2 wh, 2 wh + 1} (one wave
  // load each: 8 rows of 128 B for D = 64, 4 rows of 256 B for D = 128) of K
  // and of V; lane = (D / 8) * (row in block) + chunk. Rows past the sequence
  // end are clamped to the last row: they are masked in the softmax (K) and
  // weighted by 0 (V).
  __device__ __forceinline__ void issue(int k) const {
    if (!exists(k)) return;
    const int key0 = tile(k) * G::kBc;
    const unsigned ks = kstage(k);
    const unsigned vs = vstage(k);
    if (key0 + G::kBc <= seq) {
      // Whole tile inside the sequence: a scalar tile base plus the lane's
      // fixed offset.
      const _Float16 *const kb = kp + static_cast<size_t>(key0) * D;
      const _Float16 *const vb = vp + static_cast<size_t>(key0) * D;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        global_to_lds16_sbase_at(kb, voff[0][i], ks + 2 * lds_off[i]);
        global_to_lds16_sbase_at(vb, voff[1][i], vs + 2 * lds_off[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int in_row = row_in_tile[i] * D;
        const size_t row = static_cast<size_t>(min(key0 + row_in_tile[i], seq - 1)) * D;
        global_to_lds16_at(kp + row + (voff[0][i] / 2 - in_row), ks + 2 * lds_off[i]);
        global_to_lds16_at(vp + row + (voff[1][i] / 2 - in_row), vs + 2 * lds_off[i]);
      }
    }
  }
  // Start of main step k: this half's tiles up to k + 2 are resident and
  // visible to the whole block, then the loads of tile k + 4 are issued.
  // Its K stage last held tile k, its V stage tile k - 1: the main loop read
  // them at the end of steps k - 2 and k - 1, the masked step reads a tile
  // before its own barrier. Each wave drains its LDS reads (lgkmcnt(0))
  // before the barrier: a V read issued just before it could otherwise still
  // sit in the LDS queue when another wave's refill of that stage lands
  // (measured cost: none, the reads are needed right after anyway).
  // A plain s_barrier: __syncthreads() would add a release fence, which
  // drains every outstanding load of the ring.
  __device__ __forceinline__ void advance(int k) const {
    wait(k);
    pass(k);
  }
  // advance in two parts, for register-only work between them: this wave's
  // waits, then the barrier and the loads of tile k + 4.
  __device__ __forceinline__ void wait(int k) const {
    if (exists(k + 3))
      wait_loads<kLoadsPerTile>();
    else
      wait_loads<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  __device__ __forceinline__ void pass(int k) const {
    __builtin_amdgcn_s_barrier();
    issue(k + kAhead);
  }
};

// Block -> (b, h) with XCD affinity. The grid stays in level-major order
// (every head's heaviest query tile first), and blocks go to the 8 XCDs
// round-robin (block i on XCD i % 8). Head h is "at home" on XCD h % 8:
// within a level each XCD fills its positions with its home heads first and
// the leftover heads take the spare positions in a fixed order, so most of a
// head's blocks share one XCD's L2 (for 14 heads, 89 % of the blocks).
__host__ __device__ __forceinline__ int home_head(int i, int n_bh) {
  const int level = i / n_bh;
  const int k = i - level * n_bh;
  const int base = (level * n_bh) & 7;
  const int x = (base + k) & 7;     // XCD of this block
  const int d_x = (x - base) & 7;   // first position of XCD x in this level
  const int r = (k - d_x) >> 3;     // rank of position k among XCD x's
  const int nhome_x = (n_bh - x + 7) >> 3;
  if (r < nhome_x) return x + 8 * r;
  // A spare position: its index among all spares (XCDs in order, then rank)
  // selects the matching overflow head (XCDs in order, then head rank).
  int s = r - nhome_x;
  for (int y = 0; y < x; ++y) {
    const int npos = (n_bh - ((y - base) & 7) + 7) >> 3;
    const int nhome = (n_bh - y + 7) >> 3;
    s += npos > nhome ? npos - nhome : 0;
  }
  for (int y = 0; y < 8; ++y) {
    const int npos = (n_bh - ((y - base) & 7) + 7) >> 3;
    const int nhome = (n_bh - y + 7) >> 3;
    const int over = nhome > npos ? nhome - npos : 0;
    if (s < over) return y + 8 * (npos + s);
    s -= over;
  }
  return 0;  // unreachable: spare positions and overflow heads are equal in number
}

// Grouped queries: the placement heads of XCD x (x, x + 8, x + 16, ...) are
// given a contiguous run of query heads, in XCD order, so the query heads
// that read one K/V head (consecutive indices) mostly share an XCD and its
// L2 holds one copy of that K/V head.
__host__ __device__ __forceinline__ int grouped_head(int h, int n_bh) {
  const int x = h & 7;
  int start = 0;
  for (int y = 0; y < x; ++y) start += (n_bh - y + 7) >> 3;
  return start + (h >> 3);
}

// Work units and their blocks, planned on the host when the items do not
// fill the chip evenly (at most two per CU): the heaviest items are split
// into two key chunks, tiles [0, mid) and [mid, n_tiles) with mid =
// split_mid(n_tiles), and every block takes (up to) two units, heavy with
// light. A unit is pos | code << 20 | split << 22: item pos (numbered as in
// the kernel), code 0 for the whole key range, 1 / 2 for the first / second
// chunk, split = the item's index among the split items (its partial slots
// and counters). n_blocks = 0: no plan, blocks take items by formula.
constexpr int kPlanMaxBlocks = 384;
constexpr unsigned kNoUnit = 0xffffffffu;
struct PrefillPlan {
  int n_blocks;
  unsigned unit[2 * kPlanMaxBlocks];  // block b: unit[2 b] first, unit[2 b + 1] second
};
__host__ __device__ __forceinline__ int split_mid(int n_tiles) { return (n_tiles / 2) & ~1; }
// Partial of one row wave of one chunk: O^T accumulators (lane-major), then m
// and the row sum (or head_dim 128's per-lane share of it), one per lane.
template <int D>
constexpr int kPartOFloats = Geo<D>::kDB * 16 * kWave;
template <int D>
constexpr int kPartFloats = kPartOFloats<D> + 2 * kWave;

template <int D, bool CAUSAL, bool OUT_F32>
__global__ __launch_bounds__(kThreads, 1) void prefill_kernel(
    const _Float16 *__restrict__ q, const _Float16 *__restrict__ k,
    const _Float16 *__restrict__ v, void *__restrict__ o, int seq,
    int n_qtiles, int bh_count, int group, float c_scale, bool negate_q, bool split_all,
    const PrefillPlan plan, float *__restrict__ part, unsigned *__restrict__ counters) {
  using G = Geo<D>;
  constexpr int kBc = G::kBc;
  constexpr int kKB = G::kKB;
  constexpr int kKS = G::kKS;
  constexpr int kDB = G::kDB;
  constexpr int kDS = G::kDS;
  __shared__ __attribute__((aligned(1024))) _Float16 lds[G::kLdsHalves];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Wave-uniform (SGPR) so every stage / row-block address below is scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rw = wave & (kRowWaves - 1);  // row wave: rows [32 rw, +32)
  const int half = wave / kRowWaves;      // key half: tiles 2k + half
  const int col = lane & 31;
  _Float16 *const half_lds = lds + G::kQHalves + half * G::kHalfHalves;
  _Float16 *const q_lds = lds;
  HalfRing<D> ring;
  ring.kring = lds_addr(half_lds);
  ring.vring = ring.kring + kKStages * (2 * G::kTileHalves);
  ring.seq = seq;
  ring.half = half;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rblock = 2 * rw + i;
    const int r = rblock * G::kRowsPerLoad + lane / G::kChunks;
    const int p = lane % G::kChunks;
    ring.row_in_tile[i] = r;
    ring.voff[0][i] = 2u * static_cast<unsigned>(r * D + ((p ^ k_swz_d<D>(r)) << 3));
    ring.voff[1][i] = 2u * static_cast<unsigned>(r * D + ((p ^ v_swz_d<D>(r)) << 3));
    ring.lds_off[i] = rblock * G::kRowsPerLoad * D;
  }
  const FragOffsetsD<D> fo = frag_offsets_d<D>(lane);
  const half8 sel = rowsum_selector(lane);

  // Items are (b, h, 128-row query tile), numbered heaviest (last) query
  // tile first. Block b of the G-block grid (G >= items / 2) takes item b,
  // then item G + mirror(b) if there is one, so a block with a heavy first
  // item gets a light second one: with causal masking, items b and ~2G - b
  // sum to about the same work. The mirror reverses groups of 8 positions
  // and keeps the position mod 8, the XCD the block runs on (blocks go to
  // the 8 XCDs round-robin), which home_head uses for L2 placement. (Two
  // unrolled rounds, no loop back-edge: the body keeps its registers.)
  const int n_items = bh_count * n_qtiles;
  const int grid = static_cast<int>(gridDim.x);
  const int b_id = static_cast<int>(blockIdx.x);
  const int b_mirror = (grid & 7) == 0 ? grid - 8 * (b_id / 8 + 1) + (b_id & 7) : grid - 1 - b_id;
#pragma unroll
  for (int round = 0; round < 2; ++round) {
  int pos, code = 0, split = 0;
  if (plan.n_blocks > 0) {
    const unsigned u = plan.unit[2 * b_id + round];
    if (u == kNoUnit) break;
    pos = static_cast<int>(u & 0xfffffu);
    code = static_cast<int>((u >> 20) & 3u);
    split = static_cast<int>(u >> 22);
  } else {
    pos = round == 0 ? b_id : grid + b_mirror;
    if (pos >= n_items) break;
  }
  // The previous item's last LDS accesses (output staging) end before this
  // item's loads overwrite the LDS.
  if (round > 0) __syncthreads();
  const int qtile = n_qtiles - 1 - pos / bh_count;
  int bh = home_head(pos, bh_count);
  if (group > 1) bh = grouped_head(bh, bh_count);

  // Q and O are [B, H, S, 64], K and V [B, H / group, S, 64]: query head
  // b * H + h reads K/V head b * H / group + h / group = bh / group.
  const size_t head_off = static_cast<size_t>(bh) * seq * D;
  const size_t kv_off = static_cast<size_t>(bh / group) * seq * D;
  const int q0 = qtile * kBr;
  const int qw0 = q0 + rw * kRowsPerWave;
  const int my_q = qw0 + col;

  const int key_end = CAUSAL ? min(seq, q0 + kBr) : seq;
  const int n_tiles = (key_end + kBc - 1) / kBc;
  // This unit's tiles [tb, te): the whole range, or one chunk of it (tb is
  // even, so each half keeps the parity of its tiles).
  const int tb = code == 2 ? split_mid(n_tiles) : 0;
  const int te = code == 1 ? split_mid(n_tiles) : n_tiles;
  ring.kp = k + kv_off;
  ring.vp = v + kv_off;
  ring.t0 = tb;
  ring.n_tiles = te;
  const int wave_key_end = CAUSAL ? min(seq, qw0 + kRowsPerWave) : seq;
  // Tiles [0, 2 n_main) need no mask for any row of the block, and all its
  // rows see >= kSplitPRowsBelow keys: each half runs n_main pipelined steps
  // on them, then at most one masked pipelined step (n_steps <= n_main + 1
  // whenever n_main > 0: causal, the diagonal adds two tiles; full, the
  // ragged tail one). Blocks with short rows take the plain split-P step on
  // every tile.
  const bool static_split = CAUSAL ? q0 < kSplitPRowsBelow : seq < kSplitPRowsBelow;
  // Pass 0 rounds P to fp16 once on rows that see enough keys; blocks whose
  // row sums then show a peaky row run again with split P on every tile.
  const bool short_rows = split_all || static_split;
  const int main_end = short_rows ? 0 : (CAUSAL ? q0 / kBc : seq / kBc);
  const int n_main = max(0, min(main_end, te) - tb) / 2;
  const int n_steps = (te - tb + 1) / 2;  // steps of the longer half
  // Rows that see many keys take the lazy max; shorter ones keep m at the
  // exact running max, whose P = 1 key takes no rounding.
  const float slack =
      (CAUSAL ? q0 : seq) >= kLazyMaxRowsFrom ? kLazyMaxSlack : 0.f;

  half8 qf[kDS];
  SoftmaxState<D> st;
  auto prologue = [&]() {
    // Q: for D = 64 the tile goes to LDS (16 row blocks of 8 rows, 2 per wave;
    // K swizzle); for D = 128 each lane loads its Q^T fragments (query my_q,
    // head dims [64 g + 8 s, +8)) straight into registers. Then this half's
    // first kAhead tiles.
    if constexpr (G::kQInLds) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int rblock = 2 * wave + i;
        const int r = rblock * 8 + (lane >> 3);
        const int row = min(q0 + r, seq - 1);
        global_to_lds16(q + head_off + static_cast<size_t>(row) * D +
                            (((lane & 7) ^ k_swz(r)) << 3),
                        q_lds + rblock * 8 * D);
      }
    } else {
      const _Float16 *qrow = q + head_off + static_cast<size_t>(min(my_q, seq - 1)) * D +
                             (lane >> 5) * (D / 2);
#pragma unroll
      for (int s = 0; s < kDS; ++s) qf[s] = *reinterpret_cast<const half8 *>(qrow + 8 * s);
    }
#pragma unroll
    for (int kk = 0; kk < kAhead; ++kk) ring.issue(kk);
    // Q and tiles 0, 1 resident (tiles 2, 3 may still be in flight; the first
    // advance waits for tile 2).
    if (ring.exists(3))
      wait_loads<2 * kLoadsPerTile>();
    else if (ring.exists(2))
      wait_loads<kLoadsPerTile>();
    else
      wait_loads<0>();
    __builtin_amdgcn_s_barrier();

    // Q^T fragments: lane holds query my_q, head dims [(D / 2) g + 8 s, +8).
#pragma unroll
    for (int s = 0; s < kDS; ++s) {
      if constexpr (G::kQInLds) qf[s] = lds_b128(q_lds + rw * kRowsPerWave * D + fo.k[s]);
      if (negate_q) qf[s] = -qf[s];
    }

    st.m = kNegHuge;
    st.mt = kNegHuge;
    st.r = 0.f;
    st.lprev = 0.f;
    st.l = 0.f;
    st.lacc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) st.o[db][a] = 0.f;
  };
  auto split_steps = [&](int kk0) {
    // ---- short-row blocks: one plain split-P step per tile ---------------------
    // Tile kk is resident (waited for by an earlier advance, or by the
    // prologue); its fragments are read before the barrier that lets the load
    // of tile kk + 4 overwrite its K stage.
    for (int kk = kk0; kk < n_steps; ++kk) {
      const int key0 = ring.tile(kk) * kBc;
      const bool active = key0 < wave_key_end;
      KFrags<D> kf;
      VFrags<D> vf;
      if (active) {
        read_k(ring.kstage(kk), fo, kf);
        read_v(ring.vstage(kk), fo, vf);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the reads are done
      ring.advance(kk);
      if (active)
        slow_step<CAUSAL, D>(kf, vf, qf, sel, key0, seq, my_q, lane, c_scale, slack, st);
    }
  };
  auto merge_halves = [&]() -> float * {
    // ---- merge the two halves through LDS ---------------------------------------
    // Every load the ring issued has completed; the barrier ends every read of it.
    wait_loads<0>();
    __builtin_amdgcn_s_barrier();
    float *xbase = reinterpret_cast<float *>(lds) + rw * (G::kXchg * kWave);
    floatx4 *xg = reinterpret_cast<floatx4 *>(xbase) + lane;  // group i at xg[i * kWave]
    if (half == 1) {
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          xg[(4 * db + i) * kWave] = {st.o[db][4 * i], st.o[db][4 * i + 1], st.o[db][4 * i + 2],
                                      st.o[db][4 * i + 3]};
      xg[4 * kDB * kWave] = {st.m, kMfmaRowSum<D> ? st.lacc[0] : st.l, st.r, 0.f};
    }
    __syncthreads();
    if (half == 0) {
      const floatx4 mlr = xg[4 * kDB * kWave];
      const float m = fmaxf(st.m, mlr[0]);
      const float f0 = fast_exp2(st.m - m);
      const float f1 = fast_exp2(mlr[0] - m);
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const floatx4 o1 = xg[(4 * db + i) * kWave];
#pragma unroll
          for (int e = 0; e < 4; ++e) st.o[db][4 * i + e] = st.o[db][4 * i + e] * f0 + o1[e] * f1;
        }
      if constexpr (kMfmaRowSum<D>)
        st.lacc[0] = st.lacc[0] * f0 + mlr[1] * f1;
      else
        st.l = st.l * f0 + mlr[1] * f1;
      st.r = st.r * (f0 * f0) + mlr[2] * (f1 * f1);
      st.m = m;  // O, l and r are now in units of the merged max
    }
    return xbase;
  };

  prologue();
  // ---- pipelined main loop ---------------------------------------------------
  // Step k: MFMAs QK(k+1) [K_{k+1}, read at step k-1] and PV(k-1) [P_{k-1},
  // V_{k-1}] interleave with the softmax of S_k; the first part of QK(k+1)
  // goes ahead of the step's barrier (qk_mfma_part). S, P and the K fragments
  // alternate between even and odd steps. QK(k+1) is issued unconditionally:
  // on the last main step it reads whatever K stage k+1 holds (in bounds)
  // and the result is discarded.
  int kk = 0;
  if (n_main > 0) {
    floatx16 s_a[kKB], s_b[kKB];
    half8 p_a[kKS], p_b[kKS], p_unused[kKS];
    KFrags<D> kf;
    VFrags<D> vf;
    // alpha / rescale: the move of m that the next step applies to O before
    // its PV. pm_a, pm_b: largest weights of the P tiles in p_a, p_b.
    float alpha, pm_a, pm_b;
    bool rescale;
    read_k(ring.kstage(0), fo, kf);
    qk_mfma(kf, qf, s_a);
    read_k(ring.kstage(1), fo, kf);

    // step 0 (no PV yet)
    ring.advance(0);
    rescale = tile_max<CAUSAL, false>(s_a, 0, c_scale, slack, st, alpha, pm_a);
    qk_mfma(kf, qf, s_b);
    tile_exp<false, false>(s_a, c_scale, pm_a, st, p_a, p_unused);
    __builtin_amdgcn_sched_barrier(0);
    read_k(ring.kstage(2), fo, kf);
    read_v(ring.vstage(0), fo, vf);
    kk = 1;

    // steps kk (odd: S_kk in s_b, P_{kk-1} in p_a) and kk + 1 (even); kf and
    // vf hold K_{kk+1} and V_{kk-1}.
    for (; kk + 1 < n_main; kk += 2) {
      ring.wait(kk);
      qk_mfma_part(kf, qf, s_a, 0);
      ring.pass(kk);
      note_row_sum(st);
      rescale_o(st, alpha, rescale);
      rescale = tile_max<CAUSAL, false>(s_b, 0, c_scale, slack, st, alpha, pm_b);
      qk_mfma_part(kf, qf, s_a, 1);
      rowsum_mfma<D>(sel, p_a, st.lacc);
      pv_mfma(vf, p_a, st.o);
      tile_exp<false, false>(s_b, c_scale, pm_b, st, p_b, p_unused);
      interleave_step<D>();
      keep(p_b, st);
      read_k(ring.kstage(kk + 2), fo, kf);
      read_v(ring.vstage(kk), fo, vf);

      ring.wait(kk + 1);
      qk_mfma_part(kf, qf, s_b, 0);
      ring.pass(kk + 1);
      note_row_sum(st);
      rescale_o(st, alpha, rescale);
      rescale = tile_max<CAUSAL, false>(s_a, 0, c_scale, slack, st, alpha, pm_a);
      qk_mfma_part(kf, qf, s_b, 1);
      rowsum_mfma<D>(sel, p_b, st.lacc);
      pv_mfma(vf, p_b, st.o);
      tile_exp<false, false>(s_a, c_scale, pm_a, st, p_a, p_unused);
      interleave_step<D>();
      keep(p_a, st);
      read_k(ring.kstage(kk + 3), fo, kf);
      read_v(ring.vstage(kk + 1), fo, vf);
    }
    // Here step kk - 1 is done: S_kk in s_b, P_{kk-1} in p_a, V_{kk-1} in vf.
    // The last step of each half (causal diagonal / ragged tile) runs with a
    // masked softmax on the S that the previous step's QK produced; waves
    // that see none of that tile only drain. (Its P is not split: every row
    // of the block sees >= kSplitPRowsBelow keys.)
    // (head_dim 128: its 32-key tiles put two masked tiles in each half's
    // range; the second one takes the plain step below.)
    const bool tail = n_steps >= n_main + 1;
    if (kk < n_main) {  // one more (odd) main step; leaves S_{kk+1} in s_b, P_kk in p_a
      ring.advance(kk);
      note_row_sum(st);
      rescale_o(st, alpha, rescale);
      rescale = tile_max<CAUSAL, false>(s_b, 0, c_scale, slack, st, alpha, pm_b);
      if (tail) qk_mfma(kf, qf, s_a);
      rowsum_mfma<D>(sel, p_a, st.lacc);
      pv_mfma(vf, p_a, st.o);
      tile_exp<false, false>(s_b, c_scale, pm_b, st, p_a, p_unused);
      read_v(ring.vstage(kk), fo, vf);
      ++kk;
#pragma unroll
      for (int kb = 0; kb < kKB; ++kb) s_b[kb] = s_a[kb];
    }
    if (tail) {
      ring.advance(kk);
      const int key0 = ring.tile(kk) * kBc;
      const bool active = ring.exists(kk) && key0 < wave_key_end;
      rescale_o(st, alpha, rescale);
      rowsum_mfma<D>(sel, p_a, st.lacc);
      pv_mfma(vf, p_a, st.o);
      if (active) {
        const int ln = fresh_lane();  // (not `lane`, `my_q`: see fresh_lane)
        const int lim = (CAUSAL ? min(qw0 + (ln & 31), seq - 1) : seq - 1) - key0 - 4 * (ln >> 5);
        float pm_t;
        rescale = tile_max<CAUSAL, true>(s_b, lim, c_scale, slack, st, alpha, pm_t);
        tile_exp<true, false>(s_b, c_scale, pm_t, st, p_a, p_unused);
        read_v(ring.vstage(kk), fo, vf);
        rescale_o(st, alpha, rescale);
        rowsum_mfma<D>(sel, p_a, st.lacc);
        pv_mfma(vf, p_a, st.o);
      }
      ++kk;
    } else {
      rescale_o(st, alpha, rescale);
      rowsum_mfma<D>(sel, p_a, st.lacc);
      pv_mfma(vf, p_a, st.o);
    }
  }

  split_steps(kk);
  float *xchg = merge_halves();
  if (!short_rows) {
    // Every row of a half-0 wave now holds its final (l, r). One fp16
    // rounding of each weight perturbs the output row by about 2^-11 times
    // the root of the squared normalised weights that took it, r / l^2: a row
    // that a few keys carry (beyond its exact P = 1 key) has a large r / l^2.
    // Blocks with such a row run again with split P. Each half-0 wave leaves
    // its verdict in its own (already consumed) exchange slot; after the
    // barrier every wave reads all four.
    if (half == 0) {
      const float l_row = kMfmaRowSum<D> ? st.lacc[0] : st.l + __shfl_xor(st.l, 32);
      const float r_row = st.r + __shfl_xor(st.r, 32);
      const bool peaky = qw0 + (fresh_lane() & 31) < seq &&
                         r_row > kRedoRoundedMassAbove * l_row * l_row;
      const float verdict = __builtin_amdgcn_ballot_w64(peaky) != 0 ? 1.0f : 0.0f;
      if (lane == 0) xchg[0] = verdict;
    }
    __syncthreads();
    bool redo = false;
#pragma unroll
    for (int r = 0; r < kRowWaves; ++r)
      redo = redo || reinterpret_cast<const float *>(lds)[r * (G::kXchg * kWave)] != 0.0f;
    if (redo) {
      __syncthreads();  // every wave has read the verdicts before the LDS is reloaded
      prologue();
      split_steps(0);
      merge_halves();
    }
  }
  if (half == 1) continue;

  if (code != 0) {
    // ---- one chunk of a split item ---------------------------------------------
    // Each row wave publishes its (O, m, l) partial, waits until it is stored
    // and counts itself on the (item, row wave) counter; the second to arrive
    // merges the other chunk's partial into its own (log-sum-exp rule) and
    // writes the rows, then sets the counter back to zero.
    float l_lane = kMfmaRowSum<D> ? st.lacc[0] : st.l;
    float *mine = part + (static_cast<size_t>(2 * split + code - 1) * kRowWaves + rw) *
                             kPartFloats<D>;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) store_coherent(mine + (db * 16 + a) * kWave + lane, st.o[db][a]);
    store_coherent(mine + kPartOFloats<D> + lane, st.m);
    store_coherent(mine + kPartOFloats<D> + kWave + lane, l_lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned *const counter = counters + kRowWaves * split + rw;
    unsigned ticket = 0;
    if (lane == 0)
      ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __shfl(ticket, 0);
    if (ticket == 0) continue;
    const float *other = part + (static_cast<size_t>(2 * split + 2 - code) * kRowWaves + rw) *
                                    kPartFloats<D>;
    float o2[kDB][16];
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int a = 0; a < 16; ++a) o2[db][a] = load_coherent(other + (db * 16 + a) * kWave + lane);
    const float m2 = load_coherent(other + kPartOFloats<D> + lane);
    const float l2 = load_coherent(other + kPartOFloats<D> + kWave + lane);
    // Both products rounded, then added (no fused multiply-add): the sum is
    // the same whichever chunk arrives last, so the result does not depend on
    // the order in which the two units finish.
    const float m_all = fmaxf(st.m, m2);
    const float f1 = fast_exp2(st.m - m_all), f2 = fast_exp2(m2 - m_all);
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int a = 0; a < 16; ++a) st.o[db][a] = st.o[db][a] * f1 + o2[db][a] * f2;
      l_lane = l_lane * f1 + l2 * f2;
    }
    if constexpr (kMfmaRowSum<D>)
      st.lacc[0] = l_lane;
    else
      st.l = l_lane;
    if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- epilogue: O = O^T / l --------------------------------------------------
  // Each lane holds one query row; it writes its row's values to this row
  // wave's staging area, then the wave stores whole rows: lane i of a store
  // instruction takes 16-byte chunk i % kChunksOut of row i / kChunksOut.
  {
    using OutT = typename std::conditional<OUT_F32, float, _Float16>::type;
    constexpr int kRowBytes = G::template kOutRowBytes<OUT_F32>;
    constexpr int kChunksOut = kRowBytes / 16;          // 16-byte chunks per row
    constexpr int kRowsPerStore = kWave / kChunksOut;    // rows per store instruction
    const int lane = fresh_lane();  // shadows the kernel's: see fresh_lane
    const int col = lane & 31;
    const int g = lane >> 5;
    const float l_tot = kMfmaRowSum<D> ? st.lacc[0] : st.l + __shfl_xor(st.l, 32);
    const float inv_l = (l_tot > 0.f) ? 1.0f / l_tot : 0.f;
    char *stage = reinterpret_cast<char *>(lds) + G::kXchgBytes +
                  rw * (kRowsPerWave * kRowBytes);
    const int swz = col & (kChunksOut - 1);
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        // dims [32 db + 8 jj + 4 g, +4)
        if constexpr (OUT_F32) {
          floatx4 r;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = st.o[db][4 * jj + e] * inv_l;
          const int chunk = 8 * db + 2 * jj + g;
          *reinterpret_cast<floatx4 *>(stage + col * kRowBytes + 16 * (chunk ^ swz)) = r;
        } else {
          half4 r;
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = static_cast<_Float16>(st.o[db][4 * jj + e] * inv_l);
          const int chunk = 4 * db + jj;
          *reinterpret_cast<half4 *>(stage + col * kRowBytes + 16 * (chunk ^ swz) + 8 * g) = r;
        }
      }
    }
    // The wave reads back only what it wrote itself: its LDS operations
    // complete in order, so no barrier is needed.
    const int chunk = lane % kChunksOut;
#pragma unroll
    for (int i = 0; i < kRowsPerWave / kRowsPerStore; ++i) {
      const int r = i * kRowsPerStore + lane / kChunksOut;
      const floatx4 val =
          *reinterpret_cast<const floatx4 *>(stage + r * kRowBytes + 16 * (chunk ^ (r & (kChunksOut - 1))));
      // Non-temporal: the rows are never read back here, and a normal store
      // would take L2 lines from the K/V tiles that the head's other items
      // re-read (C3 48.2 -> 47.7 us, C2 full 28.6 -> 28.1, 21 interleaved
      // rounds on one box).
      if (qw0 + r < seq)
        __builtin_nontemporal_store(
            val, reinterpret_cast<floatx4 *>(
                     reinterpret_cast<char *>(static_cast<OutT *>(o) + head_off +
                                              static_cast<size_t>(qw0 + r) * D) +
                     16 * chunk));
    }
  }
  }  // items
}

// ---- host: the unit plan --------------------------------------------------------
// Cost of a unit in pipeline steps: its tiles over the two halves, plus what
// every unit pays once (Q and the first tiles in flight, the half merge, the
// epilogue), plus the partial store and merge of a chunk.
constexpr int kUnitOverheadSteps = 3;
constexpr int kChunkOverheadSteps = 1;
constexpr int kMinSplitTiles = 8;  // items with fewer tiles stay whole

struct PlanShape {
  int bh, n_qtiles, seq, causal, kbc, group, cu;
  bool operator<(const PlanShape &o) const {
    return std::tie(bh, n_qtiles, seq, causal, kbc, group, cu) <
           std::tie(o.bh, o.n_qtiles, o.seq, o.causal, o.kbc, o.group, o.cu);
  }
};
struct PlanEntry {
  PrefillPlan plan;
  int n_splits;
};

int item_tiles(const PlanShape &s, int pos) {
  const int qtile = s.n_qtiles - 1 - pos / s.bh;
  const int key_end = s.causal ? std::min(s.seq, qtile * kBr + kBr) : s.seq;
  return (key_end + s.kbc - 1) / s.kbc;
}

struct PlanUnit {
  int cost;
  unsigned code;
};

// Units of the plan that splits the n_split heaviest items, heaviest unit
// first. Items are numbered heaviest query tile first; the split ones are
// the first n_split in (query tile, head) order, so whether an item is split
// depends on its head and query tile only, not on the block placement (a
// grouped-query call splits the same items as one on repeated K/V heads).
void plan_units(const PlanShape &s, int n_split, std::vector<PlanUnit> &units) {
  units.clear();
  const int n_items = s.bh * s.n_qtiles;
  for (int pos = 0; pos < n_items; ++pos) {
    const int nt = item_tiles(s, pos);
    int head = home_head(pos, s.bh);
    if (s.group > 1) head = grouped_head(head, s.bh);
    const int rank = (pos / s.bh) * s.bh + head;  // (query tile, head) order
    if (rank < n_split) {
      const int mid = split_mid(nt);
      const unsigned base = static_cast<unsigned>(pos) | (static_cast<unsigned>(rank) << 22);
      units.push_back({(mid + 1) / 2 + kUnitOverheadSteps + kChunkOverheadSteps, base | (1u << 20)});
      units.push_back(
          {(nt - mid + 1) / 2 + kUnitOverheadSteps + kChunkOverheadSteps, base | (2u << 20)});
    } else {
      units.push_back({(nt + 1) / 2 + kUnitOverheadSteps, static_cast<unsigned>(pos)});
    }
  }
  std::stable_sort(units.begin(), units.end(),
                   [](const PlanUnit &a, const PlanUnit &b) { return a.cost > b.cost; });
}

// Unit costs of the plan that splits the first n_split items in (query tile,
// head) order, as a histogram (cnt[c] units of cost c); returns the unit count.
// All heads of a query tile have the same tiles, so this is per tile level.
int plan_costs(const PlanShape &s, int n_split, std::vector<int> &cnt) {
  std::fill(cnt.begin(), cnt.end(), 0);
  int n = 0;
  for (int level = 0; level < s.n_qtiles; ++level) {
    const int nt = item_tiles(s, level * s.bh);
    const int split = std::min(s.bh, std::max(0, n_split - level * s.bh));
    const int mid = split_mid(nt);
    const int whole = (nt + 1) / 2 + kUnitOverheadSteps;
    const int first = (mid + 1) / 2 + kUnitOverheadSteps + kChunkOverheadSteps;
    const int second = (nt - mid + 1) / 2 + kUnitOverheadSteps + kChunkOverheadSteps;
    cnt[whole] += s.bh - split;
    cnt[first] += split;
    cnt[second] += split;
    n += s.bh + split;
  }
  return n;
}

// Longest unit time of any block when the `g` blocks take the n units
// heaviest first: the 2 g - n heaviest alone, the others paired heaviest with
// lightest (from the cost histogram, which it consumes).
int plan_makespan(std::vector<int> &cnt, int n, int g) {
  int singles = std::max(0, 2 * g - n);
  int hi = static_cast<int>(cnt.size()) - 1, lo = 0, span = 0;
  while (hi >= 0 && singles > 0) {  // the heaviest units, alone
    if (cnt[hi] == 0) {
      --hi;
      continue;
    }
    span = std::max(span, hi);
    const int take = std::min(cnt[hi], singles);
    cnt[hi] -= take;
    singles -= take;
  }
  for (;;) {  // the rest, heaviest with lightest
    while (hi >= 0 && cnt[hi] == 0) --hi;
    while (lo < static_cast<int>(cnt.size()) && cnt[lo] == 0) ++lo;
    if (hi < 0 || lo > hi) break;
    if (lo == hi) {
      span = std::max(span, cnt[hi] >= 2 ? 2 * hi : hi);
      break;
    }
    span = std::max(span, hi + lo);
    const int take = std::min(cnt[hi], cnt[lo]);
    cnt[hi] -= take;
    cnt[lo] -= take;
  }
  return span;
}

// The plan for one shape: the number of split items that minimises the
// makespan (from the cost histograms, O(levels + max cost) per candidate), or
// no plan when splitting does not shorten it.
PlanEntry make_plan(const PlanShape &s) {
  PlanEntry e{};
  e.plan.n_blocks = 0;
  e.n_splits = 0;
  const long long n_items = static_cast<long long>(s.bh) * s.n_qtiles;
  const int g = s.cu;
  if (g > 0 && g <= kPlanMaxBlocks && n_items <= 2LL * g) {
    std::vector<int> cnt((item_tiles(s, 0) + 1) / 2 + kUnitOverheadSteps + kChunkOverheadSteps + 1);
    int n = plan_costs(s, 0, cnt);
    int best_span = plan_makespan(cnt, n, g), best_k = 0;
    const int k_max = static_cast<int>(std::min<long long>(n_items, 2LL * g - n_items));
    for (int kk = 1; kk <= k_max && item_tiles(s, kk - 1) >= kMinSplitTiles; ++kk) {
      n = plan_costs(s, kk, cnt);
      const int span = plan_makespan(cnt, n, g);
      if (span < best_span) {
        best_span = span;
        best_k = kk;
      }
    }
    if (best_k > 0 && static_cast<size_t>(kRowWaves) * best_k <= kMergeCountersPerSlot) {
      std::vector<PlanUnit> units;
      plan_units(s, best_k, units);
      const int n = static_cast<int>(units.size());
      const int singles = std::max(0, 2 * g - n);
      e.plan.n_blocks = g;
      e.n_splits = best_k;
      for (int b = 0; b < g; ++b) e.plan.unit[2 * b] = e.plan.unit[2 * b + 1] = kNoUnit;
      // Blocks go to the 8 XCDs round-robin (block b on XCD b % 8), and the
      // head of item pos is placed (home_head) for XCD pos % 8. A block is
      // taken on its heavier unit's XCD while one is free there; its lighter
      // unit is, among the remaining units of the cost the pairing asks for,
      // one of that XCD when there is one. So most units of a head share an
      // L2, as on the formula path.
      const auto xcd_of = [](unsigned code) { return static_cast<int>(code & 0xfffffu) % 8; };
      std::vector<int> free_b[8];
      for (int b = g - 1; b >= 0; --b) free_b[b % 8].push_back(b);
      const auto take_block = [&](int x) {
        for (int d = 0; d < 8; ++d) {
          std::vector<int> &f = free_b[(x + d) % 8];
          if (!f.empty()) {
            const int b = f.back();
            f.pop_back();
            return b;
          }
        }
        return -1;  // unreachable: at most g blocks are taken
      };
      for (int i = 0; i < singles && i < n; ++i) e.plan.unit[2 * take_block(xcd_of(units[i].code))] = units[i].code;
      const int n_pairs = (n - std::min(singles, n)) / 2;
      std::map<int, std::vector<unsigned>> light[8];  // cost -> codes, per XCD
      for (int j = n - n_pairs; j < n; ++j) light[xcd_of(units[j].code)][units[j].cost].push_back(units[j].code);
      for (int k = 0; k < n_pairs; ++k) {
        const unsigned heavy = units[singles + k].code;
        const int x = xcd_of(heavy);
        const int cost = units[n - 1 - k].cost;  // the k-th lightest unit's cost
        unsigned lite = kNoUnit;
        for (int d = 0; d < 8 && lite == kNoUnit; ++d) {
          auto it = light[(x + d) % 8].find(cost);
          if (it != light[(x + d) % 8].end() && !it->second.empty()) {
            lite = it->second.back();
            it->second.pop_back();
          }
        }
        const int b = take_block(x);
        e.plan.unit[2 * b] = heavy;
        e.plan.unit[2 * b + 1] = lite;
      }
    }
  }
  return e;
}

// Plans are kept per shape (a few KiB each); the cache starts over when it
// holds kPlanCacheShapes of them, so a caller cycling through many shapes
// neither grows it without bound nor pays more than one plan per shape and
// round.
constexpr size_t kPlanCacheShapes = 256;
PlanEntry prefill_plan(const PlanShape &s) {
  static std::mutex mu;
  static std::map<PlanShape, PlanEntry> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(s);
  if (it != cache.end()) return it->second;
  if (cache.size() >= kPlanCacheShapes) cache.clear();
  return cache.emplace(s, make_plan(s)).first->second;
}

template <int D>
size_t plan_workspace_bytes(const PlanEntry &e) {
  return static_cast<size_t>(e.n_splits) * 2 * kRowWaves * kPartFloats<D> * sizeof(float);
}

int current_cu_count() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess ? device_cu_count(dev) : 0;
}

template <int D, bool CAUSAL, bool OUT_F32>
void launch_one(const void *q, const void *k, const void *v, void *o, int bh,
                int seq, int group, float c_scale, bool negate_q, bool split_all,
                void *workspace, size_t workspace_bytes, hipStream_t stream) {
  const int n_qtiles = (seq + kBr - 1) / kBr;
  const long long items = static_cast<long long>(bh) * n_qtiles;
  const int cu = current_cu_count();
  // With a plan (and its workspace and counters): one block per CU. Otherwise
  // a block takes a whole CU's LDS and up to two items: one block per CU, or
  // half the items when there are more than two per CU; without a CU count,
  // one block per item.
  const PlanEntry e = prefill_plan({bh, n_qtiles, seq, CAUSAL ? 1 : 0, Geo<D>::kBc, group, cu});
  unsigned *counters = nullptr;
  const PrefillPlan *plan = nullptr;
  static const PrefillPlan no_plan{0, {}};
  if (e.plan.n_blocks > 0 && workspace != nullptr && workspace_bytes >= plan_workspace_bytes<D>(e))
    counters = merge_counters(stream, static_cast<size_t>(kRowWaves) * e.n_splits);
  if (counters != nullptr) plan = &e.plan;
  const unsigned blocks = static_cast<unsigned>(
      plan != nullptr ? plan->n_blocks
      : cu > 0        ? std::min<long long>(items, std::max<long long>(cu, (items + 1) / 2))
                      : items);
  hipLaunchKernelGGL((prefill_kernel<D, CAUSAL, OUT_F32>), dim3(blocks),
                     dim3(kThreads), 0, stream,
                     static_cast<const _Float16 *>(q),
                     static_cast<const _Float16 *>(k),
                     static_cast<const _Float16 *>(v), o, seq, n_qtiles, bh, group,
                     c_scale, negate_q, split_all, plan != nullptr ? *plan : no_plan,
                     static_cast<float *>(workspace), counters);
}

}  // namespace

// launch_d<D> and prefill_occupancy_d<D> are instantiated by the build of
// head size D only; the head_dim 64 build declares the head_dim 128 ones.
template <int D>
void launch_d(const void *q, const void *k, const void *v, void *o, bool out_f32, int bh,
              int seq, int group, bool causal, float c_scale, bool negate_q, bool split_all,
              void *ws, size_t ws_bytes, hipStream_t stream) {
  if (causal) {
    if (out_f32)
      launch_one<D, true, true>(q, k, v, o, bh, seq, group, c_scale, negate_q, split_all, ws,
                                ws_bytes, stream);
    else
      launch_one<D, true, false>(q, k, v, o, bh, seq, group, c_scale, negate_q, split_all, ws,
                                 ws_bytes, stream);
  } else {
    if (out_f32)
      launch_one<D, false, true>(q, k, v, o, bh, seq, group, c_scale, negate_q, split_all, ws,
                                 ws_bytes, stream);
    else
      launch_one<D, false, false>(q, k, v, o, bh, seq, group, c_scale, negate_q, split_all, ws,
                                  ws_bytes, stream);
  }
}

template <int D>
int prefill_occupancy_d(fa_occupancy_entry *out, int cap, int *n) {
  struct K { const char *name; const void *fn; };
  const K ks[] = {
      {D == 64 ? "prefill_kernel<causal=true>" : "prefill_kernel<causal=true, head_dim=128>",
       reinterpret_cast<const void *>(prefill_kernel<D, true, false>)},
      {D == 64 ? "prefill_kernel<causal=false>" : "prefill_kernel<causal=false, head_dim=128>",
       reinterpret_cast<const void *>(prefill_kernel<D, false, false>)},
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

template void launch_d<FA_PREFILL_D>(const void *, const void *, const void *, void *, bool, int,
                                     int, int, bool, float, bool, bool, void *, size_t,
                                     hipStream_t);
template int prefill_occupancy_d<FA_PREFILL_D>(fa_occupancy_entry *, int, int *);

#if FA_PREFILL_D == 64
extern template void launch_d<128>(const void *, const void *, const void *, void *, bool, int,
                                   int, int, bool, float, bool, bool, void *, size_t,
                                   hipStream_t);
extern template int prefill_occupancy_d<128>(fa_occupancy_entry *, int, int *);

size_t prefill_workspace_bytes(int batch, int heads, int seq, bool causal) {
  if (batch <= 0 || heads <= 0 || seq <= 0) return 0;
  const int bh = batch * heads;
  const int n_qtiles = (seq + kBr - 1) / kBr;
  const int cu = current_cu_count();
  const int c = causal ? 1 : 0;
  // The number of split items depends on the shape only (not on the K/V
  // grouping, which only permutes the heads among the blocks).
  return std::max(
      plan_workspace_bytes<64>(prefill_plan({bh, n_qtiles, seq, c, Geo<64>::kBc, 1, cu})),
      plan_workspace_bytes<128>(prefill_plan({bh, n_qtiles, seq, c, Geo<128>::kBc, 1, cu})));
}

int launch_prefill(const void *q, const void *k, const void *v, void *o,
                   bool out_f32, int batch, int heads, int kv_heads, int seq,
                   int head_dim, bool causal, float scale, void *workspace,
                   size_t workspace_bytes, hipStream_t stream) {
  const int bh = batch * heads;
  const int group = heads / kv_heads;
  const float c_scale = fabsf(scale) * kLog2e;
  const bool negate_q = scale < 0.f;
  // A scale well above 1/sqrt(D) makes rows peaky at any length (one fp16
  // rounding of P costs up to ~5e-4 at D = 128, scale 0.3): the single-
  // rounding pass would be redone for nearly every block, so every row takes
  // the split-P step from the start. Wide inputs at a standard scale are
  // caught per block by the rounded-mass check in the kernel.
  const bool split_all = fabsf(scale) * sqrtf(static_cast<float>(head_dim)) > kSplitAllWidth;
  if (head_dim == 128)
    launch_d<128>(q, k, v, o, out_f32, bh, seq, group, causal, c_scale, negate_q, split_all,
                  workspace, workspace_bytes, stream);
  else
    launch_d<64>(q, k, v, o, out_f32, bh, seq, group, causal, c_scale, negate_q, split_all,
                 workspace, workspace_bytes, stream);
  return check_hip(hipGetLastError(), "prefill_kernel launch");
}

int prefill_occupancy(fa_occupancy_entry *out, int cap, int *n) {
  const int rc = prefill_occupancy_d<64>(out, cap, n);
  return rc != FA_OK ? rc : prefill_occupancy_d<128>(out, cap, n);
}

int prefill_plan_units(int bh, int seq, int causal, int head_dim, int group, int cu,
                       unsigned *units, int cap, int *n_blocks, int *n_splits) {
  if (bh <= 0 || seq <= 0 || group <= 0 || (head_dim != 64 && head_dim != 128) || cu < 0 ||
      cap < 0 || (cap > 0 && units == nullptr) || n_blocks == nullptr || n_splits == nullptr)
    return set_error(FA_ERR_INVALID_ARGUMENT, "invalid prefill plan query");
  const int n_qtiles = (seq + kBr - 1) / kBr;
  const PlanEntry e = prefill_plan(
      {bh, n_qtiles, seq, causal ? 1 : 0, head_dim == 64 ? Geo<64>::kBc : Geo<128>::kBc, group, cu});
  *n_blocks = e.plan.n_blocks;
  *n_splits = e.n_splits;
  for (int i = 0; i < std::min(cap, 2 * e.plan.n_blocks); ++i) units[i] = e.plan.unit[i];
  return FA_OK;
}
#endif  // FA_PREFILL_D == 64

}  // namespace fa
