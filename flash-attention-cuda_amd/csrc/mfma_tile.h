// MFMA tile building blocks shared by the gfx950 attention kernels
// (prefill.hip, decode.hip): the 16-byte-chunk swizzles of a row-major
// [rows x 64] or [rows x 128] fp16 tile in LDS, direct global->LDS loads, the
// fragment offsets of v_mfma_f32_32x32x16_f16 operands read from such a tile,
// and the lane-pair max of an S^T accumulator.
//
// Operand conventions (lane l: column l % 32, half g = l / 32):
//   S^T = K Q^T : A = 32 key rows x 16 head dims, B = 16 head dims x 32
//                 queries; the 64 head dims are grouped [32 g + 8 s, +8) for
//                 k-step s, so every fragment is one 16-byte chunk of a row.
//   O^T += V^T P^T : A = V^T read from a row-major V tile with
//                 ds_read_b64_tr_b16; B = P^T taken from the S^T
//                 accumulators in their own key order.
// Accumulator element a of a 32 x 32 tile sits at row 8 (a / 4) + 4 g + a % 4
// of column l % 32.
#pragma once

#include "fa_internal.h"

namespace fa {
namespace {

typedef short short4v __attribute__((ext_vector_type(4)));

// Chunk swizzles (16-byte chunk index within a 128-byte row).
//  K, Q: a ds_read_b128 phase reads the same logical chunk of 8 (32 banks) or
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
// m0 is listed as clobbered for the reader; the compiler treats m0 as a
// reserved register and does not track it (hence the silenced warning), which
// is safe only while nothing else in the kernels defines or reads m0:
// tests/test_build_checks.py builds the gfx950 assembly of prefill.hip and
// decode.hip and fails on any other m0 use (build.py m0_problems).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
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
// The same load with the non-temporal hint, for data read exactly once per
// call (the decode's cache rows): it bypasses the normal cache-allocation
// policy, as the VALU decode's nontemporal register loads do.
__device__ __forceinline__ void global_to_lds16_nt(const void *src, const void *lds_dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(lds_dst))));
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off nt"
      :
      : "v"(src), "s"(m0)
      : "memory", "m0");
}
// The same load with a wave-uniform 64-bit base in SGPRs and a per-lane
// 32-bit byte offset (the saddr form): no per-lane address arithmetic.
__device__ __forceinline__ void global_to_lds16_sbase(const void *base, unsigned voff,
                                                      const void *lds_dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(lds_dst))));
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "s"(m0)
      : "memory", "m0");
}
// The same two loads with the LDS destination given as a byte address (a
// wave-uniform value kept from lds_addr): no generic-to-LDS pointer cast, and
// so no null check, per load.
__device__ __forceinline__ void global_to_lds16_at(const void *src, unsigned lds_dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(lds_dst);
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "s"(m0)
      : "memory", "m0");
}
__device__ __forceinline__ void global_to_lds16_sbase_at(const void *base, unsigned voff,
                                                         unsigned lds_dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(lds_dst);
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "s"(m0)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a pointer into a __shared__ array. The generic-to-LDS
// cast carries a null check; callers take it once and do their address
// arithmetic on the integer.
__device__ __forceinline__ unsigned lds_addr(const void *p) {
  return static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(p)));
}

// Wait until at most N of this thread's global->LDS loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_loads() {
  if constexpr (N == 0)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ floatx16 mfma(const half8 &a, const half8 &b,
                                         const floatx16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Row sums of P^T fragments on the matrix cores.
// v_mfma_f32_16x16x32_f16 (lane l: A[l % 16][8 (l / 16) + i],
// B[8 (l / 16) + i][l % 16], result rows 4 (l / 16) + j of column l % 16)
// reads a 32x32x16 B fragment (lane l: query l % 32, keys 8 (l / 32) + i of
// a 16-key step) as B[k][n] with k-group l / 16 and column l % 16: k-groups
// 0 and 2 hold query n, k-groups 1 and 3 query n + 16. A selector with ones
// in rows {0, 8} over k-groups {0, 2} and in rows {4, 12} over k-groups
// {1, 3} therefore puts the 16-key sum of query l % 32 into result element 0
// of lane l, for all 64 lanes (rows 0, 4, 8, 12 are element 0 of lane groups
// 0-3); elements 1-3 stay zero.
__device__ __forceinline__ floatx4 mfma16(const half8 &a, const half8 &b, const floatx4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half8 rowsum_selector(int lane) {
  const int m = lane & 15;
  const bool odd_group = (lane >> 4) & 1;
  const bool on = odd_group ? (m == 4 || m == 12) : (m == 0 || m == 8);
  const _Float16 one = static_cast<_Float16>(on ? 1.0f : 0.0f);
  half8 s;
#pragma unroll
  for (int i = 0; i < 8; ++i) s[i] = one;
  return s;
}

// Per-lane LDS offsets (in halves, relative to a tile) of every fragment a
// wave reads from a tile; loop invariant.
struct FragOffsets {
  int k[4];  // K (and Q) fragment for d-step s (32-key block 0; block 1 is +32 rows)
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
    f.v[db] = tr_row * kHeadDim + (((d >> 3) ^ v_swz(tr_row)) << 3) + (d & 7);
  }
  return f;
}

// The same building blocks for tiles of D-dim rows, D in {64, 128}. D = 64 is
// exactly the layout above. D = 128 rows are 256 B (16 chunks), so a row
// no longer shifts the bank group of a chunk and the swizzles change:
//  K, Q: a ds_read_b128 phase reads one logical chunk of 8 or 16
//     consecutive rows; chunk c of row r goes to position c ^ (r & 15),
//     16 distinct positions for any 16 consecutive rows.
//  V: a 32-lane transpose-read phase reads chunks {4 db, .., 4 db + 3} of 4
//     consecutive rows; c ^ 4 (r & 3) maps those 16 (row, chunk) pairs to 16
//     distinct positions.
// Fragment order for Q/K: k-step s, lane half g holds chunk (D / 16) g + s
// (head dims [(D / 2) g + 8 s, +8)); A and B use the same order.
template <int D>
__device__ __forceinline__ int k_swz_d(int row) {
  if constexpr (D == 64) return k_swz(row);
  else return row & 15;
}
template <int D>
__device__ __forceinline__ int v_swz_d(int row) {
  if constexpr (D == 64) return v_swz(row);
  else return (row & 3) << 2;
}

template <int D>
struct FragOffsetsD {
  int k[D / 16];  // K (and Q) fragment for d-step s (key block 0; block 1 is +32 rows)
  int v[D / 32];  // V^T transpose-read base for d-block db
};

template <int D>
__device__ __forceinline__ FragOffsetsD<D> frag_offsets_d(int lane) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  FragOffsetsD<D> f;
  const int col = lane & 31;
  const int g = lane >> 5;
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    f.k[s] = col * D + ((((D / 16) * g + s) ^ k_swz_d<D>(col)) << 3);
  const int tr_row = 4 * g + ((lane & 15) >> 2);
  const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    const int d = db * 32 + tr_dim;
    f.v[db] = tr_row * D + (((d >> 3) ^ v_swz_d<D>(tr_row)) << 3) + (d & 7);
  }
  return f;
}

typedef __attribute__((address_space(3))) const _Float16 lds_half;

// An LDS address the compiler must materialise as one register per step:
// the constant row offsets of the reads below then fold into the
// instructions' offset fields instead of being hoisted out of the loop as
// separate loop-invariant addresses.
__device__ __forceinline__ lds_half *opaque_lds(const _Float16 *p) {
  unsigned a = static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_half *)(p)));
  asm volatile("" : "+v"(a));
  return reinterpret_cast<lds_half *>(static_cast<uintptr_t>(a));
}

// LDS address base + 2 * off_halves, with base a wave-uniform tile address
// kept whole in an SGPR (so no constant part of it is split off into a
// separate vector add) and the sum opaque as in opaque_lds.
__device__ __forceinline__ unsigned uniform_lds_base(const _Float16 *p) {
  unsigned a = __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_half *)(p))));
  asm volatile("" : "+s"(a));
  return a;
}
// uniform_lds_base for a tile already given as an LDS byte address.
__device__ __forceinline__ unsigned uniform_lds_u(unsigned a) {
  a = __builtin_amdgcn_readfirstlane(a);
  asm volatile("" : "+s"(a));
  return a;
}
__device__ __forceinline__ lds_half *opaque_lds_at(unsigned base, int off_halves) {
  unsigned a = base + 2u * static_cast<unsigned>(off_halves);
  asm volatile("" : "+v"(a));
  return reinterpret_cast<lds_half *>(static_cast<uintptr_t>(a));
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


// Partials that another wave of the same launch reads: relaxed agent-scope
// atomic stores and loads, which go to the device-coherent level (sc1) on
// their own, so the only ordering needed is the writer's wait for its stores
// before it counts (no cache-wide release or acquire).
__device__ __forceinline__ void store_coherent(float *p, float x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace
}  // namespace fa
