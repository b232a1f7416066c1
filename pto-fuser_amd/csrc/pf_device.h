// Device-side building blocks for the gfx950 (CDNA4) delta-rule kernels.
//
// Everything here is written for 64-wide wavefronts and the 16x16 MFMA tiles of CDNA4:
//   bf16:  v_mfma_f32_16x16x32_bf16   (8 bf16 of A and of B per lane, fp32 accumulate)
//   fp32:  v_mfma_f32_16x16x4_f32     (1 fp32 of A and of B per lane)
//
// Lane layout of one 16x16xK MFMA (lane l, group g = l / 16, column c = l % 16):
//   A operand:  A[row = c][k in the lane's K slice]
//   B operand:  B[k in the lane's K slice][col = c]
//   D result :  D[row = 4*g + i][col = c], i = 0..3 (a floatx4 per lane)
//
// "Permuted K".  A contraction does not care in which order its K indices are visited, as long
// as A and B agree.  We choose, per 16-row D block, the K order in which lane group g consumes
// exactly the four rows 4g..4g+3 that it already holds in its D registers.  Then the output
// of one MFMA chain (a [16R x 16] D tile) is directly the B operand of the next product that
// contracts over those R*16 rows — no LDS round trip, no cross-lane shuffle.  The matching A
// operand reads, for lane (row c, group g), the columns {4g..4g+3} of each 16-column block,
// i.e. short contiguous runs of the row-major A source.
//   bf16 (K = 32 per instruction): a K-block of 32 rows = D blocks (2kb, 2kb+1); lane group g
//        supplies rows {32kb + 4g + 0..3} and {32kb + 16 + 4g + 0..3}.
//   fp32 (K = 4 per instruction): a K-block of 16 rows = D block kb, consumed by 4 MFMAs; MFMA
//        i takes row 16kb + 4g + i from lane group g.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pf {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));   // one 16-byte vector

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }

template <typename E> __device__ __forceinline__ E from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// Workgroup barrier that orders LDS traffic only.  __syncthreads() is a workgroup memory fence:
// it waits for every outstanding global load and store of the wave (vmcnt(0)) before the
// barrier, which turns register prefetches into synchronous HBM round trips.  Here the wave waits
// only for its own LDS operations (lgkmcnt(0); vmcnt and expcnt left at their maxima), so loads
// and stores to global memory stay in flight across the barrier.  Valid because no wave of these
// kernels reads global data that another wave of the same workgroup writes.
__device__ __forceinline__ void lds_barrier() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // gfx9 encoding: vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

// Index of the lower-triangular 16x16 tile (ib, jb), jb <= ib, of a 64 x 64 chunk matrix (T, the
// score) in a packed list of its ten tiles.
__device__ __forceinline__ constexpr int score_tile_index(int ib, int jb) { return ib * (ib + 1) / 2 + jb; }

// exp(x) for x <= 0, 0 for x > 0 (the reference's _safe_exp).
__device__ __forceinline__ float safe_exp(float x) { return x <= 0.f ? __expf(x) : 0.f; }

// --------------------------------------------------------------------------------------------
//  Swizzled LDS tiles.  A tile is row-major with `pitch` elements per row; its 4-element column
//  groups are XOR-permuted by row bits, group' = group ^ ((row >> RS) & RM), so that the MFMA
//  operand reads (16 rows x one group) and the transposed staging writes (rows 8 apart) spread
//  over all banks.  RM = 0 is the plain layout.  With RM = 1 a 16-byte vector (two bf16 groups)
//  stays in place and only its two 8-byte halves swap.
// --------------------------------------------------------------------------------------------
template <int RS, int RM>
struct Swz {
  static constexpr int rs = RS, rm = RM;
  __device__ __forceinline__ static int off(int row, int col, int pitch) {
    return row * pitch + ((((col >> 2) ^ ((row >> RS) & RM)) << 2) | (col & 3));
  }
  // element offset of the 4-element group holding column `col` (col % 4 == 0)
  __device__ __forceinline__ static int grp(int row, int col, int pitch) {
    return row * pitch + (((col >> 2) ^ ((row >> RS) & RM)) << 2);
  }
};

// --------------------------------------------------------------------------------------------
//  MFMA traits.  KB = contraction rows consumed per "K-block" step.
// --------------------------------------------------------------------------------------------
template <typename E> struct Mfma;

template <> struct Mfma<bf16> {
  static constexpr int KB = 32;
  // acc += A x B, A = row `row` of a swizzled tile (K-block kb, permuted K order), B = the two
  // D blocks (2kb, 2kb+1) of a register tile.
  template <class SW>
  __device__ __forceinline__ static floatx4 perm_b(floatx4 acc, const bf16* tile, int row, int pitch,
                                                   int kb, int g, const floatx4& d0,
                                                   const floatx4& d1) {
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(tile + SW::grp(row, kb * 32 + 4 * g, pitch));
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(tile + SW::grp(row, kb * 32 + 16 + 4 * g, pitch));
    bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    bf16x8 b = {(bf16)d0[0], (bf16)d0[1], (bf16)d0[2], (bf16)d0[3],
                (bf16)d1[0], (bf16)d1[1], (bf16)d1[2], (bf16)d1[3]};
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  // acc += A x B^T with both operands read as rows from memory (natural K order).
  // arow = row (lane c) of A, brow = row (lane c) of B, K-block kb.
  __device__ __forceinline__ static floatx4 rows(floatx4 acc, const bf16* arow, const bf16* brow,
                                                 int kb, int g) {
    bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + kb * 32 + 8 * g);
    bf16x8 b = *reinterpret_cast<const bf16x8*>(brow + kb * 32 + 8 * g);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int KB = 16;
  template <class SW>
  __device__ __forceinline__ static floatx4 perm_b(floatx4 acc, const float* tile, int row, int pitch,
                                                   int kb, int g, const floatx4& d0,
                                                   const floatx4& /*unused*/) {
    floatx4 a = *reinterpret_cast<const floatx4*>(tile + SW::grp(row, kb * 16 + 4 * g, pitch));
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], d0[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], d0[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], d0[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], d0[3], acc, 0, 0, 0);
    return acc;
  }
  __device__ __forceinline__ static floatx4 rows(floatx4 acc, const float* arow, const float* brow,
                                                 int kb, int g) {
    floatx4 a = *reinterpret_cast<const floatx4*>(arow + kb * 16 + 4 * g);
    floatx4 b = *reinterpret_cast<const floatx4*>(brow + kb * 16 + 4 * g);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc, 0, 0, 0);
    return acc;
  }
};

// Chain helper: acc += A[row, 0 : NKB*KB] x D, where A is row `row` of a swizzled LDS tile and D
// is a register tile of NKB*KB/16 D blocks (16 rows each) consumed in the permuted-K order.
// Only the first `kb_end` K-blocks are visited (a triangular A skips its zero blocks); NKB keeps
// every register index static.
template <typename E, int NKB, class SW>
__device__ __forceinline__ floatx4 chain(floatx4 acc, const E* tile, int row, int pitch,
                                         const floatx4* d, int kb_end, int g) {
  constexpr int per = Mfma<E>::KB / 16;  // D blocks per K-block (2 for bf16, 1 for fp32)
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    if (kb < kb_end)
      acc = Mfma<E>::template perm_b<SW>(acc, tile, row, pitch, kb, g, d[kb * per], d[kb * per + (per - 1)]);
  }
  return acc;
}

// Store four consecutive values as one vector (8 bytes of bf16 or 16 bytes of fp32).
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)a, (bf16)b, (bf16)c, (bf16)d};
}
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<floatx4*>(p) = floatx4{a, b, c, d};
}

// Four consecutive elements as fp32.
__device__ __forceinline__ floatx4 load4f(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ floatx4 load4f(const float* p) { return *reinterpret_cast<const floatx4*>(p); }

// 16-byte vector type of an element type (8 bf16 or 4 fp32).
template <typename E> struct Vec16;
template <> struct Vec16<bf16> { typedef uint4 T; static constexpr int N = 8; };
template <> struct Vec16<float> { typedef uint4 T; static constexpr int N = 4; };

}  // namespace pf
