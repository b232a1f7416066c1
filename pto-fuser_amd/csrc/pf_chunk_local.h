// K1 — the chunk-local stage of the chunked delta-rule forward, one workgroup per chunk.
//
// For chunk m (C tokens, rows m*C .. m*C+C-1 of the flattened [B*H*T, dk] token axis):
//   G     = cumsum_within_chunk(g)                                   (_gdn_full.py:63)
//   A     = strictly_lower( beta_i * safe_exp(G_i - G_j) * (k_i . k_j) )  (_gdn_full.py:73-75)
//   T     = (I + A)^-1                                                 (_gdn_full.py:76-78)
//   P     = p_scale * causal_incl_diag( (q_i . k_j) * exp(min(G_i - G_j, 0)) )
//           (_gdn_full.py:91-95; the output scale of :97 is applied here, once per score element)
//
// Mapping on CDNA4: k and q chunk tiles are staged in LDS (row pitch padded by 16 bytes so the
// MFMA operand reads are bank-conflict free per 16 lanes); the 20 lower-triangular 16x16 score
// blocks (10 of A, 10 of P) are split over the 4 waves in lists that share operand rows, and
// computed with bf16 (or fp32) MFMA; the gate/mask epilogue runs branch free in VALU on the
// accumulator registers.  The fp32 inverse (unit_lower_inverse64): the 16x16 diagonal blocks by
// forward substitution in one wave, then the off-diagonal blocks by block doubling on fp32 MFMA
// (16x16x4), the product chains kept in registers through the permuted-K layout.
#pragma once

#include <type_traits>

#include "pf_device.h"

// Barriers are LDS-only (lds_barrier): waves exchange data through LDS alone, so a barrier need
// not wait for this wave's global stores to be acknowledged (a full __syncthreads would).

namespace pf {

struct ChunkLocalArgs {
  const void* k;        // [M*C, DK]  E
  const void* q;        // [M*C, DK]  E        (needed when P is produced)
  const float* beta;    // [M*C]      fp32
  const float* g;       // [M*C]      fp32 per-token log decay; null => 0 (DeltaNet)
  float* G_out;         // [M*C]      within-chunk cumsum (optional)
  void* T_out;          // [M, C, C]  TO       (optional)
  void* P_out;          // [M, C, C]  E        (optional)
  float* A_out;         // [M, C, C]  fp32     (optional)
  int M;                // number of chunks
  int g_is_cumsum;      // 1: g already holds within-chunk cumulative sums
  int t_lower_only;     // 1: leave T's upper-right quadrant (rows < 32, columns >= 32, all zero)
                        //    unwritten: the fused forward's scan never reads it
  float p_scale;        // multiplies P (the forward's output scale)
  float* scale_out;     // if set, block 0 records p_scale here for the scan stage
  int split_p;          // with P: 1 = grid of 2M blocks, blocks M .. 2M-1 form P of chunk b - M
                        //    alone and blocks 0 .. M-1 the rest (half the products per block,
                        //    for launches whose M blocks would leave most CUs idle)
};

// (I + A)^-1 of one strictly-lower C x C block held in LDS (As, fp32, pitch C+4) into Ts (same
// layout); must be called by all 256 threads of the workgroup.  Diagonal 16x16 blocks by
// lane-parallel forward substitution, then off-diagonal blocks level by level on fp32 MFMA.
template <int C>
__device__ __forceinline__ void block_unit_lower_inverse(const float* As, float* Ts) {
  constexpr int CP = C + 4;
  constexpr int NB = C / 16;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  if (tid < 16 * NB) {
    const int r = tid >> 4, cc = tid & 15;
    const float* Ab = As + (16 * r) * CP + 16 * r;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) s = fmaf(Ab[i * CP + j], t[j], s);
      if (i > cc) t[i] = -s;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Ts[(16 * r + i) * CP + 16 * r + cc] = t[i];
  }
  lds_barrier();
#pragma unroll
  for (int L = 1; L < NB; ++L) {
    for (int j = w; j + L < NB; j += 4) {
      const int i = j + L;
      floatx4 X = zero4();
      for (int kk = j; kk < i; ++kk) {
        const float* arow = As + (16 * i + c) * CP + 16 * kk + 4 * g;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          X = __builtin_amdgcn_mfma_f32_16x16x4f32(arow[ii], Ts[(16 * kk + 4 * g + ii) * CP + 16 * j + c],
                                                   X, 0, 0, 0);
      }
      floatx4 Y = zero4();
      const float* trow = Ts + (16 * i + c) * CP + 16 * i + 4 * g;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) Y = __builtin_amdgcn_mfma_f32_16x16x4f32(trow[ii], X[ii], Y, 0, 0, 0);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) Ts[(16 * i + 4 * g + ii) * CP + 16 * j + c] = -Y[ii];
    }
    lds_barrier();
  }
}

// acc += M1[r1.., c1..] x M2[r2.., c2..] for 16 x 16 blocks of two fp32 LDS matrices with row
// pitch C + 4: four 16x16x4 MFMAs in the permuted-K order (lane (c, g) supplies A row c, columns
// 4g .. 4g+3 as one vector, and B rows 4g .. 4g+3 of column c).
template <int CP>
__device__ __forceinline__ floatx4 mm16(floatx4 acc, const float* M1, int r1, int c1, const float* M2,
                                        int r2, int c2, int c, int g) {
  const floatx4 a = *reinterpret_cast<const floatx4*>(M1 + (r1 + c) * CP + c1 + 4 * g);
#pragma unroll
  for (int ii = 0; ii < 4; ++ii)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ii], M2[(r2 + 4 * g + ii) * CP + c2 + c], acc, 0, 0, 0);
  return acc;
}
// acc += M1[r1.., c1..] x X with X a 16 x 16 register tile in the D layout (X[ii] = row 4g+ii,
// column c), which is the B operand of the permuted-K chain as it stands.
template <int CP>
__device__ __forceinline__ floatx4 mm16r(floatx4 acc, const float* M1, int r1, int c1, const floatx4& X,
                                         int c, int g) {
  const floatx4 a = *reinterpret_cast<const floatx4*>(M1 + (r1 + c) * CP + c1 + 4 * g);
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ii], X[ii], acc, 0, 0, 0);
  return acc;
}
template <int CP>
__device__ __forceinline__ void put16(float* M, int r, int cc, const floatx4& X, float sign, int c, int g) {
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) M[(r + 4 * g + ii) * CP + cc + c] = sign * X[ii];
}

// x of lane p of this lane's quad (DPP quad_perm broadcast; p folds to a constant where the
// caller's loop is unrolled).
template <int P>
__device__ __forceinline__ float quad_broadcast_c(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), P * 0x55, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_broadcast(float x, int p) {
  switch (p) {
    case 0: return quad_broadcast_c<0>(x);
    case 1: return quad_broadcast_c<1>(x);
    case 2: return quad_broadcast_c<2>(x);
    default: return quad_broadcast_c<3>(x);
  }
}

// (I + A)^-1 of one strictly-lower 64 x 64 block (As, fp32, pitch 68) into Ts, by 16-row blocks:
//   1. the four diagonal blocks by right-looking forward substitution, one wave per block, four
//      lanes per column (each holding four rows of it and those rows of A in registers);
//   2. T10 = -T11 A10 T00 and T32 = -T33 A32 T22 (two waves);
//   3. the lower-left 32 x 32 quadrant T_LL = -T_R (A_LL T_L), T_L / T_R the inverted upper-left
//      / lower-right quadrants: the four 16 x 16 tiles of X = A_LL T_L (one per wave) go to the
//      unused strictly-upper quadrant of As, then the four tiles of -T_R X.
// The off-diagonal part is three levels of at most two dependent 16 x 16 products each (a
// block-diagonal sweep would end in a chain of four).  Must be called by all 256 threads.
//
// Ts may equal As (in place): every block of T is written only after the last read of the A
// block at its position — T_ii by the wave that has read all of A_ii, T10 / T32 by the wave
// that just read A10 / A32, and T_LL a barrier after the X products read A_LL — and X lives in
// the strictly-upper quadrant, which neither A nor T occupies.
__device__ __forceinline__ void unit_lower_inverse64(float* As, float* Ts) {
  constexpr int CP = 64 + 4;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  {  // wave w inverts diagonal block w: lane = column cc (of T) x row phase p (rows 4k + p)
    const int r = w, cc = lane >> 2, p = lane & 3;
    const float* Ab = As + (16 * r) * CP + 16 * r;
    // this lane's rows of A_rr, columns 0 .. 4k+3 (A is zero on and above the diagonal)
    floatx4 arow[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int q = 0; q <= k; ++q) arow[k][q] = *reinterpret_cast<const floatx4*>(Ab + (4 * k + p) * CP + 4 * q);
    float s[4];                                        // rows 4k + p of column cc of T_rr
#pragma unroll
    for (int k = 0; k < 4; ++k) s[k] = (4 * k + p == cc) ? 1.f : 0.f;
    // right-looking substitution: once row j of the column is final, subtract its share from
    // every later row; row j comes from lane (cc, j & 3) of the quad (a DPP broadcast), so the
    // dependent chain is one broadcast and one fused multiply-add per row
#pragma unroll
    for (int j = 0; j < 15; ++j) {
      const float tj = quad_broadcast(s[j >> 2], j & 3);
#pragma unroll
      for (int k = j >> 2; k < 4; ++k) s[k] = fmaf(-arow[k][j >> 2][j & 3], tj, s[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) Ts[(16 * r + 4 * k + p) * CP + 16 * r + cc] = s[k];
  }
  lds_barrier();
  if (w < 2) {   // T10 (wave 0), T32 (wave 1)
    const int b = 32 * w;
    const floatx4 X = mm16<CP>(zero4(), As, b + 16, b, Ts, b, b, c, g);
    put16<CP>(Ts, b + 16, b, mm16r<CP>(zero4(), Ts, b + 16, b + 16, X, c, g), -1.f, c, g);
  }
  lds_barrier();
  {  // X = A_LL T_L, tile (xa, xb) by wave 2 xa + xb, into As rows 16 xa, columns 32 + 16 xb
    const int xa = w >> 1, xb = w & 1;
    floatx4 X = mm16<CP>(zero4(), As, 32 + 16 * xa, 16, Ts, 16, 16 * xb, c, g);   // A_(2+xa),1 T_1,xb
    if (xb == 0) X = mm16<CP>(X, As, 32 + 16 * xa, 0, Ts, 0, 0, c, g);           // + A_(2+xa),0 T_00
    put16<CP>(As, 16 * xa, 32 + 16 * xb, X, 1.f, c, g);
  }
  lds_barrier();
  {  // T_(2+ta),tb = -(T_(2+ta),2 X_0,tb + [ta = 1] T_33 X_1,tb)
    const int ta = w >> 1, tb = w & 1;
    floatx4 Y = mm16<CP>(zero4(), Ts, 32 + 16 * ta, 32, As, 0, 32 + 16 * tb, c, g);
    if (ta == 1) Y = mm16<CP>(Y, Ts, 48, 48, As, 16, 32 + 16 * tb, c, g);
    put16<CP>(Ts, 32 + 16 * ta, 16 * tb, Y, -1.f, c, g);
  }
  lds_barrier();
}

// Score blocks of the 64-token chunk (4 x 4 grid of 16-row blocks, lower triangle) owned by one
// wave, encoded 16 qk + 4 i + j: qk = 1 for a block of P (q rows i against k rows j), 0 for a
// block of A (k rows i against k rows j).  The lists group each wave's blocks by shared rows, so
// a wave reads every 16-row operand block it needs once per K step and feeds it to all of its
// MFMAs (with P: 18 operand reads per K step for the workgroup instead of 40):
//   A and P  w0: A row 3 + P(0,0)   w1: P row 3 + A(0,0)   w2: A rows 1-2   w3: P rows 1-2
//   A only   w0: A(3,0..1)   w1: A row 2   w2: A row 1 + A(0,0)   w3: A(3,2..3)
//   P only   w0: P(3,0..2)   w1: P(2,0..2)   w2: P row 1   w3: P(0,0) + P(3,3)
enum ScoreSet : int { kScoreA = 0, kScoreAP = 1, kScoreP = 2 };
__device__ __forceinline__ constexpr int score_count(int set, int w) {
  return set == kScoreAP ? 5 : (set == kScoreA ? ((w == 0 || w == 3) ? 2 : 3) : (w < 2 ? 3 : 2));
}
__device__ __forceinline__ constexpr int score_code(int set, int w, int b) {
  return set == kScoreAP ? (w == 0   ? (b < 4 ? 12 + b : 16)
                            : w == 1 ? (b < 4 ? 16 + 12 + b : 0)
                            : w == 2 ? (b < 2 ? 4 + b : 8 + (b - 2))
                                     : 16 + (b < 2 ? 4 + b : 8 + (b - 2)))
       : set == kScoreA  ? (w == 0   ? 12 + b
                            : w == 1 ? 8 + b
                            : w == 2 ? (b < 2 ? 4 + b : 0)
                                     : 14 + b)
                         : 16 + (w == 0   ? 12 + b
                                 : w == 1 ? 8 + b
                                 : w == 2 ? 4 + b
                                          : (b == 0 ? 0 : 15));
}

// One wave's score blocks: products, then (after the workgroup barrier that frees the k / q
// tiles) the gate / mask epilogue.  Each product is formed transposed —
// D[4g+ii][c] = sum_d k[j][d] x[i][d] with i = 16 bi + c, j = 16 bj + 4g + ii — so a lane holds
// four consecutive columns of one score row and stores them as one vector.
template <typename E, int C, int DK, int KP, int CP, int SET, int W>
__device__ __forceinline__ void score_wave(const ChunkLocalArgs& a, const E* ks, const E* qs,
                                           float* As, const float* Gs, const float* Bs, int m) {
  constexpr int N = score_count(SET, W);
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  floatx4 acc[N];
#pragma unroll
  for (int b = 0; b < N; ++b) acc[b] = zero4();
  // unrolled by two, not fully: with every K step's operand reads hoisted the kernel needs 72
  // VGPRs (seven waves per SIMD); by two it needs 61 and eight workgroups fit a CU
#pragma unroll 2
  for (int kb = 0; kb < DK / Mfma<E>::KB; ++kb) {
#pragma unroll
    for (int b = 0; b < N; ++b) {
      const int code = score_code(SET, W, b);
      const E* jrow = ks + (16 * (code & 3) + c) * KP;
      const E* irow = ((code & 16) ? qs : ks) + (16 * ((code >> 2) & 3) + c) * KP;
      acc[b] = Mfma<E>::rows(acc[b], jrow, irow, kb, g);   // equal rows: one LDS read
    }
  }
  lds_barrier();   // every wave is done reading k / q: A now overwrites them
  // Gate / mask epilogue, branch free: every exponential is evaluated (clamped to <= 0, so it is
  // finite) and the mask multiplies it in as 0 / 1 (a select would be turned back into a branch
  // around the exponential), so no lane-divergent branch splits the wave's instruction stream.
#pragma unroll
  for (int b = 0; b < N; ++b) {
    const int code = score_code(SET, W, b);
    const int i = 16 * ((code >> 2) & 3) + c, j0 = 16 * (code & 3) + 4 * g;
    const float gi = Gs[i];
    const floatx4 gj = *reinterpret_cast<const floatx4*>(Gs + j0);
    floatx4 out;
    if (!(code & 16)) {
      const float bi = Bs[i];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {   // beta_i safe_exp(G_i - G_j), strictly lower
        const float x = gi - gj[ii];
        const float keep = (i > j0 + ii && x <= 0.f) ? 1.f : 0.f;
        out[ii] = keep * bi * __expf(fminf(x, 0.f)) * acc[b][ii];
      }
      *reinterpret_cast<floatx4*>(As + i * CP + j0) = out;
    } else {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const float e = __expf(fminf(gi - gj[ii], 0.f));
        const float keep = (i >= j0 + ii) ? 1.f : 0.f;
        out[ii] = keep * a.p_scale * acc[b][ii] * e;
      }
      store4(static_cast<E*>(a.P_out) + (size_t)m * C * C + i * C + j0, out[0], out[1], out[2], out[3]);
    }
  }
  if (SET != kScoreA && (W == 0 || W == 3)) {
    // the strictly-upper blocks of P that the scan kernels read as parts of a 32-wide K block:
    // (0,1) beside P(0,0) (wave 0) and (2,3) beside P row 2 (wave 3); the other four are never read
    const int i = (W == 0 ? 0 : 32) + c, j0 = (W == 0 ? 16 : 48) + 4 * g;
    store4(static_cast<E*>(a.P_out) + (size_t)m * C * C + i * C + j0, 0.f, 0.f, 0.f, 0.f);
  }
}

// One workgroup per chunk; eight workgroups fit a CU for bf16 without P (at most 64 VGPRs and
// 17.9 KB of LDS each), so the HBM latency of one chunk's loads overlaps the other workgroups'
// products and inverse.  At the headline's 16 chunks per CU that is two generations of workgroups
// instead of three.  The fp32 tiles' LDS allows four workgroups per CU without P, two with it;
// the register target follows, so the compiler does not trade registers for residency the LDS
// cannot give.
template <typename E, bool DO_P>
struct ChunkLocalWaves {
  static constexpr int value = (sizeof(E) == 2 && !DO_P) ? 8 : DO_P ? 2 : 4;
};

template <typename E, typename TO, int C, int DK, bool DO_P, bool DO_INV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ChunkLocalWaves<E, DO_P>::value,
                                                                      ChunkLocalWaves<E, DO_P>::value)))
void chunk_local_kernel(ChunkLocalArgs a) {
  static_assert(C == 64, "the chunk-local kernel is written for 64-token chunks");
  static_assert(DK % Mfma<E>::KB == 0, "head dim must be a multiple of the MFMA K block");
  constexpr int PE = 16 / sizeof(E);
  constexpr int KP = DK + PE;   // LDS row pitch of k / q (elements)
  constexpr int CP = C + 4;     // LDS row pitch of A / T (floats)
  constexpr int VE = Vec16<E>::N;
  constexpr int NV = C * (DK / VE);                 // 16-byte vectors per k (or q) chunk tile
  constexpr int NVT = NV / 256;                     // per thread
  static_assert(NV % 256 == 0, "k/q chunk tile must divide over 256 threads");
  constexpr int KQ_BYTES = (DO_P ? 2 : 1) * C * KP * (int)sizeof(E);
  constexpr int AT_BYTES = C * CP * 4;   // A, then T in its place
  // A is written only after the last score read of k/q (a barrier apart), so it reuses the k/q
  // tiles' LDS, and the inverse runs in place: 17.9 KB per workgroup for bf16 without P, eight
  // workgroups per CU.
  constexpr int KQT_BYTES = KQ_BYTES > AT_BYTES ? KQ_BYTES : AT_BYTES;

  __shared__ __attribute__((aligned(16))) char kqt[KQT_BYTES];
  __shared__ __attribute__((aligned(16))) float Gs[C];
  __shared__ float Bs[C];
  E* ks = reinterpret_cast<E*>(kqt);
  E* qs = ks + C * KP;
  float* As = reinterpret_cast<float*>(kqt);
  float* Ts = As;

  // block role (block-uniform): P alone (split launch, second half of the grid), A, T and P in
  // one block (DO_P, no split), or A and T (no P, or the first half of a split launch)
  const bool p_only = DO_P && a.split_p && (int)blockIdx.x >= a.M;
  const bool stage_q = DO_P && (p_only || !a.split_p);
  const int m = p_only ? (int)blockIdx.x - a.M : (int)blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar branches
  const size_t row0 = (size_t)m * C;
  if (a.scale_out && !p_only && m == 0 && tid == 0) *a.scale_out = a.p_scale;

  // ---- 1. stage k (and q), gates: every load issued before the first LDS store ----------------
  {
    const u32x4* kg = reinterpret_cast<const u32x4*>(static_cast<const E*>(a.k) + row0 * DK);
    const u32x4* qg = reinterpret_cast<const u32x4*>(static_cast<const E*>(a.q) + row0 * DK);
    u32x4 kr[NVT], qr[NVT];   // native vectors (a uint4 struct copy would go through scratch)
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      kr[i] = kg[tid + 256 * i];
      qr[i] = stage_q ? qg[tid + 256 * i] : u32x4{0u, 0u, 0u, 0u};
    }
    const float x = a.g != nullptr ? a.g[row0 + (tid & (C - 1))] : 0.f;
    const float bv = a.beta[row0 + (tid & (C - 1))];
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      const int u = tid + 256 * i;
      const int r = u / (DK / VE), v = u % (DK / VE);
      *reinterpret_cast<u32x4*>(ks + r * KP + v * VE) = kr[i];
      if (stage_q) *reinterpret_cast<u32x4*>(qs + r * KP + v * VE) = qr[i];
    }
    if (w == 0) {   // G = within-chunk cumsum of g (lane = token)
      float xs = x;
      if (!a.g_is_cumsum) {
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(xs, off);
          if (lane >= off) xs += y;
        }
      }
      Gs[lane] = xs;
      Bs[lane] = bv;
      if (a.G_out && !p_only) a.G_out[row0 + lane] = xs;
    }
  }
  lds_barrier();

  // ---- 2. gated score blocks: kkt (A) and / or qk (P) ---------------------------------------------
  auto scores = [&](auto set_tag) {
    constexpr int SET = decltype(set_tag)::value;
    switch (w) {
      case 0: score_wave<E, C, DK, KP, CP, SET, 0>(a, ks, qs, As, Gs, Bs, m); break;
      case 1: score_wave<E, C, DK, KP, CP, SET, 1>(a, ks, qs, As, Gs, Bs, m); break;
      case 2: score_wave<E, C, DK, KP, CP, SET, 2>(a, ks, qs, As, Gs, Bs, m); break;
      default: score_wave<E, C, DK, KP, CP, SET, 3>(a, ks, qs, As, Gs, Bs, m); break;
    }
  };
  if constexpr (DO_P) {
    if (p_only) {
      scores(std::integral_constant<int, kScoreP>{});
      return;                                          // the whole block: no barrier follows
    }
    if (a.split_p)
      scores(std::integral_constant<int, kScoreA>{});
    else
      scores(std::integral_constant<int, kScoreAP>{});
  } else {
    scores(std::integral_constant<int, kScoreA>{});
  }
  lds_barrier();

  if (a.A_out) {
    float* Ao = a.A_out + (size_t)m * C * C;
    for (int e = tid; e < C * C; e += 256) {
      const int i = e / C, j = e % C;
      Ao[e] = (j < i) ? As[i * CP + j] : 0.f;
    }
    lds_barrier();   // the inverse overwrites A in place
  }

  if (DO_INV) {
    unit_lower_inverse64(As, Ts);
    // ---- 3. write T (lower unit-triangular, zeros above), four columns per store ---------------
    TO* To = static_cast<TO*>(a.T_out) + (size_t)m * C * C;
#pragma unroll
    for (int it = 0; it < C * C / 4 / 256; ++it) {
      const int u = tid + 256 * it;
      const int i = u / (C / 4), j0 = (u % (C / 4)) * 4;
      if (a.t_lower_only && i < 32 && j0 >= 32) continue;
      const floatx4 t4 = *reinterpret_cast<const floatx4*>(Ts + i * CP + j0);
      store4(To + i * C + j0, (j0 <= i) ? t4[0] : 0.f, (j0 + 1 <= i) ? t4[1] : 0.f,
             (j0 + 2 <= i) ? t4[2] : 0.f, (j0 + 3 <= i) ? t4[3] : 0.f);
    }
  }
}

}  // namespace pf

namespace pf {

// Standalone opaque inverse: T = (I + A)^-1 for M strictly-lower C x C fp32 blocks (the upper
// triangle and diagonal of A are ignored, as tril does).  One workgroup per block.
template <int C>
__global__ __launch_bounds__(256) void tri_inv_kernel(const float* A, float* T, int M) {
  constexpr int CP = C + 4;
  __shared__ __attribute__((aligned(16))) float As[C * CP];
  __shared__ __attribute__((aligned(16))) float Ts[C * CP];
  const int m = blockIdx.x, tid = threadIdx.x;
  const float* Ag = A + (size_t)m * C * C;
  for (int e = tid; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    As[i * CP + j] = (j < i) ? Ag[e] : 0.f;
  }
  lds_barrier();
  block_unit_lower_inverse<C>(As, Ts);
  float* To = T + (size_t)m * C * C;
  for (int e = tid; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    To[e] = (j <= i) ? Ts[i * CP + j] : 0.f;
  }
}

}  // namespace pf
