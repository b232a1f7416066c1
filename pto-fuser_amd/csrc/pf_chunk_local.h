// K1 — the chunk-local stage of the chunked delta-rule forward, one workgroup per chunk.
//
// For chunk m (C tokens, rows m*C .. m*C+C-1 of the flattened [B*H*T, dk] token axis):
//   G     = cumsum_within_chunk(g)                                   (_gdn_full.py:63)
//   A     = strictly_lower( beta_i * safe_exp(G_i - G_j) * (k_i . k_j) )  (_gdn_full.py:73-75)
//           [epi_mode 1: exp(min(G_i + log beta_i - G_j, 0)), kkt_fused.h:154-185]
//   T     = (I + A)^-1                                                 (_gdn_full.py:76-78)
//   P     = p_scale * causal_incl_diag( (q_i . k_j) * exp(min(G_i - G_j, 0)) )
//           (_gdn_full.py:91-95; the output scale of :97 is applied here, once per score element)
//
// Mapping on CDNA4: k and q chunk tiles are staged in LDS (row pitch padded by 16 bytes so the
// MFMA operand reads are bank-conflict free per half wave); the 2*NB(NB+1)/2 lower-triangular
// 16x16 score blocks are spread over the 4 waves and computed with bf16 (or fp32) MFMA; the
// gate/mask epilogue runs in VALU on the accumulator registers.  The inverse is fp32:
//   * the NB diagonal 16x16 blocks are inverted by forward substitution, one lane per column,
//     all blocks at once (16*NB lanes);
//   * off-diagonal blocks are filled level by level (block distance L = 1..NB-1) with
//       T_ij = -T_ii * sum_{k=j}^{i-1} A_ik T_kj
//     on fp32 MFMA (16x16x4), the product chain kept in registers via the permuted-K layout.
#pragma once

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
  int epi_mode;         // 0: beta_i*safe_exp(G_i-G_j)   1: exp(min(G_i+log beta_i-G_j, 0))
  int g_is_cumsum;      // 1: g already holds within-chunk cumulative sums
  float p_scale;        // multiplies P (the forward's output scale)
  float* scale_out;     // if set, block 0 records p_scale here for the scan stage
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

template <typename E, typename TO, int C, int DK, bool DO_P, bool DO_INV>
__global__ __launch_bounds__(256) void chunk_local_kernel(ChunkLocalArgs a) {
  static_assert(C % 16 == 0 && C <= 64, "chunk size must be 16, 32, 48 or 64");
  static_assert(DK % Mfma<E>::KB == 0, "head dim must be a multiple of the MFMA K block");
  constexpr int PE = 16 / sizeof(E);
  constexpr int KP = DK + PE;   // LDS row pitch of k / q (elements)
  constexpr int CP = C + 4;     // LDS row pitch of A / T (floats)
  constexpr int NB = C / 16;
  constexpr int NL = NB * (NB + 1) / 2;
  constexpr int VE = Vec16<E>::N;
  constexpr int NV = C * (DK / VE);                 // 16-byte vectors per k (or q) chunk tile
  constexpr int NVT = NV / 256;                     // per thread
  static_assert(NV % 256 == 0, "k/q chunk tile must divide over 256 threads");
  constexpr int KQ_BYTES = (DO_P ? 2 : 1) * C * KP * (int)sizeof(E);
  constexpr int AT_BYTES = (DO_INV ? 2 : 1) * C * CP * 4;
  // A and T are written only after the last score read of k/q (a barrier apart), so they reuse
  // the k/q tiles' LDS: 35 KB per workgroup for bf16, four workgroups per CU.
  constexpr int KQT_BYTES = KQ_BYTES > AT_BYTES ? KQ_BYTES : AT_BYTES;

  __shared__ __attribute__((aligned(16))) char kqt[KQT_BYTES];
  __shared__ __attribute__((aligned(16))) float Gs[C];
  __shared__ float Bs[C];
  E* ks = reinterpret_cast<E*>(kqt);
  E* qs = ks + C * KP;
  float* As = reinterpret_cast<float*>(kqt);
  float* Ts = As + C * CP;

  const int m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const size_t row0 = (size_t)m * C;
  if (a.scale_out && m == 0 && tid == 0) *a.scale_out = a.p_scale;

  // ---- 1. stage k (and q), gates: every load issued before the first LDS store ----------------
  {
    const uint4* kg = reinterpret_cast<const uint4*>(static_cast<const E*>(a.k) + row0 * DK);
    const uint4* qg = reinterpret_cast<const uint4*>(static_cast<const E*>(a.q) + row0 * DK);
    uint4 kr[NVT], qr[NVT];
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      kr[i] = kg[tid + 256 * i];
      qr[i] = DO_P ? qg[tid + 256 * i] : make_uint4(0u, 0u, 0u, 0u);
    }
    float x = 0.f, bv = 0.f;
    if (tid < C) {
      x = a.g != nullptr ? a.g[row0 + tid] : 0.f;
      bv = a.beta[row0 + tid];
    }
#pragma unroll
    for (int i = 0; i < NVT; ++i) {
      const int u = tid + 256 * i;
      const int r = u / (DK / VE), v = u % (DK / VE);
      *reinterpret_cast<uint4*>(ks + r * KP + v * VE) = kr[i];
      if (DO_P) *reinterpret_cast<uint4*>(qs + r * KP + v * VE) = qr[i];
    }
    if (w == 0) {
      if (!a.g_is_cumsum) {
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float y = __shfl_up(x, off);
          if (lane >= off) x += y;
        }
      }
      if (lane < C) {
        Gs[lane] = x;
        Bs[lane] = bv;
        if (a.G_out) a.G_out[row0 + lane] = x;
      }
    }
  }
  lds_barrier();

  // ---- 2. gated score blocks: kkt (A) and, optionally, qk (P) -------------------------------
  // Wave w owns the blocks x = w, w+4, ... of the list [kk blocks | qk blocks]; their MFMA chains
  // are interleaved (independent accumulators), and each product is formed transposed —
  // D[4g+ii][c] = sum_d b[j][d] a[i][d] with i = 16 bi + c, j = 16 bj + 4g + ii — so a lane holds
  // four consecutive columns of one score row and stores them as one vector.
  {
    constexpr int NSB = NL * (DO_P ? 2 : 1), NPW = (NSB + 3) / 4;
    floatx4 acc[NPW];
    int bI[NPW], bJ[NPW];
    bool isqk[NPW], valid[NPW];
#pragma unroll
    for (int sb = 0; sb < NPW; ++sb) {
      const int x = w + 4 * sb;
      valid[sb] = x < NSB;
      isqk[sb] = x >= NL;
      int idx = isqk[sb] ? x - NL : x, bi = 0;
      while (idx > bi) { idx -= bi + 1; ++bi; }
      bI[sb] = valid[sb] ? bi : 0;
      bJ[sb] = valid[sb] ? idx : 0;
      acc[sb] = zero4();
    }
#pragma unroll
    for (int kb = 0; kb < DK / Mfma<E>::KB; ++kb) {
#pragma unroll
      for (int sb = 0; sb < NPW; ++sb) {
        if (!valid[sb]) continue;
        const E* jrow = ks + (16 * bJ[sb] + c) * KP;                    // k rows j
        const E* irow = (isqk[sb] ? qs : ks) + (16 * bI[sb] + c) * KP;  // k or q rows i
        acc[sb] = Mfma<E>::rows(acc[sb], jrow, irow, kb, g);
      }
    }
    lds_barrier();   // every wave is done reading k / q: A now overwrites them
#pragma unroll
    for (int sb = 0; sb < NPW; ++sb) {
      if (!valid[sb]) continue;
      const int i = 16 * bI[sb] + c, j0 = 16 * bJ[sb] + 4 * g;
      const float gi = Gs[i];
      const floatx4 gj = *reinterpret_cast<const floatx4*>(Gs + j0);
      floatx4 out;
      if (!isqk[sb]) {
        const float bi = Bs[i];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const float coef = a.epi_mode == 0 ? bi * safe_exp(gi - gj[ii])
                                             : __expf(fminf(gi + __logf(bi) - gj[ii], 0.f));
          out[ii] = (i > j0 + ii) ? coef * acc[sb][ii] : 0.f;
        }
        *reinterpret_cast<floatx4*>(As + i * CP + j0) = out;
      } else {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          out[ii] = (i >= j0 + ii) ? a.p_scale * acc[sb][ii] * __expf(fminf(gi - gj[ii], 0.f)) : 0.f;
        store4(static_cast<E*>(a.P_out) + (size_t)m * C * C + i * C + j0, out[0], out[1], out[2], out[3]);
      }
    }
  }
  if (DO_P) {  // zero the strictly-upper 16x16 blocks of P (the scan reads whole K blocks)
    uint4* P = reinterpret_cast<uint4*>(static_cast<E*>(a.P_out) + (size_t)m * C * C);
    for (int u = tid; u < C * C / VE; u += 256) {
      const int i = u / (C / VE), j0 = (u % (C / VE)) * VE;
      if ((j0 >> 4) > (i >> 4)) P[u] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  lds_barrier();

  if (a.A_out) {
    float* Ao = a.A_out + (size_t)m * C * C;
    for (int e = tid; e < C * C; e += 256) {
      const int i = e / C, j = e % C;
      Ao[e] = (j < i) ? As[i * CP + j] : 0.f;
    }
  }

  if (DO_INV) {
    block_unit_lower_inverse<C>(As, Ts);

    // ---- 4. write T (lower unit-triangular, zeros above), four columns per store ----------
    TO* To = static_cast<TO*>(a.T_out) + (size_t)m * C * C;
    for (int u = tid; u < C * C / 4; u += 256) {
      const int i = u / (C / 4), j0 = (u % (C / 4)) * 4;
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
