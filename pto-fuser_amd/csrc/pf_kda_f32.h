// KDA forward for fp32 operands: the two stages of the bf16 kernels (pf_kda.h) with fp32 tiles and
// the fp32 MFMA (v_mfma_f32_16x16x4f32), written for exactness rather than throughput (no config
// of the benchmark runs KDA in fp32).  Mathematics (examples/attention/_kda_full.py:42-76), per
// chain and chunk of C tokens, G = within-chunk cumsum of g [C, dk], a = k e^G, b = k e^-G:
//
//   A = strictly_lower(beta_i (a b^T)_ij),  T = (I + A)^-1,  W = T diag(beta) a,  U = T diag(beta) v
//   stage 2:  v_new = U - W S,  o = QE S + P v_new,  S <- diag(e^{G_last}) S + KR^T v_new
//
// with QE = scale q e^G, KR = k e^{G_last - G}, P = causal_incl(QE b^T).
//
// Stage 1 (kda_local_f32_kernel): one 256-thread workgroup per chunk; a, b and qe in LDS (fp32,
// 132-float rows, so that the 16 rows of an MFMA operand read fall in 16 different bank groups),
// the 20 score blocks over the GDN chunk-local kernel's lists, the inverse in place, then W and U
// with the T rows as the A operand.  Stage 2 (kda_scan_f32_kernel): one workgroup of two waves per
// (chain, 32-column slice); each wave holds 16 state columns (fp32, MFMA D layout) through the
// chain, and every chunk's W, QE, KR, P and U slice are copied into LDS before its products.
#pragma once

#include <type_traits>

#include "pf_chunk_local.h"
#include "pf_gfx950.h"

namespace pf {

struct KdaLocalF32Args {
  const float* q;       // [M*C, DK]
  const float* k;       // [M*C, DK]
  const float* v;       // [M*C, DV]
  const float* g;       // [M*C, DK] per-token, per-channel log decay (cumsummed here)
  const float* beta;    // [M*C]
  float scale;
  float* W;             // [M, C, DK]
  float* U;             // [M, C, DV]
  float* QE;            // [M*C, DK]
  float* KR;            // [M*C, DK]
  float* P;             // [M, C, C]   lower blocks only (the scan reads no other)
  float* DEC;           // [M, DK]     e^{G_last}
};

template <int C, int DK>
__global__ __launch_bounds__(256) void kda_local_f32_kernel(KdaLocalF32Args a) {
  static_assert(C == 64 && DK == 128, "the fp32 KDA kernels are written for C 64, dk = dv = 128");
  constexpr int RP = DK + 4;           // fp32 row tiles
  constexpr int CP = C + 4;            // A / T
  constexpr int TILE = C * RP;
  // LDS: a | b | qe row tiles, then A; the g staging [C][DK] aliases a and b until the gated
  // operands are formed; after the scores T replaces A in place and the v tile takes b's rows.
  static_assert(C * DK <= 2 * TILE, "g staging fits the a and b tiles");
  __shared__ __attribute__((aligned(16))) float tiles[3 * TILE];
  __shared__ __attribute__((aligned(16))) float As[C * CP];
  __shared__ __attribute__((aligned(16))) float Bs[C];
  float* at = tiles;
  float* bt = tiles + TILE;
  float* qt = tiles + 2 * TILE;
  float* gsm = tiles;
  float* vt = bt;

  const int m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const size_t row0 = (size_t)m * C;
  const int rb = tid >> 4, vc = (tid & 15) * 8;    // rows rb + 16 i, columns vc .. vc+7

  // ---- 1. loads; g to LDS ----------------------------------------------------------------
  floatx4 kr[4][2], qr[4][2], vr[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const size_t e = (row0 + rb + 16 * i) * DK + vc;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      kr[i][h] = *reinterpret_cast<const floatx4*>(a.k + e + 4 * h);
      qr[i][h] = *reinterpret_cast<const floatx4*>(a.q + e + 4 * h);
      vr[i][h] = *reinterpret_cast<const floatx4*>(a.v + e + 4 * h);
      *reinterpret_cast<floatx4*>(gsm + (rb + 16 * i) * DK + vc + 4 * h) =
          *reinterpret_cast<const floatx4*>(a.g + e + 4 * h);
    }
  }
  if (tid < C) Bs[tid] = a.beta[row0 + tid];
  lds_barrier();

  // ---- 2. within-chunk cumsum per channel (thread = column x half of the rows; the second
  //         half's entries get the first half's total when read below) ------------------------
  {
    const int col = tid & (DK - 1), h = tid >> 7;
    float x[C / 2];
#pragma unroll
    for (int r = 0; r < C / 2; ++r) x[r] = gsm[(h * (C / 2) + r) * DK + col];
#pragma unroll
    for (int r = 1; r < C / 2; ++r) x[r] += x[r - 1];
#pragma unroll
    for (int r = 0; r < C / 2; ++r) gsm[(h * (C / 2) + r) * DK + col] = x[r];
  }
  lds_barrier();

  // ---- 3. gated operands ------------------------------------------------------------------
  float G[4][8], gl[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float half = gsm[(C / 2 - 1) * DK + vc + e];
    gl[e] = gsm[(C - 1) * DK + vc + e] + half;         // G_last of column vc + e
#pragma unroll
    for (int i = 0; i < 4; ++i)
      G[i][e] = gsm[(rb + 16 * i) * DK + vc + e] + ((rb + 16 * i) >= C / 2 ? half : 0.f);
  }
  lds_barrier();                                       // the g staging is overwritten below
  if (tid < 16) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      *reinterpret_cast<floatx4*>(a.DEC + (size_t)m * DK + vc + 4 * h) =
          floatx4{__expf(gl[4 * h]), __expf(gl[4 * h + 1]), __expf(gl[4 * h + 2]), __expf(gl[4 * h + 3])};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rb + 16 * i;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      floatx4 av, bv, qv, rv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gg = G[i][4 * h + e];
        const float eg = __expf(gg), ebg = __expf(-gg);
        av[e] = kr[i][h][e] * eg;
        bv[e] = kr[i][h][e] * ebg;
        qv[e] = a.scale * qr[i][h][e] * eg;
        rv[e] = kr[i][h][e] * __expf(gl[4 * h + e] - gg);
      }
      const size_t e0 = (row0 + r) * DK + vc + 4 * h;
      *reinterpret_cast<floatx4*>(a.QE + e0) = qv;
      *reinterpret_cast<floatx4*>(a.KR + e0) = rv;
      *reinterpret_cast<floatx4*>(at + r * RP + vc + 4 * h) = av;
      *reinterpret_cast<floatx4*>(bt + r * RP + vc + 4 * h) = bv;
      *reinterpret_cast<floatx4*>(qt + r * RP + vc + 4 * h) = qv;
    }
  }
  lds_barrier();

  // ---- 4. scores: the GDN chunk-local kernel's block lists (score_code with P): A = beta_i
  //         (a_i . b_j) strictly lower into As, P = qe_i . b_j (lower, with its diagonal) to HBM
  {
    constexpr int N = 5;
    floatx4 acc[N];
#pragma unroll
    for (int b = 0; b < N; ++b) acc[b] = zero4();
    auto products = [&](auto wtag) {
      constexpr int WW = decltype(wtag)::value;
#pragma unroll
      for (int kb = 0; kb < DK / 16; ++kb) {
#pragma unroll
        for (int b = 0; b < N; ++b) {
          const int code = score_code(kScoreAP, WW, b);
          const float* jrow = bt + (16 * (code & 3) + c) * RP;
          const float* irow = ((code & 16) ? qt : at) + (16 * ((code >> 2) & 3) + c) * RP;
          acc[b] = Mfma<float>::rows(acc[b], jrow, irow, kb, g);
        }
      }
    };
    switch (w) {
      case 0: products(std::integral_constant<int, 0>{}); break;
      case 1: products(std::integral_constant<int, 1>{}); break;
      case 2: products(std::integral_constant<int, 2>{}); break;
      default: products(std::integral_constant<int, 3>{}); break;
    }
    // each product is formed transposed: acc[ii] = (x_i . b_j), i = 16 bi + c, j = 16 bj + 4g + ii
#pragma unroll
    for (int b = 0; b < N; ++b) {
      const int code = score_code(kScoreAP, w, b);
      const int i = 16 * ((code >> 2) & 3) + c, j0 = 16 * (code & 3) + 4 * g;
      floatx4 out;
      if (!(code & 16)) {
        const float bi = Bs[i];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) out[ii] = (i > j0 + ii) ? bi * acc[b][ii] : 0.f;
        *reinterpret_cast<floatx4*>(As + i * CP + j0) = out;
      } else {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) out[ii] = (i >= j0 + ii) ? acc[b][ii] : 0.f;
        *reinterpret_cast<floatx4*>(a.P + (size_t)m * C * C + i * C + j0) = out;
      }
    }
  }
  lds_barrier();

  // ---- 5. T = (I + A)^-1 in place; the v tile into b's rows ---------------------------------
  unit_lower_inverse64(As, As);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) *reinterpret_cast<floatx4*>(vt + (rb + 16 * i) * RP + vc + 4 * h) = vr[i][h];
  lds_barrier();

  // ---- 6. W = T diag(beta) a, U = T diag(beta) v: wave w owns column blocks 2w, 2w+1 ---------
  //         (A operand = T rows, lane (c, g) T[16 ib + c][4 kk + g]; B = beta_j x[j][16 db + c])
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    floatx4 accW[2], accU[2];
#pragma unroll
    for (int d2 = 0; d2 < 2; ++d2) accW[d2] = accU[d2] = zero4();
    for (int kk = 0; kk < 4 * ib + 4; ++kk) {        // T lower triangular: j <= 16 ib + 15
      const int j = 4 * kk + g;
      const float t = As[(16 * ib + c) * CP + j];
      const float bj = Bs[j];
#pragma unroll
      for (int d2 = 0; d2 < 2; ++d2) {
        const int col = 16 * (2 * w + d2) + c;
        accW[d2] = __builtin_amdgcn_mfma_f32_16x16x4f32(t, bj * at[j * RP + col], accW[d2], 0, 0, 0);
        accU[d2] = __builtin_amdgcn_mfma_f32_16x16x4f32(t, bj * vt[j * RP + col], accU[d2], 0, 0, 0);
      }
    }
    // lane (c, g) holds D[4g + ii][c] of the tile: rows 16 ib + 4g + ii, column 16 db + c
#pragma unroll
    for (int d2 = 0; d2 < 2; ++d2)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const size_t e = ((size_t)m * C + 16 * ib + 4 * g + ii) * DK + 16 * (2 * w + d2) + c;
        a.W[e] = accW[d2][ii];
        a.U[e] = accU[d2][ii];
      }
  }
}

struct KdaScanF32Args {
  const float* W;       // [BH*NC, C, DK]
  const float* U;       // [BH*NC, C, DV]
  const float* QE;      // [BH*T, DK]
  const float* KR;      // [BH*T, DK]
  const float* P;       // [BH*NC, C, C]  (lower blocks read)
  const float* DEC;     // [BH*NC, DK]
  const float* h0;      // [BH, DK, DV] or null
  float* o;             // [BH*T, DV]
  float* h_final;       // [BH, DK, DV] or null
  int BH, NC;
};

template <int C, int DK, int DV>
__global__ __launch_bounds__(128) void kda_scan_f32_kernel(KdaScanF32Args a) {
  static_assert(C == 64 && DK == 128 && DV == 128, "the fp32 KDA kernels are written for C 64, dk = dv = 128");
  constexpr int RP = DK + 4, PP = C + 4, UP = 32 + 4;
  __shared__ __attribute__((aligned(16))) float Ws[C * RP];
  __shared__ __attribute__((aligned(16))) float Qs[C * RP];
  __shared__ __attribute__((aligned(16))) float Ks[C * RP];
  __shared__ __attribute__((aligned(16))) float Ps[C * PP];
  __shared__ __attribute__((aligned(16))) float Us[C * UP];
  __shared__ __attribute__((aligned(16))) float Ds[DK];

  const int bh = blockIdx.x / (DV / 32), slice = blockIdx.x % (DV / 32);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col0 = 32 * slice, mycol = col0 + 16 * w + c;   // this lane's state / o column
  const size_t Tlen = (size_t)a.NC * C;

  floatx4 S[DK / 16];                                  // rows 16 r + 4g + ii, column mycol
#pragma unroll
  for (int r = 0; r < DK / 16; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + mycol] : 0.f;

  for (int ch = 0; ch < a.NC; ++ch) {
    const size_t m = (size_t)bh * a.NC + ch;
    // ---- the chunk's images into LDS (128 threads, 16-byte copies) ----
    for (int u = tid; u < C * DK / 4; u += 128) {
      const int r = u / (DK / 4), q4 = u % (DK / 4);
      *reinterpret_cast<floatx4*>(Ws + r * RP + 4 * q4) = *reinterpret_cast<const floatx4*>(a.W + (m * C + r) * DK + 4 * q4);
      *reinterpret_cast<floatx4*>(Qs + r * RP + 4 * q4) = *reinterpret_cast<const floatx4*>(a.QE + (m * C + r) * DK + 4 * q4);
      *reinterpret_cast<floatx4*>(Ks + r * RP + 4 * q4) = *reinterpret_cast<const floatx4*>(a.KR + (m * C + r) * DK + 4 * q4);
    }
    for (int u = tid; u < C * C / 4; u += 128) {
      const int r = u / (C / 4), q4 = u % (C / 4);
      *reinterpret_cast<floatx4*>(Ps + r * PP + 4 * q4) = *reinterpret_cast<const floatx4*>(a.P + (m * C + r) * C + 4 * q4);
    }
    for (int u = tid; u < C * 8; u += 128) {
      const int r = u / 8, q4 = u % 8;
      *reinterpret_cast<floatx4*>(Us + r * UP + 4 * q4) = *reinterpret_cast<const floatx4*>(a.U + (m * C + r) * DV + col0 + 4 * q4);
    }
    if (tid < DK / 4) *reinterpret_cast<floatx4*>(Ds + 4 * tid) = *reinterpret_cast<const floatx4*>(a.DEC + m * DK + 4 * tid);
    lds_barrier();

    // ---- Y = W S, (QE S), v_new = U - Y (token tile ib: lane (c, g) rows 16 ib + 4g + ii) ----
    floatx4 VN[C / 16], QS[C / 16];
#pragma unroll
    for (int ib = 0; ib < C / 16; ++ib) {
      floatx4 y = zero4(), qs = zero4();
#pragma unroll
      for (int r = 0; r < DK / 16; ++r) {
        const floatx4 wa = *reinterpret_cast<const floatx4*>(Ws + (16 * ib + c) * RP + 16 * r + 4 * g);
        const floatx4 qa = *reinterpret_cast<const floatx4*>(Qs + (16 * ib + c) * RP + 16 * r + 4 * g);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          y = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[ii], S[r][ii], y, 0, 0, 0);
          qs = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[ii], S[r][ii], qs, 0, 0, 0);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) VN[ib][ii] = Us[(16 * ib + 4 * g + ii) * UP + 16 * w + c] - y[ii];
      QS[ib] = qs;
    }
    // ---- o = QE S + P v_new (P lower triangular by 16-token blocks) -> HBM ----
#pragma unroll
    for (int ib = 0; ib < C / 16; ++ib) {
      floatx4 o4 = QS[ib];
#pragma unroll
      for (int jb = 0; jb <= ib; ++jb) {
        const floatx4 pa = *reinterpret_cast<const floatx4*>(Ps + (16 * ib + c) * PP + 16 * jb + 4 * g);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ii], VN[jb][ii], o4, 0, 0, 0);
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        __builtin_nontemporal_store(o4[ii], a.o + ((size_t)bh * Tlen + (size_t)ch * C + 16 * ib + 4 * g + ii) * DV + mycol);
    }
    // ---- S <- diag(e^{G_last}) S + KR^T v_new  (A operand lane (c, g): KR[t][16 r + c]) ----
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) {
      floatx4 acc;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) acc[ii] = Ds[16 * r + 4 * g + ii] * S[r][ii];
#pragma unroll
      for (int jb = 0; jb < C / 16; ++jb)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Ks[(16 * jb + 4 * g + ii) * RP + 16 * r + c], VN[jb][ii], acc, 0, 0, 0);
      S[r] = acc;
    }
    lds_barrier();                                     // the images are read: next chunk's copies
  }
  if (a.h_final) {
#pragma unroll
    for (int r = 0; r < DK / 16; ++r)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        a.h_final[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + mycol] = S[r][ii];
  }
}

}  // namespace pf
