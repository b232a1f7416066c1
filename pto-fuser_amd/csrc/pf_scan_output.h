// K2 — the inter-chunk state scan fused with the output stage.
//
// One workgroup per (chain bh = (b,h), dv tile of 16*NW columns); wave w owns 16 columns of the
// state.  The state S[DK x 16] of a wave lives in registers (fp32, the MFMA D layout) for the
// whole sequential chunk loop; per-chunk snapshots are never written to HBM.  Per chunk c:
//
//   Y     = k_c S                                    (A = k rows from LDS, B = S registers)
//   QS    = q_c S
//   r     = beta (v - e^G * Y)
//   v_new = T_c r          ( = U - W S  with W = T beta k e^G, U = T beta v; _gdn_full.py:79-84)
//   o_c   = scale * (e^G * QS + P_c v_new)                              (_gdn_full.py:88-97)
//   S     = e^{G_last} S + k_c^T (v_new * e^{G_last - G})               (_gdn_full.py:86-87)
//
// T_c = (I+A)^-1, P_c (gated causal score) and G (within-chunk cumsum) come from K1.  Every
// product chains register to register through the permuted-K MFMA layout; k_c^T for the state
// update is staged transposed in LDS.  The tiles of one chain are mapped to the same XCD so the
// per-chunk k/q/T/P reads of the sibling workgroups hit one L2.
#pragma once

#include "pf_device.h"

namespace pf {

struct ScanOutArgs {
  const void* q;        // [BH*T, DK]  E
  const void* k;        // [BH*T, DK]  E
  const void* v;        // [BH*T, DV]  E
  const float* beta;    // [BH*T]
  const float* G;       // [BH*T] within-chunk cumsum (from K1); null => 0
  const void* Tm;       // [M, C, C]   E
  const void* P;        // [M, C, C]   E
  const float* h0;      // [BH, DK, DV] or null
  float* o;             // [BH*T, DV]
  float* h_final;       // [BH, DK, DV] or null
  int BH;
  int NC;               // chunks per chain
  float scale;
};

template <typename E, int C, int DK, int DV, int NW>
__global__ __launch_bounds__(64 * NW) void scan_output_kernel(ScanOutArgs a) {
  constexpr int PE = 16 / sizeof(E);
  constexpr int KP = DK + PE;
  constexpr int TP = C + PE;
  constexpr int NT = DV / (16 * NW);
  constexpr int NTHR = 64 * NW;
  constexpr int VE = Vec16<E>::N;
  constexpr int KB = Mfma<E>::KB;
  constexpr int NKB_D = DK / KB;
  constexpr int NKB_C = C / KB;
  constexpr int MB = C / 16;
  static_assert(DV % (16 * NW) == 0, "dv tile");
  static_assert(C % KB == 0 && C <= 64 && NTHR >= C, "chunk size");

  __shared__ __attribute__((aligned(16))) E ks[C * KP];
  __shared__ __attribute__((aligned(16))) E qs[C * KP];
  __shared__ __attribute__((aligned(16))) E kts[DK * TP];
  __shared__ __attribute__((aligned(16))) E ts[C * TP];
  __shared__ __attribute__((aligned(16))) E ps[C * TP];
  __shared__ float Gs[C], Bs[C];

  int bh, tile;
  const int bid = blockIdx.x;
  if (a.BH % 8 == 0) {  // the NT tiles of one chain share an XCD (dispatch is round-robin on XCDs)
    const int grp = bid / (8 * NT), within = bid % (8 * NT);
    bh = grp * 8 + (within % 8);
    tile = within / 8;
  } else {
    bh = bid / NT;
    tile = bid % NT;
  }
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int col = tile * 16 * NW + w * 16 + c;

  floatx4 S[DK / 16];
#pragma unroll
  for (int r = 0; r < DK / 16; ++r) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + col] : 0.f;
  }

  const E* kbase = static_cast<const E*>(a.k);
  const E* qbase = static_cast<const E*>(a.q);
  const E* vbase = static_cast<const E*>(a.v);

  for (int ch = 0; ch < a.NC; ++ch) {
    const size_t m = (size_t)bh * a.NC + ch;
    const size_t tok0 = m * C;
    // ---- stage the chunk: k (row-major and transposed), q, T, P, G, beta -------------------
    {
      const E* kg = kbase + tok0 * DK;
      for (int u = tid; u < (C / 4) * (DK / VE); u += NTHR) {
        const int t0 = (u / (DK / VE)) * 4, d0 = (u % (DK / VE)) * VE;
        uint4 x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = *reinterpret_cast<const uint4*>(kg + (size_t)(t0 + j) * DK + d0);
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(ks + (t0 + j) * KP + d0) = x[j];
        const E* xe = reinterpret_cast<const E*>(x);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          E* dst = kts + (d0 + e) * TP + t0;
          dst[0] = xe[e];
          dst[1] = xe[VE + e];
          dst[2] = xe[2 * VE + e];
          dst[3] = xe[3 * VE + e];
        }
      }
      const uint4* qg = reinterpret_cast<const uint4*>(qbase + tok0 * DK);
      for (int i = tid; i < C * (DK / VE); i += NTHR)
        *reinterpret_cast<uint4*>(qs + (i / (DK / VE)) * KP + (i % (DK / VE)) * VE) = qg[i];
      const uint4* tg = reinterpret_cast<const uint4*>(static_cast<const E*>(a.Tm) + m * C * C);
      const uint4* pg = reinterpret_cast<const uint4*>(static_cast<const E*>(a.P) + m * C * C);
      for (int i = tid; i < C * (C / VE); i += NTHR) {
        const int r = i / (C / VE), v = (i % (C / VE)) * VE;
        *reinterpret_cast<uint4*>(ts + r * TP + v) = tg[i];
        *reinterpret_cast<uint4*>(ps + r * TP + v) = pg[i];
      }
      if (tid < C) {
        Gs[tid] = a.G ? a.G[tok0 + tid] : 0.f;
        Bs[tid] = a.beta[tok0 + tid];
      }
    }
    __syncthreads();

    // ---- Y = k S and QS = q S --------------------------------------------------------------
    floatx4 Y[MB], QS[MB], R[MB], VN[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      Y[mb] = chain<E, NKB_D>(zero4(), ks + (16 * mb + c) * KP, S, NKB_D, g);
      QS[mb] = chain<E, NKB_D>(zero4(), qs + (16 * mb + c) * KP, S, NKB_D, g);
    }
    // ---- r = beta (v - e^G Y) ---------------------------------------------------------------
    const E* vcol = vbase + tok0 * DV + col;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int t = 16 * mb + 4 * g + ii;
        R[mb][ii] = Bs[t] * (to_f32(vcol[(size_t)t * DV]) - __expf(Gs[t]) * Y[mb][ii]);
      }
    }
    // ---- v_new = T r (T lower triangular: K blocks up to the diagonal) ----------------------
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      VN[mb] = chain<E, NKB_C>(zero4(), ts + (16 * mb + c) * TP, R, (16 * mb + 16 + KB - 1) / KB, g);
    // ---- o = scale (e^G QS + P v_new) -------------------------------------------------------
    float* ocol = a.o + tok0 * DV + col;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const floatx4 O = chain<E, NKB_C>(zero4(), ps + (16 * mb + c) * TP, VN, (16 * mb + 16 + KB - 1) / KB, g);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int t = 16 * mb + 4 * g + ii;
        ocol[(size_t)t * DV] = a.scale * (__expf(Gs[t]) * QS[mb][ii] + O[ii]);
      }
    }
    // ---- S = e^{G_last} S + k^T (v_new e^{G_last - G}) --------------------------------------
    const float gl = Gs[C - 1];
    const float dl = __expf(gl);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) VN[mb][ii] *= __expf(gl - Gs[16 * mb + 4 * g + ii]);
    }
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) S[r] = chain<E, NKB_C>(S[r] * dl, kts + (16 * r + c) * TP, VN, NKB_C, g);
    __syncthreads();
  }

  if (a.h_final) {
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) a.h_final[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + col] = S[r][ii];
    }
  }
}

}  // namespace pf
