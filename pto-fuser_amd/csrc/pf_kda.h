// KDA — the chunked delta rule with a per-channel (per key dimension) decay, fused into two
// kernels for bf16 operands on gfx950.  Mathematics (examples/attention/_kda_full.py:42-76), per
// chain and chunk of C tokens, G = within-chunk cumsum of the per-token, per-channel log decay
// g [C, dk], a = k e^G, b = k e^-G (element-wise):
//
//   A    = strictly_lower( beta_i (a b^T)_ij )            T = (I + A)^-1
//   W    = T diag(beta) a,   U = T diag(beta) v           (the WY form)
//   v_new = U - W S
//   o    = scale (q e^G) S + scale causal_incl((q e^G) b^T) v_new
//   S   <- diag(e^{G_last}) (S + b^T v_new)     (= diag(e^{G_last}) S + (k e^{G_last - G})^T v_new)
//
// Stage 1 (kda_local_kernel, one workgroup per chunk) does what needs the whole chunk's gates at
// once: the cumsum, the gated operands, A and the inverse; it writes W, TB = T diag(beta),
// QE = scale q e^G, KB = b (bf16) and the chunk decay e^{G_last} (fp32), W, TB, QE and KB as
// whole 128-byte lines stored non-temporally (they are far larger than the caches and read only
// by stage 2: stored through the caches they cost stage 2 4 % of its time).  Stage 2
// (kda_scan_split_kernel, pf_kda_scan.h, one workgroup per (chain, 32-column slice)) carries S in
// registers through the chain:
//
//   U = TB v,  P = causal_incl(QE KB^T),  Y = W S,  v_new = U - Y,
//   o^T = v_new^T P^T + (QE S)^T,  S <- e^{G_last} (.) (S + KB^T v_new)
//
// so its chunk images hold the already-gated operands and the per-channel decay is one multiply
// of the state rows per chunk.  U and the score are formed in stage 2 from what it stages anyway
// (v, QE, KB) rather than written by stage 1: stage 1 then reads no v and writes neither U
// (16 KiB per chunk) nor P (6 KiB), only the 64 x 64 TB (8 KiB).
#pragma once

#include "pf_chunk_local.h"
#include "pf_gfx950.h"

namespace pf {

// ============================== stage 1: chunk-local ==============================

struct KdaLocalArgs {
  const bf16* q;        // [M*C, DK]
  const bf16* k;        // [M*C, DK]
  const float* g;       // [M*C, DK] per-token, per-channel log decay (cumsummed here)
  const float* beta;    // [M*C]
  float scale;
  bf16* W;              // [M, C, DK]  T diag(beta) (k e^G)
  bf16* TB;             // [M, C, C]   T diag(beta), zeros above the diagonal
  bf16* QE;             // [M*C, DK]   scale q e^G
  bf16* KB;             // [M*C, DK]   k e^-G
  float* DEC;           // [M, DK]     e^{G_last}
};

// Row tiles of stage 1 use the swizzle of the stage-2 k tile: element (r, col) lives at
// r*KP + 4*((col/4) ^ ((r >> 2) & 3)) + col%4 with KP = DK + 16, so both the row reads of the A
// products and the transposed reads of the W products are free of bank conflicts.
template <int KP>
__device__ __forceinline__ int kda_swz(int r, int col) {
  return r * KP + 4 * ((col >> 2) ^ ((r >> 2) & 3)) + (col & 3);
}

// One wave's blocks of A for the KDA chunk (the GDN kernel's A lists, score_code): products over
// the swizzled a / b tiles, then the mask epilogue (A scaled by beta_i into LDS).
template <int C, int KP, int CP, int W>
__device__ __forceinline__ void kda_score_wave(const bf16* at, const bf16* bt, float* As, const float* Bs) {
  constexpr int N = score_count(kScoreA, W);
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int rd = c * KP + 4 * (g ^ ((c >> 2) & 3));   // row c, K groups g and g+4 of each 32-block
  floatx4 acc[N];
#pragma unroll
  for (int b = 0; b < N; ++b) acc[b] = zero4();
#pragma unroll
  for (int kb = 0; kb < 128 / 32; ++kb) {
#pragma unroll
    for (int b = 0; b < N; ++b) {
      const int code = score_code(kScoreA, W, b);
      const bf16* jp = bt + 16 * (code & 3) * KP + rd + 32 * kb;
      const bf16* ip = at + 16 * ((code >> 2) & 3) * KP + rd + 32 * kb;
      const bf16x8 ja = cat8(*reinterpret_cast<const bf16x4*>(jp), *reinterpret_cast<const bf16x4*>(jp + 16));
      const bf16x8 ib = cat8(*reinterpret_cast<const bf16x4*>(ip), *reinterpret_cast<const bf16x4*>(ip + 16));
      acc[b] = mfma_bf16(ja, ib, acc[b]);   // equal rows: one LDS read
    }
  }
#pragma unroll
  for (int b = 0; b < N; ++b) {
    const int code = score_code(kScoreA, W, b);
    const int i = 16 * ((code >> 2) & 3) + c, j0 = 16 * (code & 3) + 4 * g;
    floatx4 out;
    const float bi = Bs[i];
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) out[ii] = (i > j0 + ii) ? bi * acc[b][ii] : 0.f;
    *reinterpret_cast<floatx4*>(As + i * CP + j0) = out;
  }
}

template <int C, int DK, int DV>
__global__ __launch_bounds__(256) void kda_local_kernel(KdaLocalArgs a) {
  static_assert(C == 64 && DK == 128 && DV == 128, "the KDA kernels are written for C 64, dk = dv = 128");
  constexpr int KP = DK + 16;          // bf16 row tiles: 288-byte rows
  constexpr int CP = C + 4;            // fp32 A / T
  constexpr int TPB = C + 8;           // bf16 T diag(beta)
  constexpr int TILE = C * KP;         // elements of one row tile
  // LDS regions, by phase:
  //   [0, 3 TILE) bf16 : tiles a | b | (spare)   (the fp32 g staging [C][DK] aliases the start)
  //   [3 TILE, ..) fp32: A [C][CP]
  // after the products of A: T (fp32) takes the third tile, T diag(beta) (bf16) takes A, and W
  // passes through the b tile on its way to HBM.
  static_assert(C * CP * 4 <= TILE * 2 && C * DK * 4 <= 3 * TILE * 2 && C * TPB * 2 <= C * CP * 4, "LDS aliasing");
  __shared__ __attribute__((aligned(16))) bf16 tiles[3 * TILE];
  __shared__ __attribute__((aligned(16))) float As[C * CP];
  __shared__ __attribute__((aligned(16))) float Bs[C];
  bf16* at = tiles;
  bf16* bt = tiles + TILE;
  float* gsm = reinterpret_cast<float*>(tiles);
  float* Ts = reinterpret_cast<float*>(tiles + 2 * TILE);
  bf16* Tb = reinterpret_cast<bf16*>(As);

  const int m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const size_t row0 = (size_t)m * C;
  // this thread's 16-byte vectors: rows rb + 16 i (i = 0..3), columns vc .. vc+7
  const int rb = tid >> 4, vc = (tid & 15) * 8;

  // ---- 1. loads; g to LDS ----------------------------------------------------------------
  uint4 kr[4], qr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const size_t e = (row0 + rb + 16 * i) * DK + vc;
    kr[i] = *reinterpret_cast<const uint4*>(a.k + e);
    qr[i] = *reinterpret_cast<const uint4*>(a.q + e);
    const floatx4 g0 = *reinterpret_cast<const floatx4*>(a.g + e);
    const floatx4 g1 = *reinterpret_cast<const floatx4*>(a.g + e + 4);
    *reinterpret_cast<floatx4*>(gsm + (rb + 16 * i) * DK + vc) = g0;
    *reinterpret_cast<floatx4*>(gsm + (rb + 16 * i) * DK + vc + 4) = g1;
  }
  if (tid < C) Bs[tid] = a.beta[row0 + tid];
  lds_barrier();

  // ---- 2. within-chunk cumsum per channel: thread = (column, half); the second half adds the
  //         first half's total when it reads G below ----------------------------------------
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
  float G[4][8];
  float egl[8];
  {
    float h0[8], gl[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h0[e] = gsm[(C / 2 - 1) * DK + vc + e];
      gl[e] = gsm[(C - 1) * DK + vc + e] + h0[e];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        G[i][e] = gsm[(rb + 16 * i) * DK + vc + e] + ((rb + 16 * i) >= C / 2 ? h0[e] : 0.f);
#pragma unroll
    for (int e = 0; e < 8; ++e) egl[e] = __expf(gl[e]);
  }
  lds_barrier();                                       // g staging is overwritten below
  if (tid < 16) {
#pragma unroll
    for (int e = 0; e < 8; e += 4)
      *reinterpret_cast<floatx4*>(a.DEC + (size_t)m * DK + vc + e) = floatx4{egl[e], egl[e + 1], egl[e + 2], egl[e + 3]};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rb + 16 * i;
    const bf16x8 kx = __builtin_bit_cast(bf16x8, kr[i]), qx = __builtin_bit_cast(bf16x8, qr[i]);
    bf16x8 av, bv, qv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float eg = __expf(G[i][e]), ebg = __expf(-G[i][e]);
      const float kf = (float)kx[e];
      av[e] = (bf16)(kf * eg);
      bv[e] = (bf16)(kf * ebg);
      qv[e] = (bf16)(a.scale * (float)qx[e] * eg);
    }
    const size_t e0 = (row0 + r) * DK + vc;
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, qv), reinterpret_cast<u32x4*>(a.QE + e0));
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, bv), reinterpret_cast<u32x4*>(a.KB + e0));
    // swizzled row tiles: two 4-element groups per vector
    const int o0 = kda_swz<KP>(r, vc), o1 = kda_swz<KP>(r, vc + 4);
    *reinterpret_cast<bf16x4*>(at + o0) = bf16x4{av[0], av[1], av[2], av[3]};
    *reinterpret_cast<bf16x4*>(at + o1) = bf16x4{av[4], av[5], av[6], av[7]};
    *reinterpret_cast<bf16x4*>(bt + o0) = bf16x4{bv[0], bv[1], bv[2], bv[3]};
    *reinterpret_cast<bf16x4*>(bt + o1) = bf16x4{bv[4], bv[5], bv[6], bv[7]};
  }
  lds_barrier();

  // ---- 4. A = beta_i (a b^T) strictly lower (fp32, LDS) ------------------------------------
  // The 10 lower 16x16 blocks are split over the waves as in the GDN chunk-local kernel (lists
  // that share operand rows), each product formed transposed so a lane holds four consecutive
  // columns of one row.
  switch (__builtin_amdgcn_readfirstlane(w)) {
    case 0: kda_score_wave<C, KP, CP, 0>(at, bt, As, Bs); break;
    case 1: kda_score_wave<C, KP, CP, 1>(at, bt, As, Bs); break;
    case 2: kda_score_wave<C, KP, CP, 2>(at, bt, As, Bs); break;
    default: kda_score_wave<C, KP, CP, 3>(at, bt, As, Bs); break;
  }
  lds_barrier();

  // ---- 5. T = (I + A)^-1 (fp32) ------------------------------------------------------------
  unit_lower_inverse64(As, Ts);

  // ---- 6. T diag(beta) as bf16 (in A's space) ----------------------------------------------
  for (int u = tid; u < C * C / 4; u += 256) {
    const int i = u / (C / 4), j0 = (u % (C / 4)) * 4;
    const floatx4 t4 = *reinterpret_cast<const floatx4*>(Ts + i * CP + j0);
    const floatx4 b4 = *reinterpret_cast<const floatx4*>(Bs + j0);
    store4(Tb + i * TPB + j0, (j0 <= i) ? t4[0] * b4[0] : 0.f, (j0 + 1 <= i) ? t4[1] * b4[1] : 0.f,
           (j0 + 2 <= i) ? t4[2] * b4[2] : 0.f, (j0 + 3 <= i) ? t4[3] * b4[3] : 0.f);
  }
  lds_barrier();
  // TB to HBM for stage 2: vector u = tid + 256 h (h = 0, 1) is row u / 8, columns 8 (u % 8) ..,
  // so each store instruction writes eight whole 128-byte rows
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int u = tid + 256 * h, i = u >> 3, j0 = 8 * (u & 7);
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(Tb + i * TPB + j0),
                                reinterpret_cast<u32x4*>(a.TB + ((size_t)m * C + i) * C + j0));
  }

  // ---- 7. W^T = a^T (T diag beta)^T ---------------------------------------------------------
  // Wave w owns the 16-row blocks mb = 2w, 2w+1 of the dk dimension.  A operand: a^T by
  // transpose reads (lane (c,g) gets rows j = 32kb + 4g + 0..3 and +16 of column 16mb + c);
  // B operand: rows i = 16nb + c of T diag(beta) at the same (permuted) j.  The D registers hold
  // W[i][16mb + 4g .. +3]: four consecutive columns.
  {
    floatx4 accW[2][4];
#pragma unroll
    for (int mb2 = 0; mb2 < 2; ++mb2)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) accW[mb2][nb] = zero4();
    const int tr = (4 * g + (c >> 2)) * KP + 4 * ((c & 3) ^ g);     // transposed reads
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int kb = 0; kb <= (nb >> 1); ++kb) {                    // T is lower triangular
        const bf16* tp = Tb + (16 * nb + c) * TPB + 32 * kb + 4 * g;
        const bf16x8 tbv = cat8(*reinterpret_cast<const bf16x4*>(tp), *reinterpret_cast<const bf16x4*>(tp + 16));
#pragma unroll
        for (int mb2 = 0; mb2 < 2; ++mb2) {
          const int mb = 2 * w + mb2;
          const bf16* ap = at + 32 * kb * KP + tr + 16 * mb;
          accW[mb2][nb] = mfma_bf16(cat8(lds_read_tr(ap), lds_read_tr(ap + 16 * KP)), tbv, accW[mb2][nb]);
        }
      }
    }
    // staged in the b tile (free since A was formed), then written as whole rows: a store
    // instruction of four scattered 32-byte pieces per row was measured 7 % slower for the kernel
#pragma unroll
    for (int mb2 = 0; mb2 < 2; ++mb2)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        store4(bt + (16 * nb + c) * KP + 16 * (2 * w + mb2) + 4 * g, accW[mb2][nb][0], accW[mb2][nb][1],
               accW[mb2][nb][2], accW[mb2][nb][3]);
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(bt + (rb + 16 * i) * KP + vc),
                                  reinterpret_cast<u32x4*>(a.W + (row0 + rb + 16 * i) * DK + vc));
  }
}

// ============================== stage 2: scan + output ==============================

struct KdaScanArgs {
  const bf16* W;        // [BH*NC, C, DK]
  const bf16* TB;       // [BH*NC, C, C]   T diag(beta)
  const bf16* v;        // [BH*T, DV]
  const bf16* QE;       // [BH*T, DK]
  const bf16* KB;       // [BH*T, DK]      k e^-G
  const float* DEC;     // [BH*NC, DK]
  const float* h0;      // [BH, DK, DV] or null
  float* o;             // [BH*T, DV]
  float* h_final;       // [BH, DK, DV] or null
  int BH;
  int NC;
};

}  // namespace pf
