// KDA — the chunked delta rule with a per-channel (per key dimension) decay, fused into two
// kernels for bf16 operands on gfx950.  Mathematics (examples/attention/_kda_full.py:42-76), per
// chain and chunk of C tokens, G = within-chunk cumsum of the per-token, per-channel log decay
// g [C, dk], a = k e^G, b = k e^-G (element-wise):
//
//   A    = strictly_lower( beta_i (a b^T)_ij )            T = (I + A)^-1
//   W    = T diag(beta) a,   U = T diag(beta) v           (the WY form)
//   v_new = U - W S
//   o    = scale (q e^G) S + scale causal_incl((q e^G) b^T) v_new
//   S   <- diag(e^{G_last}) S + (k e^{G_last - G})^T v_new
//
// Stage 1 (kda_local_kernel, one workgroup per chunk) does everything that does not depend on S:
// the cumsum, the gated operands, A, the inverse, W, U and the score P; it writes W, U,
// QE = scale q e^G, KR = k e^{G_last - G}, P = causal_incl(QE b^T) (bf16) and the chunk decay
// e^{G_last} (fp32).  Stage 2 (kda_scan_kernel, one workgroup per (chain, 32-column slice))
// carries S in registers through the chain:
//
//   Y = W S,  v_new = U - Y,  o^T = v_new^T P^T + (QE S)^T,  S <- e^{G_last} (.) S + KR^T v_new
//
// so its chunk images hold the already-gated operands and the per-channel decay is one multiply
// of the state rows per chunk.  Two compute waves each hold 16 state columns through the whole
// chain; four loader waves keep three chunks in flight in registers, write each chunk into the
// free half of a double-buffered LDS stage (swizzled rows, 16-byte stores) and store the o tiles
// the compute waves stage in LDS.
#pragma once

#include "pf_chunk_local.h"
#include "pf_gfx950.h"

namespace pf {

// ============================== stage 1: chunk-local ==============================

struct KdaLocalArgs {
  const bf16* q;        // [M*C, DK]
  const bf16* k;        // [M*C, DK]
  const bf16* v;        // [M*C, DV]
  const float* g;       // [M*C, DK] per-token, per-channel log decay (cumsummed here)
  const float* beta;    // [M*C]
  float scale;
  bf16* W;              // [M, C, DK]  T diag(beta) (k e^G)
  bf16* U;              // [M, C, DV]  T diag(beta) v
  bf16* QE;             // [M*C, DK]   scale q e^G
  bf16* KR;             // [M*C, DK]   k e^{G_last - G}
  bf16* P;              // [M, C, C]   causal_incl(QE (k e^-G)^T); upper blocks (0,1), (2,3) zero
  float* DEC;           // [M, DK]     e^{G_last}
};

// Row tiles of stage 1 use the swizzle of the stage-2 k tile: element (r, col) lives at
// r*KP + 4*((col/4) ^ ((r >> 2) & 3)) + col%4 with KP = DK + 16, so both the row reads of the score
// products and the transposed reads of the W/U products are free of bank conflicts.
template <int KP>
__device__ __forceinline__ int kda_swz(int r, int col) {
  return r * KP + 4 * ((col >> 2) ^ ((r >> 2) & 3)) + (col & 3);
}

// One wave's score blocks of the KDA chunk (the GDN kernel's lists, score_code): products over
// the swizzled a / b / qe tiles, then the mask epilogue (A scaled by beta_i into LDS, P to global).
template <int C, int KP, int CP, int W>
__device__ __forceinline__ void kda_score_wave(const bf16* at, const bf16* bt, const bf16* qt, float* As,
                                               const float* Bs, bf16* P) {
  constexpr int N = score_count(kScoreAP, W);
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int rd = c * KP + 4 * (g ^ ((c >> 2) & 3));   // row c, K groups g and g+4 of each 32-block
  floatx4 acc[N];
#pragma unroll
  for (int b = 0; b < N; ++b) acc[b] = zero4();
#pragma unroll
  for (int kb = 0; kb < 128 / 32; ++kb) {
#pragma unroll
    for (int b = 0; b < N; ++b) {
      const int code = score_code(kScoreAP, W, b);
      const bf16* jp = bt + 16 * (code & 3) * KP + rd + 32 * kb;
      const bf16* ip = ((code & 16) ? qt : at) + 16 * ((code >> 2) & 3) * KP + rd + 32 * kb;
      const bf16x8 ja = cat8(*reinterpret_cast<const bf16x4*>(jp), *reinterpret_cast<const bf16x4*>(jp + 16));
      const bf16x8 ib = cat8(*reinterpret_cast<const bf16x4*>(ip), *reinterpret_cast<const bf16x4*>(ip + 16));
      acc[b] = mfma_bf16(ja, ib, acc[b]);   // equal rows: one LDS read
    }
  }
#pragma unroll
  for (int b = 0; b < N; ++b) {
    const int code = score_code(kScoreAP, W, b);
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
      store4(P + i * C + j0, out[0], out[1], out[2], out[3]);
    }
  }
  if (W == 0 || W == 3) {   // the upper blocks (0,1) and (2,3) the scan reads; see score_wave
    const int i = (W == 0 ? 0 : 32) + c, j0 = (W == 0 ? 16 : 48) + 4 * g;
    store4(P + i * C + j0, 0.f, 0.f, 0.f, 0.f);
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
  //   [0, 3 TILE) bf16 : tiles a | b | qe   (the fp32 g staging [C][DK] aliases the start)
  //   [3 TILE, ..) fp32: A [C][CP]
  // after the scores: T (fp32) takes the qe tile, the v tile takes the b tile, T diag(beta)
  // (bf16) takes A.
  static_assert(C * CP * 4 <= TILE * 2 && C * DK * 4 <= 3 * TILE * 2 && C * TPB * 2 <= C * CP * 4, "LDS aliasing");
  __shared__ __attribute__((aligned(16))) bf16 tiles[3 * TILE];
  __shared__ __attribute__((aligned(16))) float As[C * CP];
  __shared__ __attribute__((aligned(16))) float Bs[C];
  bf16* at = tiles;
  bf16* bt = tiles + TILE;
  bf16* qt = tiles + 2 * TILE;
  float* gsm = reinterpret_cast<float*>(tiles);
  float* Ts = reinterpret_cast<float*>(qt);
  bf16* vt = bt;
  bf16* Tb = reinterpret_cast<bf16*>(As);

  const int m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const size_t row0 = (size_t)m * C;
  // this thread's 16-byte vectors: rows rb + 16 i (i = 0..3), columns vc .. vc+7
  const int rb = tid >> 4, vc = (tid & 15) * 8;

  // ---- 1. loads; g to LDS ----------------------------------------------------------------
  uint4 kr[4], qr[4], vr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const size_t e = (row0 + rb + 16 * i) * DK + vc;
    kr[i] = *reinterpret_cast<const uint4*>(a.k + e);
    qr[i] = *reinterpret_cast<const uint4*>(a.q + e);
    vr[i] = *reinterpret_cast<const uint4*>(a.v + (row0 + rb + 16 * i) * DV + vc);
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
    bf16x8 av, bv, qv, rv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float eg = __expf(G[i][e]), ebg = __expf(-G[i][e]);
      const float kf = (float)kx[e];
      av[e] = (bf16)(kf * eg);
      bv[e] = (bf16)(kf * ebg);
      qv[e] = (bf16)(a.scale * (float)qx[e] * eg);
      rv[e] = (bf16)(kf * ebg * egl[e]);
    }
    const size_t e0 = (row0 + r) * DK + vc;
    *reinterpret_cast<bf16x8*>(a.QE + e0) = qv;
    *reinterpret_cast<bf16x8*>(a.KR + e0) = rv;
    // swizzled row tiles: two 4-element groups per vector
    const int o0 = kda_swz<KP>(r, vc), o1 = kda_swz<KP>(r, vc + 4);
    *reinterpret_cast<bf16x4*>(at + o0) = bf16x4{av[0], av[1], av[2], av[3]};
    *reinterpret_cast<bf16x4*>(at + o1) = bf16x4{av[4], av[5], av[6], av[7]};
    *reinterpret_cast<bf16x4*>(bt + o0) = bf16x4{bv[0], bv[1], bv[2], bv[3]};
    *reinterpret_cast<bf16x4*>(bt + o1) = bf16x4{bv[4], bv[5], bv[6], bv[7]};
    *reinterpret_cast<bf16x4*>(qt + o0) = bf16x4{qv[0], qv[1], qv[2], qv[3]};
    *reinterpret_cast<bf16x4*>(qt + o1) = bf16x4{qv[4], qv[5], qv[6], qv[7]};
  }
  lds_barrier();

  // ---- 4. scores: A = beta_i (a b^T) strictly lower (fp32, LDS), P = causal_incl(qe b^T) --------
  // The 20 lower 16x16 blocks are split over the waves as in the GDN chunk-local kernel (lists
  // that share operand rows: b rows on the j side of every block, a rows for A and qe rows for
  // P on the i side), each product formed transposed so a lane holds four consecutive columns
  // of one score row.
  switch (__builtin_amdgcn_readfirstlane(w)) {
    case 0: kda_score_wave<C, KP, CP, 0>(at, bt, qt, As, Bs, a.P + (size_t)m * C * C); break;
    case 1: kda_score_wave<C, KP, CP, 1>(at, bt, qt, As, Bs, a.P + (size_t)m * C * C); break;
    case 2: kda_score_wave<C, KP, CP, 2>(at, bt, qt, As, Bs, a.P + (size_t)m * C * C); break;
    default: kda_score_wave<C, KP, CP, 3>(at, bt, qt, As, Bs, a.P + (size_t)m * C * C); break;
  }
  lds_barrier();

  // ---- 5. T = (I + A)^-1 (fp32) ------------------------------------------------------------
  unit_lower_inverse64(As, Ts);

  // ---- 6. T diag(beta) as bf16 (in A's space), the v tile (in b's space) -------------------
  for (int u = tid; u < C * C / 4; u += 256) {
    const int i = u / (C / 4), j0 = (u % (C / 4)) * 4;
    const floatx4 t4 = *reinterpret_cast<const floatx4*>(Ts + i * CP + j0);
    const floatx4 b4 = *reinterpret_cast<const floatx4*>(Bs + j0);
    store4(Tb + i * TPB + j0, (j0 <= i) ? t4[0] * b4[0] : 0.f, (j0 + 1 <= i) ? t4[1] * b4[1] : 0.f,
           (j0 + 2 <= i) ? t4[2] * b4[2] : 0.f, (j0 + 3 <= i) ? t4[3] * b4[3] : 0.f);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rb + 16 * i;
    const bf16x8 vx = __builtin_bit_cast(bf16x8, vr[i]);
    *reinterpret_cast<bf16x4*>(vt + kda_swz<KP>(r, vc)) = bf16x4{vx[0], vx[1], vx[2], vx[3]};
    *reinterpret_cast<bf16x4*>(vt + kda_swz<KP>(r, vc + 4)) = bf16x4{vx[4], vx[5], vx[6], vx[7]};
  }
  lds_barrier();

  // ---- 7. W^T = a^T (T diag beta)^T, U^T = v^T (T diag beta)^T ------------------------------
  // Wave w owns the 16-row blocks mb = 2w, 2w+1 of the dk (dv) dimension.  A operand: a^T / v^T
  // by transpose reads (lane (c,g) gets rows j = 32kb + 4g + 0..3 and +16 of column 16mb + c);
  // B operand: rows i = 16nb + c of T diag(beta) at the same (permuted) j.  The D registers hold
  // W[i][16mb + 4g .. +3]: four consecutive columns, one 8-byte store.
  {
    floatx4 accW[2][4], accU[2][4];
#pragma unroll
    for (int mb2 = 0; mb2 < 2; ++mb2)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        accW[mb2][nb] = zero4();
        accU[mb2][nb] = zero4();
      }
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
          const bf16* vp = vt + 32 * kb * KP + tr + 16 * mb;
          accW[mb2][nb] = mfma_bf16(cat8(lds_read_tr(ap), lds_read_tr(ap + 16 * KP)), tbv, accW[mb2][nb]);
          accU[mb2][nb] = mfma_bf16(cat8(lds_read_tr(vp), lds_read_tr(vp + 16 * KP)), tbv, accU[mb2][nb]);
        }
      }
    }
#pragma unroll
    for (int mb2 = 0; mb2 < 2; ++mb2)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const size_t e = ((size_t)m * C + 16 * nb + c) * DK + 16 * (2 * w + mb2) + 4 * g;
        const floatx4 x = accW[mb2][nb], y = accU[mb2][nb];
        store4(a.W + e, x[0], x[1], x[2], x[3]);
        store4(a.U + e, y[0], y[1], y[2], y[3]);
      }
  }
}

// ============================== stage 2: scan + output ==============================

struct KdaScanArgs {
  const bf16* W;        // [BH*NC, C, DK]
  const bf16* U;        // [BH*NC, C, DV]
  const bf16* QE;       // [BH*T, DK]
  const bf16* KR;       // [BH*T, DK]
  const bf16* P;        // [BH*NC, C, C]
  const float* DEC;     // [BH*NC, DK]
  const float* h0;      // [BH, DK, DV] or null
  float* o;             // [BH*T, DV]
  float* h_final;       // [BH, DK, DV] or null
  int BH;
  int NC;
};

// LDS image of one chunk (C = 64, DK = 128, 32-column tile).  W, QE, KR: the GDN k / q layout
// (288-byte rows, Swz<2,3>); P: 144-byte rows, half swap on row bit 3; U: the tile's 32 columns,
// 96-byte rows, read transposed.
template <int C, int DK, int TW>
struct KdaStage {
  static constexpr int KP = DK + 16;
  static constexpr int TP = C + 8;
  static constexpr int UP = TW + 16;
  bf16 ws[C * KP];
  bf16 qs[C * KP];
  bf16 ks[C * KP];
  bf16 ps[C * TP];
  bf16 us[C * UP];
  float dec[DK];
};

// Loader register image of one chunk: W, QE, KR 1024 vectors each; P 512; U 256; dec 32.
template <int NLW>
struct KdaRegs {
  static constexpr int NK = 1024 / (64 * NLW), NP = 512 / (64 * NLW), NU = 256 / (64 * NLW);
  uint4 w[NK], q[NK], k[NK], p[NP], u[NU];
  uint4 d;
};

template <int C, int DK, int DV, int NLW>
__global__ __launch_bounds__(64 * (2 + NLW)) __attribute__((amdgpu_waves_per_eu(1, 1)))
void kda_scan_kernel(KdaScanArgs a) {
  constexpr int NWC = 2, TW = 32;
  using Stage = KdaStage<C, DK, TW>;
  using Regs = KdaRegs<NLW>;
  constexpr int KP = Stage::KP, TP = Stage::TP, UP = Stage::UP;
  constexpr int NT = DV / TW;
  static_assert(C == 64 && DK == 128 && NLW == 4, "tile shapes of the KDA scan kernel are fixed");

  __shared__ __attribute__((aligned(16))) Stage st[2];
  constexpr int OP = TW + 4;
  __shared__ __attribute__((aligned(16))) float ost[2][C * OP];

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
  const int NC = a.NC;
  const int col0 = tile * TW;
  const uint32_t Tlen = (uint32_t)NC * C;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.W + (size_t)bh * Tlen * DK, Tlen * DK * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.QE + (size_t)bh * Tlen * DK, Tlen * DK * 2);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.KR + (size_t)bh * Tlen * DK, Tlen * DK * 2);
  const __amdgpu_buffer_rsrc_t ru = make_rsrc(a.U + (size_t)bh * Tlen * DV, Tlen * DV * 2);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.P + (size_t)bh * NC * C * C, (uint32_t)NC * C * C * 2);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.DEC + (size_t)bh * NC * DK, (uint32_t)NC * DK * 4);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.o + (size_t)bh * Tlen * DV, Tlen * DV * 4);

  if (w >= NWC) {
    // =========================== loader waves ===========================
    const int lt = tid - 64 * NWC;
    __builtin_amdgcn_s_setprio(3);
    // W / QE / KR rows (16 vectors per row): row = a0 | a1<<1 | i0<<2 | a2<<3 | a3<<4 | i1<<5
    const int ka = lt >> 4, kvec = lt & 15;
    const int krow_l = (ka & 3) | (((ka >> 2) & 1) << 3) | ((ka >> 3) << 4);
    const uint32_t k_voff = (uint32_t)(krow_l * DK + kvec * 8) * 2;
    const int k_lds = krow_l * KP + 8 * (kvec ^ ((ka >> 2) & 1));   // Swz<2,3>: slot ^= row bit 3
    auto krow_i = [](int i) -> int { return ((i & 1) << 2) | (((i >> 1) & 1) << 5); };
    // P rows (8 vectors per row): row = a0 | a1<<1 | a2<<2 | i0<<3 | a3<<4 | a4<<5
    const int ta = lt >> 3, tvec = lt & 7;
    const int prow_l = (ta & 7) | ((ta >> 3) << 4);
    const uint32_t p_voff = (uint32_t)(prow_l * C + tvec * 8) * 2;
    const int p_lds = prow_l * TP + 8 * tvec;
    auto prow_i = [](int i) -> int { return (i & 1) << 3; };
    // U tile (4 vectors per row): row = lt >> 2, columns col0 + 8 (lt & 3)
    const int urow = lt >> 2, uvec = lt & 3;
    const uint32_t u_voff = (uint32_t)(urow * DV + col0 + uvec * 8) * 2;
    // dec: 32 vectors of 4 floats (lanes 32.. repeat lanes 0..31: no branch around a load)
    const uint32_t d_voff = (uint32_t)(lt & 31) * 16;

    auto load_chunk = [&](Regs& r, int ch) {
      const uint32_t k_s = (uint32_t)ch * C * DK * 2;
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const uint32_t rowi = krow_i(i);
        r.w[i] = buf_load16(rw, k_voff, k_s + rowi * DK * 2);
        r.q[i] = buf_load16(rq, k_voff, k_s + rowi * DK * 2);
        r.k[i] = buf_load16(rk, k_voff, k_s + rowi * DK * 2);
      }
      const uint32_t p_s = (uint32_t)ch * C * C * 2;
#pragma unroll
      for (int i = 0; i < Regs::NP; ++i) r.p[i] = buf_load16(rp, p_voff, p_s + prow_i(i) * C * 2);
      const uint32_t u_s = (uint32_t)ch * C * DV * 2;
#pragma unroll
      for (int i = 0; i < Regs::NU; ++i) r.u[i] = buf_load16(ru, u_voff, u_s + (uint32_t)(16 * NLW * i) * DV * 2);
      r.d = buf_load16(rd, d_voff, (uint32_t)ch * DK * 4);
    };
    auto store_chunk = [&](Stage& s, const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const int rowi = krow_i(i);
        put16(s.ws + k_lds + rowi * KP, r.w[i], (i & 1) != 0);
        put16(s.qs + k_lds + rowi * KP, r.q[i], (i & 1) != 0);
        put16(s.ks + k_lds + rowi * KP, r.k[i], (i & 1) != 0);
      }
#pragma unroll
      for (int i = 0; i < Regs::NP; ++i) put16(s.ps + p_lds + prow_i(i) * TP, r.p[i], (i & 1) != 0);
#pragma unroll
      for (int i = 0; i < Regs::NU; ++i) *reinterpret_cast<uint4*>(s.us + (urow + 16 * NLW * i) * UP + 8 * uvec) = r.u[i];
      if (lt < 32) *reinterpret_cast<uint4*>(s.dec + 4 * lt) = r.d;
    };
    const int orow_l = lt >> 3, oseg = lt & 7;
    const uint32_t o_voff = (uint32_t)(orow_l * DV + col0 + 4 * oseg) * 4;
    auto store_o = [&](const float* os, int ch) {
#pragma unroll
      for (int i = 0; i < (C * TW / 4) / (64 * NLW); ++i) {
        const int row = orow_l + (64 * NLW / 8) * i;
        const floatx4 x = *reinterpret_cast<const floatx4*>(os + row * OP + 4 * oseg);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), ro, o_voff + (uint32_t)((64 * NLW / 8) * i * DV) * 4,
                                               (uint32_t)ch * C * DV * 4, kCachePolicyNT);   // streamed
      }
    };
    // Same schedule as the GDN scan kernel: step j (between barriers j and j+1) issues the loads
    // of chunk j+2, writes out the o of chunk j-2, stores chunk j into buffer j & 1; three
    // register sets rotate.  The compute waves pass NC + 1 barriers (one before the first chunk,
    // one after each); so do the loaders: barrier 1, the steps 1 .. NC-1, barrier NC + 1.  With
    // one chunk there is no step and no o two chunks back.
    const int last = NC - 1;
    Regs r0, r1, r2;
    auto step = [&](Regs& ld, Regs& sd, int j, bool with_o) {
      load_chunk(ld, min(j + 2, last));
      if (with_o) store_o(ost[j & 1], j - 2);
      store_chunk(st[j & 1], sd);
      lds_barrier();
    };
    load_chunk(r0, 0);
    load_chunk(r1, min(1, last));
    load_chunk(r2, min(2, last));
    store_chunk(st[0], r0);
    lds_barrier();                                       // barrier 1
    if (NC > 1) {
      step(r0, r1, 1, false);
      int j = 2;
      for (; j + 2 < NC; j += 3) {
        step(r1, r2, j, true);
        step(r2, r0, j + 1, true);
        step(r0, r1, j + 2, true);
      }
      if (j < NC) step(r1, r2, j, true);
      if (j + 1 < NC) step(r2, r0, j + 1, true);
      store_o(ost[NC & 1], NC - 2);
    }
    lds_barrier();                                       // barrier NC + 1
    store_o(ost[(NC - 1) & 1], NC - 1);
  } else {
    // =========================== compute waves ===========================
    const int cbase = 16 * w;
    const int colw = col0 + cbase + c;
    const int kq_rd = c * KP + 4 * (g ^ ((c >> 2) & 3));             // W / QE rows, permuted K
    const int kt_rd = (4 * g + (c >> 2)) * KP + 4 * ((c & 3) ^ g);   // transposed A of KR^T
    const int tp_rd = c * TP + 4 * (g ^ (c >> 3));                   // P rows, permuted K
    const int u_rd = (4 * g + (c >> 2)) * UP + cbase + 4 * (c & 3);  // transposed U column
    const int o_lds = c * OP + cbase + 4 * g;

    floatx4 S[DK / 16];
#pragma unroll
    for (int r = 0; r < DK / 16; ++r)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + colw] : 0.f;

    auto compute_chunk = [&](const Stage& s, int ch) {
      bf16x8 SB[DK / 32];
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) SB[kb] = pack8(S[2 * kb], S[2 * kb + 1]);
      floatx4 Y[4], QT[4], VN[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        Y[mb] = zero4();
        QT[mb] = zero4();
      }
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const bf16* wp = s.ws + kq_rd + 16 * mb * KP + 32 * kb;
          const bf16* qp = s.qs + kq_rd + 16 * mb * KP + 32 * kb;
          const bf16x8 wa = cat8(*reinterpret_cast<const bf16x4*>(wp), *reinterpret_cast<const bf16x4*>(wp + 16));
          const bf16x8 qa = cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16));
          Y[mb] = mfma_bf16(wa, SB[kb], Y[mb]);        // (W S)[t][n]
          QT[mb] = mfma_bf16(SB[kb], qa, QT[mb]);      // (QE S)^T[n][t]
        }
      }
      // v_new = U - W S
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16x4 uu = lds_read_tr(s.us + u_rd + 16 * mb * UP);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) VN[mb][ii] = (float)uu[ii] - Y[mb][ii];
      }
      const bf16x8 VB0 = pack8(VN[0], VN[1]), VB1 = pack8(VN[2], VN[3]);
      // o^T = v_new^T P^T + (QE S)^T
      float* os = ost[ch & 1];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16* pp = s.ps + tp_rd + 16 * mb * TP;
        const bf16x8 p0 = cat8(*reinterpret_cast<const bf16x4*>(pp), *reinterpret_cast<const bf16x4*>(pp + 16));
        floatx4 OT = mfma_bf16(VB0, p0, QT[mb]);
        if (mb >= 2) {
          const bf16x8 p1 = cat8(*reinterpret_cast<const bf16x4*>(pp + 32), *reinterpret_cast<const bf16x4*>(pp + 48));
          OT = mfma_bf16(VB1, p1, OT);
        }
        *reinterpret_cast<floatx4*>(os + o_lds + 16 * mb * OP) = OT;
      }
      // S <- e^{G_last} (.) S + KR^T v_new  (the decay scales the state rows = key channels)
#pragma unroll
      for (int r = 0; r < DK / 16; ++r) {
        const floatx4 d4 = *reinterpret_cast<const floatx4*>(s.dec + 16 * r + 4 * g);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) S[r][ii] *= d4[ii];
      }
#pragma unroll
      for (int r = 0; r < DK / 16; ++r) {
        const bf16* k0 = s.ks + kt_rd + 16 * r;
        const bf16x8 a0 = cat8(lds_read_tr(k0), lds_read_tr(k0 + 16 * KP));
        const bf16x8 a1 = cat8(lds_read_tr(k0 + 32 * KP), lds_read_tr(k0 + 48 * KP));
        const floatx4 acc = mfma_bf16(a0, VB0, S[r]);
        S[r] = mfma_bf16(a1, VB1, acc);
      }
    };

    lds_barrier();
    for (int ch = 0; ch < NC; ch += 2) {
      compute_chunk(st[0], ch);
      lds_barrier();
      if (ch + 1 >= NC) break;
      compute_chunk(st[1], ch + 1);
      lds_barrier();
    }
    if (a.h_final) {
#pragma unroll
      for (int r = 0; r < DK / 16; ++r)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          a.h_final[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + colw] = S[r][ii];
    }
  }
}

}  // namespace pf
