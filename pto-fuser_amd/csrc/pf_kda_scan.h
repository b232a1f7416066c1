// KDA stage 2 for bf16 operands on gfx950: the state scan fused with the output, every chunk
// split over four MFMA waves (one per SIMD) by token block and state row block, two workgroup
// barriers per chunk.
//
// Workgroup = one chain bh x one slice of 32 state columns (NT = 2 column tiles of 16).  Stage 1
// (kda_local_kernel) leaves per chunk the gated images W = T diag(beta) (k e^G),
// TB = T diag(beta), QE = scale q e^G, KB = k e^-G and the chunk decay e^{G_last} per key
// channel, so the recurrence needs no T r step:
//
//   U = TB v,  P = causal_incl(QE KB^T),  Y = W S,  v_new = U - Y,  o = QE S + P v_new,
//   S <- e^{G_last} (.) (S + KB^T v_new).
//
// U and P do not depend on the state: each wave forms its 16 rows of U (TB's rows of its tokens
// against the slice's v tile, 2 or 4 products) beside Y, and the ten 16 x 16 tiles of P are
// spread three, three, two, two over the waves (each tile P^T = KB_jb QE_ib^T, a wave's own QE
// rows from the registers of Y's phase), the tiles (2,0), (3,0) and (3,1) reaching their
// owners through PX.  The gates are inside QE and KB, so the tiles need only the causal mask.
//
// Compute wave w owns tokens 16w..16w+15 of every chunk (its rows of Y, v_new and o) and state
// rows 32w..32w+31 (fp32, MFMA D layout, in registers for the whole chain).  The two products
// that contract over what another wave owns go through LDS exchange tiles in the MFMA operand
// layout, one 16-byte slot per lane (every exchange read one contiguous 1 KiB ds_read_b128):
//
//   SB  the bf16 state, [4 row blocks][NT][64 lanes]: each wave publishes its 32 rows after the
//       update (its two 16-row D blocks are exactly one permuted-K B fragment); every wave reads
//       all four as the B operand of W S and the A operand of (QE S)^T;
//   VX  v_new in bf16, [2 token blocks of 32][NT][64 lanes]: wave w fills half (w & 1) of block
//       w >> 1; it is the A operand of o^T = v_new^T P^T (causal: blocks 0..w>>1) and the B
//       operand of the state update (both blocks).
//
//   phase 1  U = TB v, Y = W S~, (QE S~)^T, v_new = U - Y -> VX; P's tiles                 B1
//   phase 2  o^T = v_new^T P^T + (QE S~)^T -> HBM; S~ <- e^{G_last} (.) (S~ + KB^T VX) -> SB  B2
//
// SB is read in phase 1 and written in phase 2, VX the other way round, so one copy of each
// suffices.  Per wave and chunk: 2 or 4 products for U, 8 for W S, 8 for (QE S)^T, 8 or 12 for
// P's tiles, 2 or 4 for P v_new and 8 for the update.  The per-channel decay is one multiply of the 32 state values a lane holds.
//
// Four loader waves own the loads: chunk c+3's loads issued while the compute waves work on chunk
// c (three rotating register sets), chunk c+1 written into the free half of a double-buffered LDS
// stage (W, QE, KB rows swizzled for the permuted-K operand reads and the transposed KB^T reads,
// the v tile row-major, the decay), W, v and the decay in the first phase, QE and KB in the
// second.  TB has one LDS copy: it is read only in phase 1, so chunk c+1's TB is written in the
// second phase of interval c.  The compute waves store their o rows
// themselves: two 16-byte stores per lane, non-temporal, after lanes c and c + 8 swap the halves
// of a token's 128-byte row so that every store instruction writes whole lines.
#pragma once

#include "pf_gfx950.h"
#include "pf_kda.h"

namespace pf {

// LDS image of one KDA chunk (C = 64, DK = 128, NCOL = 32 columns).
template <int C, int DK, int NCOL>
struct KdaSplitStage {
  static constexpr int KP = DK + 16;   // W, QE, KB rows: Swz<2,3>
  static constexpr int TP = C + 8;     // TB rows (the single copy outside the stage): Swz<3,1>
  static constexpr int UP = NCOL + 8;  // v tile rows (row-major, read transposed)
  bf16 ws[C * KP];
  bf16 qs[C * KP];
  bf16 ks[C * KP];
  bf16 vs[C * UP];
  float dec[DK];
};

// Loader register image of one chunk (W, QE, KB: 1024 16-byte vectors each; TB: 512; v: 8 NCOL;
// the decay: 32).
template <int NLW, int NCOL>
struct KdaSplitRegs {
  static constexpr int NK = 1024 / (64 * NLW), NTR = 512 / (64 * NLW);
  static constexpr int NV = (8 * NCOL + 64 * NLW - 1) / (64 * NLW);
  uint4 w[NK], q[NK], k[NK], t[NTR], u[NV];
  uint4 d;
};

template <int C, int DK, int DV, int NLW>
__global__ __launch_bounds__(64 * (4 + NLW)) __attribute__((amdgpu_waves_per_eu(2, 2)))
void kda_scan_split_kernel(KdaScanArgs a) {
  constexpr int NT = 2, NCOL = 16 * NT;
  using Stage = KdaSplitStage<C, DK, NCOL>;
  using Regs = KdaSplitRegs<NLW, NCOL>;
  constexpr int KP = Stage::KP, TP = Stage::TP, UP = Stage::UP;
  constexpr int NS = DV / NCOL;                 // slices per chain
  constexpr int FRAG = 64 * 8;                  // bf16 elements of one operand fragment
  static_assert(C == 64 && DK == 128 && DV == 128 && NLW == 4,
                "tile shapes of the KDA split scan kernel: C 64, DK = DV 128, 32 columns");

  __shared__ __attribute__((aligned(16))) Stage st[2];
  __shared__ __attribute__((aligned(16))) bf16 TBs[C * TP];        // TB of the current chunk
  __shared__ __attribute__((aligned(16))) bf16 SB[4 * NT * FRAG];
  __shared__ __attribute__((aligned(16))) bf16 VX[2 * NT * FRAG];
  __shared__ __attribute__((aligned(16))) bf16 PX[3 * 64 * 4];   // P tiles (2,0) (3,0) (3,1)

  int bh, slice;
  const int bid = blockIdx.x;
  if (a.BH % 8 == 0) {  // the slices of one chain share an XCD (dispatch is round-robin on XCDs)
    const int grp = bid / (8 * NS), within = bid % (8 * NS);
    bh = grp * 8 + (within % 8);
    slice = within / 8;
  } else {
    bh = bid / NS;
    slice = bid % NS;
  }
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int NC = a.NC;
  const int col0 = slice * NCOL;
  const uint32_t Tlen = (uint32_t)NC * C;

  if (w >= 4) {
    // =========================== loader waves ===========================
    const int lt = tid - 256;                            // 0 .. 64*NLW-1
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.W + (size_t)bh * Tlen * DK, Tlen * DK * 2);
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.QE + (size_t)bh * Tlen * DK, Tlen * DK * 2);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.KB + (size_t)bh * Tlen * DK, Tlen * DK * 2);
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(a.v + (size_t)bh * Tlen * DV, Tlen * DV * 2);
    const __amdgpu_buffer_rsrc_t rtb = make_rsrc(a.TB + (size_t)bh * NC * C * C, (uint32_t)NC * C * C * 2);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.DEC + (size_t)bh * NC * DK, (uint32_t)NC * DK * 4);
    // W / QE / KB rows (16 vectors of 8 per row): vec = lt & 15, a = lt >> 4; the vector index i
    // supplies the row bits that decide the swizzle's half swap, so the swap is compile-time:
    // row = a0 | a1<<1 | i0<<2 | a2<<3 | a3<<4 | i1<<5
    const int ka = lt >> 4, kvec = lt & 15;
    const int krow_l = (ka & 3) | (((ka >> 2) & 1) << 3) | ((ka >> 3) << 4);
    const uint32_t k_voff = (uint32_t)(krow_l * DK + kvec * 8) * 2;
    const int k_lds = krow_l * KP + 8 * (kvec ^ ((ka >> 2) & 1));   // Swz<2,3>: slot ^= row bit 3
    auto krow_i = [](int i) -> int { return ((i & 1) << 2) | (((i >> 1) & 1) << 5); };
    // TB rows (8 vectors per row): vec = lt & 7, a = lt >> 3;
    // row = a0 | a1<<1 | a2<<2 | i0<<3 | a3<<4 | a4<<5
    const int ta = lt >> 3, tvec = lt & 7;
    const int prow_l = (ta & 7) | ((ta >> 3) << 4);
    const uint32_t p_voff = (uint32_t)(prow_l * C + tvec * 8) * 2;
    const int p_lds = prow_l * TP + 8 * tvec;
    auto prow_i = [](int i) -> int { return (i & 1) << 3; };
    // v tile (NCOL / 8 vectors per row): vector u = lt + 64 NLW i
    constexpr int VPR = NCOL / 8, VSTEP = 64 * NLW / VPR;
    static_assert(C * VPR == 64 * NLW * Regs::NV, "the v tile divides over the loader lanes");
    const int urow_l = lt / VPR, uvec = lt % VPR;
    const uint32_t u_voff = (uint32_t)(urow_l * DV + col0 + uvec * 8) * 2;
    // decay: 32 vectors of 4 floats (lanes 32.. repeat lanes 0..31: no branch around a load)
    const uint32_t d_voff = (uint32_t)(lt & 31) * 16;

    auto load_wq = [&](Regs& r, int ch) {
      const uint32_t k_s = (uint32_t)ch * C * DK * 2;
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const uint32_t rowi = krow_i(i);
        r.w[i] = buf_load16(rw, k_voff, k_s + rowi * DK * 2);
        r.q[i] = buf_load16(rq, k_voff, k_s + rowi * DK * 2);
      }
    };
    auto load_kpud = [&](Regs& r, int ch) {
      const uint32_t k_s = (uint32_t)ch * C * DK * 2;
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) r.k[i] = buf_load16(rk, k_voff, k_s + krow_i(i) * DK * 2);
      const uint32_t p_s = (uint32_t)ch * C * C * 2;
#pragma unroll
      for (int i = 0; i < Regs::NTR; ++i) r.t[i] = buf_load16(rtb, p_voff, p_s + prow_i(i) * C * 2);
      const uint32_t u_s = (uint32_t)ch * C * DV * 2;
#pragma unroll
      for (int i = 0; i < Regs::NV; ++i) r.u[i] = buf_load16(ru, u_voff, u_s + (uint32_t)(VSTEP * i) * DV * 2);
      r.d = buf_load16(rd, d_voff, (uint32_t)ch * DK * 4);
    };
    auto store_wpud = [&](Stage& s, const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) put16(s.ws + k_lds + krow_i(i) * KP, r.w[i], (i & 1) != 0);
#pragma unroll
      for (int i = 0; i < Regs::NV; ++i)
        *reinterpret_cast<uint4*>(s.vs + (urow_l + VSTEP * i) * UP + uvec * 8) = r.u[i];
      if (lt < 32) *reinterpret_cast<uint4*>(s.dec + 4 * lt) = r.d;
    };
    auto store_qk = [&](Stage& s, const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        put16(s.qs + k_lds + krow_i(i) * KP, r.q[i], (i & 1) != 0);
        put16(s.ks + k_lds + krow_i(i) * KP, r.k[i], (i & 1) != 0);
      }
    };
    auto store_tb = [&](const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NTR; ++i) put16(TBs + p_lds + prow_i(i) * TP, r.t[i], (i & 1) != 0);
    };

    // Interval j (the compute waves work on chunk j from stage j & 1): chunk j+3's loads go into
    // the register set that held chunk j, chunk j+1 (loaded two intervals earlier) into stage
    // (j+1) & 1.  Chunk m lives in register set m % 3; past the end the loads repeat the last
    // chunk.  Every interval is straight-line code, so the compiler's wait counts stay exact and
    // two chunks stay in flight.
    const int last = NC - 1;
    Regs r0, r1, r2;
    auto interval = [&](Regs& ld, Regs& nx, int j) {
      const int nl = min(j + 3, last);
      Stage& sn = st[(j + 1) & 1];
      load_wq(ld, nl);
      store_wpud(sn, nx);
      lds_barrier();                                     // B1
      load_kpud(ld, nl);
      store_qk(sn, nx);
      store_tb(nx);                                      // chunk j's TB was read before B1
      lds_barrier();                                     // B2
    };
    load_wq(r0, 0);
    load_kpud(r0, 0);
    load_wq(r1, min(1, last));
    load_kpud(r1, min(1, last));
    load_wq(r2, min(2, last));
    load_kpud(r2, min(2, last));
    store_wpud(st[0], r0);
    store_qk(st[0], r0);
    store_tb(r0);
    lds_barrier();                                       // start: stage 0 and SB ready
    if (NC > 1) {
      interval(r0, r1, 0);
      int j = 1;
      for (; j + 3 < NC; j += 3) {                       // intervals j..j+2 write chunks j+1..j+3
        interval(r1, r2, j);
        interval(r2, r0, j + 1);
        interval(r0, r1, j + 2);
      }
      // 1 <= NC - j <= 3 intervals remain, the last of which writes no chunk
      if (j + 1 < NC) interval(r1, r2, j);
      if (j + 2 < NC) interval(r2, r0, j + 1);
    }
    lds_barrier();                                       // the last interval writes no chunk
    lds_barrier();
  } else {
    // =========================== compute waves ===========================
    const int cw = __builtin_amdgcn_readfirstlane(w);   // wave-uniform
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.o + (size_t)bh * Tlen * DV, Tlen * DV * 4);
    const int tok0 = 16 * cw;                            // this wave's token block
    // per-lane LDS element offsets
    const int kq_rd = (tok0 + c) * KP + 4 * (g ^ ((c >> 2) & 3));          // W / QE rows
    const int kt_rd = (4 * g + (c >> 2)) * KP + 4 * ((c & 3) ^ g) + 32 * cw; // KB^T, rows 32cw..
    const int kj_rd = c * KP + 4 * (g ^ ((c >> 2) & 3));                   // KB / QE rows 16 b + c
    const int p_rd = (tok0 + c) * TP + 4 * (g ^ (c >> 3));                // TB rows
    const int v_rd = (4 * g + (c >> 2)) * UP + 4 * (c & 3);                // v, transposed read
    const int frag = lane * 8;                                             // lane's exchange slot
    const int xhalf = 4 * (cw & 1), xblk = cw >> 1;                        // this wave's VX slot

    floatx4 S[2][NT];                                    // rows 32cw + 16r + 4g + i, column c
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          S[r][nt][ii] = a.h0 ? a.h0[((size_t)bh * DK + 32 * cw + 16 * r + 4 * g + ii) * DV + col0 + 16 * nt + c] : 0.f;
    auto publish = [&]() {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        *reinterpret_cast<bf16x8*>(SB + (cw * NT + nt) * FRAG + frag) = pack8(S[0][nt], S[1][nt]);
    };
    publish();
    lds_barrier();                                       // start

    for (int ch = 0; ch < NC; ++ch) {
      const Stage& s = st[ch & 1];
      // ---- phase 1: U = TB v, Y = W S~, (QE S~)^T for this wave's 16 tokens, v_new = U - Y -> VX
      // U's products: A = TB rows of the wave's tokens (lower triangular: key blocks 0..cw>>1),
      // B = the v tile read transposed (lane (c, g): tokens 32 kb + 4 g + 0..3 and + 16,
      // column 16 nt + c), so lane (c, g) gets U[tok0 + 4 g + i][16 nt + c] like Y
      floatx4 U[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) U[nt] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (kb == 0 || cw >= 2) {
          const bf16* tp = TBs + p_rd + 32 * kb;
          const bf16x8 ta = cat8(*reinterpret_cast<const bf16x4*>(tp), *reinterpret_cast<const bf16x4*>(tp + 16));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const bf16* vp = s.vs + v_rd + 32 * kb * UP + 16 * nt;
            U[nt] = mfma_bf16(ta, cat8(lds_read_tr(vp), lds_read_tr(vp + 16 * UP)), U[nt]);
          }
        }
      }
      floatx4 Y[NT], QT[NT];
      bf16x8 qf[DK / 32];                                 // QE rows, kept for P's tiles
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) { Y[nt] = zero4(); QT[nt] = zero4(); }
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) {
        const bf16* wp = s.ws + kq_rd + 32 * kb;
        const bf16* qp = s.qs + kq_rd + 32 * kb;
        const bf16x8 wf = cat8(*reinterpret_cast<const bf16x4*>(wp), *reinterpret_cast<const bf16x4*>(wp + 16));
        qf[kb] = cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bf16x8 sb = *reinterpret_cast<const bf16x8*>(SB + (kb * NT + nt) * FRAG + frag);
          Y[nt] = mfma_bf16(wf, sb, Y[nt]);               // (W S~)[t][n]
          QT[nt] = mfma_bf16(sb, qf[kb], QT[nt]);         // (QE S~)^T[n][t]
        }
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        bf16x4 vb;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) vb[ii] = (bf16)(U[nt][ii] - Y[nt][ii]);
        *reinterpret_cast<bf16x4*>(VX + (xblk * NT + nt) * FRAG + frag + xhalf) = vb;
      }
      // P's tiles: tile (ib, jb) (query tokens 16 ib .., key tokens 16 jb .., jb <= ib) is
      // P^T = KB_jb QE_ib^T, so lane (c, g) holds P[16 ib + c][16 jb + 4 g + i]; tiles (ib, 2 kb)
      // and (ib, 2 kb + 1) together are the permuted-K B fragment of o^T = v_new^T P^T for key
      // block kb.  Three, three, two and two tiles per wave; a wave's own QE rows come from qf.
      bf16x4 ptl[4];                                     // this wave's own tiles (ib = cw)
      {
        auto tile = [&](int ib, int jb, bool own_q) -> bf16x4 {
          floatx4 acc = zero4();
#pragma unroll
          for (int kb = 0; kb < DK / 32; ++kb) {
            const bf16* kp = s.ks + kj_rd + 16 * jb * KP + 32 * kb;
            const bf16* qp = s.qs + kj_rd + 16 * ib * KP + 32 * kb;
            const bf16x8 kr = cat8(*reinterpret_cast<const bf16x4*>(kp), *reinterpret_cast<const bf16x4*>(kp + 16));
            const bf16x8 qr = own_q ? qf[kb] : cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16));
            acc = mfma_bf16(kr, qr, acc);
          }
          bf16x4 out;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) out[ii] = (bf16)((jb < ib || c >= 4 * g + ii) ? acc[ii] : 0.f);
          return out;
        };
        const bf16x4 z4 = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) ptl[jb] = z4;
        if (cw == 0) {
          ptl[0] = tile(0, 0, true);
          *reinterpret_cast<bf16x4*>(PX + (0 * 64 + lane) * 4) = tile(2, 0, false);
          *reinterpret_cast<bf16x4*>(PX + (1 * 64 + lane) * 4) = tile(3, 0, false);
        } else if (cw == 1) {
          ptl[0] = tile(1, 0, true);
          ptl[1] = tile(1, 1, true);
          *reinterpret_cast<bf16x4*>(PX + (2 * 64 + lane) * 4) = tile(3, 1, false);
        } else if (cw == 2) {
          ptl[1] = tile(2, 1, true);
          ptl[2] = tile(2, 2, true);
        } else {
          ptl[2] = tile(3, 2, true);
          ptl[3] = tile(3, 3, true);
        }
      }
      lds_barrier();                                     // B1
      // ---- phase 2: o^T = v_new^T P^T + (QE S~)^T -> HBM; S~ update -> SB ----
      {
        floatx4 OT[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) OT[nt] = QT[nt];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          if (kb == 0 || cw >= 2) {
            bf16x4 lo = ptl[2 * kb], hi = ptl[2 * kb + 1];
            if (kb == 0 && cw == 2) lo = *reinterpret_cast<const bf16x4*>(PX + (0 * 64 + lane) * 4);
            if (kb == 0 && cw == 3) {
              lo = *reinterpret_cast<const bf16x4*>(PX + (1 * 64 + lane) * 4);
              hi = *reinterpret_cast<const bf16x4*>(PX + (2 * 64 + lane) * 4);
            }
            const bf16x8 pb = cat8(lo, hi);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
              OT[nt] = mfma_bf16(*reinterpret_cast<const bf16x8*>(VX + (kb * NT + nt) * FRAG + frag), pb, OT[nt]);
          }
        }
        // lane (c, g) holds o[token tok0 + c][columns 16 nt + 4g .. +3]; a token's 32 columns
        // are one 128-byte line: lanes c and c + 8 of a row swap halves (DPP row rotate by 8) so
        // that each store instruction writes eight whole lines, tokens 0..7 then 8..15 of the
        // block, non-temporal (o is never read here)
        const bool hi = c >= 8;
        floatx4 sa, sb;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const float send = hi ? OT[0][ii] : OT[1][ii];
          const float recv = __int_as_float(__builtin_amdgcn_update_dpp(
              __float_as_int(send), __float_as_int(send), 0x128, 0xf, 0xf, false));   // row_ror:8
          sa[ii] = hi ? recv : OT[0][ii];                // token c & 7, columns 16 hi + 4g ..
          sb[ii] = hi ? OT[1][ii] : recv;                // token 8 + (c & 7), same columns
        }
        const uint32_t col = col0 + (hi ? 16 : 0) + 4 * g;
        const uint32_t ra = (uint32_t)(((size_t)ch * C + tok0 + (c & 7)) * DV + col) * 4;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sa), ro, ra, 0, kCachePolicyNT);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sb), ro, ra + 8 * DV * 4, 0,
                                               kCachePolicyNT);
      }
      // S~ <- e^{G_last} (.) (S~ + KB^T v_new)  (the decay scales the state rows = key channels;
      // e^{G_last} KB^T is the (k e^{G_last - G})^T of the recurrence)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const bf16* k0 = s.ks + kt_rd + 16 * r;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const bf16x8 at = cat8(lds_read_tr(k0 + 32 * kb * KP), lds_read_tr(k0 + (32 * kb + 16) * KP));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            S[r][nt] = mfma_bf16(at, *reinterpret_cast<const bf16x8*>(VX + (kb * NT + nt) * FRAG + frag), S[r][nt]);
        }
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const floatx4 d4 = *reinterpret_cast<const floatx4*>(s.dec + 32 * cw + 16 * r + 4 * g);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) S[r][nt][ii] *= d4[ii];
      }
      publish();
      lds_barrier();                                     // B2
    }
    if (a.h_final) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii)
            a.h_final[((size_t)bh * DK + 32 * cw + 16 * r + 4 * g + ii) * DV + col0 + 16 * nt + c] = S[r][nt][ii];
    }
  }
}

}  // namespace pf
