// Stage 2 for bf16 operands on gfx950: the state scan fused with the output stage, with every
// chunk's work split over four MFMA waves (one per SIMD) by token block and state row block.
//
// Workgroup = one chain bh x one slice of NCOL = 16*NT state columns.  Per chunk c (C = 64, DK =
// 128), with T = (I+A)^-1 and G from stage 1 and the gated causal score
// P = scale causal_incl(q k^T ⊙ e^{min(G_i - G_j, 0)}) formed here:
//
//   Y = k S,  r = beta v - beta e^G Y,  v_new = T r,
//   o = scale e^G (q S) + P v_new,  S <- e^{G_last} S + k^T (v_new e^{G_last - G}).
//
// Compute wave w (w = 0..3) owns tokens 16w..16w+15 of every chunk (its rows of Y, q S, r, v_new
// and o) and state rows 32w..32w+31 (fp32, MFMA D layout, for the whole chain).  The products
// that contract over what another wave owns go through small LDS exchange tiles in the MFMA
// operand layout, one 16-byte slot per lane, so every exchange read is one contiguous 1 KiB
// ds_read_b128 per fragment:
//
//   SB  the bf16 state, [4 row blocks][NT][64 lanes]: each wave publishes its 32 rows after the
//       update (its two 16-row D blocks are exactly one permuted-K B fragment), every wave reads
//       all four as the B operand of k S and the A operand of (q S)^T;
//   RX  r in bf16, [2 token blocks of 32][NT][64 lanes]: wave w fills half (w & 1) of block
//       w >> 1 (its D registers are the lane's permuted-K half); wave w reads blocks 0..w>>1 for
//       v_new = T r (T is lower triangular);
//   VX  v_new in bf16, the A operand of o^T = v_new^T P^T (causal: blocks 0..w>>1);
//   VXs v_new e^{G_last - G} / f in bf16, the B operand of the state update (both blocks).
//
// Three workgroup barriers per chunk: after RX is written (B1), after VX / VXs (B2), after the
// state is published and the chunk's stage buffer released (B3).  Per wave and chunk: 16 MFMAs
// for k S and q S, 2 or 4 for T r, 2 or 4 for P v_new, 8 for the update (NT = 2), and 8 or 12
// for the score: its ten 16x16 tiles (4 MFMAs each) are formed in phase B from the staged k and
// q rows (a wave's own blocks from its registers), three, three, two and two per wave so that the
// phase carries the same number of products on every wave; the tiles (2,0), (3,0) and (3,1)
// reach their owners through PX.  Their gates come from two small tables the loader writes per
// chunk (no exponential in the compute waves unless G rises or a block decays steeply).  P
// never goes through HBM, and stage 1 reads no q.
//
// NLW loader waves (the rest of the workgroup) own the loads: chunk c+3's loads issued while the
// compute waves work on chunk c (three rotating register sets), and chunk c+1 written into the
// free half of a double-buffered LDS stage (k and q rows swizzled for the permuted-K operand
// reads and the transposed k^T reads, T rows, the v tile row-major, per-token gate tables).
// Both are spread over the three phases of the interval (k's loads and LDS rows in the first,
// T's and q's loads, T's rows and the score gates in the second, v, the per-token gates and q's
// rows in the third), and the
// loader waves run at the default wave priority: a burst of loads or LDS writes issued at once,
// or at a raised priority, was measured to stall the compute waves sharing the SIMDs (one phase
// lost up to 1 000 cycles; q's loads in the first phase beside k's cost 5 % of the kernel).
// The compute waves store their o rows themselves, 16-byte stores: with 32-column slices two per
// lane, non-temporal, after lanes c and c + 8 swap the halves of a token's 128-byte row so that
// every store instruction writes whole lines; with 16-column slices one per lane, through the
// cache (the line's other half comes from the neighbouring slice's workgroup).  The loaders also carry the deferred state decay: the compute waves hold
// S~ = S / f with a running factor f folded into the gate tables, and multiply it back only when
// the loader flags a renormalisation (f below e^-60, or the last chunk, so the final state is
// exact).
#pragma once

#include <type_traits>

#include "pf_gfx950.h"
#include "pf_scan_args.h"

namespace pf {

// LDS image of one chunk.
template <int C, int DK, int NCOL>
struct SplitStage {
  static constexpr int KP = DK + 16;   // k, q rows: Swz<2,3>
  static constexpr int TP = C + 8;     // T rows: Swz<3,1>
  static constexpr int VP = NCOL + 8;  // v tile rows (bf16, row-major)
  bf16 ks[C * KP];
  bf16 qs[C * KP];
  bf16 ts[C * TP];
  bf16 vs[C * VP];
  float GT[C];    // G_t (within-chunk cumulative log decay)
  float BT[C];    // beta_t
  float BEG[C];   // beta_t e^{G_t} f_c
  float EGS[C];   // scale e^{G_t} f_c
  float EL[C];    // e^{G_last - G_t} / f_{c+1}
  float CB[C];    // score gate, key side: e^{G_{16 (t / 16)} - G_t}
  float RA[160];  // score gate, query side: scale e^{G_{16 ib + c} - G_{16 jb}}, [tile(ib, jb)][c]
  float DL[4];    // [0] factor for the state at this chunk's update, [1] nonzero: apply it,
                  // [2] nonzero: the score gates are evaluated per element (CB, RA not valid)
};

// Decay inside one 16-token block (G at its start minus G at its end) up to which the factored
// score gate e^{G_i - G_j} = e^{G_i - G_m} e^{G_m - G_j} is used: its key factor stays below e^80.
constexpr float kScoreGateSpan = 80.f;

// Loader register image of one chunk (k, q: 1024 16-byte vectors each; T: 512; v: 8 NCOL).
template <int NLW, int NCOL>
struct SplitRegs {
  static constexpr int NK = 1024 / (64 * NLW), NTR = 512 / (64 * NLW);
  static constexpr int NV = (8 * NCOL + 64 * NLW - 1) / (64 * NLW);
  uint4 k[NK], q[NK], t[NTR], v[NV];
  float g, b;
};

template <int C, int DK, int DV, int NT, int NLW>
__global__ __launch_bounds__(64 * (4 + NLW)) __attribute__((amdgpu_waves_per_eu(2, 2)))
void scan_split_kernel(ScanOutArgs a) {
  constexpr int NCOL = 16 * NT;
  using Stage = SplitStage<C, DK, NCOL>;
  using Regs = SplitRegs<NLW, NCOL>;
  constexpr int KP = Stage::KP, TP = Stage::TP, VP = Stage::VP;
  constexpr int NS = DV / NCOL;                 // slices per chain
  constexpr int FRAG = 64 * 8;                  // bf16 elements of one operand fragment
  static_assert(C == 64 && DK == 128 && (NT == 1 || NT == 2) && (NLW == 2 || NLW == 4),
                "tile shapes of the split scan kernel: C 64, DK 128, 16 or 32 columns");

  __shared__ __attribute__((aligned(16))) Stage st[2];
  __shared__ __attribute__((aligned(16))) bf16 SB[4 * NT * FRAG];
  __shared__ __attribute__((aligned(16))) bf16 RX[2 * NT * FRAG];
  __shared__ __attribute__((aligned(16))) bf16 VX[2 * NT * FRAG];
  __shared__ __attribute__((aligned(16))) bf16 VXs[2 * NT * FRAG];
  __shared__ __attribute__((aligned(16))) bf16 PX[3 * 64 * 4];   // score tiles (2,0) (3,0) (3,1)

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
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(static_cast<const bf16*>(a.k) + (size_t)bh * Tlen * DK, Tlen * DK * 2);
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(static_cast<const bf16*>(a.q) + (size_t)bh * Tlen * DK, Tlen * DK * 2);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(static_cast<const bf16*>(a.v) + (size_t)bh * Tlen * DV, Tlen * DV * 2);
    const __amdgpu_buffer_rsrc_t rt = make_rsrc(static_cast<const bf16*>(a.Tm) + (size_t)bh * NC * C * C, (uint32_t)NC * C * C * 2);
    const float* Gc = a.G + (size_t)bh * Tlen;
    const float* Bc = a.beta + (size_t)bh * Tlen;
    const float oscale = *a.scale;
    // k / q rows (16 vectors of 8 per row): vec = lt & 15, a = lt >> 4; the vector index i
    // supplies the row bits that decide the swizzle's half swap, so the swap is compile-time
    //   NLW 2: row = a0 | a1<<1 | i0<<2 | a2<<3 | i1<<4 | i2<<5
    //   NLW 4: row = a0 | a1<<1 | i0<<2 | a2<<3 | a3<<4 | i1<<5
    const int ka = lt >> 4, kvec = lt & 15;
    const int krow_l = (ka & 3) | (((ka >> 2) & 1) << 3) | (NLW == 4 ? ((ka >> 3) << 4) : 0);
    const uint32_t kq_voff = (uint32_t)(krow_l * DK + kvec * 8) * 2;
    const int kq_lds = krow_l * KP + 8 * (kvec ^ ((ka >> 2) & 1));   // Swz<2,3>: slot ^= row bit 3
    auto krow_i = [](int i) -> int {
      return NLW == 2 ? ((i & 1) << 2) | (((i >> 1) & 1) << 4) | (((i >> 2) & 1) << 5)
                      : ((i & 1) << 2) | (((i >> 1) & 1) << 5);
    };
    // T rows (8 vectors per row): vec = lt & 7, a = lt >> 3
    //   NLW 2: row = a0 | a1<<1 | a2<<2 | i0<<3 | a3<<4 | i1<<5
    //   NLW 4: row = a0 | a1<<1 | a2<<2 | i0<<3 | a3<<4 | a4<<5
    const int ta = lt >> 3, tvec = lt & 7;
    const int trow_l = (ta & 7) | ((ta >> 3) << 4);
    const uint32_t t_voff = (uint32_t)(trow_l * C + tvec * 8) * 2;
    const int t_lds = trow_l * TP + 8 * tvec;
    auto trow_i = [](int i) -> int { return NLW == 2 ? ((i & 1) << 3) | (((i >> 1) & 1) << 5) : ((i & 1) << 3); };
    // v tile (NCOL / 8 vectors per row): vector u = lt + 64 NLW i; lanes past the tile's vectors
    // repeat one (load only)
    constexpr int VPR = NCOL / 8, V_VECS = C * VPR, VSTEP = 64 * NLW / VPR;
    const int vu = lt % V_VECS;
    const bool v_owner = V_VECS >= 64 * NLW || lt < V_VECS;
    const int vrow_l = vu / VPR, vvec = vu % VPR;
    const uint32_t v_voff = (uint32_t)(vrow_l * DV + col0 + vvec * 8) * 2;
    float Lrun = 0.f;                                   // log of the state factor f_c

    auto load_kq = [&](Regs& r, int ch) {
      const uint32_t kq_s = (uint32_t)ch * C * DK * 2;
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const uint32_t rowi = krow_i(i);
        r.k[i] = buf_load16(rk, kq_voff, kq_s + rowi * DK * 2);
      }
    };
    auto load_q = [&](Regs& r, int ch) {
      const uint32_t kq_s = (uint32_t)ch * C * DK * 2;
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const uint32_t rowi = krow_i(i);
        r.q[i] = buf_load16(rq, kq_voff, kq_s + rowi * DK * 2);
      }
    };
    auto load_t = [&](Regs& r, int ch) {
      const uint32_t t_s = (uint32_t)ch * C * C * 2;
#pragma unroll
      for (int i = 0; i < Regs::NTR; ++i) {
        const uint32_t rowi = trow_i(i);
        r.t[i] = buf_load16(rt, t_voff, t_s + rowi * C * 2);
      }
    };
    auto load_vg = [&](Regs& r, int ch) {
      const uint32_t v_s = (uint32_t)ch * C * DV * 2;
#pragma unroll
      for (int i = 0; i < Regs::NV; ++i)
        r.v[i] = buf_load16(rv, v_voff, v_s + (uint32_t)(VSTEP * i) * DV * 2);
      // every lane loads (lanes past the first loader wave repeat its rows): no branch around a
      // load, so the compiler's wait counts stay exact
      r.g = Gc[(size_t)ch * C + (lt & (C - 1))];
      r.b = Bc[(size_t)ch * C + (lt & (C - 1))];
    };
    auto store_k = [&](Stage& s, const Regs& r) {       // halves already in swizzled order
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) put16(s.ks + kq_lds + krow_i(i) * KP, r.k[i], (i & 1) != 0);
    };
    auto store_q = [&](Stage& s, const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) put16(s.qs + kq_lds + krow_i(i) * KP, r.q[i], (i & 1) != 0);
    };
    auto store_t = [&](Stage& s, const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NTR; ++i) {
        const int rowi = trow_i(i);
        put16(s.ts + t_lds + rowi * TP, r.t[i], (i & 1) != 0);
      }
    };
    auto store_vg = [&](Stage& s, const Regs& r, int ch) {
      if (v_owner) {
#pragma unroll
        for (int i = 0; i < Regs::NV; ++i)
          *reinterpret_cast<uint4*>(s.vs + (vrow_l + VSTEP * i) * VP + vvec * 8) = r.v[i];
      }
      // gate tables with the deferred state factor f_c = e^{Lrun}
      const float gl = __shfl(r.g, C - 1);                // G_last (log of the chunk decay)
      const float Ln = Lrun + gl;                         // log(e^{G_last} f_c)
      const bool renorm = Ln < kLogFactorFloor || ch == NC - 1;
      const float Lnext = renorm ? 0.f : Ln;
      if (lt < C) {
        const float eg = __expf(r.g + Lrun);
        s.GT[lt] = r.g;
        s.BT[lt] = r.b;
        s.BEG[lt] = r.b * eg;
        s.EGS[lt] = oscale * eg;
        s.EL[lt] = __expf(gl - r.g - Lnext);
        if (lt == 0) {
          s.DL[0] = __expf(Ln);
          s.DL[1] = renorm ? 1.f : 0.f;
        }
      }
      Lrun = Lnext;
    };

    // Score gate tables of a chunk.  P[i][j] = scale e^{min(G_i - G_j, 0)} (q_i . k_j) for
    // j <= i; with G non-increasing through the chunk (every g <= 0) the clamp is inactive and,
    // with m = 16 jb the first token of j's block, e^{G_i - G_j} = RA (<= scale: i >= m) * CB[j]
    // (>= 1, at most e^kScoreGateSpan): two finite factors, and no exponential in the compute
    // waves.  Any other chunk (a g > 0, a steeper block, a non-finite G) sets DL[2] and takes the
    // per-element path.  Loader wave lw writes the RA column jb = lw (lanes = query tokens, G from
    // its own lane and the block starts read as scalars); wave 0 also CB and the flag.
    auto store_gates = [&](Stage& s, const Regs& r) {
      const int t = lt & (C - 1), lw = lt >> 6;
      float gb[4], ge[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        gb[b] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r.g), 16 * b));
        ge[b] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r.g), 16 * b + 15));
      }
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
        if (jb % NLW == lw && t >= 16 * jb)
          s.RA[score_tile_index(t >> 4, jb) * 16 + (t & 15)] = oscale * __expf(r.g - gb[jb]);
      if (lw == 0) {
        const float gblk = t < 16 ? gb[0] : t < 32 ? gb[1] : t < 48 ? gb[2] : gb[3];
        s.CB[t] = __expf(gblk - r.g);
        // G_{t-1} from the neighbouring lane (DPP wave shift right by one)
        const float gprev = __int_as_float(__builtin_amdgcn_update_dpp(
            __float_as_int(r.g), __float_as_int(r.g), 0x138, 0xf, 0xf, false));
        bool ok = t == 0 || r.g <= gprev;
#pragma unroll
        for (int b = 0; b < 4; ++b) ok = ok && gb[b] - ge[b] <= kScoreGateSpan;
        const bool fact = __all(ok);
        if (t == 0) s.DL[2] = fact ? 0.f : 1.f;
      }
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
      load_kq(ld, nl);
      store_k(sn, nx);
      lds_barrier();                                     // B1
      load_t(ld, nl);
      load_q(ld, nl);
      store_t(sn, nx);
      store_gates(sn, nx);
      lds_barrier();                                     // B2
      load_vg(ld, nl);
      store_vg(sn, nx, j + 1);
      store_q(sn, nx);
      lds_barrier();                                     // B3
    };
    auto final_interval = [&]() {                        // writes no chunk
      lds_barrier();
      lds_barrier();
      lds_barrier();
    };
    load_kq(r0, 0);
    load_q(r0, 0);
    load_t(r0, 0);
    load_vg(r0, 0);
    load_kq(r1, min(1, last));
    load_q(r1, min(1, last));
    load_t(r1, min(1, last));
    load_vg(r1, min(1, last));
    load_kq(r2, min(2, last));
    load_q(r2, min(2, last));
    load_t(r2, min(2, last));
    load_vg(r2, min(2, last));
    store_k(st[0], r0);
    store_q(st[0], r0);
    store_t(st[0], r0);
    store_gates(st[0], r0);
    store_vg(st[0], r0, 0);
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
    final_interval();
  } else {
    // =========================== compute waves ===========================
    const int cw = __builtin_amdgcn_readfirstlane(w);   // wave-uniform
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.o + (size_t)bh * Tlen * DV, Tlen * DV * 4);
    const int tok0 = 16 * cw;                            // this wave's token block
    // per-lane LDS element offsets
    const int kq_rd = (tok0 + c) * KP + 4 * (g ^ ((c >> 2) & 3));          // k / q rows
    const int kt_rd = (4 * g + (c >> 2)) * KP + 4 * ((c & 3) ^ g) + 32 * cw; // k^T, rows 32cw..
    const int t_rd = (tok0 + c) * TP + 4 * (g ^ (c >> 3));                // T rows
    const int kj_rd = c * KP + 4 * (g ^ ((c >> 2) & 3));                   // k / q rows 16 b + c
    const float oscale = *a.scale;
    const int v_rd = (tok0 + 4 * g + (c >> 2)) * VP + 4 * (c & 3);         // v, transposed read
    const int frag = lane * 8;                                             // lane's exchange slot
    const int xhalf = 4 * (cw & 1), xblk = cw >> 1;                        // this wave's RX/VX slot

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
      // ---- phase A: Y = k S~ and (q S~)^T for this wave's 16 tokens, r -> RX ----
      floatx4 Y[NT], QT[NT];
      bf16x8 kf[DK / 32], qf[DK / 32];                    // k, q rows, kept for the score
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) { Y[nt] = zero4(); QT[nt] = zero4(); }
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) {
        const bf16* kp = s.ks + kq_rd + 32 * kb;
        const bf16* qp = s.qs + kq_rd + 32 * kb;
        kf[kb] = cat8(*reinterpret_cast<const bf16x4*>(kp), *reinterpret_cast<const bf16x4*>(kp + 16));
        qf[kb] = cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bf16x8 sb = *reinterpret_cast<const bf16x8*>(SB + (kb * NT + nt) * FRAG + frag);
          Y[nt] = mfma_bf16(kf[kb], sb, Y[nt]);           // (k S~)[t][n]
          QT[nt] = mfma_bf16(sb, qf[kb], QT[nt]);         // (q S~)^T[n][t]
        }
      }
      {
        const floatx4 bt = *reinterpret_cast<const floatx4*>(s.BT + tok0 + 4 * g);
        const floatx4 beg = *reinterpret_cast<const floatx4*>(s.BEG + tok0 + 4 * g);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bf16x4 v4 = lds_read_tr(s.vs + v_rd + 16 * nt);
          bf16x4 rb;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) rb[ii] = (bf16)fmaf(-beg[ii], Y[nt][ii], bt[ii] * (float)v4[ii]);
          *reinterpret_cast<bf16x4*>(RX + (xblk * NT + nt) * FRAG + frag + xhalf) = rb;
        }
      }
      lds_barrier();                                     // B1
      // ---- phase B: v_new = T r for this wave's tokens -> VX, VXs ----
      floatx4 VN[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) VN[nt] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (kb == 0 || cw >= 2) {
          const bf16* tp = s.ts + t_rd + 32 * kb;
          const bf16x8 ta = cat8(*reinterpret_cast<const bf16x4*>(tp), *reinterpret_cast<const bf16x4*>(tp + 16));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            VN[nt] = mfma_bf16(ta, *reinterpret_cast<const bf16x8*>(RX + (kb * NT + nt) * FRAG + frag), VN[nt]);
        }
      }
      {
        const floatx4 el = *reinterpret_cast<const floatx4*>(s.EL + tok0 + 4 * g);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          bf16x4 vb, vs;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            vb[ii] = (bf16)VN[nt][ii];
            vs[ii] = (bf16)(VN[nt][ii] * el[ii]);
          }
          *reinterpret_cast<bf16x4*>(VX + (xblk * NT + nt) * FRAG + frag + xhalf) = vb;
          *reinterpret_cast<bf16x4*>(VXs + (xblk * NT + nt) * FRAG + frag + xhalf) = vs;
        }
      }
      // The causal score, formed here from the staged k and q rows instead of read from stage 1.
      // Tile (ib, jb) (query tokens 16 ib .., key tokens 16 jb .., jb <= ib) is P^T = k_jb q_ib^T,
      // so lane (c, g) holds P[16 ib + c][16 jb + 4 g + ii], and tiles (ib, 2 kb), (ib, 2 kb + 1)
      // together are the permuted-K B fragment of o^T = v_new^T P^T for key block kb.  Gate and
      // mask as in stage 1: P[i][j] = scale (q_i . k_j) e^{min(G_i - G_j, 0)} for j <= i.  The ten
      // tiles are spread three, three, two, two over the waves so that each wave's phase carries
      // the same number of products; (2,0), (3,0) (wave 0) and (3,1) (wave 1) reach their owners
      // through PX after B2.
      // A wave's own k and q rows (block cw) come from the registers of phase A, so every tile
      // reads at most one operand block from LDS.
      bf16x4 ptl[4];                                     // this wave's own tiles (ib = cw)
      {
        // one straight-line copy of the score block per gate path (a branch inside each tile
        // would keep the scheduler from overlapping one tile's gating with the next's products)
        const bool gate_exact = __builtin_amdgcn_readfirstlane(__float_as_int(s.DL[2])) != 0;
        auto score_tiles = [&](auto exact_tag) {
          constexpr bool kExact = decltype(exact_tag)::value;
          auto tile = [&](int ib, int jb, bool own_k, bool own_q) -> bf16x4 {
            floatx4 acc = zero4();
#pragma unroll
            for (int kb = 0; kb < DK / 32; ++kb) {
              const bf16* kp = s.ks + kj_rd + 16 * jb * KP + 32 * kb;
              const bf16* qp = s.qs + kj_rd + 16 * ib * KP + 32 * kb;
              const bf16x8 kr = own_k ? kf[kb] : cat8(*reinterpret_cast<const bf16x4*>(kp), *reinterpret_cast<const bf16x4*>(kp + 16));
              const bf16x8 qr = own_q ? qf[kb] : cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16));
              acc = mfma_bf16(kr, qr, acc);
            }
            bf16x4 out;
            if constexpr (!kExact) {
              const float ra = s.RA[score_tile_index(ib, jb) * 16 + c];
              const floatx4 cb = *reinterpret_cast<const floatx4*>(s.CB + 16 * jb + 4 * g);
#pragma unroll
              for (int ii = 0; ii < 4; ++ii)
                out[ii] = (bf16)((jb < ib || c >= 4 * g + ii) ? acc[ii] * (ra * cb[ii]) : 0.f);
            } else {
              const float gi = s.GT[16 * ib + c];
              const floatx4 gj = *reinterpret_cast<const floatx4*>(s.GT + 16 * jb + 4 * g);
#pragma unroll
              for (int ii = 0; ii < 4; ++ii) {
                const float keep = (jb < ib || c >= 4 * g + ii) ? oscale : 0.f;
                out[ii] = (bf16)(keep * acc[ii] * __expf(fminf(gi - gj[ii], 0.f)));
              }
            }
            return out;
          };
          if (cw == 0) {
            ptl[0] = tile(0, 0, true, true);
            *reinterpret_cast<bf16x4*>(PX + (0 * 64 + lane) * 4) = tile(2, 0, true, false);
            *reinterpret_cast<bf16x4*>(PX + (1 * 64 + lane) * 4) = tile(3, 0, true, false);
          } else if (cw == 1) {
            ptl[0] = tile(1, 0, false, true);
            ptl[1] = tile(1, 1, true, true);
            *reinterpret_cast<bf16x4*>(PX + (2 * 64 + lane) * 4) = tile(3, 1, true, false);
          } else if (cw == 2) {
            ptl[1] = tile(2, 1, false, true);
            ptl[2] = tile(2, 2, true, true);
          } else {
            ptl[2] = tile(3, 2, false, true);
            ptl[3] = tile(3, 3, true, true);
          }
        };
        const bf16x4 z4 = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) ptl[jb] = z4;
        if (gate_exact)
          score_tiles(std::true_type{});
        else
          score_tiles(std::false_type{});
      }
      lds_barrier();                                     // B2
      // ---- phase C: o^T = v_new^T P^T + scale e^G f (q S~)^T -> HBM; S~ update -> SB ----
      {
        floatx4 OT[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) OT[nt] = zero4();
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
        // lane (c, g) holds o[token tok0 + c][columns 16 nt + 4g .. +3]: one 16-byte store each,
        // non-temporal (o is never read here; streaming it past L2 leaves the cache to the k, q
        // and T lines the chain's other column slices read: 7 % of the kernel's time)
        const float egs = s.EGS[tok0 + c];
        if constexpr (NT == 2) {
          // a token's 32 columns are one 128-byte line: lanes c and c + 8 of a row swap halves
          // (DPP row rotate by 8) so that each store instruction writes eight whole lines, tokens
          // 0..7 then 8..15 of the block (two half-line stores reach memory apart when streamed)
          floatx4 v0, v1;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            v0[ii] = fmaf(egs, QT[0][ii], OT[0][ii]);
            v1[ii] = fmaf(egs, QT[1][ii], OT[1][ii]);
          }
          const bool hi = c >= 8;
          floatx4 sa, sb;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const float send = hi ? v0[ii] : v1[ii];
            const float recv = __int_as_float(__builtin_amdgcn_update_dpp(
                __float_as_int(send), __float_as_int(send), 0x128, 0xf, 0xf, false));   // row_ror:8
            sa[ii] = hi ? recv : v0[ii];                 // token c & 7, columns 16 hi + 4g ..
            sb[ii] = hi ? v1[ii] : recv;                 // token 8 + (c & 7), same columns
          }
          const uint32_t col = col0 + (hi ? 16 : 0) + 4 * g;
          const uint32_t ra = (uint32_t)(((size_t)ch * C + tok0 + (c & 7)) * DV + col) * 4;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sa), ro, ra, 0, kCachePolicyNT);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sb), ro, ra + 8 * DV * 4, 0,
                                                 kCachePolicyNT);
        } else {
          // 16-column slices: the other half of each 128-byte line comes from the neighbouring
          // slice's workgroup (same XCD), so o is stored through the cache, where the halves
          // meet before write-back (streamed, they reached memory apart: o written 12 % over its
          // size, at the same speed)
          const uint32_t ooff = (uint32_t)(((size_t)ch * C + tok0 + c) * DV + col0 + 4 * g) * 4;
          floatx4 val;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) val[ii] = fmaf(egs, QT[0][ii], OT[0][ii]);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, val), ro, ooff, 0, 0);
        }
      }
      if (s.DL[1] != 0.f) {
        const float m = s.DL[0];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) S[r][nt] *= m;
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const bf16* k0 = s.ks + kt_rd + 16 * r;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const bf16x8 at = cat8(lds_read_tr(k0 + 32 * kb * KP), lds_read_tr(k0 + (32 * kb + 16) * KP));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            S[r][nt] = mfma_bf16(at, *reinterpret_cast<const bf16x8*>(VXs + (kb * NT + nt) * FRAG + frag), S[r][nt]);
        }
      }
      publish();
      lds_barrier();                                     // B3
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
