// K2 for bf16 operands on gfx950 — the state scan fused with the output stage, with the chunk
// operands staged row-major only and read transposed through LDS transpose loads.
//
// Same mathematics and workgroup decomposition as the generic kernel (pf_scan_output.h): one
// workgroup per (chain bh, 32-column dv tile), NWC compute waves (16*NCB state columns each, the
// state register-resident in fp32) and NLW loader waves, two LDS chunk buffers, one barrier per
// chunk.  Per chunk c, with v, beta, G, T and the pre-scaled P from K1:
//
//   Y = k S,  r = beta v - beta e^G Y,  v_new = T r,
//   o = scale e^G (q S) + P v_new,  S <- e^{G_last} S + k^T (v_new e^{G_last - G}).
//
// Work moved off the compute waves (which bound the kernel: every chunk is a serial chain of
// dependent MFMAs, and the waves stall between instructions, so instructions per chunk are the
// currency):
//   * the loader stages beta*v in fp32, already transposed to the accumulator layout, and the gate
//     tables beta e^G, scale e^G, e^{G_last - G} (the exponentials once per row, not per lane);
//   * the per-chunk decay e^{G_last} of the state is deferred: the compute waves hold
//     S~ = S / f with a running factor f folded into the gate tables, and multiply the state only
//     when the loader decides to renormalise (f below e^-60, or the last chunk, so the final state
//     is exact) — 32 multiplies per chunk become a rare branch;
//   * the output is produced transposed (o^T = v_new^T P^T + (S^T q^T) scale e^G, the same
//     registers with the MFMA operands swapped), so each lane holds four consecutive output
//     columns and stores them as one 16-byte vector.
//
// gfx950 specifics:
//   * k^T, the A operand of the state update, is read straight out of the row-major k tile with
//     ds_read_b64_tr_b16: within each 16-lane group, lane l receives element (l & 3) of the
//     4-element words addressed by lanes 4j + (l >> 2), j = 0..3.  Lane (c, g) therefore
//     addresses k[32kb + 4g + (c >> 2)][16r + 4(c & 3) .. +3] and receives
//     k[32kb + 4g + j][16r + c], j = 0..3 — the permuted-K operand of the MFMA chain.
//   * every bf16 tile is written by the loader as whole 16-byte row vectors and swizzled (Swz) so
//     that the row writes, the MFMA operand reads and the transpose reads are all free of LDS bank
//     conflicts; the loader's lane-to-row mapping makes the swizzle's half-swap bit a compile-time
//     constant, so no data is shuffled;
//   * global traffic uses raw buffer loads/stores with a per-chain descriptor: the chunk advance
//     is a scalar offset, the lane part a constant vector offset.
#pragma once

#include "pf_scan_output.h"

namespace pf {

typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Store of a 16-byte row vector into a Swz<RS,1> tile slot whose 8-byte halves are swapped when
// `swap` (a compile-time constant at every call): the halves change places in registers and the
// LDS store stays one conflict-free 16-byte write (two 8-byte stores would conflict).
__device__ __forceinline__ void put16(bf16* dst, const uint4& x, bool swap) {
  *reinterpret_cast<uint4*>(dst) = swap ? make_uint4(x.z, x.w, x.x, x.y) : x;
}

// Transposed 8-byte LDS read (see the header comment); p is an LDS address.
__device__ __forceinline__ bf16x4 lds_read_tr(const bf16* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(const_cast<bf16*>(p)));
  return __builtin_bit_cast(bf16x4, v);
}

__device__ __forceinline__ bf16x8 cat8(const bf16x4& lo, const bf16x4& hi) {
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ bf16x8 pack8(const floatx4& d0, const floatx4& d1) {
  return bf16x8{(bf16)d0[0], (bf16)d0[1], (bf16)d0[2], (bf16)d0[3],
                (bf16)d1[0], (bf16)d1[1], (bf16)d1[2], (bf16)d1[3]};
}

__device__ __forceinline__ floatx4 mfma_bf16(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// LDS image of one chunk, C = 64, DK = 128, tile width TW = 32 or 16.
template <int C, int DK, int TW>
struct TrStage {
  static constexpr int KP = DK + 16;   // k, q: Swz<2,3>
  static constexpr int TP = C + 8;     // T, P: Swz<3,1>
  static constexpr int BP = C + 4;     // beta v, fp32, transposed: [tile column][row], 4-row
                                       // groups swizzled: group' = group ^ 2 (column >> 3)
  bf16 ks[C * KP];
  bf16 qs[C * KP];
  bf16 ts[C * TP];
  bf16 ps[C * TP];
  float bv[TW * BP];
  float BEG[C];   // beta_t e^{G_t} f_c
  float EGS[C];   // scale e^{G_t} f_c
  float EL[C];    // e^{G_last - G_t} / f_{c+1}
  float DL[4];    // [0] factor for the state at this chunk's update, [1] nonzero: apply it
};

// Loader register image of one chunk; NLW loader waves share the tile (k, q: 1024 vectors;
// T, P: 512; v: 8 TW — per thread NK, NTP, NV; with fewer v vectors than loader lanes the extra
// lanes repeat a vector's load and skip its store).
template <int NLW, int TW>
struct TrRegs {
  static constexpr int NK = 1024 / (64 * NLW), NTP = 512 / (64 * NLW);
  static constexpr int NV = (8 * TW + 64 * NLW - 1) / (64 * NLW);
  uint4 k[NK], q[NK], t[NTP], p[NTP], v[NV];
  float vb[NV];   // beta of each v row this lane stages
  float g, b;
};

#ifndef PF_TR_LOADER_PRIO
#define PF_TR_LOADER_PRIO 3
#endif

// Renormalisation threshold of the deferred state decay (log of the smallest factor kept).
constexpr float kLogFactorFloor = -60.f;

template <int C, int DK, int DV, int NWC, int NLW, int NCB>
__global__ __launch_bounds__(64 * (NWC + NLW)) __attribute__((amdgpu_waves_per_eu(1, 1)))
void scan_output_tr_kernel(ScanOutArgs a) {
  constexpr int TW = 16 * NWC * NCB;
  using Stage = TrStage<C, DK, TW>;
  using Regs = TrRegs<NLW, TW>;
  constexpr int KP = Stage::KP, TP = Stage::TP, BP = Stage::BP;
  constexpr int NT = DV / TW;
  static_assert(C == 64 && DK == 128 && (TW == 32 || TW == 16) && (NLW == 2 || NLW == 4),
                "tile shapes of the transpose-read kernel: C 64, DK 128, 32- or 16-column tile");

  __shared__ __attribute__((aligned(16))) Stage st[2];
  // o of chunk c (fp32, [C][OP]) is staged in ost[c & 1] by the compute waves and written to HBM
  // by the loader waves one interval later, so the compute waves never issue a vector-memory
  // instruction (theirs would queue behind the loader's loads and stall the MFMA chain).
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
  const uint32_t Tlen = (uint32_t)NC * C;            // tokens per chain

  // per-chain buffer descriptors (every offset below is relative to the chain's first element)
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(static_cast<const bf16*>(a.k) + (size_t)bh * Tlen * DK, Tlen * DK * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(static_cast<const bf16*>(a.q) + (size_t)bh * Tlen * DK, Tlen * DK * 2);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(static_cast<const bf16*>(a.v) + (size_t)bh * Tlen * DV, Tlen * DV * 2);
  const __amdgpu_buffer_rsrc_t rt = make_rsrc(static_cast<const bf16*>(a.Tm) + (size_t)bh * NC * C * C, (uint32_t)NC * C * C * 2);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(static_cast<const bf16*>(a.P) + (size_t)bh * NC * C * C, (uint32_t)NC * C * C * 2);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.o + (size_t)bh * Tlen * DV, Tlen * DV * 4);
  const float* Gc = a.G + (size_t)bh * Tlen;          // always written by K1
  const float* Bc = a.beta + (size_t)bh * Tlen;

  if (w >= NWC) {
    // =========================== loader waves ===========================
    // (the gate tables are filled by loader threads lt < C, i.e. the first loader wave)
    const int lt = tid - 64 * NWC;                       // 0 .. 64*NLW-1
#if PF_TR_LOADER_PRIO
    // loader waves share SIMDs with the compute waves: let their few instructions go first
    __builtin_amdgcn_s_setprio(PF_TR_LOADER_PRIO);
#endif
    const float oscale = *a.scale;
    // Row mappings: the lane part of each row index is fixed per thread, the vector index i
    // supplies the bits that decide the swizzle's half swap (so the swap is compile-time).
    // k / q (16 vectors per row): vec = lt & 15, a = lt >> 4;
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
    // T / P (8 vectors per row): vec = lt & 7, a = lt >> 3;
    //   NLW 2: row = a0 | a1<<1 | a2<<2 | i0<<3 | a3<<4 | i1<<5
    //   NLW 4: row = a0 | a1<<1 | a2<<2 | i0<<3 | a3<<4 | a4<<5
    const int ta = lt >> 3, tvec = lt & 7;
    const int trow_l = (ta & 7) | ((ta >> 3) << 4);
    const uint32_t tp_voff = (uint32_t)(trow_l * C + tvec * 8) * 2;
    const int tp_lds = trow_l * TP + 8 * tvec;
    auto trow_i = [](int i) -> int { return NLW == 2 ? ((i & 1) << 3) | (((i >> 1) & 1) << 5) : ((i & 1) << 3); };
    // (T's upper-right quadrant, rows < 32 and columns >= 32, is staged with the rest of each
    // 128-byte row but never used: the products of rows 0..31 stop at K block 0, and K1 leaves it
    // unwritten.)
    // v (TW / 8 vectors per row of the tile): vector u = lt + 64 NLW i, row = u / (TW / 8),
    // columns 8 vvec .. +7; lanes past the tile's 8 TW vectors repeat one (load only)
    constexpr int VPR = TW / 8, V_VECS = C * VPR, VSTEP = 64 * NLW / VPR;
    const int vu = lt % V_VECS;
    const bool v_owner = V_VECS >= 64 * NLW || lt < V_VECS;
    const int vrow_l = vu / VPR, vvec = vu % VPR;
    const uint32_t v_voff = (uint32_t)(vrow_l * DV + col0 + vvec * 8) * 2;
    float Lrun = 0.f;                                   // log of the state factor f_c

    auto load_chunk = [&](Regs& r, int ch) {
      const uint32_t kq_s = (uint32_t)ch * C * DK * 2;
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const uint32_t rowi = krow_i(i);
        r.k[i] = buf_load16(rk, kq_voff, kq_s + rowi * DK * 2);
        r.q[i] = buf_load16(rq, kq_voff, kq_s + rowi * DK * 2);
      }
      const uint32_t tp_s = (uint32_t)ch * C * C * 2;
#pragma unroll
      for (int i = 0; i < Regs::NTP; ++i) {
        const uint32_t rowi = trow_i(i);
        r.t[i] = buf_load16(rt, tp_voff, tp_s + rowi * C * 2);
        r.p[i] = buf_load16(rp, tp_voff, tp_s + rowi * C * 2);
      }
      const uint32_t v_s = (uint32_t)ch * C * DV * 2;
#pragma unroll
      for (int i = 0; i < Regs::NV; ++i) {
        r.v[i] = buf_load16(rv, v_voff, v_s + (uint32_t)(VSTEP * i) * DV * 2);
        r.vb[i] = Bc[(size_t)ch * C + vrow_l + VSTEP * i];
      }
      // every lane loads (lanes past the first loader wave repeat its rows): no branch around a
      // load, so the compiler's wait counts stay exact and two chunks stay in flight
      r.g = Gc[(size_t)ch * C + (lt & (C - 1))];
      r.b = Bc[(size_t)ch * C + (lt & (C - 1))];
    };
    auto store_chunk = [&](Stage& s, const Regs& r, int ch) {
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {                // halves already in swizzled order
        const int rowi = krow_i(i);
        put16(s.ks + kq_lds + rowi * KP, r.k[i], (i & 1) != 0);
        put16(s.qs + kq_lds + rowi * KP, r.q[i], (i & 1) != 0);
      }
#pragma unroll
      for (int i = 0; i < Regs::NTP; ++i) {
        const int rowi = trow_i(i);
        put16(s.ts + tp_lds + rowi * TP, r.t[i], (i & 1) != 0);
        put16(s.ps + tp_lds + rowi * TP, r.p[i], (i & 1) != 0);
      }
      if (v_owner) {
#pragma unroll
        for (int i = 0; i < Regs::NV; ++i) {
          const int row = vrow_l + VSTEP * i;
          const bf16x8 x = __builtin_bit_cast(bf16x8, r.v[i]);
          const int prow = (((row >> 2) ^ (2 * vvec)) << 2) | (row & 3);
#pragma unroll
          for (int e = 0; e < 8; ++e) s.bv[(vvec * 8 + e) * BP + prow] = (float)x[e] * r.vb[i];
        }
      }
      // gate tables with the deferred state factor f_c = e^{Lrun}
      const float gl = __shfl(r.g, C - 1);                // G_last (log of the chunk decay)
      const float Ln = Lrun + gl;                         // log(e^{G_last} f_c)
      const bool renorm = Ln < kLogFactorFloor || ch == NC - 1;
      const float Lnext = renorm ? 0.f : Ln;
      if (lt < C) {
        const float eg = __expf(r.g + Lrun);
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

    // o rows of a staged chunk: TW / 4 16-byte vectors per row, C TW / (256 NLW) per thread
    constexpr int OPR = TW / 4;
    const int orow_l = lt / OPR, oseg = lt % OPR;
    const uint32_t o_voff = (uint32_t)(orow_l * DV + col0 + 4 * oseg) * 4;
    auto store_o = [&](const float* os, int ch) {
#pragma unroll
      for (int i = 0; i < (C * TW / 4) / (64 * NLW); ++i) {
        const int row = orow_l + (64 * NLW / OPR) * i;
        const floatx4 x = *reinterpret_cast<const floatx4*>(os + row * OP + 4 * oseg);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), ro, o_voff + (uint32_t)((64 * NLW / OPR) * i * DV) * 4,
                                               (uint32_t)ch * C * DV * 4, 0);
      }
    };

    // Barrier j (j = 1 .. NC+1) follows the compute of chunk j-2.  Step j (between barriers j and
    // j+1, j = 1 .. NC-1) first issues the loads of chunk j+2, then writes out the o of chunk
    // j-2, then stores chunk j (loaded two steps earlier) into buffer j & 1.  Three register sets
    // rotate, so a chunk's loads have two whole steps to land; the loop body is straight-line
    // with one back edge (conditional code inside it makes the compiler's wait counts
    // conservative); past the end the loads repeat the last chunk.
    const int last = NC - 1;
    Regs r0, r1, r2;
    auto step = [&](Regs& ld, Regs& sd, int j, bool with_o) {
      load_chunk(ld, min(j + 2, last));
      if (with_o) store_o(ost[j & 1], j - 2);
      store_chunk(st[j & 1], sd, j);
      lds_barrier();
    };
    load_chunk(r0, 0);
    load_chunk(r1, min(1, last));
    load_chunk(r2, min(2, last));
    store_chunk(st[0], r0, 0);
    lds_barrier();                                       // barrier 1
    step(r0, r1, 1, false);                              // the host launches NC >= 2 only
    int j = 2;
    for (; j + 2 < NC; j += 3) {
      step(r1, r2, j, true);
      step(r2, r0, j + 1, true);
      step(r0, r1, j + 2, true);
    }
    if (j < NC) step(r1, r2, j, true);
    if (j + 1 < NC) step(r2, r0, j + 1, true);
    store_o(ost[NC & 1], NC - 2);
    lds_barrier();                                       // barrier NC + 1
    store_o(ost[(NC - 1) & 1], NC - 1);
  } else {
    // =========================== compute waves ===========================
    // Wave w owns NCB blocks of 16 state columns; every LDS A operand it reads (k, q, T, P, k^T)
    // feeds the NCB blocks' MFMAs.
    const int cbase = w * 16 * NCB;                      // first tile column of this wave
    const int colw = col0 + cbase + c;                   // column of block cb: colw + 16 cb
    // per-lane LDS element offsets (see the swizzle derivations in the header comment)
    const int kq_rd = c * KP + 4 * (g ^ ((c >> 2) & 3));             // k / q rows, permuted K
    const int kt_rd = (4 * g + (c >> 2)) * KP + 4 * ((c & 3) ^ g);   // transposed A of k^T
    const int tp_rd = c * TP + 4 * (g ^ (c >> 3));                   // T / P rows, permuted K
    const int bv_col = cbase + c;                                    // beta v column (tile)
    // transposed output: lane holds token 16 mb + c, columns 4g .. 4g+3 of its 16-column block
    const int o_lds = c * OP + cbase + 4 * g;

    floatx4 S[NCB][DK / 16];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
      for (int r = 0; r < DK / 16; ++r)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          S[cb][r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + colw + 16 * cb] : 0.f;

    auto compute_chunk = [&](const Stage& s, int ch) {
      // bf16 state, one per 32-row K block: the B operand of k S and the A operand of S^T q^T
      bf16x8 SB[NCB][DK / 32];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int kb = 0; kb < DK / 32; ++kb) SB[cb][kb] = pack8(S[cb][2 * kb], S[cb][2 * kb + 1]);
      floatx4 Y[NCB][4], QT[NCB][4], R[NCB][4], VN[NCB][4];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          Y[cb][mb] = zero4();
          QT[cb][mb] = zero4();
        }
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const bf16* kp = s.ks + kq_rd + 16 * mb * KP + 32 * kb;
          const bf16* qp = s.qs + kq_rd + 16 * mb * KP + 32 * kb;
          const bf16x8 ka = cat8(*reinterpret_cast<const bf16x4*>(kp), *reinterpret_cast<const bf16x4*>(kp + 16));
          const bf16x8 qa = cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16));
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            Y[cb][mb] = mfma_bf16(ka, SB[cb][kb], Y[cb][mb]);      // (k S)[t][n]
            QT[cb][mb] = mfma_bf16(SB[cb][kb], qa, QT[cb][mb]);    // (q S)^T[n][t]
          }
        }
      }
      // r = beta v - beta e^G f Y~
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const floatx4 beg = *reinterpret_cast<const floatx4*>(s.BEG + 16 * mb + 4 * g);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          const int n = bv_col + 16 * cb;
          const floatx4 bvv = *reinterpret_cast<const floatx4*>(s.bv + n * BP + 4 * ((4 * mb + g) ^ (2 * (n >> 3))));
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) R[cb][mb][ii] = fmaf(-beg[ii], Y[cb][mb][ii], bvv[ii]);
        }
      }
      // v_new = T r (lower triangular: K block 1 only for rows 32..63)
      bf16x8 RB0[NCB], RB1[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        RB0[cb] = pack8(R[cb][0], R[cb][1]);
        RB1[cb] = pack8(R[cb][2], R[cb][3]);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16* tp = s.ts + tp_rd + 16 * mb * TP;
        const bf16x8 t0 = cat8(*reinterpret_cast<const bf16x4*>(tp), *reinterpret_cast<const bf16x4*>(tp + 16));
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) VN[cb][mb] = mfma_bf16(t0, RB0[cb], zero4());
        if (mb >= 2) {
          const bf16x8 t1 = cat8(*reinterpret_cast<const bf16x4*>(tp + 32), *reinterpret_cast<const bf16x4*>(tp + 48));
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) VN[cb][mb] = mfma_bf16(t1, RB1[cb], VN[cb][mb]);
        }
      }
      // o^T = v_new^T P^T + (scale e^G f) (S~^T q^T): v_new is the A operand as it stands
      bf16x8 VB0[NCB], VB1[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        VB0[cb] = pack8(VN[cb][0], VN[cb][1]);
        VB1[cb] = pack8(VN[cb][2], VN[cb][3]);
      }
      float* os = ost[ch & 1];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16* pp = s.ps + tp_rd + 16 * mb * TP;
        const bf16x8 p0 = cat8(*reinterpret_cast<const bf16x4*>(pp), *reinterpret_cast<const bf16x4*>(pp + 16));
        const float egs = s.EGS[16 * mb + c];
        floatx4 OT[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) OT[cb] = mfma_bf16(VB0[cb], p0, zero4());
        if (mb >= 2) {
          const bf16x8 p1 = cat8(*reinterpret_cast<const bf16x4*>(pp + 32), *reinterpret_cast<const bf16x4*>(pp + 48));
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) OT[cb] = mfma_bf16(VB1[cb], p1, OT[cb]);
        }
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          floatx4 val;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) val[ii] = fmaf(egs, QT[cb][mb][ii], OT[cb][ii]);
          *reinterpret_cast<floatx4*>(os + o_lds + 16 * mb * OP + 16 * cb) = val;
        }
      }
      // S~ <- (renormalise ? e^{G_last} f_c : 1) S~ + k^T (v_new e^{G_last - G} / f_{c+1})
      bf16x8 UB0[NCB], UB1[NCB];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const floatx4 el = *reinterpret_cast<const floatx4*>(s.EL + 16 * mb + 4 * g);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) VN[cb][mb][ii] *= el[ii];
      }
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        UB0[cb] = pack8(VN[cb][0], VN[cb][1]);
        UB1[cb] = pack8(VN[cb][2], VN[cb][3]);
      }
      if (s.DL[1] != 0.f) {
        const float m = s.DL[0];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
          for (int r = 0; r < DK / 16; ++r) S[cb][r] *= m;
      }
#pragma unroll
      for (int r = 0; r < DK / 16; ++r) {
        const bf16* k0 = s.ks + kt_rd + 16 * r;
        const bf16x8 a0 = cat8(lds_read_tr(k0), lds_read_tr(k0 + 16 * KP));
        const bf16x8 a1 = cat8(lds_read_tr(k0 + 32 * KP), lds_read_tr(k0 + 48 * KP));
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          const floatx4 acc = mfma_bf16(a0, UB0[cb], S[cb][r]);
          S[cb][r] = mfma_bf16(a1, UB1[cb], acc);
        }
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
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int r = 0; r < DK / 16; ++r)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii)
            a.h_final[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + colw + 16 * cb] = S[cb][r][ii];
    }
  }
}

}  // namespace pf
