// K2 — the inter-chunk state scan fused with the output stage.
//
// One workgroup per (chain bh = (b,h), dv tile of 16*NWC columns), NWC compute waves + 2 loader
// waves.  Compute wave w owns 16 columns of the state S[DK x 16], held in registers (fp32, MFMA
// D layout) for the whole sequential chunk loop; per-chunk snapshots are never written to HBM.
// Per chunk c:
//
//   Y     = k_c S                                    (A = k rows from LDS, B = S registers)
//   QS    = q_c S
//   r     = beta (v - e^G * Y)
//   v_new = T_c r          ( = U - W S  with W = T beta k e^G, U = T beta v; _gdn_full.py:79-84)
//   o_c   = scale * e^G * QS + P_c v_new   (P carries the scale from K1)  (_gdn_full.py:88-97)
//   S     = e^{G_last} S + k_c^T (v_new * e^{G_last - G})               (_gdn_full.py:86-87)
//
// T_c = (I+A)^-1, P_c (gated causal score) and G (within-chunk cumsum) come from K1.  Every
// product chains register to register through the permuted-K MFMA layout.
//
// Warp specialisation: the loader waves own all global loads.  They keep the operands of the
// next two chunks in flight in registers and write chunk c+1's LDS image (k row-major and
// transposed for the state update, q, T, P, the v tile transposed, G, beta) into the second of
// two LDS buffers while the compute waves work on chunk c from the first; one workgroup barrier
// per chunk swaps the roles of the buffers.  The compute waves touch global memory only to store
// o.  The tiles of one chain are mapped to the same XCD so the sibling workgroups' per-chunk
// k/q/T/P reads share one L2.
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
  const float* scale;   // device scalar: the output scale K1 applied to P (written by K1)
};

constexpr int kLoaderWaves = 2;

// LDS image of one chunk for a workgroup whose tile is TW columns wide.
template <typename E, int C, int DK, int TW>
struct ChunkStage {
  static constexpr int PE = 16 / sizeof(E);
  static constexpr int KP = DK + PE;   // k / q row pitch
  static constexpr int TP = C + PE;    // kT / T / P / vT row pitch
  E ks[C * KP];
  E qs[C * KP];
  E kts[DK * TP];
  E ts[C * TP];
  E ps[C * TP];
  E vts[TW * TP];
  float Bs[C];    // beta
  float BEG[C];   // beta e^{G_t}
  float EG[C];    // scale e^{G_t}
  float EL[C];    // e^{G_last - G_t}
  float DL[4];    // [0] = e^{G_last}
};

// Swizzle of each LDS tile (see Swz): bf16 tiles swap 8-byte halves by row bit 3 (k/q/T/P/vT)
// or permute all 16 groups by row bits 3..6 (kT, written transposed 8 rows apart); fp32 tiles
// are conflict-free unswizzled except kT.
template <typename E> struct StageSwz;
template <> struct StageSwz<bf16> {
  using Rows = Swz<3, 1>;     // ks, qs, ts, ps, vts
  using KT = Swz<3, 15>;      // kts
};
template <> struct StageSwz<float> {
  using Rows = Swz<0, 0>;
  using KT = Swz<3, 3>;
};

// Register image of one chunk's operands for one loader thread.  k and v move as units of 4
// tokens x one 16-byte vector so they can be written row-major and transposed.
template <typename E, int C, int DK, int TW>
struct ChunkRegs {
  static constexpr int NTHR = 64 * kLoaderWaves;
  static constexpr int VE = Vec16<E>::N;
  static constexpr int NK = (C / 4) * (DK / VE) / NTHR;     // k units per thread
  static constexpr int NQ = C * (DK / VE) / NTHR;           // q vectors per thread
  static constexpr int NTP = C * (C / VE) / NTHR;           // T (and P) vectors per thread
  static constexpr int VU = (C / 4) * (TW / VE);            // v units in the tile
  static constexpr int NV = (VU + NTHR - 1) / NTHR;         // v units per thread (ceil)
  static_assert((C / 4) * (DK / VE) % NTHR == 0 && C * (DK / VE) % NTHR == 0 &&
                    C * (C / VE) % NTHR == 0 && C <= NTHR,
                "chunk tile does not divide over the loader waves");
  uint4 k[NK][4];
  uint4 q[NQ];
  uint4 t[NTP];
  uint4 p[NTP];
  uint4 v[NV][4];
  float g, b, gl;
};

// A 16-byte row vector stored into a Swz<RS, 1> bf16 tile: the vector keeps its slot, its two
// 8-byte halves swap on rows whose bit RS is set.
__device__ __forceinline__ uint4 swap_halves_if(const uint4& x, bool swap) {
  return swap ? make_uint4(x.z, x.w, x.x, x.y) : x;
}

__device__ __forceinline__ uint32_t word_of(const uint4& x, int i) {
  return i == 0 ? x.x : i == 1 ? x.y : i == 2 ? x.z : x.w;
}

// Element e of each of four 16-byte row vectors (one per token of a unit), packed into one
// transposed LDS store.  Pure register arithmetic (e is a compile-time constant after unrolling).
__device__ __forceinline__ void store_col4(bf16* dst, const uint4* x, int e) {
  const int wi = e >> 1, sh = (e & 1) * 16;
  const uint32_t a0 = (word_of(x[0], wi) >> sh) & 0xFFFFu, a1 = (word_of(x[1], wi) >> sh) & 0xFFFFu;
  const uint32_t a2 = (word_of(x[2], wi) >> sh) & 0xFFFFu, a3 = (word_of(x[3], wi) >> sh) & 0xFFFFu;
  *reinterpret_cast<uint2*>(dst) = make_uint2(a0 | (a1 << 16), a2 | (a3 << 16));
}
__device__ __forceinline__ void store_col4(float* dst, const uint4* x, int e) {
  *reinterpret_cast<uint4*>(dst) =
      make_uint4(word_of(x[0], e), word_of(x[1], e), word_of(x[2], e), word_of(x[3], e));
}

// 16-byte row vector into a row-swizzled tile: the vector keeps its slot and, for a bf16 tile
// with RM = 1, its two 8-byte halves swap on rows whose bit RS is set (see Swz).
template <class SW, typename E>
__device__ __forceinline__ void put_row16(E* tile, int row, int col, int pitch, uint4 x) {
  static_assert(SW::rm <= 1, "a row swizzle may only swap the halves of a 16-byte vector");
  const bool swap = sizeof(E) == 2 && (((row >> SW::rs) & SW::rm) != 0);
  *reinterpret_cast<uint4*>(tile + row * pitch + col) = swap_halves_if(x, swap);
}

template <typename E, int C, int DK, int DV, int NWC, int NBUF>
__global__ __launch_bounds__(64 * (NWC + kLoaderWaves)) __attribute__((amdgpu_waves_per_eu(1, 1)))
void scan_output_kernel(ScanOutArgs a) {
  const float oscale = *a.scale;
  constexpr int TW = 16 * NWC;
  using Stage = ChunkStage<E, C, DK, TW>;
  using Regs = ChunkRegs<E, C, DK, TW>;
  constexpr int KP = Stage::KP;
  constexpr int TP = Stage::TP;
  constexpr int NT = DV / TW;
  constexpr int VE = Vec16<E>::N;
  constexpr int LTHR = Regs::NTHR;
  constexpr int KB = Mfma<E>::KB;
  constexpr int NKB_D = DK / KB;
  constexpr int NKB_C = C / KB;
  constexpr int MB = C / 16;
  static_assert(DV % TW == 0, "dv tile");
  static_assert(C % KB == 0 && C <= 64, "chunk size");
  static_assert(NBUF == 1 || NBUF == 2, "one or two LDS chunk buffers");

  __shared__ __attribute__((aligned(16))) Stage st[NBUF];

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
  const bool is_loader = w >= NWC;
  const int ltid = tid - 64 * NWC;           // loader thread index (valid when is_loader)
  const int col0 = tile * TW;
  const int col = col0 + w * 16 + c;         // this compute lane's dv column
  const size_t m0 = (size_t)bh * a.NC;

  const E* kbase = static_cast<const E*>(a.k);
  const E* qbase = static_cast<const E*>(a.q);
  const E* vbase = static_cast<const E*>(a.v);
  const E* tbase = static_cast<const E*>(a.Tm);
  const E* pbase = static_cast<const E*>(a.P);

  using RowsSwz = typename StageSwz<E>::Rows;
  using KTSwz = typename StageSwz<E>::KT;

  // ---- loader: global -> registers for chunk m -------------------------------------------------
  // k units are 4 tokens x one 16-byte vector, d fastest across lanes (coalesced rows); v units
  // are token-fastest so their transposed LDS writes of one row are contiguous.
  auto load_chunk = [&](Regs& r, size_t m) {
    const size_t tok0 = m * C;
    const E* kg = kbase + tok0 * DK;
#pragma unroll
    for (int i = 0; i < Regs::NK; ++i) {
      const int u = ltid + i * LTHR;
      const int t0 = (u / (DK / VE)) * 4, d0 = (u % (DK / VE)) * VE;
#pragma unroll
      for (int j = 0; j < 4; ++j) r.k[i][j] = *reinterpret_cast<const uint4*>(kg + (size_t)(t0 + j) * DK + d0);
    }
    const uint4* qg = reinterpret_cast<const uint4*>(qbase + tok0 * DK);
#pragma unroll
    for (int i = 0; i < Regs::NQ; ++i) r.q[i] = qg[ltid + i * LTHR];
    const uint4* tg = reinterpret_cast<const uint4*>(tbase + m * C * C);
    const uint4* pg = reinterpret_cast<const uint4*>(pbase + m * C * C);
#pragma unroll
    for (int i = 0; i < Regs::NTP; ++i) {
      r.t[i] = tg[ltid + i * LTHR];
      r.p[i] = pg[ltid + i * LTHR];
    }
    const E* vg = vbase + tok0 * DV + col0;
#pragma unroll
    for (int i = 0; i < Regs::NV; ++i) {
      const int u = ltid + i * LTHR;
      if (u < Regs::VU) {
        const int t0 = (u % (C / 4)) * 4, c0 = (u / (C / 4)) * VE;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.v[i][j] = *reinterpret_cast<const uint4*>(vg + (size_t)(t0 + j) * DV + c0);
      }
    }
    r.g = 0.f;
    r.b = 0.f;
    if (ltid < C) {
      r.g = a.G ? a.G[tok0 + ltid] : 0.f;
      r.b = a.beta[tok0 + ltid];
    }
  };


  // ---- loader: registers -> LDS image of the chunk ----------------------------------------------
  auto store_chunk = [&](Stage& s, const Regs& r) {
#pragma unroll
    for (int i = 0; i < Regs::NK; ++i) {
      const int u = ltid + i * LTHR;
      const int t0 = (u / (DK / VE)) * 4, d0 = (u % (DK / VE)) * VE;
#pragma unroll
      for (int j = 0; j < 4; ++j) put_row16<RowsSwz>(s.ks, t0 + j, d0, KP, r.k[i][j]);
#pragma unroll
      for (int e = 0; e < VE; ++e) store_col4(s.kts + KTSwz::grp(d0 + e, t0, TP), r.k[i], e);
    }
#pragma unroll
    for (int i = 0; i < Regs::NQ; ++i) {
      const int u = ltid + i * LTHR;
      put_row16<RowsSwz>(s.qs, u / (DK / VE), (u % (DK / VE)) * VE, KP, r.q[i]);
    }
#pragma unroll
    for (int i = 0; i < Regs::NTP; ++i) {
      const int u = ltid + i * LTHR;
      const int rr = u / (C / VE), vv = (u % (C / VE)) * VE;
      put_row16<RowsSwz>(s.ts, rr, vv, TP, r.t[i]);
      put_row16<RowsSwz>(s.ps, rr, vv, TP, r.p[i]);
    }
#pragma unroll
    for (int i = 0; i < Regs::NV; ++i) {
      const int u = ltid + i * LTHR;
      if (u < Regs::VU) {
        const int t0 = (u % (C / 4)) * 4, c0 = (u / (C / 4)) * VE;
#pragma unroll
        for (int e = 0; e < VE; ++e) store_col4(s.vts + RowsSwz::grp(c0 + e, t0, TP), r.v[i], e);
      }
    }
    // gate tables: the exponentials are taken once per chunk here, not per lane in the compute
    const float gl = __shfl(r.g, C - 1);
    if (ltid < C) {
      s.Bs[ltid] = r.b;
      s.BEG[ltid] = r.b * __expf(r.g);
      s.EG[ltid] = oscale * __expf(r.g);
      s.EL[ltid] = __expf(gl - r.g);
      if (ltid == 0) s.DL[0] = __expf(gl);
    }
  };

  // ---- compute: one chunk from LDS image s, state S in registers --------------------------------
  floatx4 S[DK / 16];
  auto compute_chunk = [&](const Stage& s, size_t m) {
    const size_t tok0 = m * C;
    floatx4 Y[MB], QS[MB], R[MB], VN[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      Y[mb] = chain<E, NKB_D, RowsSwz>(zero4(), s.ks, 16 * mb + c, KP, S, NKB_D, g);
      QS[mb] = chain<E, NKB_D, RowsSwz>(zero4(), s.qs, 16 * mb + c, KP, S, NKB_D, g);
    }
    // r = beta (v - e^G Y); v rows 4g..4g+3 of block mb are one 4-element group of the vT tile
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const floatx4 vv = load4f(s.vts + RowsSwz::grp(w * 16 + c, 16 * mb + 4 * g, TP));
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int t = 16 * mb + 4 * g + ii;
        R[mb][ii] = s.Bs[t] * vv[ii] - s.BEG[t] * Y[mb][ii];
      }
    }
    // v_new = T r (T lower triangular: K blocks up to the diagonal)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      VN[mb] = chain<E, NKB_C, RowsSwz>(zero4(), s.ts, 16 * mb + c, TP, R, (16 * mb + 16 + KB - 1) / KB, g);
    // o = scale e^G QS + P v_new   (P is pre-scaled)
    float* ocol = a.o + tok0 * DV + col;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const floatx4 O = chain<E, NKB_C, RowsSwz>(zero4(), s.ps, 16 * mb + c, TP, VN, (16 * mb + 16 + KB - 1) / KB, g);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int t = 16 * mb + 4 * g + ii;
        __builtin_nontemporal_store(s.EG[t] * QS[mb][ii] + O[ii], ocol + (size_t)t * DV);   // streamed
      }
    }
    // S = e^{G_last} S + k^T (v_new e^{G_last - G})
    const float dl = s.DL[0];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) VN[mb][ii] *= s.EL[16 * mb + 4 * g + ii];
    }
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) S[r] = chain<E, NKB_C, KTSwz>(S[r] * dl, s.kts, 16 * r + c, TP, VN, NKB_C, g);
  };

  auto init_state = [&]() {
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + col] : 0.f;
    }
  };
  auto store_state = [&]() {
    if (!a.h_final) return;
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        a.h_final[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + col] = S[r][ii];
    }
  };

  const int NC = a.NC;
  if constexpr (NBUF == 2) {
    // Iteration ch: compute waves consume buffer ch&1; loader waves write chunk ch+1 (held in the
    // register set it was loaded into) to buffer (ch+1)&1 and refill that set with chunk ch+3.
    // The two roles run separate loops (disjoint register live ranges) with the same barrier
    // sequence; both are unrolled by two so the buffer and register-set choice is static.
    if (is_loader) {
      Regs ra, rb;
      load_chunk(ra, m0);
      store_chunk(st[0], ra);
      if (NC > 1) load_chunk(rb, m0 + 1);
      if (NC > 2) load_chunk(ra, m0 + 2);
      lds_barrier();
      for (int ch = 0; ch < NC; ch += 2) {
        if (ch + 1 < NC) {
          store_chunk(st[NBUF - 1], rb);
          if (ch + 3 < NC) load_chunk(rb, m0 + ch + 3);
        }
        lds_barrier();
        if (ch + 1 >= NC) break;
        if (ch + 2 < NC) {
          store_chunk(st[0], ra);
          if (ch + 4 < NC) load_chunk(ra, m0 + ch + 4);
        }
        lds_barrier();
      }
    } else {
      init_state();
      lds_barrier();
      for (int ch = 0; ch < NC; ch += 2) {
        compute_chunk(st[0], m0 + ch);
        lds_barrier();
        if (ch + 1 >= NC) break;
        compute_chunk(st[NBUF - 1], m0 + ch + 1);
        lds_barrier();
      }
      store_state();
    }
  } else {
    // One buffer (operand images too large to double): the loader refills it between two
    // barriers after the compute waves are done with it; the next chunk's global loads are
    // still in flight during the current chunk's compute.
    if (is_loader) {
      Regs ra;
      load_chunk(ra, m0);
      store_chunk(st[0], ra);
      if (NC > 1) load_chunk(ra, m0 + 1);
      lds_barrier();
      for (int ch = 0; ch < NC; ++ch) {
        lds_barrier();
        if (ch + 1 < NC) {
          store_chunk(st[0], ra);
          if (ch + 2 < NC) load_chunk(ra, m0 + ch + 2);
        }
        lds_barrier();
      }
    } else {
      init_state();
      lds_barrier();
      for (int ch = 0; ch < NC; ++ch) {
        compute_chunk(st[0], m0 + ch);
        lds_barrier();
        lds_barrier();
      }
      store_state();
    }
  }
}

}  // namespace pf
