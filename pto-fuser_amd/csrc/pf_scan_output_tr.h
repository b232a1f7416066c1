// K2 for bf16 operands on gfx950 — the state scan fused with the output stage, with the chunk
// operands staged row-major only and read transposed through LDS transpose loads.
//
// Same mathematics and workgroup decomposition as the generic kernel (pf_scan_output.h): one
// workgroup per (chain bh, 32-column dv tile), two compute waves (16 state columns each, state
// register-resident in fp32) and two loader waves, two LDS chunk buffers, one barrier per chunk:
//
//   Y = k S,  QS = q S,  r = beta (v - e^G Y),  v_new = T r,
//   o = scale (e^G QS + P v_new),  S = e^{G_last} S + k^T (v_new e^{G_last - G}).
//
// What is specific to gfx950 and bf16:
//   * k^T, the A operand of the state update, is read straight out of the row-major k tile with
//     ds_read_b64_tr_b16: within each 16-lane group, lane l receives element (l & 3) of the
//     4-element words addressed by lanes 4j + (l >> 2), j = 0..3.  Lane (c, g) therefore
//     addresses k[32kb + 4g + (c >> 2)][16r + 4(c & 3) .. +3] and receives
//     k[32kb + 4g + j][16r + c], j = 0..3 — the permuted-K operand of the MFMA chain.  The v
//     tile is read into the accumulator layout the same way.  No transposed copy is staged.
//   * every tile is written by the loader as whole 16-byte row vectors and swizzled (Swz) so that
//     the row writes, the MFMA operand reads and the transpose reads are all free of LDS bank
//     conflicts; the loader's lane-to-row mapping makes the swizzle's half-swap bit a
//     compile-time constant, so no data is shuffled;
//   * global traffic uses raw buffer loads/stores with a per-chain descriptor: the chunk advance
//     is a scalar offset, the lane part a constant vector offset, rows a small immediate.
#pragma once

#include "pf_scan_output.h"

namespace pf {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
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

// LDS image of one chunk (bf16), C = 64, DK = 128, tile width TW = 32.
template <int C, int DK, int TW>
struct TrStage {
  static constexpr int KP = DK + 16;   // k, q: Swz<2,3>
  static constexpr int TP = C + 8;     // T, P: Swz<3,1>
  static constexpr int VP = TW + 16;   // v: unswizzled
  bf16 ks[C * KP];
  bf16 qs[C * KP];
  bf16 ts[C * TP];
  bf16 ps[C * TP];
  bf16 vs[C * VP];
  float Bs[C];
  float EG[C];
  float EL[C];
  float DL[4];
};

// Loader register image of one chunk; NLW loader waves share the tile (k, q: 1024 vectors;
// T, P: 512; v: 256 — per thread NK, NT, NV).
template <int NLW>
struct TrRegs {
  static constexpr int NK = 1024 / (64 * NLW), NTP = 512 / (64 * NLW), NV = 256 / (64 * NLW);
  uint4 k[NK], q[NK], t[NTP], p[NTP], v[NV];
  float g, b;
};

template <int C, int DK, int DV, int NWC, int NLW>
__global__ __launch_bounds__(64 * (NWC + NLW)) __attribute__((amdgpu_waves_per_eu(1, 1)))
void scan_output_tr_kernel(ScanOutArgs a) {
  constexpr int TW = 16 * NWC;
  using Stage = TrStage<C, DK, TW>;
  using Regs = TrRegs<NLW>;
  constexpr int KP = Stage::KP, TP = Stage::TP, VP = Stage::VP;
  constexpr int NT = DV / TW;
  static_assert(C == 64 && DK == 128 && TW == 32 && (NLW == 2 || NLW == 4),
                "tile shapes of the transpose-read kernel are fixed: C 64, DK 128, 32-column tile");

  __shared__ __attribute__((aligned(16))) Stage st[2];

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
  const float* Gc = a.G ? a.G + (size_t)bh * Tlen : nullptr;
  const float* Bc = a.beta + (size_t)bh * Tlen;

  if (w >= NWC) {
    // =========================== loader waves ===========================
    // (the gate tables below are filled by loader threads lt < C, i.e. the first loader wave)
    const int lt = tid - 64 * NWC;                       // 0 .. 64*NLW-1
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
    // v (4 vectors per row of the tile): row = (lt >> 2) + (16*NLW) i, vec = lt & 3
    const int vrow_l = lt >> 2, vvec = lt & 3;
    const uint32_t v_voff = (uint32_t)(vrow_l * DV + col0 + vvec * 8) * 2;
    const int v_lds = vrow_l * VP + vvec * 8;

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
      for (int i = 0; i < Regs::NV; ++i) r.v[i] = buf_load16(rv, v_voff, v_s + (uint32_t)(16 * NLW * i) * DV * 2);
      r.g = 0.f;
      r.b = 0.f;
      if (lt < C) {
        r.g = Gc ? Gc[(size_t)ch * C + lt] : 0.f;
        r.b = Bc[(size_t)ch * C + lt];
      }
    };
    auto store_chunk = [&](Stage& s, const Regs& r) {
#pragma unroll
      for (int i = 0; i < Regs::NK; ++i) {
        const int rowi = krow_i(i);
        const bool swap = (i & 1) != 0;                   // Swz<2,3> bit 0 = row bit 2 = i0
        *reinterpret_cast<uint4*>(s.ks + kq_lds + rowi * KP) = swap_halves_if(r.k[i], swap);
        *reinterpret_cast<uint4*>(s.qs + kq_lds + rowi * KP) = swap_halves_if(r.q[i], swap);
      }
#pragma unroll
      for (int i = 0; i < Regs::NTP; ++i) {
        const int rowi = trow_i(i);
        const bool swap = (i & 1) != 0;                   // Swz<3,1> bit 0 = row bit 3 = i0
        *reinterpret_cast<uint4*>(s.ts + tp_lds + rowi * TP) = swap_halves_if(r.t[i], swap);
        *reinterpret_cast<uint4*>(s.ps + tp_lds + rowi * TP) = swap_halves_if(r.p[i], swap);
      }
#pragma unroll
      for (int i = 0; i < Regs::NV; ++i) *reinterpret_cast<uint4*>(s.vs + v_lds + 16 * NLW * i * VP) = r.v[i];
      const float gl = __shfl(r.g, C - 1);
      if (lt < C) {
        s.Bs[lt] = r.b;
        s.EG[lt] = __expf(r.g);
        s.EL[lt] = __expf(gl - r.g);
        if (lt == 0) s.DL[0] = __expf(gl);
      }
    };

    Regs ra, rb;
    load_chunk(ra, 0);
    store_chunk(st[0], ra);
    if (NC > 1) load_chunk(rb, 1);
    if (NC > 2) load_chunk(ra, 2);
    lds_barrier();
    for (int ch = 0; ch < NC; ch += 2) {
      if (ch + 1 < NC) {
        store_chunk(st[1], rb);
        if (ch + 3 < NC) load_chunk(rb, ch + 3);
      }
      lds_barrier();
      if (ch + 1 >= NC) break;
      if (ch + 2 < NC) {
        store_chunk(st[0], ra);
        if (ch + 4 < NC) load_chunk(ra, ch + 4);
      }
      lds_barrier();
    }
  } else {
    // =========================== compute waves ===========================
    const int col = col0 + w * 16 + c;
    // per-lane LDS element offsets (see the swizzle derivations in the header comment)
    const int kq_rd = c * KP + 4 * (g ^ ((c >> 2) & 3));             // A of k S / q S
    const int kt_rd = (4 * g + (c >> 2)) * KP + 4 * ((c & 3) ^ g);   // transposed A of k^T
    const int tp_rd = c * TP + 4 * (g ^ (c >> 3));                   // A of T r / P v_new
    const int v_rd = (4 * g + (c >> 2)) * VP + 16 * w + 4 * (c & 3); // v rows 4g.. of col c
    const uint32_t o_voff = (uint32_t)(4 * g * DV + col) * 4;

    floatx4 S[DK / 16];
#pragma unroll
    for (int r = 0; r < DK / 16; ++r) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + col] : 0.f;
    }

    auto compute_chunk = [&](const Stage& s, int ch) {
      // bf16 B operands of the state, one per 32-row K block
      bf16x8 SB[DK / 32];
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) SB[kb] = pack8(S[2 * kb], S[2 * kb + 1]);
      floatx4 Y[4], QS[4], R[4], VN[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        Y[mb] = zero4();
        QS[mb] = zero4();
      }
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const bf16* kp = s.ks + kq_rd + 16 * mb * KP + 32 * kb;
          const bf16* qp = s.qs + kq_rd + 16 * mb * KP + 32 * kb;
          Y[mb] = mfma_bf16(cat8(*reinterpret_cast<const bf16x4*>(kp), *reinterpret_cast<const bf16x4*>(kp + 16)),
                            SB[kb], Y[mb]);
          QS[mb] = mfma_bf16(cat8(*reinterpret_cast<const bf16x4*>(qp), *reinterpret_cast<const bf16x4*>(qp + 16)),
                             SB[kb], QS[mb]);
        }
      }
      // r = beta (v - e^G Y)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16x4 vv = lds_read_tr(s.vs + v_rd + 16 * mb * VP);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int t = 16 * mb + 4 * g + ii;
          R[mb][ii] = s.Bs[t] * ((float)vv[ii] - s.EG[t] * Y[mb][ii]);
        }
      }
      // v_new = T r (lower triangular: K block 1 only for rows 32..63)
      const bf16x8 RB0 = pack8(R[0], R[1]), RB1 = pack8(R[2], R[3]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16* tp = s.ts + tp_rd + 16 * mb * TP;
        VN[mb] = mfma_bf16(cat8(*reinterpret_cast<const bf16x4*>(tp), *reinterpret_cast<const bf16x4*>(tp + 16)),
                           RB0, zero4());
        if (mb >= 2)
          VN[mb] = mfma_bf16(cat8(*reinterpret_cast<const bf16x4*>(tp + 32), *reinterpret_cast<const bf16x4*>(tp + 48)),
                             RB1, VN[mb]);
      }
      // o = scale (e^G QS + P v_new)
      const bf16x8 VB0 = pack8(VN[0], VN[1]), VB1 = pack8(VN[2], VN[3]);
      const uint32_t o_s = (uint32_t)ch * C * DV * 4;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const bf16* pp = s.ps + tp_rd + 16 * mb * TP;
        floatx4 O = mfma_bf16(cat8(*reinterpret_cast<const bf16x4*>(pp), *reinterpret_cast<const bf16x4*>(pp + 16)),
                              VB0, zero4());
        if (mb >= 2)
          O = mfma_bf16(cat8(*reinterpret_cast<const bf16x4*>(pp + 32), *reinterpret_cast<const bf16x4*>(pp + 48)),
                        VB1, O);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int t = 16 * mb + 4 * g + ii;
          const float val = a.scale * (s.EG[t] * QS[mb][ii] + O[ii]);
          // the builtin takes the 32 data bits as an unsigned int: pass the float's bits
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, val), ro, o_voff,
                                                o_s + (uint32_t)(16 * mb + ii) * DV * 4, 0);
        }
      }
      // S = e^{G_last} S + k^T (v_new e^{G_last - G})
      const float dl = s.DL[0];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) VN[mb][ii] *= s.EL[16 * mb + 4 * g + ii];
      }
      const bf16x8 UB0 = pack8(VN[0], VN[1]), UB1 = pack8(VN[2], VN[3]);
#pragma unroll
      for (int r = 0; r < DK / 16; ++r) {
        const bf16* k0 = s.ks + kt_rd + 16 * r;
        floatx4 acc = S[r] * dl;
        acc = mfma_bf16(cat8(lds_read_tr(k0), lds_read_tr(k0 + 16 * KP)), UB0, acc);
        acc = mfma_bf16(cat8(lds_read_tr(k0 + 32 * KP), lds_read_tr(k0 + 48 * KP)), UB1, acc);
        S[r] = acc;
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
      for (int r = 0; r < DK / 16; ++r) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          a.h_final[((size_t)bh * DK + 16 * r + 4 * g + ii) * DV + col] = S[r][ii];
      }
    }
  }
}

}  // namespace pf
