// Stage 2 for fp32 operands with every chunk's work split over four waves: the state scan fused
// with the output, for short sequences and few chains, where one wave walking a chain's whole
// chunk (pf_scan_output.h) leaves the chain's latency as the forward's time.
//
// Workgroup = one chain bh x one 16-column slice (grid BH * DV / 16), four waves.  Wave w owns
// state rows 32w .. 32w+31 (fp32, MFMA D layout, in registers for the whole chain).  Per chunk
// (T, P, G from stage 1; fp32 MFMA 16x16x4 throughout):
//
//   1.  partial Y_w = k[:, rows of w] S_w and (q S)_w for all 64 tokens     -> LDS
//   2a. wave w: Y = sum of the partials and r = beta v - beta e^G Y for token tiles 0..w, and
//       v_new of token tile w = sum_jb T[w][jb] r_jb (T is lower triangular)   -> LDS
//   2b. every wave reads all of v_new; wave w: o of token tile 3 - w = scale e^G (sum of the
//       q S partials) + P v_new -> HBM (o tiles 3..0 balance the v_new tiles 0..3: 20 products
//       per wave); S_w <- e^{G_last} S_w + k[:, rows of w]^T (e^{G_last - G} v_new)
//
// so every wave carries 64 + 20 + 32 products per chunk instead of one wave's ~460 (forming all
// of v_new in every wave, as an earlier version did, took 64 + 40 + 4..16 + 32 and was 6 %
// slower at 64 chunks per chain).  The next chunk is loaded into registers while a chunk is
// computed.  q is last read in step 1, and T and P (kept as their ten lower 16x16 tiles, in two
// buffers) are read from the current buffer in step 2, so the next chunk's q, T and P are written
// into LDS during step 2, and its q, T and P loads for the chunk after issued then; only k (read
// by step 2's update), v and the gate tables are written between the two barriers that end a
// chunk.
#pragma once

#include "pf_scan_output.h"

namespace pf {

template <int C, int DK, int DV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void scan_split_f32_kernel(ScanOutArgs a) {
  static_assert(C == 64 && DK == 128 && DV % 16 == 0, "tile shapes of the fp32 split scan: C 64, DK 128");
  constexpr int KP = DK + 4, VP = 16 + 4;
  constexpr int NK = C * DK / 4 / 256, NT = C * C / 4 / 256;   // float4 copies per thread
  // T and P as their ten lower-triangular 16x16 tiles, tile (ib, jb) at score_tile_index(ib, jb),
  // rows padded to 20 floats; two buffers, so a chunk's tiles are written while the previous
  // chunk's are read
  constexpr int TR = 20, TT = 16 * TR, TB = 10 * TT;
  __shared__ __attribute__((aligned(16))) float ks[C * KP];
  __shared__ __attribute__((aligned(16))) float qs[C * KP];
  __shared__ __attribute__((aligned(16))) float tsb[2][TB];
  __shared__ __attribute__((aligned(16))) float psb[2][TB];
  __shared__ __attribute__((aligned(16))) float vs[C * VP];
  __shared__ __attribute__((aligned(16))) float Bs[C], BEG[C], EG[C], EL[C], DL[4];
  __shared__ __attribute__((aligned(16))) floatx4 YP[4 * 4 * 64];   // [wave][token tile][lane]
  __shared__ __attribute__((aligned(16))) floatx4 QP[4 * 4 * 64];
  __shared__ __attribute__((aligned(16))) floatx4 VX[4 * 64];      // v_new, [token tile][lane]

  constexpr int NS = DV / 16;
  const int bh = blockIdx.x / NS, col0 = 16 * (blockIdx.x % NS);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NC = a.NC;
  const size_t Tlen = (size_t)NC * C;
  const float* kb = static_cast<const float*>(a.k) + (size_t)bh * Tlen * DK;
  const float* qb = static_cast<const float*>(a.q) + (size_t)bh * Tlen * DK;
  const float* vb = static_cast<const float*>(a.v) + (size_t)bh * Tlen * DV;
  const float* tb = static_cast<const float*>(a.Tm) + (size_t)bh * NC * C * C;
  const float* pb = static_cast<const float*>(a.P) + (size_t)bh * NC * C * C;
  const float oscale = *a.scale;

  // ---- one chunk: global -> registers -> LDS ----
  floatx4 rk[NK], rq[NK], rt[NT], rp[NT], rv;
  float rg = 0.f, rb = 0.f;
  // thread tid holds T / P rows 16 i + tid / 16, columns 4 (tid % 16) .. : tile (i, (tid % 16) / 4)
  const int t_row = tid >> 4, t_jb = (tid & 15) >> 2, t_col = 4 * (tid & 3);
  auto load_qtp = [&](int ch) {
    const size_t t0 = (size_t)ch * C;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int u = tid + 256 * i, row = u >> 5, q4 = u & 31;
      rq[i] = *reinterpret_cast<const floatx4*>(qb + (t0 + row) * DK + 4 * q4);
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int u = tid + 256 * i, row = u >> 4, q4 = u & 15;
      rt[i] = *reinterpret_cast<const floatx4*>(tb + ((size_t)ch * C + row) * C + 4 * q4);
      rp[i] = *reinterpret_cast<const floatx4*>(pb + ((size_t)ch * C + row) * C + 4 * q4);
    }
  };
  auto store_qtp = [&](int ch) {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int u = tid + 256 * i, row = u >> 5, q4 = u & 31;
      *reinterpret_cast<floatx4*>(qs + row * KP + 4 * q4) = rq[i];
    }
    float* tsd = tsb[ch & 1];
    float* psd = psb[ch & 1];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if (t_jb <= i) {
        const int off = score_tile_index(i, t_jb) * TT + t_row * TR + t_col;
        *reinterpret_cast<floatx4*>(tsd + off) = rt[i];
        *reinterpret_cast<floatx4*>(psd + off) = rp[i];
      }
    }
  };
  auto load = [&](int ch) {
    const size_t t0 = (size_t)ch * C;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int u = tid + 256 * i, row = u >> 5, q4 = u & 31;
      rk[i] = *reinterpret_cast<const floatx4*>(kb + (t0 + row) * DK + 4 * q4);
    }
    rv = *reinterpret_cast<const floatx4*>(vb + (t0 + (tid >> 2)) * DV + col0 + 4 * (tid & 3));
    if (tid < C) {
      rg = a.G ? a.G[(size_t)bh * Tlen + t0 + tid] : 0.f;
      rb = a.beta[(size_t)bh * Tlen + t0 + tid];
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int u = tid + 256 * i, row = u >> 5, q4 = u & 31;
      *reinterpret_cast<floatx4*>(ks + row * KP + 4 * q4) = rk[i];
    }
    *reinterpret_cast<floatx4*>(vs + (tid >> 2) * VP + 4 * (tid & 3)) = rv;
    if (w == 0) {                                     // lane = token
      const float gl = __shfl(rg, C - 1);
      Bs[lane] = rb;
      BEG[lane] = rb * __expf(rg);
      EG[lane] = oscale * __expf(rg);
      EL[lane] = __expf(gl - rg);
      if (lane == 0) DL[0] = __expf(gl);
    }
  };

  floatx4 S[2];                                       // rows 32w + 16r + 4g + ii, column col0 + c
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 32 * w + 16 * r + 4 * g + ii) * DV + col0 + c] : 0.f;

  load(0);
  load_qtp(0);
  store();
  store_qtp(0);
  lds_barrier();
  if (NC > 1) {
    load(1);
    load_qtp(1);
  }

  for (int ch = 0; ch < NC; ++ch) {
    // ---- 1. partial products over this wave's 32 state rows ----
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      floatx4 y = zero4(), qy = zero4();
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const floatx4 ka = *reinterpret_cast<const floatx4*>(ks + (16 * ib + c) * KP + 32 * w + 16 * r + 4 * g);
        const floatx4 qa = *reinterpret_cast<const floatx4*>(qs + (16 * ib + c) * KP + 32 * w + 16 * r + 4 * g);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          y = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[ii], S[r][ii], y, 0, 0, 0);
          qy = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[ii], S[r][ii], qy, 0, 0, 0);
        }
      }
      YP[(w * 4 + ib) * 64 + lane] = y;
      QP[(w * 4 + ib) * 64 + lane] = qy;
    }
    lds_barrier();
    // q of this chunk is read: the next chunk's q, and its T and P into the other buffer
    if (ch + 1 < NC) {
      store_qtp(ch + 1);
      if (ch + 2 < NC) load_qtp(ch + 2);
    }
    const float* ts = tsb[ch & 1];
    const float* ps = psb[ch & 1];
    // ---- 2a. wave w: r for token tiles 0..w, v_new tile w = sum_jb T[w][jb] r_jb -> VX ----
    {
      floatx4 V = zero4();
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        if (jb <= w) {
          floatx4 Y = YP[jb * 64 + lane];
#pragma unroll
          for (int w2 = 1; w2 < 4; ++w2) Y += YP[(w2 * 4 + jb) * 64 + lane];
          floatx4 R;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int t = 16 * jb + 4 * g + ii;
            R[ii] = Bs[t] * vs[t * VP + c] - BEG[t] * Y[ii];
          }
          const floatx4 ta = *reinterpret_cast<const floatx4*>(ts + score_tile_index(w, jb) * TT + c * TR + 4 * g);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) V = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[ii], R[ii], V, 0, 0, 0);
        }
      }
      VX[w * 64 + lane] = V;
    }
    lds_barrier();
    // ---- 2b. every wave: all of v_new; o for token tile 3 - w; the update of rows 32w .. ----
    floatx4 VN[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) VN[ib] = VX[ib * 64 + lane];
    {
      const int ot = 3 - w;                            // o tiles 3..0 balance v_new tiles 0..3
      floatx4 O = QP[ot * 64 + lane];
#pragma unroll
      for (int w2 = 1; w2 < 4; ++w2) O += QP[(w2 * 4 + ot) * 64 + lane];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) O[ii] *= EG[16 * ot + 4 * g + ii];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        if (jb <= ot) {
          const floatx4 pa = *reinterpret_cast<const floatx4*>(ps + score_tile_index(ot, jb) * TT + c * TR + 4 * g);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) O = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ii], VN[jb][ii], O, 0, 0, 0);
        }
      }
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        __builtin_nontemporal_store(O[ii], a.o + ((size_t)bh * Tlen + (size_t)ch * C + 16 * ot + 4 * g + ii) * DV + col0 + c);
    }
    {
      const float dl = DL[0];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        floatx4 acc = S[r] * dl;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int t = 16 * jb + 4 * g + ii;
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[t * KP + 32 * w + 16 * r + c], EL[t] * VN[jb][ii], acc, 0, 0, 0);
          }
        S[r] = acc;
      }
    }
    lds_barrier();                                     // the chunk's image and partials are read
    if (ch + 1 < NC) {
      store();
      lds_barrier();
      if (ch + 2 < NC) load(ch + 2);
    }
  }
  if (a.h_final) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        a.h_final[((size_t)bh * DK + 32 * w + 16 * r + 4 * g + ii) * DV + col0 + c] = S[r][ii];
  }
}

}  // namespace pf
