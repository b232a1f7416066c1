// Stage 2 for fp32 operands: the state scan fused with the output, every chunk's work split over
// four waves so that the chain's latency (the forward's time at few chains) is a quarter of one
// wave walking the whole chunk.
//
// Workgroup = one chain bh x one 16-column slice (grid BH * DV / 16), four waves.  Wave w owns
// state rows 32w .. 32w+31 (fp32, MFMA D layout, in registers for the whole chain).  Per chunk
// (T, P, G from stage 1; fp32 MFMA 16x16x4 throughout):
//
//   1.  partial Y_w = k[:, rows of w] S_w and (q S)_w for all 64 tokens     -> LDS
//   2a. wave w: Y = sum of the partials and r = beta v - beta e^G Y for token tiles 0..w, and
//       v_new of token tile w = sum_jb T[w][jb] r_jb (T is lower triangular)   -> LDS; the sum
//       of the q S partials of token tile 3 - w
//   2b. every wave reads all of v_new; wave w: o of token tile 3 - w = scale e^G (q S) +
//       P v_new -> HBM (o tiles 3..0 balance the v_new tiles 0..3: 20 products
//       per wave); S_w <- e^{G_last} S_w + k[:, rows of w]^T (e^{G_last - G} v_new)
//
// so every wave carries 64 + 20 + 32 products per chunk instead of one wave's ~460 (forming all
// of v_new in every wave, as an earlier version did, took 64 + 40 + 4..16 + 32 and was 6 %
// slower at 64 chunks per chain).  The next chunk is loaded into registers while a chunk is
// computed and written into LDS where its last reader is done: each wave's own slice of k and q
// (the only columns it reads) after its own last read, T, P and the gate tables (two buffers:
// T and P as their ten lower 16x16 tiles) after the barrier that ends step 1, v after the one
// that ends step 2a.  Two barriers per chunk, and no copy section between them: every exchange
// tile is last read before the second, so the next chunk's first step may overwrite them.
#pragma once

#include "pf_scan_args.h"

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
  __shared__ __attribute__((aligned(16))) float Bs[2][C], BEG[2][C], EG[2][C], EL[2][C], DL[2][4];
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

  // ---- chunk data: global -> registers -> LDS.  Wave w reads only columns 32w .. 32w+31 of the
  //      k and q rows (its state rows), so it loads and writes that slice itself and refills it
  //      after its own last read, with no workgroup barrier; T, P and the gate tables (two
  //      buffers) are written after B1, v after B2 (its last read is in step 2a) ----
  floatx4 rk[8], rq[8], rt[NT], rp[NT], rv;
  float rg = 0.f, rb = 0.f;
  static_assert(NK == 8, "64 rows x 32 columns of k (or q) per wave: eight float4 per lane");
  auto kq_lds = [&](int i) { const int u = lane + 64 * i; return (u >> 3) * KP + 32 * w + 4 * (u & 7); };
  auto kq_mem = [&](int i) { const int u = lane + 64 * i; return (size_t)(u >> 3) * DK + 32 * w + 4 * (u & 7); };
  auto load_k = [&](int ch) {
#pragma unroll
    for (int i = 0; i < 8; ++i) rk[i] = *reinterpret_cast<const floatx4*>(kb + (size_t)ch * C * DK + kq_mem(i));
  };
  auto load_q = [&](int ch) {
#pragma unroll
    for (int i = 0; i < 8; ++i) rq[i] = *reinterpret_cast<const floatx4*>(qb + (size_t)ch * C * DK + kq_mem(i));
  };
  auto store_k = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<floatx4*>(ks + kq_lds(i)) = rk[i];
  };
  auto store_q = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<floatx4*>(qs + kq_lds(i)) = rq[i];
  };
  // thread tid holds T / P rows 16 i + tid / 16, columns 4 (tid % 16) .. : tile (i, (tid % 16) / 4)
  const int t_row = tid >> 4, t_jb = (tid & 15) >> 2, t_col = 4 * (tid & 3);
  auto load_tpg = [&](int ch) {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int u = tid + 256 * i, row = u >> 4, q4 = u & 15;
      rt[i] = *reinterpret_cast<const floatx4*>(tb + ((size_t)ch * C + row) * C + 4 * q4);
      rp[i] = *reinterpret_cast<const floatx4*>(pb + ((size_t)ch * C + row) * C + 4 * q4);
    }
    // every thread loads (threads 64.. repeat the first wave's tokens): no branch around a load;
    // G is the stage-1 workspace's cumsum, always present for this kernel
    rg = a.G[(size_t)bh * Tlen + (size_t)ch * C + (tid & (C - 1))];
    rb = a.beta[(size_t)bh * Tlen + (size_t)ch * C + (tid & (C - 1))];
  };
  auto store_tpg = [&](int ch) {
    const int b = ch & 1;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if (t_jb <= i) {
        const int off = score_tile_index(i, t_jb) * TT + t_row * TR + t_col;
        *reinterpret_cast<floatx4*>(tsb[b] + off) = rt[i];
        *reinterpret_cast<floatx4*>(psb[b] + off) = rp[i];
      }
    }
    if (w == 0) {                                     // lane = token
      const float gl = __shfl(rg, C - 1);
      Bs[b][lane] = rb;
      BEG[b][lane] = rb * __expf(rg);
      EG[b][lane] = oscale * __expf(rg);
      EL[b][lane] = __expf(gl - rg);
      if (lane == 0) DL[b][0] = __expf(gl);
    }
  };
  auto load_v = [&](int ch) {
    rv = *reinterpret_cast<const floatx4*>(vb + ((size_t)ch * C + (tid >> 2)) * DV + col0 + 4 * (tid & 3));
  };
  auto store_v = [&]() { *reinterpret_cast<floatx4*>(vs + (tid >> 2) * VP + 4 * (tid & 3)) = rv; };

  floatx4 S[2];                                       // rows 32w + 16r + 4g + ii, column col0 + c
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = a.h0 ? a.h0[((size_t)bh * DK + 32 * w + 16 * r + 4 * g + ii) * DV + col0 + c] : 0.f;

  load_k(0);
  load_q(0);
  load_tpg(0);
  load_v(0);
  store_k();
  store_q();
  store_tpg(0);
  store_v();
  lds_barrier();
  load_k(min(1, NC - 1));
  load_q(min(1, NC - 1));
  load_tpg(min(1, NC - 1));
  load_v(min(1, NC - 1));

  // Past the end the loads repeat the last chunk and the copies write what no one reads again
  // (a wave's own slices after its last read, the other T / P / gate buffer, v after its last
  // read): the loop body is straight-line code, so the compiler's wait counts stay exact and a
  // copy waits only for its own loads, issued a chunk earlier.
  const int last = NC - 1;
  for (int ch = 0; ch < NC; ++ch) {
    const int cb = ch & 1;
    const int nx2 = min(ch + 2, last);
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
    store_q();                                         // this wave's q slice is read
    load_q(nx2);
    lds_barrier();                                     // B1: partials written
    store_tpg(ch + 1);                                 // the other T / P / gate buffer is free
    load_tpg(nx2);
    const float* ts = tsb[cb];
    const float* ps = psb[cb];
    // ---- 2a. wave w: r for token tiles 0..w, v_new tile w = sum_jb T[w][jb] r_jb -> VX; the
    //      (q S) partials of its o tile 3 - w summed here, so no exchange is read after B2 ----
    const int ot = 3 - w;                              // o tiles 3..0 balance v_new tiles 0..3
    floatx4 O = QP[ot * 64 + lane];
#pragma unroll
    for (int w2 = 1; w2 < 4; ++w2) O += QP[(w2 * 4 + ot) * 64 + lane];
    {
      floatx4 V = zero4(), V2 = zero4();                 // two accumulators: shorter chains
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
            R[ii] = Bs[cb][t] * vs[t * VP + c] - BEG[cb][t] * Y[ii];
          }
          const floatx4 ta = *reinterpret_cast<const floatx4*>(ts + score_tile_index(w, jb) * TT + c * TR + 4 * g);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            if (ii & 1) V2 = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[ii], R[ii], V2, 0, 0, 0);
            else V = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[ii], R[ii], V, 0, 0, 0);
          }
        }
      }
      VX[w * 64 + lane] = V + V2;
    }
    lds_barrier();                                     // B2: v_new written, v read
    store_v();
    load_v(nx2);
    // ---- 2b. every wave: all of v_new; o for token tile 3 - w; the update of rows 32w .. ----
    floatx4 VN[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) VN[ib] = VX[ib * 64 + lane];
    {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) O[ii] *= EG[cb][16 * ot + 4 * g + ii];
      floatx4 O2 = zero4();
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        if (jb <= ot) {
          const floatx4 pa = *reinterpret_cast<const floatx4*>(ps + score_tile_index(ot, jb) * TT + c * TR + 4 * g);
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            if (ii & 1) O2 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ii], VN[jb][ii], O2, 0, 0, 0);
            else O = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ii], VN[jb][ii], O, 0, 0, 0);
          }
        }
      }
      O += O2;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        __builtin_nontemporal_store(O[ii], a.o + ((size_t)bh * Tlen + (size_t)ch * C + 16 * ot + 4 * g + ii) * DV + col0 + c);
    }
    {
      const float dl = DL[cb][0];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        floatx4 acc = S[r] * dl, acc2 = zero4();        // two accumulators: shorter chains
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int t = 16 * jb + 4 * g + ii;
            if (ii & 1)
              acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[t * KP + 32 * w + 16 * r + c], EL[cb][t] * VN[jb][ii], acc2, 0, 0, 0);
            else
              acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[t * KP + 32 * w + 16 * r + c], EL[cb][t] * VN[jb][ii], acc, 0, 0, 0);
          }
        S[r] = acc + acc2;
      }
    }
    store_k();                                         // this wave's k slice is read
    load_k(nx2);
    // no third barrier: the next chunk's step 1 writes YP (last read in 2a) and QP (last read
    // in 2a), its 2a writes VX after B1 (every wave then is past this 2b), and T, P and the gate
    // tables alternate between two buffers
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
