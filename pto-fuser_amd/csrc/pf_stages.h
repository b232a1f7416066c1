// Stage kernels behind the compile stack's fused nodes (the reference's FusedKernelRegistry keys,
// src/pto_fuser/fused.py:396-588).  Each is one launch over independent units, with no workspace:
//
//   gated_qk_kernel   L = (a' b'^T) * exp(min(G_i + log beta_i - G_j, 0)) * mask
//                     a' = a (.* a_scale), b' = b (.* b_scale) — the scalar-gate epilogue of
//                     kkt_fused.h:154-185 (kkt_gated*, gated_qk*) and, with the operand scales and
//                     no gate, the per-channel prologue of prologue_fused.h:37-107 (qk_prologue*).
//   qkv_flash_kernel  o = causal_incl(the same score) v, the score kept on chip
//                     (qkv_flash_native*, qkv_fused.h:62-175; qkvp_flash_native*,
//                     qkv_prologue_fused.h:99-187).
//   scan_state_kernel chunk_h_scan: h_out[c] = S;  S = decay (.) S + k^T (u - w S), scalar decay
//                     per chunk or a per-row (per key channel) decay vector
//                     (scan_fused.h:198-262; vec_recurrence_perdim :143-180).
//
// Row addressing.  The reference runs these stages on two layouts: the native batch [M, C, D]
// (heads outer) and the "mega" token layout [nc*C, H, D] (= [1, T, H, D]).  Both are described
// by one rule: chunk m = c*H + h, token i of it lives at row (c*C + i)*H + h.  H = 1 is the native
// layout.  Gates follow the same rule with row length 1, scores with row length C.
//
// gfx950 mapping: 256-thread workgroups (4 waves) per chunk for the two score kernels, every
// 16x16 output block one MFMA chain (bf16 16x16x32 or fp32 16x16x4); the scan keeps its
// [D x 16] state slice in registers across the whole chunk loop, one wave per 16 columns.
#pragma once

#include "pf_device.h"

// Barriers are LDS-only (lds_barrier): waves exchange data through LDS alone, so a barrier need
// not wait for this wave's global stores to be acknowledged (a full __syncthreads would).

namespace pf {

template <typename E> struct VecT;
template <> struct VecT<bf16> { typedef bf16x8 T; };
template <> struct VecT<float> { typedef floatx4 T; };

// Copy a C x D tile (rows `row_stride` elements apart) into LDS with row pitch `pitch`,
// multiplying element-wise by `scale` (same addressing, fp32) when it is given.
template <typename E, int C, int D, int NTHR>
__device__ __forceinline__ void stage_tile(const E* src, size_t row_stride, const float* scale,
                                           E* dst, int pitch) {
  constexpr int VE = Vec16<E>::N, PER_ROW = D / VE;
  typedef typename VecT<E>::T V;
  for (int u = threadIdx.x; u < C * PER_ROW; u += NTHR) {
    const int i = u / PER_ROW, d0 = (u % PER_ROW) * VE;
    V x = __builtin_bit_cast(V, *reinterpret_cast<const uint4*>(src + i * row_stride + d0));
    if (scale) {
      const float* s = scale + i * row_stride + d0;
#pragma unroll
      for (int e = 0; e < VE; ++e) x[e] = from_f32<E>(to_f32(x[e]) * s[e]);
    }
    *reinterpret_cast<V*>(dst + i * pitch + d0) = x;
  }
}

__device__ __forceinline__ void store_out(void* base, size_t idx, float v, int out_f32) {
  if (out_f32) static_cast<float*>(base)[idx] = v;
  else static_cast<bf16*>(base)[idx] = (bf16)v;
}

// Lower-triangular block (bi >= bj) number x of an NB x NB block grid, row-major over the
// triangle: 0 -> (0,0), 1 -> (1,0), 2 -> (1,1), 3 -> (2,0) ...
__device__ __forceinline__ void tri_block(int x, int& bi, int& bj) {
  bi = 0;
  while (x > bi) { x -= bi + 1; ++bi; }
  bj = x;
}

struct GatedQkArgs {
  const void* a;        // rows of a  (E)
  const void* b;        // rows of b  (E)
  const float* a_scale; // same addressing as a, or null
  const float* b_scale; // same addressing as b, or null
  const float* g;       // per-token within-chunk cumulative log decay, or null (0)
  const float* beta;    // per-token beta, or null (1)
  const float* mask;    // [C, C] multiplier, or null (use `causal`)
  void* L;              // scores, row length C, fp32 or bf16
  int H;                // heads interleaved in the row index (1 = native [M, C, D])
  int causal;           // without mask: 1 keeps i >= j, 0 keeps i > j
  int out_f32;          // 1: L is fp32, 0: bf16
};

template <typename E, int C, int D>
__global__ __launch_bounds__(256) void gated_qk_kernel(GatedQkArgs p) {
  constexpr int PE = 16 / sizeof(E), KP = D + PE, NB = C / 16;
  __shared__ __attribute__((aligned(16))) E sa[C * KP];
  __shared__ __attribute__((aligned(16))) E sb[C * KP];
  __shared__ float Gs[C], Ls[C];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int m = blockIdx.x, ch = m / p.H, h = m % p.H;
  const size_t rs = (size_t)p.H * D, base = ((size_t)ch * C * p.H + h) * D;
  stage_tile<E, C, D, 256>(static_cast<const E*>(p.a) + base, rs, p.a_scale ? p.a_scale + base : nullptr, sa, KP);
  stage_tile<E, C, D, 256>(static_cast<const E*>(p.b) + base, rs, p.b_scale ? p.b_scale + base : nullptr, sb, KP);
  if (tid < C) {
    const size_t gi = ((size_t)ch * C + tid) * p.H + h;
    Gs[tid] = p.g ? p.g[gi] : 0.f;
    Ls[tid] = p.beta ? __logf(p.beta[gi]) : 0.f;
  }
  lds_barrier();
  const size_t lrs = (size_t)p.H * C, lbase = ((size_t)ch * C * p.H + h) * C;
  for (int x = w; x < NB * NB; x += 4) {
    const int bi = x / NB, bj = x % NB, j = 16 * bj + c;
    if (bj > bi && !p.mask) {            // strictly-upper blocks of a triangular mask are zero
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) store_out(p.L, lbase + (16 * bi + 4 * g + ii) * lrs + j, 0.f, p.out_f32);
      continue;
    }
    floatx4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < D / Mfma<E>::KB; ++kb)
      acc = Mfma<E>::rows(acc, sa + (16 * bi + c) * KP, sb + (16 * bj + c) * KP, kb, g);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 16 * bi + 4 * g + ii;
      const float mk = p.mask ? p.mask[i * C + j] : ((p.causal ? i >= j : i > j) ? 1.f : 0.f);
      const float coef = __expf(fminf(Gs[i] + Ls[i] - Gs[j], 0.f));
      store_out(p.L, lbase + i * lrs + j, mk == 0.f ? 0.f : acc[ii] * coef * mk, p.out_f32);
    }
  }
}

struct QkvFlashArgs {
  const void* q;        // [M, C, D] E
  const void* k;        // [M, C, D] E
  const void* v;        // [M, C, D] E
  const float* q_scale; // [M, C, D] or null
  const float* k_scale; // [M, C, D] or null
  const float* g;       // [M, C] or null
  const float* beta;    // [M, C] or null
  float* o;             // [M, C, D] fp32
};

template <int A, int B> struct MaxI { static constexpr int v = A > B ? A : B; };

template <typename E, int C, int D>
__global__ __launch_bounds__(256) void qkv_flash_kernel(QkvFlashArgs p) {
  constexpr int PE = 16 / sizeof(E), KP = D + PE, LP = C + PE, VP = C + PE, VE = Vec16<E>::N;
  constexpr int NB = C / 16, NL = NB * (NB + 1) / 2, NPW = (NL + 3) / 4;
  // phase 1: rx = q tile, ry = k tile;  phase 2: rx = score (operand type), ry = v^T
  __shared__ __attribute__((aligned(16))) E rx[MaxI<C * KP, C * LP>::v];
  __shared__ __attribute__((aligned(16))) E ry[MaxI<C * KP, D * VP>::v];
  __shared__ float Gs[C], Ls[C];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const size_t m = blockIdx.x, row0 = m * C;
  stage_tile<E, C, D, 256>(static_cast<const E*>(p.q) + row0 * D, D, p.q_scale ? p.q_scale + row0 * D : nullptr, rx, KP);
  stage_tile<E, C, D, 256>(static_cast<const E*>(p.k) + row0 * D, D, p.k_scale ? p.k_scale + row0 * D : nullptr, ry, KP);
  if (tid < C) {
    Gs[tid] = p.g ? p.g[row0 + tid] : 0.f;
    Ls[tid] = p.beta ? __logf(p.beta[row0 + tid]) : 0.f;
  }
  lds_barrier();
  floatx4 acc[NPW];
#pragma unroll
  for (int s = 0; s < NPW; ++s) {
    acc[s] = zero4();
    const int x = w + 4 * s;
    if (x < NL) {
      int bi, bj;
      tri_block(x, bi, bj);
#pragma unroll
      for (int kb = 0; kb < D / Mfma<E>::KB; ++kb)
        acc[s] = Mfma<E>::rows(acc[s], rx + (16 * bi + c) * KP, ry + (16 * bj + c) * KP, kb, g);
    }
  }
  lds_barrier();
#pragma unroll
  for (int s = 0; s < NPW; ++s) {
    const int x = w + 4 * s;
    if (x < NL) {
      int bi, bj;
      tri_block(x, bi, bj);
      const int j = 16 * bj + c;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int i = 16 * bi + 4 * g + ii;
        const float coef = __expf(fminf(Gs[i] + Ls[i] - Gs[j], 0.f));
        rx[i * LP + j] = from_f32<E>(i >= j ? acc[s][ii] * coef : 0.f);
      }
    }
  }
  for (int e = tid; e < C * C; e += 256) {
    const int i = e / C, j = e % C;
    if ((j >> 4) > (i >> 4)) rx[i * LP + j] = from_f32<E>(0.f);
  }
  {
    typedef typename VecT<E>::T V;
    const E* vg = static_cast<const E*>(p.v) + row0 * D;
    for (int u = tid; u < C * (D / VE); u += 256) {
      const int t = u / (D / VE), n0 = (u % (D / VE)) * VE;
      const V x = __builtin_bit_cast(V, *reinterpret_cast<const uint4*>(vg + (size_t)t * D + n0));
#pragma unroll
      for (int e = 0; e < VE; ++e) ry[(n0 + e) * VP + t] = x[e];
    }
  }
  lds_barrier();
  // o[t, n] = sum_{t' <= t} S[t, t'] v[t', n]: (C/16) x (D/16) blocks over the four waves
  float* o = p.o + row0 * D;
  for (int x = w; x < NB * (D / 16); x += 4) {
    const int bi = x / (D / 16), bn = x % (D / 16);
    floatx4 r = zero4();
#pragma unroll
    for (int kb = 0; kb < C / Mfma<E>::KB; ++kb)
      if (kb * Mfma<E>::KB <= 16 * bi + 15)
        r = Mfma<E>::rows(r, rx + (16 * bi + c) * LP, ry + (16 * bn + c) * VP, kb, g);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) o[(size_t)(16 * bi + 4 * g + ii) * D + 16 * bn + c] = r[ii];
  }
}

struct ScanStateArgs {
  const void* w;        // [B, nc, C, H, D] E
  const void* u;        // [B, nc, C, H, D] E
  const void* k;        // [B, nc, C, H, D] E
  const float* decay;   // [B, H, nc] (scalar) or [B, H, nc, D] (per row)
  const float* h0;      // [B, H, D, D] or null (zero)
  void* h_out;          // [B, nc, H, D, D] fp32 or bf16
  float* final_state;   // [B, H, D, D] or null
  int H, NC, perdim, out_f32;
};

// One workgroup per (b, h, 16*NW-column slice of the state); wave w owns 16 columns.
template <typename E, int C, int D, int NW>
__global__ __launch_bounds__(64 * NW) void scan_state_kernel(ScanStateArgs p) {
  constexpr int PE = 16 / sizeof(E), KP = D + PE, TP = C + PE, VE = Vec16<E>::N;
  constexpr int NKB_D = D / Mfma<E>::KB, NKB_C = C / Mfma<E>::KB, MB = C / 16, NTHR = 64 * NW;
  constexpr int TW = 16 * NW, NT = D / TW;
  using SW = Swz<0, 0>;
  typedef typename VecT<E>::T V;
  __shared__ __attribute__((aligned(16))) E ws[C * KP];
  __shared__ __attribute__((aligned(16))) E kts[D * TP];
  __shared__ __attribute__((aligned(16))) E us[C * TW];
  __shared__ float dec[D];

  const int bh = blockIdx.x / NT, tile = blockIdx.x % NT;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int col = tile * TW + w * 16 + c;
  const size_t rs = (size_t)p.H * D;    // token row stride of [.., C, H, D]

  floatx4 S[D / 16];
#pragma unroll
  for (int r = 0; r < D / 16; ++r)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
      S[r][ii] = p.h0 ? p.h0[((size_t)bh * D + 16 * r + 4 * g + ii) * D + col] : 0.f;

  for (int ch = 0; ch < p.NC; ++ch) {
    const size_t base = (((size_t)b * p.NC + ch) * C * p.H + h) * D;   // token 0 of chunk, head h
    const E* wg = static_cast<const E*>(p.w) + base;
    const E* ug = static_cast<const E*>(p.u) + base;
    const E* kg = static_cast<const E*>(p.k) + base;
    for (int i = tid; i < C * (D / VE); i += NTHR) {
      const int t = i / (D / VE), d0 = (i % (D / VE)) * VE;
      *reinterpret_cast<uint4*>(ws + t * KP + d0) = *reinterpret_cast<const uint4*>(wg + t * rs + d0);
      const V x = __builtin_bit_cast(V, *reinterpret_cast<const uint4*>(kg + t * rs + d0));
#pragma unroll
      for (int e = 0; e < VE; ++e) kts[(d0 + e) * TP + t] = x[e];
    }
    for (int i = tid; i < C * TW; i += NTHR) us[i] = ug[(i / TW) * rs + tile * TW + (i % TW)];
    for (int i = tid; i < D; i += NTHR)
      dec[i] = p.perdim ? p.decay[((size_t)bh * p.NC + ch) * D + i] : p.decay[(size_t)bh * p.NC + ch];
    lds_barrier();

    // snapshot before the update
    const size_t hbase = (((size_t)b * p.NC + ch) * p.H + h) * D * D;
#pragma unroll
    for (int r = 0; r < D / 16; ++r)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        store_out(p.h_out, hbase + (size_t)(16 * r + 4 * g + ii) * D + col, S[r][ii], p.out_f32);
    // vc = u - w S   (token rows 16mb + 4g + ii, column col)
    floatx4 Vc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const floatx4 X = chain<E, NKB_D, SW>(zero4(), ws, 16 * mb + c, KP, S, NKB_D, g);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) Vc[mb][ii] = to_f32(us[(16 * mb + 4 * g + ii) * TW + w * 16 + c]) - X[ii];
    }
    // S = decay (.) S + k^T vc   (per-row decay scales state row d)
#pragma unroll
    for (int r = 0; r < D / 16; ++r) {
      floatx4 sd;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) sd[ii] = S[r][ii] * dec[16 * r + 4 * g + ii];
      S[r] = chain<E, NKB_C, SW>(sd, kts, 16 * r + c, TP, Vc, NKB_C, g);
    }
    lds_barrier();
  }
  if (p.final_state) {
#pragma unroll
    for (int r = 0; r < D / 16; ++r)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        p.final_state[((size_t)bh * D + 16 * r + 4 * g + ii) * D + col] = S[r][ii];
  }
}

}  // namespace pf
