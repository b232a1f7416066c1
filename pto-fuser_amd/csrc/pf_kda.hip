// extern "C" entry points of the fused KDA forward (declared in include/pto_fuser_hip.h).
#include <hip/hip_runtime.h>

#include <new>

#include "../../include/pto_fuser_hip.h"
#include "pf_kda.h"
#include "pf_kda_scan.h"
#include "pf_kda_f32.h"
#include "pf_status.h"
#include "pf_workspace.h"

namespace {

using pf::bf16;

constexpr size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

using KdaWorkspace = pf::Workspace;

// Byte layout of the KDA workspace, M = B*H*T/C chunks:
//   fp32 operands  [ W | U | QE | KR  (each M*C*128 fp32) | P (M*C*C fp32) | DEC (M*128 fp32) ]
//   bf16 operands  [ W (M*C*128) | T diag(beta) (M*C*C) | QE | k e^-G (M*C*128 each) | DEC ]
// (bf16 stage 2 forms U and the score itself: nothing in P's place.)
struct KdaLayout {
  size_t w_off, u_off, q_off, k_off, p_off, d_off, total;
  KdaLayout(size_t M, int C, int D, int dtype) {
    const bool b16 = dtype == PF_DTYPE_BF16;
    const size_t esize = b16 ? sizeof(bf16) : sizeof(float);
    const size_t tile = align256(M * C * D * esize);
    const size_t square = align256(M * C * C * esize);
    w_off = 0;
    u_off = w_off + tile;
    q_off = u_off + (b16 ? square : tile);
    k_off = q_off + tile;
    p_off = k_off + tile;
    d_off = p_off + (b16 ? 0 : square);
    total = d_off + align256(M * D * sizeof(float));
  }
};

// bf16 operands (pf_kda.h) or fp32 operands (the fp32 kernels of pf_kda_f32.h); dk = dv = 128.
// 64-token chunks in the kernels; a caller's chunk size of 128 runs them over T / 64 chunks (the
// chunked forward's result does not depend on the chunk size), with T a multiple of 128.
constexpr int kChunk = 64;

bool kda_shape_ok(int B, int H, int T, int C, int DK, int DV, int dtype) {
  return B > 0 && H > 0 && T > 0 && T <= pf::kMaxChainTokens && (C == 64 || C == 128) &&
         DK == 128 && DV == 128 && T % C == 0 &&
         (dtype == PF_DTYPE_BF16 || dtype == PF_DTYPE_F32);
}

}  // namespace

extern "C" {

size_t pf_kda_workspace_bytes(int B, int H, int T, int C, int DK, int DV, int dtype) {
  if (!kda_shape_ok(B, H, T, C, DK, DV, dtype)) return 0;
  return KdaLayout((size_t)B * H * (T / kChunk), kChunk, DK, dtype).total;
}

void* pf_kda_create(void) { return pf::workspace_create(); }

int pf_kda_reserve(void* ws, int B, int H, int T, int C, int DK, int DV, int dtype) {
  const size_t bytes = pf_kda_workspace_bytes(B, H, T, C, DK, DV, dtype);
  if (bytes == 0) return PF_ERR_ARG;
  return pf::workspace_reserve(static_cast<KdaWorkspace*>(ws), bytes);
}

void* pf_kda_setup(int B, int H, int T, int C, int DK, int DV, int dtype) {
  if (pf_kda_workspace_bytes(B, H, T, C, DK, DV, dtype) == 0) return nullptr;
  KdaWorkspace* ws = pf::workspace_create();
  if (ws && pf_kda_reserve(ws, B, H, T, C, DK, DV, dtype) != PF_OK) {
    pf::workspace_destroy(ws);
    return nullptr;
  }
  return ws;
}

void pf_kda_teardown(void* ws) { pf::workspace_destroy(static_cast<KdaWorkspace*>(ws)); }

int pf_kda_exec(const void* q, const void* k, const void* v, const float* beta, const float* g,
                const float* h0, float* o, float* h_final, int B, int H, int T, int C, int DK,
                int DV, int dtype, float scale, void* ws, void* stream) {
  if (!kda_shape_ok(B, H, T, C, DK, DV, dtype)) return PF_ERR_ARG;
  const KdaWorkspace* w = static_cast<const KdaWorkspace*>(ws);
  const size_t M = (size_t)B * H * (T / kChunk);
  const KdaLayout lay(M, kChunk, DK, dtype);
  if (!w || !w->base || w->bytes < lay.total) return PF_ERR_WORKSPACE;
  if (!q || !k || !v || !beta || !g || !o) return PF_ERR_ARG;
  constexpr int KC = 64, KD = 128;
  char* base = static_cast<char*>(w->base);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PF_DTYPE_F32) {
    pf::KdaLocalF32Args la{};
    la.q = static_cast<const float*>(q);
    la.k = static_cast<const float*>(k);
    la.v = static_cast<const float*>(v);
    la.g = g;
    la.beta = beta;
    la.scale = scale;
    la.W = reinterpret_cast<float*>(base + lay.w_off);
    la.U = reinterpret_cast<float*>(base + lay.u_off);
    la.QE = reinterpret_cast<float*>(base + lay.q_off);
    la.KR = reinterpret_cast<float*>(base + lay.k_off);
    la.P = reinterpret_cast<float*>(base + lay.p_off);
    la.DEC = reinterpret_cast<float*>(base + lay.d_off);
    pf::LaunchScope scope;
    pf::kda_local_f32_kernel<KC, KD><<<dim3((unsigned)M), dim3(256), 0, s>>>(la);
    pf::KdaScanF32Args sa{};
    sa.W = la.W;
    sa.U = la.U;
    sa.QE = la.QE;
    sa.KR = la.KR;
    sa.P = la.P;
    sa.DEC = la.DEC;
    sa.h0 = h0;
    sa.o = o;
    sa.h_final = h_final;
    sa.BH = B * H;
    sa.NC = T / kChunk;
    pf::kda_scan_f32_kernel<KC, KD, KD><<<dim3((unsigned)(B * H * (KD / 32))), dim3(128), 0, s>>>(sa);
    return scope.status();
  }

  pf::KdaLocalArgs la{};
  la.q = static_cast<const bf16*>(q);
  la.k = static_cast<const bf16*>(k);
  la.g = g;
  la.beta = beta;
  la.scale = scale;
  la.W = reinterpret_cast<bf16*>(base + lay.w_off);
  la.TB = reinterpret_cast<bf16*>(base + lay.u_off);
  la.QE = reinterpret_cast<bf16*>(base + lay.q_off);
  la.KB = reinterpret_cast<bf16*>(base + lay.k_off);
  la.DEC = reinterpret_cast<float*>(base + lay.d_off);
  pf::LaunchScope scope;
  pf::kda_local_kernel<KC, KD, KD><<<dim3((unsigned)M), dim3(256), 0, s>>>(la);
  const int st = scope.status();
  if (st != PF_OK) return st;

  pf::KdaScanArgs sa{};
  sa.W = la.W;
  sa.TB = la.TB;
  sa.v = static_cast<const bf16*>(v);
  sa.QE = la.QE;
  sa.KB = la.KB;
  sa.DEC = la.DEC;
  sa.h0 = h0;
  sa.o = o;
  sa.h_final = h_final;
  sa.BH = B * H;
  sa.NC = T / kChunk;
  constexpr int NLW = 4;
  const unsigned grid = (unsigned)(B * H * (KD / 32));
  pf::kda_scan_split_kernel<KC, KD, KD, NLW><<<dim3(grid), dim3(64 * (4 + NLW)), 0, s>>>(sa);
  return scope.status();
}

}  // extern "C"
