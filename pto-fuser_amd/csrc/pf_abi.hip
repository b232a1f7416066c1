// extern "C" entry points of libptofuser_hip.so (declared in include/pto_fuser_hip.h).
//
// Host-side contract checks happen here, before anything is enqueued; kernels are launched only
// on the caller's stream, and no exec allocates or synchronises.
#include <hip/hip_runtime.h>

#include <mutex>
#include <new>

#include "../../include/pto_fuser_hip.h"
#include "pf_chunk_local.h"
#include "pf_status.h"
#include "pf_workspace.h"
#include "pf_scan_args.h"
#include "pf_scan_split.h"
#include "pf_scan_split_f32.h"

namespace {

// loader waves of the bf16 split scan kernel for 32-column and for 16-column slices
constexpr int kSplitLoaderWaves = 4, kSplit16LoaderWaves = 4;

using pf::bf16;

using GdnWorkspace = pf::Workspace;

constexpr size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

size_t elem_size(int dtype) { return dtype == PF_DTYPE_BF16 ? 2 : 4; }

bool valid_dtype(int dtype) { return dtype == PF_DTYPE_F32 || dtype == PF_DTYPE_BF16; }

// Byte layout of the fused-forward workspace:
//   [ T (M*C*C E) | P (M*C*C E, pre-scaled; fp32 only) | G (M*C fp32) | output scale (fp32, 256 B) ].
// The bf16 scan forms P from the q and k rows it stages, so the bf16 layout has no P.
struct GdnLayout {
  size_t t_off, p_off, g_off, s_off, total;
  GdnLayout(size_t M, int C, int dtype) {
    const size_t cc = M * C * C * elem_size(dtype);
    t_off = 0;
    p_off = align256(cc);
    g_off = p_off + (dtype == PF_DTYPE_BF16 ? 0 : align256(cc));
    s_off = g_off + align256(M * C * sizeof(float));
    total = s_off + 256;
  }
};

// The kernels' chunk: every forward runs 64-token chunks.  A caller's chunk size of 128 (the
// reference's) is served by the same kernels over T / 64 chunks: the chunked forward's result does
// not depend on the chunk size (each is an exact regrouping of the token recurrence), so only the
// blocking of the arithmetic differs; T must then be a multiple of 128, as the caller's chunking
// implies.
constexpr int kChunk = 64;

bool gdn_shape_ok(int B, int H, int T, int C, int DK, int DV, int dtype) {
  return B > 0 && H > 0 && T > 0 && T <= pf::kMaxChainTokens && (C == 64 || C == 128) && DK == 128 &&
         DV == 128 && T % C == 0 && valid_dtype(dtype);
}

// CUs of the device current at the first call (queried once, thread-safe; 256, MI355X's count,
// if the query fails).
int device_cu_count() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      return n;
    return 256;
  }();
  return cus;
}

template <typename E>
void chunk_local_launch(const void* q, const void* k, const float* beta, const float* g,
                       float scale, char* base, size_t M, hipStream_t stream) {
  constexpr int C = 64, DK = 128;
  const GdnLayout lay(M, C, std::is_same<E, bf16>::value ? PF_DTYPE_BF16 : PF_DTYPE_F32);
  pf::ChunkLocalArgs a{};
  a.k = k;
  a.q = q;
  a.beta = beta;
  a.g = g;
  a.G_out = reinterpret_cast<float*>(base + lay.g_off);
  a.T_out = base + lay.t_off;
  a.P_out = std::is_same<E, bf16>::value ? nullptr : base + lay.p_off;
  a.A_out = nullptr;
  a.M = static_cast<int>(M);
  a.g_is_cumsum = 0;
  a.t_lower_only = 1;   // the scan kernels read T's rows 0..31 up to column 31 only
  a.p_scale = scale;
  a.scale_out = reinterpret_cast<float*>(base + lay.s_off);
  if constexpr (std::is_same<E, bf16>::value) {   // no P: the bf16 scan forms it from its q, k rows
    pf::chunk_local_kernel<E, E, C, DK, false, true><<<dim3((unsigned)M), dim3(256), 0, stream>>>(a);
  } else {
    // fp32 with P: when the chunks fit one generation of workgroups (short sequences, few
    // chains), P gets workgroups of its own, which halves each workgroup's products
    a.split_p = M <= (size_t)device_cu_count() ? 1 : 0;
    const unsigned grid = (unsigned)(a.split_p ? 2 * M : M);
    pf::chunk_local_kernel<E, E, C, DK, true, true><<<dim3(grid), dim3(256), 0, stream>>>(a);
  }
}

template <typename E>
void scan_output_launch(const void* q, const void* k, const void* v, const float* beta,
                       const float* h0, float* o, float* h_final, int BH, int NC,
                       char* base, hipStream_t stream) {
  constexpr int C = 64, DK = 128, DV = 128;
  const size_t M = (size_t)BH * NC;
  const GdnLayout lay(M, C, std::is_same<E, bf16>::value ? PF_DTYPE_BF16 : PF_DTYPE_F32);
  pf::ScanOutArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.beta = beta;
  a.G = reinterpret_cast<const float*>(base + lay.g_off);
  a.Tm = base + lay.t_off;
  a.P = base + lay.p_off;
  a.h0 = h0;
  a.o = o;
  a.h_final = h_final;
  a.BH = BH;
  a.NC = NC;
  a.scale = reinterpret_cast<const float*>(base + lay.s_off);
  if constexpr (std::is_same<E, bf16>::value) {
    // bf16: one workgroup per (chain, 32-column slice), or 16-column slices when 32 would leave
    // CUs idle (fewer than 8 chains per 32 CUs: long sequences at small batch); four MFMA waves
    // split every chunk (pf_scan_split.h)
    if ((size_t)BH * (DV / 32) < (size_t)device_cu_count())
      pf::scan_split_kernel<C, DK, DV, 1, kSplit16LoaderWaves>
          <<<dim3((unsigned)(BH * (DV / 16))), dim3(64 * (4 + kSplit16LoaderWaves)), 0, stream>>>(a);
    else
      pf::scan_split_kernel<C, DK, DV, 2, kSplitLoaderWaves>
          <<<dim3((unsigned)(BH * (DV / 32))), dim3(64 * (4 + kSplitLoaderWaves)), 0, stream>>>(a);
  } else {
    // fp32: one workgroup per (chain, 16-column slice), every chunk split over four waves
    // (pf_scan_split_f32.h)
    pf::scan_split_f32_kernel<C, DK, DV><<<dim3((unsigned)(BH * (DV / 16))), dim3(256), 0, stream>>>(a);
  }
}

// Both stages of the forward on the workspace at `base` (the layout of GdnLayout).
int gdn_forward_on(char* base, const void* q, const void* k, const void* v, const float* beta,
                   const float* g, const float* h0, float* o, float* h_final, int B, int H, int T,
                   int C, int dtype, float scale, hipStream_t s) {
  const size_t M = (size_t)B * H * (T / kChunk);
  pf::LaunchScope scope;
  if (dtype == PF_DTYPE_BF16) {
    chunk_local_launch<bf16>(q, k, beta, g, scale, base, M, s);
    scan_output_launch<bf16>(q, k, v, beta, h0, o, h_final, B * H, T / kChunk, base, s);
  } else {
    chunk_local_launch<float>(q, k, beta, g, scale, base, M, s);
    scan_output_launch<float>(q, k, v, beta, h0, o, h_final, B * H, T / kChunk, base, s);
  }
  return scope.status();
}

// Shared host checks of the three GDN entry points.
int gdn_check(int B, int H, int T, int C, int DK, int DV, int dtype, const void* ws) {
  if (!gdn_shape_ok(B, H, T, C, DK, DV, dtype)) return PF_ERR_ARG;
  const GdnWorkspace* w = static_cast<const GdnWorkspace*>(ws);
  if (!w || !w->base || w->bytes < GdnLayout((size_t)B * H * (T / kChunk), kChunk, dtype).total)
    return PF_ERR_WORKSPACE;
  return PF_OK;
}

// ---- the allocation-free forward ---------------------------------------------------------
// Its workspace is this file-scope array, 40 MiB: the bf16 headline shape (B4 H16 T4096, 4096
// chunks: T 32 MiB, G 1 MiB) fits with room to spare; bf16 up to 4 964 chunks of 64 tokens, fp32
// (T and P) up to 1 270.  Every GPU the library runs on holds one copy until the process ends.
constexpr size_t kStaticScratchBytes = size_t(40) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// Device address of `scratch` on the current device, resolved once per device with
// hipGetSymbolAddress (in host code the array's name is only a host-side stand-in, never a
// device address).  Returns nullptr with *status set when the lookup fails.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

void* scratch_on_current_device(int* status) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *status = e != hipSuccess ? static_cast<int>(e) : PF_ERR_ARG;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *status = e != hipSuccess ? static_cast<int>(e) : PF_ERR_ARG;
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

const char* pf_status_string(int status) {
  switch (status) {
    case PF_OK: return "ok";
    case PF_ERR_ARG: return "invalid argument (shape, dtype or pointer contract)";
    case PF_ERR_WORKSPACE: return "workspace missing or too small for this call";
    case PF_ERR_ALLOC: return "workspace allocation failed";
    case PF_ERR_SCRATCH: return "input needs more than the static scratch of pf_gdn_exec_static";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

int pf_abi_version(void) { return 2; }

#ifndef PF_SOURCE_HASH
#define PF_SOURCE_HASH "unknown"
#endif
const char* pf_source_hash(void) { return PF_SOURCE_HASH; }

size_t pf_gdn_workspace_bytes(int B, int H, int T, int C, int DK, int DV, int dtype) {
  if (!gdn_shape_ok(B, H, T, C, DK, DV, dtype)) return 0;
  return GdnLayout((size_t)B * H * (T / kChunk), kChunk, dtype).total;
}

void* pf_gdn_create(void) { return pf::workspace_create(); }

int pf_gdn_reserve(void* ws, int B, int H, int T, int C, int DK, int DV, int dtype) {
  const size_t bytes = pf_gdn_workspace_bytes(B, H, T, C, DK, DV, dtype);
  if (bytes == 0) return PF_ERR_ARG;
  return pf::workspace_reserve(static_cast<GdnWorkspace*>(ws), bytes);
}

void* pf_gdn_setup(int B, int H, int T, int C, int DK, int DV, int dtype) {
  if (pf_gdn_workspace_bytes(B, H, T, C, DK, DV, dtype) == 0) return nullptr;
  GdnWorkspace* ws = pf::workspace_create();
  if (ws && pf_gdn_reserve(ws, B, H, T, C, DK, DV, dtype) != PF_OK) {
    pf::workspace_destroy(ws);
    return nullptr;
  }
  return ws;
}

void pf_gdn_teardown(void* ws) { pf::workspace_destroy(static_cast<GdnWorkspace*>(ws)); }

int pf_gdn_chunk_local_exec(const void* q, const void* k, const float* beta, const float* g,
                            int B, int H, int T, int C, int DK, int DV, int dtype, float scale,
                            void* ws, void* stream) {
  const int st = gdn_check(B, H, T, C, DK, DV, dtype, ws);
  if (st != PF_OK) return st;
  if (!q || !k || !beta) return PF_ERR_ARG;
  const GdnWorkspace* w = static_cast<const GdnWorkspace*>(ws);
  const size_t M = (size_t)B * H * (T / kChunk);
  hipStream_t s = static_cast<hipStream_t>(stream);
  pf::LaunchScope scope;
  if (dtype == PF_DTYPE_BF16)
    chunk_local_launch<bf16>(q, k, beta, g, scale, static_cast<char*>(w->base), M, s);
  else
    chunk_local_launch<float>(q, k, beta, g, scale, static_cast<char*>(w->base), M, s);
  return scope.status();
}

int pf_gdn_scan_output_exec(const void* q, const void* k, const void* v, const float* beta,
                            const float* h0, float* o, float* h_final, int B, int H, int T, int C,
                            int DK, int DV, int dtype, void* ws, void* stream) {
  const int st = gdn_check(B, H, T, C, DK, DV, dtype, ws);
  if (st != PF_OK) return st;
  if (!q || !k || !v || !beta || !o) return PF_ERR_ARG;
  const GdnWorkspace* w = static_cast<const GdnWorkspace*>(ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  pf::LaunchScope scope;
  if (dtype == PF_DTYPE_BF16)
    scan_output_launch<bf16>(q, k, v, beta, h0, o, h_final, B * H, T / kChunk,
                             static_cast<char*>(w->base), s);
  else
    scan_output_launch<float>(q, k, v, beta, h0, o, h_final, B * H, T / kChunk,
                              static_cast<char*>(w->base), s);
  return scope.status();
}

int pf_gdn_exec(const void* q, const void* k, const void* v, const float* beta, const float* g,
                const float* h0, float* o, float* h_final, int B, int H, int T, int C, int DK,
                int DV, int dtype, float scale, void* ws, void* stream) {
  const int st = gdn_check(B, H, T, C, DK, DV, dtype, ws);
  if (st != PF_OK) return st;
  if (!q || !k || !v || !beta || !o) return PF_ERR_ARG;
  return gdn_forward_on(static_cast<char*>(static_cast<GdnWorkspace*>(ws)->base), q, k, v, beta,
                        g, h0, o, h_final, B, H, T, C, dtype, scale,
                        static_cast<hipStream_t>(stream));
}

int pf_gdn_exec_static(const void* q, const void* k, const void* v, const float* beta,
                       const float* g, const float* h0, float* o, float* h_final, int B, int H,
                       int T, int C, int DK, int DV, int dtype, float scale, void* stream) {
  if (!gdn_shape_ok(B, H, T, C, DK, DV, dtype)) return PF_ERR_ARG;
  if (GdnLayout((size_t)B * H * (T / kChunk), kChunk, dtype).total > kStaticScratchBytes)
    return PF_ERR_SCRATCH;
  if (!q || !k || !v || !beta || !o) return PF_ERR_ARG;
  int st = PF_OK;
  void* base = scratch_on_current_device(&st);
  if (!base) return st;
  return gdn_forward_on(static_cast<char*>(base), q, k, v, beta, g, h0, o, h_final, B, H, T, C,
                        dtype, scale, static_cast<hipStream_t>(stream));
}

int pf_kkt_inv_exec(const void* k, const float* g, const float* beta, float* A_out, float* T_out,
                    int M, int C, int DK, int dtype, int g_is_cumsum, void* stream) {
  if (M <= 0 || C != 64 || DK != 128 || !valid_dtype(dtype)) return PF_ERR_ARG;
  if (!k || !beta || !T_out) return PF_ERR_ARG;
  pf::ChunkLocalArgs a{};
  a.k = k;
  a.q = nullptr;
  a.beta = beta;
  a.g = g;
  a.G_out = nullptr;
  a.T_out = T_out;
  a.P_out = nullptr;
  a.A_out = A_out;
  a.M = M;
  a.g_is_cumsum = g_is_cumsum ? 1 : 0;
  a.t_lower_only = 0;   // T_out is the caller's: the whole matrix, zeros above the diagonal
  a.p_scale = 1.f;
  a.scale_out = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  pf::LaunchScope scope;
  if (dtype == PF_DTYPE_BF16)
    pf::chunk_local_kernel<bf16, float, 64, 128, false, true><<<dim3((unsigned)M), dim3(256), 0, s>>>(a);
  else
    pf::chunk_local_kernel<float, float, 64, 128, false, true><<<dim3((unsigned)M), dim3(256), 0, s>>>(a);
  return scope.status();
}

int pf_tri_inv_exec(const float* A, float* T_out, int M, int C, void* stream) {
  if (M <= 0 || !A || !T_out) return PF_ERR_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  pf::LaunchScope scope;
  switch (C) {
    case 16: pf::tri_inv_kernel<16><<<dim3((unsigned)M), dim3(256), 0, s>>>(A, T_out, M); break;
    case 32: pf::tri_inv_kernel<32><<<dim3((unsigned)M), dim3(256), 0, s>>>(A, T_out, M); break;
    case 48: pf::tri_inv_kernel<48><<<dim3((unsigned)M), dim3(256), 0, s>>>(A, T_out, M); break;
    case 64: pf::tri_inv_kernel<64><<<dim3((unsigned)M), dim3(256), 0, s>>>(A, T_out, M); break;
    case 128: pf::tri_inv_kernel<128><<<dim3((unsigned)M), dim3(256), 0, s>>>(A, T_out, M); break;
    default: return PF_ERR_ARG;
  }
  return scope.status();
}

}  // extern "C"
