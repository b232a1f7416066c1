// extern "C" entry points of the stage kernels (declared in include/pto_fuser_hip.h).
// Shapes are runtime arguments dispatched onto compile-time instantiations; anything outside the
// supported set is rejected on the host with PF_ERR_ARG before a launch.
#include <hip/hip_runtime.h>

#include "../../include/pto_fuser_hip.h"
#include "pf_stages.h"
#include "pf_status.h"

namespace {

using pf::bf16;


// Supported (C, D): C in {16, 32, 64, 128} (bf16 needs C >= 32: one bf16 MFMA contracts 32 rows),
// D in {64, 128}.
bool stage_shape_ok(int C, int D, int dtype) {
  if (dtype != PF_DTYPE_F32 && dtype != PF_DTYPE_BF16) return false;
  if (D != 64 && D != 128) return false;
  if (C != 16 && C != 32 && C != 64 && C != 128) return false;
  return !(dtype == PF_DTYPE_BF16 && C < 32);
}

// Calls f.template operator()<E, C, D>() for the runtime (dtype, C, D).
template <class F>
int dispatch(int dtype, int C, int D, F&& f) {
#define PF_STAGE_CASE(E, CC, DD) \
  if (C == CC && D == DD) return f.template operator()<E, CC, DD>();
  if (dtype == PF_DTYPE_BF16) {
    PF_STAGE_CASE(bf16, 32, 64) PF_STAGE_CASE(bf16, 32, 128)
    PF_STAGE_CASE(bf16, 64, 64) PF_STAGE_CASE(bf16, 64, 128)
    PF_STAGE_CASE(bf16, 128, 64) PF_STAGE_CASE(bf16, 128, 128)
  } else {
    PF_STAGE_CASE(float, 16, 64) PF_STAGE_CASE(float, 16, 128)
    PF_STAGE_CASE(float, 32, 64) PF_STAGE_CASE(float, 32, 128)
    PF_STAGE_CASE(float, 64, 64) PF_STAGE_CASE(float, 64, 128)
    PF_STAGE_CASE(float, 128, 64) PF_STAGE_CASE(float, 128, 128)
  }
#undef PF_STAGE_CASE
  return PF_ERR_ARG;
}

struct GatedQkLaunch {
  pf::GatedQkArgs a;
  unsigned grid;
  hipStream_t s;
  template <typename E, int C, int D>
  int operator()() {
    pf::LaunchScope scope;
    pf::gated_qk_kernel<E, C, D><<<dim3(grid), dim3(256), 0, s>>>(a);
    return scope.status();
  }
};

struct QkvFlashLaunch {
  pf::QkvFlashArgs a;
  unsigned grid;
  hipStream_t s;
  template <typename E, int C, int D>
  int operator()() {
    pf::LaunchScope scope;
    pf::qkv_flash_kernel<E, C, D><<<dim3(grid), dim3(256), 0, s>>>(a);
    return scope.status();
  }
};

struct ScanLaunch {
  pf::ScanStateArgs a;
  int BH;
  hipStream_t s;
  template <typename E, int C, int D>
  int operator()() {
    constexpr int NW = 2;
    const unsigned grid = (unsigned)(BH * (D / (16 * NW)));
    pf::LaunchScope scope;
    pf::scan_state_kernel<E, C, D, NW><<<dim3(grid), dim3(64 * NW), 0, s>>>(a);
    return scope.status();
  }
};

}  // namespace

extern "C" {

int pf_gated_qk_exec(const void* a, const void* b, const float* a_scale, const float* b_scale,
                     const float* g, const float* beta, const float* mask, void* L, int nc, int H,
                     int C, int D, int dtype, int causal, int out_dtype, void* stream) {
  if (!a || !b || !L || nc <= 0 || H <= 0 || !stage_shape_ok(C, D, dtype)) return PF_ERR_ARG;
  if (out_dtype != PF_DTYPE_F32 && out_dtype != PF_DTYPE_BF16) return PF_ERR_ARG;
  if ((size_t)nc * H > 0x7fffffffu) return PF_ERR_ARG;
  GatedQkLaunch l{};
  l.a = pf::GatedQkArgs{a, b, a_scale, b_scale, g, beta, mask, L, H, causal ? 1 : 0,
                        out_dtype == PF_DTYPE_F32 ? 1 : 0};
  l.grid = (unsigned)(nc * H);
  l.s = static_cast<hipStream_t>(stream);
  return dispatch(dtype, C, D, l);
}

int pf_qkv_flash_exec(const void* q, const void* k, const void* v, const float* q_scale,
                      const float* k_scale, const float* g, const float* beta, float* o, int M,
                      int C, int D, int dtype, void* stream) {
  if (!q || !k || !v || !o || M <= 0 || !stage_shape_ok(C, D, dtype)) return PF_ERR_ARG;
  QkvFlashLaunch l{};
  l.a = pf::QkvFlashArgs{q, k, v, q_scale, k_scale, g, beta, o};
  l.grid = (unsigned)M;
  l.s = static_cast<hipStream_t>(stream);
  return dispatch(dtype, C, D, l);
}

int pf_scan_exec(const void* w, const void* u, const void* k, const float* decay,
                 const float* h0, void* h_out, float* final_state, int B, int H, int nc, int C,
                 int D, int dtype, int perdim, int out_dtype, void* stream) {
  if (!w || !u || !k || !decay || !h_out || B <= 0 || H <= 0 || nc <= 0) return PF_ERR_ARG;
  if (!stage_shape_ok(C, D, dtype)) return PF_ERR_ARG;
  if (out_dtype != PF_DTYPE_F32 && out_dtype != PF_DTYPE_BF16) return PF_ERR_ARG;
  ScanLaunch l{};
  l.a = pf::ScanStateArgs{w, u, k, decay, h0, h_out, final_state, H, nc, perdim ? 1 : 0,
                          out_dtype == PF_DTYPE_F32 ? 1 : 0};
  l.BH = B * H;
  l.s = static_cast<hipStream_t>(stream);
  return dispatch(dtype, C, D, l);
}

// The stage kernels hold no state between calls: setup returns NULL (the recipe's workspace
// handle) and teardown accepts it, so a recipe that names setup_sym / teardown_sym binds them.
void* pf_gated_qk_setup(void) { return nullptr; }
void pf_gated_qk_teardown(void* ws) { (void)ws; }
void* pf_qkv_flash_setup(void) { return nullptr; }
void pf_qkv_flash_teardown(void* ws) { (void)ws; }
void* pf_scan_setup(void) { return nullptr; }
void pf_scan_teardown(void* ws) { (void)ws; }

}  // extern "C"
