// Device workspace handle shared by the fused forwards: one grow-only device buffer.
//
// A handle is created empty (no allocation) and sized by `reserve`, which allocates only when the
// requested size exceeds what it holds.  Growing waits for the device to go idle before freeing
// the old buffer, so work still queued on it finishes first.  After the first reserve for the
// largest shape a caller uses, later reserves allocate nothing (safe under HIP graph capture).
#pragma once

#include <hip/hip_runtime.h>

#include <new>

#include "../../include/pto_fuser_hip.h"

namespace pf {

struct Workspace {
  void* base = nullptr;
  size_t bytes = 0;
};

inline Workspace* workspace_create() { return new (std::nothrow) Workspace(); }

inline int workspace_reserve(Workspace* w, size_t bytes) {
  if (!w || bytes == 0) return PF_ERR_ARG;
  if (w->bytes >= bytes) return PF_OK;
  if (w->base) {
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return static_cast<int>(e);
    (void)hipFree(w->base);
    w->base = nullptr;
    w->bytes = 0;
  }
  if (hipMalloc(&w->base, bytes) != hipSuccess) {
    w->base = nullptr;
    return PF_ERR_ALLOC;
  }
  w->bytes = bytes;
  return PF_OK;
}

inline void workspace_destroy(Workspace* w) {
  if (!w) return;
  if (w->base) (void)hipFree(w->base);
  delete w;
}

}  // namespace pf
