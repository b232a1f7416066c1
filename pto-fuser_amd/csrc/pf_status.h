// Launch status of the extern "C" entry points.
//
// hipGetLastError() returns (and clears) the last error of ANY earlier runtime call on this
// thread, so reading it only after a launch would report an unrelated earlier failure as this
// call's.  Every exec therefore takes a LaunchScope before its first launch: the constructor
// clears whatever error is pending (it belongs to an earlier call, whose own caller had its chance
// to read it), and status() afterwards reports only what the launches in between left.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/pto_fuser_hip.h"

namespace pf {

struct LaunchScope {
  LaunchScope() { (void)hipGetLastError(); }
  int status() const {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? PF_OK : static_cast<int>(e);
  }
};

}  // namespace pf
