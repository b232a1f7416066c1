// Launch arguments of the stage-2 kernels (the state scan fused with the output): the bf16 split
// scan (pf_scan_split.h) and the fp32 split scan (pf_scan_split_f32.h).
#pragma once

#include "pf_device.h"

namespace pf {

struct ScanOutArgs {
  const void* q;        // [BH*T, DK]  E
  const void* k;        // [BH*T, DK]  E
  const void* v;        // [BH*T, DV]  E
  const float* beta;    // [BH*T]
  const float* G;       // [BH*T] within-chunk cumsum of the log decay, from stage 1
  const void* Tm;       // [M, C, C]   E  (I + A)^-1 per chunk, from stage 1
  const void* P;        // [M, C, C]   E  gated causal score (fp32 operands only), from stage 1
  const float* h0;      // [BH, DK, DV] or null
  float* o;             // [BH*T, DV]
  float* h_final;       // [BH, DK, DV] or null
  int BH;
  int NC;               // chunks per chain
  const float* scale;   // device scalar: the output scale (written by stage 1)
};

}  // namespace pf
