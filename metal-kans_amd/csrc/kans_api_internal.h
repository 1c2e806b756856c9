// Internal declarations shared by the runtime and kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include "kans_common.h"
#include "../../include/kans_hip.h"

namespace kans {

// One fused dense launch (see kans_dense.hip).
struct DenseLaunch {
  int dtype, basis, has_base;
  int x_dtype, y_dtype;  // element types of X and Y: dtype, or DT_F32
  const void* X; long ldx;
  const void* Wt; int nob_pad;
  const void* bias;
  void* Y; long ldy;
  float* part;          // split workspace (splits * B * D_out floats) or null
  int B, D_in, D_out, nfb;
  BasisParams bp;
  int wm, nb, splits;   // tile config
};

}  // namespace kans

int kans_fail(int code, const char* fmt, ...);
hipStream_t kans_default_stream();
