// Host-side helpers shared by the launchers of the C ABI (include/flashlazy.h).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

#include "flashlazy.h"

namespace fla {

// alpha-specialised code paths: 1 -> alpha = 1.5 (p = t^2), 2 -> alpha = 2 (p = t), 0 -> any.
inline int alpha_mode(float alpha) {
  if (fabsf(alpha - 1.5f) < 1e-7f) return 1;
  if (fabsf(alpha - 2.0f) < 1e-7f) return 2;
  return 0;
}

}  // namespace fla
