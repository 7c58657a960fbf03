// CROWN adaptive ReLU relaxation of one neuron, in registers.
// Same arithmetic, in the same order and precision, as _make_slopes
// (verify_zono_bnb.py:503-522):
//   lb_r = min(lo, 0); ub_r = max(max(hi, 0), lb_r + 1e-8)
//   up_s = ub_r / (ub_r - lb_r); up_t = -lb_r * up_s
//   active = lo >= 0; dead = hi <= 0; unstable = !active && !dead
//   lo_s = 1 if active, (up_s > 0.5) if unstable, else 0
// Division is IEEE correctly rounded (the library is built without
// fast-math), so up_s / up_t are bit-identical to the fp32 torch values.
#pragma once
#include <hip/hip_runtime.h>

struct Relax {
  float lo_s, up_s, up_t;
  bool active, dead, unstable;
};

__device__ __forceinline__ Relax relax(float lo, float hi) {
  Relax s;
  const float lb_r = fminf(lo, 0.f);
  const float ub_r = fmaxf(fmaxf(hi, 0.f), lb_r + 1e-8f);
  s.up_s = ub_r / (ub_r - lb_r);
  s.up_t = -lb_r * s.up_s;
  s.active = lo >= 0.f;
  s.dead = hi <= 0.f;
  s.unstable = !s.active && !s.dead;
  s.lo_s = s.active ? 1.f : ((s.unstable && s.up_s > 0.5f) ? 1.f : 0.f);
  return s;
}
