// Shared helpers for the vibecheck_amd HIP library (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vibecheck_amd.h"

#define VC_WAVE 64

typedef float v4f __attribute__((ext_vector_type(4)));

// One 16x16x4 fp32 MFMA step on a single 16x16 block.
// Operand layout for lane l (0..63), g = l / 16, r = l % 16:
//   a  = A[row r][k g]          (A is 16 x 4)
//   b  = B[k g][col r]          (B is 4 x 16)
//   acc[i] = D[row 4*g + i][col r]
__device__ __forceinline__ v4f mfma16x16x4(float a, float b, v4f acc) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
}

#define VC_LAUNCH_CHECK()                                   \
  do {                                                      \
    hipError_t _e = hipGetLastError();                      \
    if (_e != hipSuccess) return VC_ERR_LAUNCH;             \
  } while (0)

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static inline int vc_blocks(int64_t n, int threads) {
  int64_t b = (n + threads - 1) / threads;
  if (b < 1) b = 1;
  if (b > 1048576) b = 1048576;
  return (int)b;
}

// Compensated accumulation (Knuth TwoSum): s holds the rounded running sum,
// c the accumulated rounding error; the result is s + c.  Exact as written
// because the library is compiled without contraction or reassociation.
__device__ __forceinline__ void two_sum_acc(float& s, float& c, float t) {
  const float x = s + t;
  const float bp = x - s;
  const float err = (s - (x - bp)) + (t - bp);
  s = x;
  c += err;
}

struct KSum {
  float s = 0.f, c = 0.f;
  __device__ __forceinline__ void add(float t) { two_sum_acc(s, c, t); }
  __device__ __forceinline__ float value() const { return s + c; }
};

// Wave-wide sum of compensated partials, compensated through the tree.
__device__ __forceinline__ float wave_sum_comp(KSum k) {
  float s = k.s, c = k.c;
  for (int o = 32; o > 0; o >>= 1) {
    const float so = __shfl_xor(s, o, 64);
    const float co = __shfl_xor(c, o, 64);
    two_sum_acc(s, c, so);
    c += co;
  }
  return s + c;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// torch.optim.Adam's scalars (amsgrad off, no weight decay), rounded to fp32
// the way torch rounds them: the lerp/addcmul weights 1 - beta are formed in
// double and then cast, like torch's Python-float scalars.
struct AdamConst {
  float w1, b2, w2, eps, neg_step, bc2;
};

// The Adam constants of the (up to VC_ALPHA_CHUNK, vibecheck_amd.h)
// iterations one alpha-CROWN launch runs back to back.
struct AdamChunk {
  AdamConst c[VC_ALPHA_CHUNK];
  int n;
};

// vc_alpha_control over n_it consecutive iterations (lbs: n_it x n),
// stopping at the first stop (vc_elementwise.hip).  stop_host (nullable):
// two pinned words, [0] set at a stop, [1] = it0 + n_it once all n_it
// iterations have been taken.
int alpha_control_chunk(float* best, const float* lbs, int64_t n, int it0, int n_it, double eps,
                        float* ctl, int32_t* stop_host, hipStream_t stream);

static inline AdamConst adam_const(double b1, double b2, double eps, double step_size,
                                   double bc2_sqrt) {
  AdamConst c;
  c.w1 = (float)(1.0 - b1);
  c.b2 = (float)b2;
  c.w2 = (float)(1.0 - b2);
  c.eps = (float)eps;
  c.neg_step = (float)(-step_size);
  c.bc2 = (float)bc2_sqrt;
  return c;
}

// One Adam update of one parameter p with gradient g (of the loss), in
// torch's operation order and rounding:
//   exp_avg.lerp_(g, w1)             m = fma(w1, g - m, m)   (w1 < 0.5)
//   exp_avg_sq.mul_(b2).addcmul_(g, g, value=w2)
//                                    v = fma(w2 * g, g, v * b2)
//   denom = sqrt(v) / bc2 + eps;  p.addcdiv_(m, denom, value=-step)
//                                    p + (-step * m) / denom
// sqrt and divide correctly rounded.
__device__ __forceinline__ float adam_update(float p, float g, float& m, float& v,
                                             const AdamConst& c) {
  m = c.w1 < 0.5f ? __builtin_fmaf(c.w1, g - m, m) : __builtin_fmaf(c.w1 - 1.f, g - m, g);
  v = __builtin_fmaf(c.w2 * g, g, v * c.b2);
  const float denom = __fdiv_rn(__fsqrt_rn(v), c.bc2) + c.eps;
  return p + __fdiv_rn(c.neg_step * m, denom);
}

// ---- reductions within a row of 16 lanes (lanes 16 g .. 16 g + 15) by DPP
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror:
// each step adds the value of a partner lane of the same row, so after the
// four steps every lane holds its row's total, bit-identical across the row.
__device__ __forceinline__ int dpp_row_xchg(int v, int step) {
  switch (step) {
    case 0: return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
    case 1: return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
    case 2: return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);
    default: return __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true);
  }
}

__device__ __forceinline__ float row_sum16(float v) {
#pragma unroll
  for (int s = 0; s < 4; ++s) v += __int_as_float(dpp_row_xchg(__float_as_int(v), s));
  return v;
}

__device__ __forceinline__ double row_sum16(double v) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_row_xchg((int)(b & 0xffffffffll), s);
    const int hi = dpp_row_xchg((int)(b >> 32), s);
    v += __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
  }
  return v;
}

// Sum over the wave (every lane active): DPP row sums, then the four row
// totals read from lanes 0, 16, 32, 48 and added in a fixed order.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v = row_sum16(v);
  const long long b = __double_as_longlong(v);
  double r[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), 16 * k);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), 16 * k);
    r[k] = __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
  }
  return (r[0] + r[1]) + (r[2] + r[3]);
}

// The value of lane 16 g (row position 0) in every lane of row g (exact:
// the other lanes contribute zeros).
__device__ __forceinline__ float row_bcast0(float v, int r) { return row_sum16(r == 0 ? v : 0.f); }
