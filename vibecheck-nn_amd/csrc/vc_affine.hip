// Constant elementwise ops and residual merges: the add / sub / mul ops of
// the gg graph in the interval forward, the zonotope forward and the CROWN
// backward (verify_zono_bnb.py:1132-1148, 3213-3265, 3501-3536, 4455-4533,
// 4686-4712).  All HBM-bound streaming kernels: each value is read and
// written once, with the constant vector (n floats) staying in L2.
#include <hip/hip_runtime.h>

#include "vc_common.h"

namespace {

constexpr int NT = 256;

// torch.minimum / torch.maximum on floats: a NaN operand is returned; of two
// equal values the first.
__device__ __forceinline__ float t_min(float a, float b) {
  return a != a ? a : (b != b ? b : (b < a ? b : a));
}
__device__ __forceinline__ float t_max(float a, float b) {
  return a != a ? a : (b != b ? b : (a < b ? b : a));
}

// out = x + v, x - v or x * v per element; element i of a row of n is
// (t / inner) % n, its constant v[i] (v[0] for a scalar).  INNER1: inner == 1.
template <bool INNER1>
__global__ __launch_bounds__(NT) void k_affine_ew(const float* __restrict__ x, int64_t total,
                                                  int n, int64_t inner,
                                                  const float* __restrict__ v, int nv, int mode,
                                                  float* __restrict__ out) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    float c;
    if (nv == 1) {
      c = v[0];
    } else {
      const int64_t e = INNER1 ? t : t / inner;
      c = v[(int)(e % n)];
    }
    const float a = x[t];
    out[t] = mode == 0 ? a + c : (mode == 1 ? a - c : a * c);
  }
}

// Interval times a constant: lo = min(s l, s h), hi = max(s l, s h).
__global__ __launch_bounds__(NT) void k_interval_mul(const float* __restrict__ l,
                                                     const float* __restrict__ h, int64_t total,
                                                     int n, const float* __restrict__ s, int ns,
                                                     float* __restrict__ lo,
                                                     float* __restrict__ hi) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const float c = ns == 1 ? s[0] : s[(int)(t % n)];
    const float a = c * l[t], b = c * h[t];
    lo[t] = t_min(a, b);
    hi[t] = t_max(a, b);
  }
}

__global__ __launch_bounds__(NT) void k_add_ew(const float* __restrict__ a,
                                               const float* __restrict__ b, int64_t total,
                                               float* __restrict__ out) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x)
    out[t] = a[t] + b[t];
}

// Generators of a residual merge, per (domain, neuron) row: the first
// `shared` columns summed (both branches carry the fork point's noise
// there), then a's own columns, then b's own columns.
__global__ __launch_bounds__(NT) void k_zono_merge(const float* __restrict__ Ga, int Ka,
                                                   const float* __restrict__ Gb, int Kb,
                                                   int shared, int64_t rows, int Kout,
                                                   float* __restrict__ Gout) {
  const int64_t total = rows * Kout;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / Kout;
    const int k = (int)(t - r * Kout);
    float v;
    if (k < shared)
      v = Ga[r * Ka + k] + Gb[r * Kb + k];
    else if (k < Ka)
      v = Ga[r * Ka + k];
    else
      v = Gb[r * Kb + (k - Ka + shared)];
    Gout[t] = v;
  }
}

// acc[m] += sign * sum_i ew[row, i] v[i] (row m, or m % R for rows shared
// by every domain): fp32 products summed in fp64, one rounding into acc.
// One wavefront per row.
__global__ __launch_bounds__(NT) void k_rows_bias_dot(const float* __restrict__ ew, int64_t M,
                                                      int R, int n, int shared,
                                                      const float* __restrict__ v, int nv,
                                                      float sign, float* __restrict__ acc) {
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t m = w0; m < M; m += nw) {
    const float* x = ew + (shared ? m % R : m) * (int64_t)n;
    double p = 0.0;
    for (int i = lane; i < n; i += 64) p += (double)(x[i] * (nv == 1 ? v[0] : v[i]));
    p = wave_sum_f64(p);
    if (lane == 0) acc[m] = (float)((double)acc[m] + (double)sign * p);
  }
}

}  // namespace

extern "C" int vc_affine_ew(const float* x, int64_t outer, int n, int64_t inner,
                            const float* v, int nv, int mode, float* out, vc_stream_t stream) {
  if (!x || !v || !out || outer < 0 || n <= 0 || inner <= 0 || mode < 0 || mode > 2)
    return VC_ERR_ARG;
  if (nv != 1 && nv != n) return VC_ERR_ARG;
  const int64_t total = outer * (int64_t)n * inner;
  if (total == 0) return VC_OK;
  if (inner == 1)
    hipLaunchKernelGGL(k_affine_ew<true>, dim3(vc_blocks(total, NT)), dim3(NT), 0,
                       (hipStream_t)stream, x, total, n, inner, v, nv, mode, out);
  else
    hipLaunchKernelGGL(k_affine_ew<false>, dim3(vc_blocks(total, NT)), dim3(NT), 0,
                       (hipStream_t)stream, x, total, n, inner, v, nv, mode, out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_interval_mul(const float* l, const float* h, int64_t B, int n, const float* s,
                               int ns, float* lo, float* hi, vc_stream_t stream) {
  if (!l || !h || !s || !lo || !hi || B < 0 || n <= 0 || (ns != 1 && ns != n))
    return VC_ERR_ARG;
  const int64_t total = B * (int64_t)n;
  if (total == 0) return VC_OK;
  hipLaunchKernelGGL(k_interval_mul, dim3(vc_blocks(total, NT)), dim3(NT), 0,
                     (hipStream_t)stream, l, h, total, n, s, ns, lo, hi);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_add_ew(const float* a, const float* b, int64_t total, float* out,
                         vc_stream_t stream) {
  if (!a || !b || !out || total < 0) return VC_ERR_ARG;
  if (total == 0) return VC_OK;
  hipLaunchKernelGGL(k_add_ew, dim3(vc_blocks(total, NT)), dim3(NT), 0, (hipStream_t)stream, a,
                     b, total, out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_zono_merge(const float* Ga, int Ka, const float* Gb, int Kb, int shared,
                             int64_t rows, float* Gout, vc_stream_t stream) {
  if (rows < 0 || Ka < 0 || Kb < 0 || shared < 0 || shared > Ka || shared > Kb || !Gout)
    return VC_ERR_ARG;
  if ((Ka > 0 && !Ga) || (Kb > 0 && !Gb)) return VC_ERR_ARG;
  const int Kout = Ka + Kb - shared;
  if (rows == 0 || Kout == 0) return VC_OK;
  hipLaunchKernelGGL(k_zono_merge, dim3(vc_blocks(rows * Kout, NT)), dim3(NT), 0,
                     (hipStream_t)stream, Ga, Ka, Gb, Kb, shared, rows, Kout, Gout);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_rows_bias_dot(const float* ew, int64_t M, int R, int n, int shared,
                                const float* v, int nv, float sign, float* acc,
                                vc_stream_t stream) {
  if (!ew || !v || !acc || M < 0 || R <= 0 || n <= 0 || (nv != 1 && nv != n)) return VC_ERR_ARG;
  if (!shared && M % R) return VC_ERR_ARG;
  if (M == 0) return VC_OK;
  hipLaunchKernelGGL(k_rows_bias_dot, dim3(vc_blocks(M * 64, NT)), dim3(NT), 0,
                     (hipStream_t)stream, ew, M, R, n, shared, v, nv, sign, acc);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
