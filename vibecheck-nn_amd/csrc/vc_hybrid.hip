// Per-query alpha-CROWN of the hybrid freeze / replay verifier
// (verify_hybrid_acasxu.py:164-318): the elementwise pieces around the
// shared backward and gradient sweep.
//   - d lb / d alpha with one alpha per backward row (no sum over rows);
//   - intersection of a layer's bounds with its seeded CROWN bounds;
//   - the running best bound with the sum the loop's early stop reads;
//   - the running best spec bound with the input linearization of each
//     leaf's last improving evaluation.
#include "vc_common.h"
#include "vc_relax.h"

namespace {

constexpr int NT = 256;

// galpha[m, j] = gE[m, j] * max(P[m, j], 0) where neuron j of row m's domain
// is unstable, else 0 (P shared by all domains when p_bcast: row m % R).
__global__ void k_alpha_grad_rows(const float* gE, const float* P, int p_bcast, int64_t M, int R,
                                  int n, const float* lo, const float* hi, float* ga) {
  const int64_t total = M * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / n;
    const int j = (int)(i - m * n);
    const int64_t d = m / R;
    const float p = P[p_bcast ? (m - d * R) * n + j : i];
    const Relax s = relax(lo[d * n + j], hi[d * n + j]);
    ga[i] = s.unstable ? gE[i] * fmaxf(p, 0.f) : 0.f;
  }
}

// lo' = max(lo, sl[:, j]), hi' = min(hi, -sl[:, n + j]), lo' = min(lo', hi')
// (sl: the lower bounds of the seeded rows [+I; -I], (B, 2n)).
__global__ void k_bound_tighten(float* lo, float* hi, const float* sl, int64_t B, int n) {
  const int64_t total = B * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / n;
    const int j = (int)(i - b * n);
    const float l = fmaxf(lo[i], sl[b * 2 * n + j]);
    const float h = fminf(hi[i], -sl[b * 2 * n + n + j]);
    lo[i] = fminf(l, h);
    hi[i] = h;
  }
}

// best = max(best, lb) (a copy when init), out[0] = the sum of best, accumulated
// in fp64 and rounded once to fp32: the correctly rounded value of the fp32
// sum the reference's early stop reads (verify_hybrid_acasxu.py:210, 246).
__global__ __launch_bounds__(1024) void k_best_sum(float* best, const float* lb, int64_t n,
                                                   int init, double* out) {
  __shared__ double part[16];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float b = init ? lb[i] : fmaxf(best[i], lb[i]);
    best[i] = b;
    s += (double)b;
  }
  s = wave_sum_f64(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += part[w];
    *out = (double)(float)t;
  }
}

// Per leaf b: imp[q] = lb > best; best = where(imp, lb, best); when any
// query improved, bestA[b] = A[b] (Q x n_in).  One wavefront per leaf.
__global__ __launch_bounds__(NT) void k_best_rows_A(float* best, const float* lb, float* bestA,
                                                    const float* A, int64_t B, int Q, int n_in,
                                                    int init) {
  const int lane = threadIdx.x & 63;
  for (int64_t b = (blockIdx.x * (int64_t)NT + threadIdx.x) >> 6; b < B;
       b += ((int64_t)gridDim.x * NT) >> 6) {
    int any = 0;
    for (int q = lane; q < Q; q += 64) {
      const float v = lb[b * Q + q];
      const bool imp = init || v > best[b * Q + q];
      if (imp) best[b * Q + q] = v;
      any |= imp;
    }
    for (int o = 32; o > 0; o >>= 1) any |= __shfl_xor(any, o, 64);
    if (any) {
      const int64_t off = b * (int64_t)Q * n_in;
      for (int64_t k = lane; k < (int64_t)Q * n_in; k += 64) bestA[off + k] = A[off + k];
    }
  }
}

// out[b] = group[b] when it lies in [0, n_groups), else 0 and *bad = 1
// (written only by a thread that found a bad index).
__global__ void k_group_clamp(const int64_t* __restrict__ group, int64_t B, int64_t n_groups,
                              int64_t* __restrict__ out, int32_t* __restrict__ bad) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < B;
       b += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = group[b];
    const bool ok = (uint64_t)g < (uint64_t)n_groups;
    out[b] = ok ? g : 0;
    if (!ok) *bad = 1;
  }
}

}  // namespace

extern "C" int vc_alpha_grad_rows(const float* gE, const float* P, int p_bcast, int64_t M, int R,
                                  int n, const float* relu_lo, const float* relu_hi,
                                  float* galpha, vc_stream_t stream) {
  if (M < 0 || R <= 0 || n <= 0 || M % R) return VC_ERR_ARG;
  if (M == 0) return VC_OK;
  if (!gE || !P || !relu_lo || !relu_hi || !galpha) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_alpha_grad_rows, dim3(vc_blocks(M * n, NT)), dim3(NT), 0,
                     (hipStream_t)stream, gE, P, p_bcast, M, R, n, relu_lo, relu_hi, galpha);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_bound_tighten(float* lo, float* hi, const float* sl, int64_t B, int n,
                                vc_stream_t stream) {
  if (B < 0 || n <= 0) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  if (!lo || !hi || !sl) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_bound_tighten, dim3(vc_blocks(B * n, NT)), dim3(NT), 0,
                     (hipStream_t)stream, lo, hi, sl, B, n);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_group_clamp(const int64_t* group, int64_t B, int64_t n_groups, int64_t* out,
                              int32_t* bad, vc_stream_t stream) {
  if (!group || !out || !bad || B < 0 || n_groups < 1) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_group_clamp, dim3(vc_blocks(B, 256)), dim3(256), 0, (hipStream_t)stream,
                     group, B, n_groups, out, bad);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_best_sum(float* best, const float* lb, int64_t n, int init, double* out,
                           vc_stream_t stream) {
  if (!best || !lb || !out || n <= 0) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_best_sum, dim3(1), dim3(1024), 0, (hipStream_t)stream, best, lb, n, init,
                     out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_best_rows_with_A(float* best, const float* lb, float* best_A, const float* A,
                                   int64_t B, int Q, int n_in, int init, vc_stream_t stream) {
  if (B < 0 || Q <= 0 || n_in <= 0) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  if (!best || !lb || !best_A || !A) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_best_rows_A, dim3(vc_blocks(B * 64, NT)), dim3(NT), 0,
                     (hipStream_t)stream, best, lb, best_A, A, B, Q, n_in, init);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
