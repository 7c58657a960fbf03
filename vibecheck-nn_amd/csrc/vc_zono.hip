// Zonotope ReLU (verify_zono_bnb.py:3175-3211): bounds from the generator
// abs-sums, the parallelogram relaxation lam = hi/(hi-lo),
// mu = -hi*lo/(2(hi-lo)) on unstable neurons, and one new generator column
// per unstable neuron placed at its rank within the domain.
#include "vc_common.h"

namespace {

constexpr int NT = 256;

// One wave per (b, j) row: s = sum_k |G|; lo = c - s; hi = c + s.
// rank[b, j] temporarily holds the unstable flag.
__global__ void k_zono_bounds(const float* c, const float* G, int64_t rows, int K, float* lo,
                              float* hi, int32_t* flag) {
  const int lane = threadIdx.x & 63;
  for (int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6; row < rows;
       row += ((int64_t)gridDim.x * blockDim.x) >> 6) {
    KSum ks;
    for (int k = lane; k < K; k += 64) ks.add(fabsf(G[row * K + k]));
    const float s = wave_sum_comp(ks);
    if (lane == 0) {
      const float l = c[row] - s, h = c[row] + s;
      lo[row] = l;
      hi[row] = h;
      flag[row] = (l < 0.f && h > 0.f) ? 1 : 0;
    }
  }
}

// One block per domain: exclusive scan of the flags over j, in place.
__global__ void k_zono_rank(int32_t* rank, int n, int32_t* cnt) {
  __shared__ int wsum[NT / 64];
  __shared__ int carry;
  const int64_t b = blockIdx.x;
  int32_t* rb = rank + b * (int64_t)n;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int j0 = 0; j0 < n; j0 += NT) {
    const int j = j0 + threadIdx.x;
    const int v = j < n ? rb[j] : 0;
    int x = v;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int off = carry;
    int tot = 0;
    for (int i = 0; i < NT / 64; ++i) {
      if (i < w) off += wsum[i];
      tot += wsum[i];
    }
    if (j < n) rb[j] = v ? off + x - v : -1;
    __syncthreads();
    if (threadIdx.x == 0) carry += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) cnt[b] = carry;
}

__global__ void k_zono_apply(const float* c, const float* G, const float* lo, const float* hi,
                             const int32_t* rank, int64_t rows, int K, int Kn, float* c_out,
                             float* G_out) {
#pragma clang fp contract(off)
  const int Ko = K + Kn;
  const int Kt = Ko > 0 ? Ko : 1;
  const int64_t total = rows * (int64_t)Kt;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / Kt;
    const int k = (int)(i % Kt);
    const float l = lo[row], h = hi[row];
    const bool ust = l < 0.f && h > 0.f;
    const bool dead = h <= 0.f;
    const float lam = ust ? h / (h - l) : (dead ? 0.f : 1.f);
    float v;
    if (k < K) {
      v = G[row * K + k] * lam;
    } else {
      const float mu = ust ? (-h * l) / (2.f * (h - l)) : 0.f;
      v = (ust && rank[row] == k - K) ? mu : 0.f;
    }
    if (Ko > 0) G_out[row * Ko + k] = v;
    if (k == 0) {
      const float mu = ust ? (-h * l) / (2.f * (h - l)) : 0.f;
      c_out[row] = lam * c[row] + mu;
    }
  }
}

// k_zono_apply for long rows (K + Kn >= 256): one wavefront per (b, j)
// row, lambda and mu computed once per row (every lane the same values),
// the row streamed with consecutive lanes on consecutive columns.  Same
// operations per element as k_zono_apply, without its per-element 64-bit
// division and relaxation.
__global__ void k_zono_apply_rows(const float* c, const float* G, const float* lo,
                                  const float* hi, const int32_t* rank, int64_t rows, int K,
                                  int Kn, float* c_out, float* G_out) {
#pragma clang fp contract(off)
  const int Ko = K + Kn;
  const int lane = threadIdx.x & 63;
  for (int64_t row = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6; row < rows;
       row += ((int64_t)gridDim.x * blockDim.x) >> 6) {
    const float l = lo[row], h = hi[row];
    const bool ust = l < 0.f && h > 0.f;
    const bool dead = h <= 0.f;
    const float lam = ust ? h / (h - l) : (dead ? 0.f : 1.f);
    const float mu = ust ? (-h * l) / (2.f * (h - l)) : 0.f;
    const float* g = G + row * K;
    float* o = G_out + row * Ko;
    for (int k = lane; k < K; k += 64) o[k] = g[k] * lam;
    const int rk = ust ? rank[row] : -1;
    for (int k = K + lane; k < Ko; k += 64) o[k] = (k - K == rk) ? mu : 0.f;
    if (lane == 0) c_out[row] = lam * c[row] + mu;
  }
}

}  // namespace

extern "C" int vc_zono_relu_bounds(const float* c, const float* G, int64_t B, int n, int K,
                                   float* lo, float* hi, int32_t* rank, int32_t* cnt,
                                   vc_stream_t stream) {
  if (!c || !lo || !hi || !rank || !cnt || B < 0 || n <= 0 || K < 0) return VC_ERR_ARG;
  if (K > 0 && !G) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  if (B > 2147483647LL) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int64_t rows = B * (int64_t)n;
  hipLaunchKernelGGL(k_zono_bounds, dim3(vc_blocks(rows * 64, NT)), dim3(NT), 0, st, c, G,
                     rows, K, lo, hi, rank);
  hipLaunchKernelGGL(k_zono_rank, dim3((unsigned)B), dim3(NT), 0, st, rank, n, cnt);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_zono_relu_apply(const float* c, const float* G, const float* lo,
                                  const float* hi, const int32_t* rank, int64_t B, int n,
                                  int K, int K_new, float* c_out, float* G_out,
                                  vc_stream_t stream) {
  if (!c || !lo || !hi || !rank || !c_out || B < 0 || n <= 0 || K < 0 || K_new < 0)
    return VC_ERR_ARG;
  if ((K + K_new > 0 && !G_out) || (K > 0 && !G)) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  const int64_t rows = B * (int64_t)n;
  if (K + K_new >= 256)
    hipLaunchKernelGGL(k_zono_apply_rows, dim3(vc_blocks(rows * 64, NT)), dim3(NT), 0,
                       (hipStream_t)stream, c, G, lo, hi, rank, rows, K, K_new, c_out, G_out);
  else
    hipLaunchKernelGGL(k_zono_apply, dim3(vc_blocks(rows * (K + K_new > 0 ? K + K_new : 1), NT)),
                       dim3(NT), 0, (hipStream_t)stream, c, G, lo, hi, rank, rows, K, K_new,
                       c_out, G_out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
