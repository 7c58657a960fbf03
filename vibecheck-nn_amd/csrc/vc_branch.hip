// Selections of the input-split BaB beyond the widest-axis bisection:
//   - the split-dimension scores and their top K per leaf, and the 2^K-way
//     split of a leaf on its top K dimensions (verify_graph.py:13236-13423);
//   - the boundary band of leaves that get alpha-CROWN: unclosed leaves
//     whose worst disjunct's best bound is above -eps, the best
//     alpha_max_leaves of them first (verify_graph.py:12938-12950).
#include "vc_common.h"

namespace {

constexpr int NT = 256;
constexpr int kMaxK = 8;  // dimensions split at once (2^8 children per leaf)

// Score of input dimension i of one leaf, in the reference's fp32 operation
// order (verify_graph.py:13271-13285):
//   mode 0 (widest):    w_i = xh_i - xl_i
//   mode 1 (SB sum):    w_i * sum_q |A_q,i|            (q ascending)
//   mode 2 (SB margin): max_q (max(|A_q,i|, thr) * w_i / 2 + lb_q * mw)
__device__ __forceinline__ float branch_score(const float* xl, const float* xh, const float* A,
                                              const float* lb, int Q, int n, int i, int mode,
                                              float thr, float mw) {
  const float w = xh[i] - xl[i];
  if (mode == 0) return w;
  if (mode == 1) {
    float s = 0.f;
    for (int q = 0; q < Q; ++q) s += fabsf(A[(int64_t)q * n + i]);
    return w * s;
  }
  float best = -INFINITY;
  for (int q = 0; q < Q; ++q) {
    const float a = fmaxf(fabsf(A[(int64_t)q * n + i]), thr);
    best = fmaxf(best, (a * w) / 2.f + lb[q] * mw);
  }
  return best;
}

// (value, index) order of the selection: larger value first, then lower
// index (torch.argmax's first maximum; for K > 1 a stable descending sort).
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// One wavefront per leaf: K rounds of a wave-wide best-(value, index) over
// the dimensions not yet chosen.
__global__ __launch_bounds__(NT) void k_branch_topk(const float* xl, const float* xh,
                                                    const float* A, const float* lb, int64_t B,
                                                    int Q, int n, int mode, float thr, float mw,
                                                    int K, int64_t* dims, uint8_t* usable) {
  const int lane = threadIdx.x & 63;
  for (int64_t b = (blockIdx.x * (int64_t)NT + threadIdx.x) >> 6; b < B;
       b += ((int64_t)gridDim.x * NT) >> 6) {
    const float* l = xl + b * n;
    const float* h = xh + b * n;
    const float* Ab = A ? A + b * (int64_t)Q * n : nullptr;
    const float* lbb = lb ? lb + b * Q : nullptr;
    int chosen[kMaxK];
    for (int k = 0; k < K; ++k) {
      float bv = -INFINITY;
      int bi = n;
      for (int i = lane; i < n; i += 64) {
        bool taken = false;
        for (int c = 0; c < k; ++c) taken |= chosen[c] == i;
        if (taken) continue;
        const float v = branch_score(l, h, Ab, lbb, Q, n, i, mode, thr, mw);
        if (bi == n || better(v, i, bv, bi)) {
          bv = v;
          bi = i;
        }
      }
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oi < n && (bi == n || better(ov, oi, bv, bi))) {
          bv = ov;
          bi = oi;
        }
      }
      chosen[k] = bi;
      if (lane == 0) dims[b * K + k] = bi;
    }
    if (usable && lane == 0) usable[b] = (double)(h[chosen[0]] - l[chosen[0]]) > 1e-12;
  }
}

// The dimensions of a leaf's K split dimensions that can be split (width
// > 1e-12, compared in double as the reference's float() does), in order.
__device__ __forceinline__ int usable_dims(const float* l, const float* h, const int64_t* d,
                                           int K, int* u) {
  int ku = 0;
  for (int k = 0; k < K; ++k) {
    const int64_t j = d[k];
    if ((double)(h[j] - l[j]) > 1e-12) u[ku++] = (int)j;
  }
  return ku;
}

// Children per leaf (2^K_u, or 0 when no dimension is usable), their
// exclusive prefix sum into offsets[0..B] and the degenerate-leaf count.
// One workgroup of NP threads scans the leaves in tiles, carrying the sum.
constexpr int NP = 1024;
__global__ __launch_bounds__(NP) void k_split_plan(const float* xl, const float* xh,
                                                   const int64_t* dims, int64_t B, int n, int K,
                                                   int64_t* offsets, int64_t* n_degenerate) {
  __shared__ int64_t part[NP];
  __shared__ int64_t carry;
  __shared__ int64_t ndeg;
  if (threadIdx.x == 0) {
    carry = 0;
    ndeg = 0;
  }
  __syncthreads();
  for (int64_t t0 = 0; t0 < B; t0 += NP) {
    const int64_t b = t0 + threadIdx.x;
    int64_t c = 0;
    if (b < B) {
      int u[kMaxK];
      const int ku = usable_dims(xl + b * n, xh + b * n, dims + b * K, K, u);
      c = ku > 0 ? (int64_t(1) << ku) : 0;
      if (ku == 0) atomicAdd(reinterpret_cast<unsigned long long*>(&ndeg), 1ull);
    }
    part[threadIdx.x] = c;
    __syncthreads();
    // inclusive Hillis-Steele scan of the tile
    for (int o = 1; o < NP; o <<= 1) {
      const int64_t v = threadIdx.x >= o ? part[threadIdx.x - o] : 0;
      __syncthreads();
      part[threadIdx.x] += v;
      __syncthreads();
    }
    if (b < B) offsets[b] = carry + part[threadIdx.x] - c;
    __syncthreads();
    if (threadIdx.x == NP - 1) carry += part[NP - 1];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    offsets[B] = carry;
    *n_degenerate = ndeg;
  }
}

// Leaf b writes its 2^K_u children at rows offsets[b] + combo: bit k of
// combo picks the high half (lower end = midpoint) of its k-th usable
// dimension, else the low half (upper end = midpoint).
__global__ __launch_bounds__(NT) void k_split_multi(const float* xl, const float* xh,
                                                    const int64_t* dims, const int64_t* offsets,
                                                    int64_t B, int n, int K, float* oxl,
                                                    float* oxh) {
  for (int64_t b = blockIdx.x * (int64_t)NT + threadIdx.x; b < B;
       b += (int64_t)gridDim.x * NT) {
    const float* l = xl + b * n;
    const float* h = xh + b * n;
    int u[kMaxK];
    const int ku = usable_dims(l, h, dims + b * K, K, u);
    if (ku == 0) continue;
    float mid[kMaxK];
    for (int k = 0; k < ku; ++k) mid[k] = (l[u[k]] + h[u[k]]) / 2.f;
    const int64_t o0 = offsets[b];
    for (int combo = 0; combo < (1 << ku); ++combo) {
      float* cl = oxl + (o0 + combo) * n;
      float* ch = oxh + (o0 + combo) * n;
      for (int j = 0; j < n; ++j) {
        cl[j] = l[j];
        ch[j] = h[j];
      }
      for (int k = 0; k < ku; ++k) {
        if ((combo >> k) & 1)
          cl[u[k]] = mid[k];
        else
          ch[u[k]] = mid[k];
      }
    }
  }
}

// Band keys: key[b] = min over disjuncts of (max over the disjunct's
// queries of lb[b, q]) (the worst disjunct's best bound); cand[b] = the
// leaf is not closed and key > neg_eps (the reference compares with
// -alpha_eps in the tensor's fp32).
__global__ void k_band_keys(const float* lb, int64_t B, int Q, const int32_t* dptr,
                            const int32_t* qidx, int nd, const uint8_t* closed, float neg_eps,
                            float* keys, uint8_t* cand) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < B;
       b += (int64_t)gridDim.x * blockDim.x) {
    float worst = INFINITY;
    for (int d = 0; d < nd; ++d) {
      float best = -INFINITY;
      for (int t = dptr[d]; t < dptr[d + 1]; ++t) best = fmaxf(best, lb[b * Q + qidx[t]]);
      worst = fminf(worst, best);
    }
    keys[b] = worst;
    cand[b] = !closed[b] && worst > neg_eps;
  }
}

// Rank selection: candidate i (leaf idx[i], idx ascending) has rank =
// #{j : key_j > key_i, or key_j == key_i and j < i}; the first k_max ranks
// go to out[rank], so out holds the best k_max leaves in descending key
// order, ties in leaf order.  The keys are compared through LDS tiles.
__global__ __launch_bounds__(NT) void k_rank_select(const float* keys, const int64_t* idx,
                                                    int64_t C, int64_t k_max, int64_t* out) {
  __shared__ float tile[NT];
  for (int64_t i0 = (int64_t)blockIdx.x * NT; i0 < C; i0 += (int64_t)gridDim.x * NT) {
    const int64_t i = i0 + threadIdx.x;
    const float ki = i < C ? keys[idx[i]] : 0.f;
    int64_t rank = 0;
    for (int64_t j0 = 0; j0 < C; j0 += NT) {
      __syncthreads();
      if (j0 + threadIdx.x < C) tile[threadIdx.x] = keys[idx[j0 + threadIdx.x]];
      __syncthreads();
      const int m = C - j0 < NT ? (int)(C - j0) : NT;
      for (int t = 0; t < m; ++t) {
        const float kj = tile[t];
        rank += (kj > ki || (kj == ki && j0 + t < i)) ? 1 : 0;
      }
    }
    if (i < C && rank < k_max) out[rank] = idx[i];
  }
}

}  // namespace

extern "C" int vc_branch_topk(const float* xl, const float* xh, const float* A, const float* lb,
                              int64_t B, int Q, int n, int mode, float thr, float mw, int K,
                              int64_t* dims, uint8_t* usable, vc_stream_t stream) {
  if (!xl || !xh || !dims || B < 0 || n <= 0 || K < 1 || K > kMaxK || K > n) return VC_ERR_ARG;
  if (mode < 0 || mode > 2) return VC_ERR_ARG;
  if (mode > 0 && (!A || Q <= 0)) return VC_ERR_ARG;
  if (mode == 2 && !lb) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_branch_topk, dim3(vc_blocks(B * 64, NT)), dim3(NT), 0,
                     (hipStream_t)stream, xl, xh, A, lb, B, Q, n, mode, thr, mw, K, dims, usable);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_split_multi_plan(const float* xl, const float* xh, const int64_t* dims,
                                   int64_t B, int n, int K, int64_t* offsets,
                                   int64_t* n_degenerate, vc_stream_t stream) {
  if (!offsets || !n_degenerate || B < 0 || n <= 0 || K < 1 || K > kMaxK) return VC_ERR_ARG;
  if (B > 0 && (!xl || !xh || !dims)) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_split_plan, dim3(1), dim3(NP), 0, (hipStream_t)stream, xl, xh, dims, B,
                     n, K, offsets, n_degenerate);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_split_multi(const float* xl, const float* xh, const int64_t* dims,
                              const int64_t* offsets, int64_t B, int n, int K, float* out_xl,
                              float* out_xh, vc_stream_t stream) {
  if (B < 0 || n <= 0 || K < 1 || K > kMaxK) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  if (!xl || !xh || !dims || !offsets || !out_xl || !out_xh) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_split_multi, dim3(vc_blocks(B, NT)), dim3(NT), 0, (hipStream_t)stream, xl,
                     xh, dims, offsets, B, n, K, out_xl, out_xh);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_alpha_band_keys(const float* lb, int64_t B, int Q, const int32_t* d_ptr,
                                  const int32_t* q_idx, int n_disj, const uint8_t* closed,
                                  float neg_eps, float* keys, uint8_t* cand, vc_stream_t stream) {
  if (B < 0 || Q <= 0 || n_disj <= 0) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  if (!lb || !d_ptr || !q_idx || !closed || !keys || !cand) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_band_keys, dim3(vc_blocks(B, NT)), dim3(NT), 0, (hipStream_t)stream, lb, B,
                     Q, d_ptr, q_idx, n_disj, closed, neg_eps, keys, cand);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_rank_select_desc(const float* keys, const int64_t* idx, int64_t C,
                                   int64_t k_max, int64_t* out, vc_stream_t stream) {
  if (C < 0 || k_max < 0) return VC_ERR_ARG;
  if (C == 0 || k_max == 0) return VC_OK;
  if (!keys || !idx || !out) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_rank_select, dim3(vc_blocks(C, NT)), dim3(NT), 0, (hipStream_t)stream,
                     keys, idx, C, k_max, out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
