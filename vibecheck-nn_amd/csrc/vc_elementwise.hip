// Elementwise, reduction and integer/indexing kernels: ReLU relaxation,
// IBP relu, concretization, CROWN intersection, alpha-CROWN reductions and
// Adam, closure, halfspace clipping, compaction, widest-axis bisection.
#include <algorithm>

#include "vc_common.h"
#include "vc_relax.h"
#include "vc_mlp_common.h"

namespace {

constexpr int NT = 256;

__global__ void k_fill_u8(uint8_t* p, int64_t n, uint8_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void k_make_slopes(const float* lo, const float* hi, int64_t n, float* lo_s,
                              float* up_s, float* up_t, uint8_t* act, uint8_t* dead,
                              uint8_t* unst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    Relax s = relax(lo[i], hi[i]);
    lo_s[i] = s.lo_s;
    up_s[i] = s.up_s;
    up_t[i] = s.up_t;
    if (act) act[i] = s.active;
    if (dead) dead[i] = s.dead;
    if (unst) unst[i] = s.unstable;
  }
}

__global__ void k_alpha_init(const float* lo, const float* hi, int64_t n, float* alpha) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    Relax s = relax(lo[i], hi[i]);
    alpha[i] = (s.unstable && s.up_s > 0.5f) ? 1.f : 0.f;
  }
}

__global__ void k_ibp_relu(const float* l, const float* h, int64_t B, int n,
                           const float* rlo, const float* rhi, const float* cl,
                           const float* ch, float* sb_lo, float* sb_hi, float* post_lo,
                           float* post_hi) {
  const int64_t total = B * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int j = (int)(i % n);
    // NULL l/h: an unbounded input interval, so the root bounds give it.
    float lo = l ? l[i] : -INFINITY, hi = h ? h[i] : INFINITY;
    if (rlo) {
      lo = fmaxf(lo, rlo[j]);
      hi = fminf(hi, rhi[j]);
    }
    if (cl) {
      lo = fmaxf(lo, cl[i]);
      hi = fminf(hi, ch[i]);
    }
    hi = fmaxf(hi, lo);
    sb_lo[i] = lo;
    sb_hi[i] = hi;
    if (post_lo) {
      post_lo[i] = fmaxf(lo, 0.f);
      post_hi[i] = fmaxf(hi, 0.f);
    }
  }
}

// torch.clamp(min=0) / clamp(max=0): NaN stays NaN
__device__ __forceinline__ float pos_part(float a) { return a < 0.f ? 0.f : a; }
__device__ __forceinline__ float neg_part(float a) { return a > 0.f ? 0.f : a; }

__device__ __forceinline__ bool aligned16_dev(const void* p) {
  return ((uintptr_t)p & 15) == 0;
}

// One concretization term pos(a) l + neg(a) h.  Each product is rounded to
// fp32 as torch rounds the elementwise products; at most one of them is
// non-zero, so their fp32 sum is exact, and the sum over i runs in fp64.
__device__ __forceinline__ double conc_term(float a, float l, float h) {
  return (double)(pos_part(a) * l + neg_part(a) * h);
}


// lb[m] = acc[m] + sum_i pos(A) xl + sum_i neg(A) xh.  One wave takes
// CR = 4 consecutive rows at a time and keeps all their loads in flight.
// VEC: n % 4 == 0 and 16-byte aligned rows, float4 loads (1 KB per wave
// instruction); A is streamed once, so its loads bypass the caches that
// hold the domains' xl/xh rows.
constexpr int CR = 4;

template <bool VEC>
__global__ __launch_bounds__(256) void k_concretize_wave(const float* A, int a_bcast,
                                                         const float* acc, const float* xl,
                                                         const float* xh, int64_t M, int R,
                                                         int n, float* lb) {
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t m0 = w0 * CR; m0 < M; m0 += nw * CR) {
    const float* a[CR];
    const float* l[CR];
    const float* h[CR];
    double s[CR];
#pragma unroll
    for (int k = 0; k < CR; ++k) {
      const int64_t m = min(m0 + k, M - 1);  // past the end: recompute the last row
      const int64_t d = m / R;
      a[k] = A + (a_bcast ? m % R : m) * (int64_t)n;
      l[k] = xl + d * n;
      h[k] = xh + d * n;
      s[k] = 0.0;
    }
    if (VEC && l[0] == l[CR - 1]) {
      // the CR rows share one domain: its xl/xh loaded once for all of them
      const int n4 = n >> 2;
#pragma unroll 2
      for (int i = lane; i < n4; i += 64) {
        v4f x[CR];
#pragma unroll
        for (int k = 0; k < CR; ++k)
          x[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(a[k]) + i);
        const v4f p = reinterpret_cast<const v4f*>(l[0])[i];
        const v4f q = reinterpret_cast<const v4f*>(h[0])[i];
#pragma unroll
        for (int k = 0; k < CR; ++k)
#pragma unroll
          for (int c = 0; c < 4; ++c) s[k] += conc_term(x[k][c], p[c], q[c]);
      }
    } else if (VEC) {
      const int n4 = n >> 2;
      for (int i = lane; i < n4; i += 64) {
        v4f x[CR];
#pragma unroll
        for (int k = 0; k < CR; ++k)
          x[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(a[k]) + i);
#pragma unroll
        for (int k = 0; k < CR; ++k) {
          const v4f p = reinterpret_cast<const v4f*>(l[k])[i];
          const v4f q = reinterpret_cast<const v4f*>(h[k])[i];
#pragma unroll
          for (int c = 0; c < 4; ++c) s[k] += conc_term(x[k][c], p[c], q[c]);
        }
      }
    } else {
      for (int i = lane; i < n; i += 64) {
#pragma unroll
        for (int k = 0; k < CR; ++k) s[k] += conc_term(a[k][i], l[k][i], h[k][i]);
      }
    }
#pragma unroll
    for (int k = 0; k < CR; ++k) {
      const double t = wave_sum_f64(s[k]);
      if (lane == k && m0 + k < M) lb[m0 + k] = (float)((double)acc[m0 + k] + t);
    }
  }
}

// Narrow inputs (n <= 32): one thread per row.
constexpr int CT = 256, CT_MAXN = 32;

__global__ __launch_bounds__(CT) void k_concretize_thread(const float* A, int a_bcast,
                                                          const float* acc, const float* xl,
                                                          const float* xh, int64_t M, int R,
                                                          int n, float* lb) {
  for (int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; m < M;
       m += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = m / R;
    const float* a = A + (a_bcast ? m % R : m) * (int64_t)n;
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += conc_term(a[i], xl[d * n + i], xh[d * n + i]);
    lb[m] = (float)((double)acc[m] + s);
  }
}

// Narrow inputs, A per row: each workgroup takes RPT x CT consecutive
// rows.  Its rows of A (RPT CT n floats, contiguous) and its domains'
// boxes (contiguous too) are staged into LDS with float4 loads that cover
// the whole span (a row of 5 floats is not 16-byte aligned, so per-thread
// loads would touch every cache line once per input); every load of the
// workgroup, its rows' acc included, is issued before the one barrier.
// Each thread then sums its rows (tid, tid + CT, ...) from LDS in
// k_concretize_thread's order, so the results are the same.
template <int RPT>
__global__ __launch_bounds__(CT) void k_concretize_tile(const float* __restrict__ A,
                                                        const float* __restrict__ acc,
                                                        const float* __restrict__ xl,
                                                        const float* __restrict__ xh,
                                                        int64_t M, int R, int n,
                                                        float* __restrict__ lb) {
  extern __shared__ float csm[];
  constexpr int TR = RPT * CT;  // rows per workgroup
  const int64_t m0 = (int64_t)blockIdx.x * TR;
  const int rows = (int)min((int64_t)TR, M - m0);
  const int64_t d0 = m0 / R;
  const int nd = (int)((m0 + rows - 1) / R - d0 + 1);  // domains of this tile
  // the boxes' span [d0 n, (d0 + nd) n), from the 16-byte boundary at or
  // below its start when both box arrays allow float4 loads
  const int64_t b0 = d0 * n;
  const bool bvec = aligned16_dev(xl) && aligned16_dev(xh);
  const int bsh = bvec ? (int)(b0 & 3) : 0;  // floats before the span's start
  const int bcnt = nd * n + bsh;
  float* sa = csm;                               // [TR * n]
  float* sl = sa + TR * n;                       // [bcnt], rounded up to 4
  float* sh = sl + ((bcnt + 3) & ~3);            // [bcnt]
  float av[RPT];
  {
    // A's span [m0 n, (m0 + rows) n): 16-byte aligned at m0 n (TR n is a
    // multiple of 4) when A is
    const float* src = A + m0 * n;
    const int cnt = rows * n;
    const int c4 = cnt >> 2;
    for (int k = threadIdx.x; k < c4; k += CT)
      *reinterpret_cast<float4*>(sa + 4 * k) = reinterpret_cast<const float4*>(src)[k];
    for (int k = 4 * c4 + threadIdx.x; k < cnt; k += CT) sa[k] = src[k];
  }
  if (bvec) {
    const float4* pl = reinterpret_cast<const float4*>(xl + (b0 - bsh));
    const float4* ph = reinterpret_cast<const float4*>(xh + (b0 - bsh));
    // the last float4 may reach past the span: only its in-span floats
    // are stored (the loads stay inside the box arrays, which end at a
    // span's end or later)
    const int c4 = (bcnt + 3) >> 2;
    const int64_t lim = (int64_t)(M / R) * n - (b0 - bsh);  // floats left in the arrays
    for (int k = threadIdx.x; k < c4; k += CT) {
      if (4 * (int64_t)k + 4 <= lim) {
        *reinterpret_cast<float4*>(sl + 4 * k) = pl[k];
        *reinterpret_cast<float4*>(sh + 4 * k) = ph[k];
      } else {
        for (int c = 0; c < 4 && 4 * (int64_t)k + c < lim; ++c) {
          sl[4 * k + c] = xl[b0 - bsh + 4 * k + c];
          sh[4 * k + c] = xh[b0 - bsh + 4 * k + c];
        }
      }
    }
  } else {
    for (int k = threadIdx.x; k < bcnt; k += CT) {
      sl[k] = xl[b0 + k];
      sh[k] = xh[b0 + k];
    }
  }
#pragma unroll
  for (int q = 0; q < RPT; ++q) {
    const int r = q * CT + threadIdx.x;
    av[q] = r < rows ? acc[m0 + r] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < RPT; ++q) {
    const int r = q * CT + threadIdx.x;
    if (r < rows) {
      const int64_t m = m0 + r;
      const int dl = (int)(m / R - d0) * n + bsh;
      const float* a = sa + r * n;
      double s = 0.0;
      for (int i = 0; i < n; ++i) s += conc_term(a[i], sl[dl + i], sh[dl + i]);
      lb[m] = (float)((double)av[q] + s);
    }
  }
}

// One relaxed element: e = pos(x) lo_s + neg(x) up_s (+ beta), and the
// neg(x) up_t term of acc, for the slopes s (ls: lo_s, or the alpha slope).
__device__ __forceinline__ float relax_apply(float x, const Relax& s, float ls, bool has_beta,
                                             float bt, double& p) {
  const float ep = pos_part(x), en = neg_part(x);
  float e = ep * ls + en * s.up_s;
  if (has_beta) e = e + bt;
  p += (double)(en * s.up_t);
  return e;
}

__device__ __forceinline__ float lo_slope(const Relax& s, bool has_alpha, float a) {
  return has_alpha ? (s.active ? 1.f : (s.unstable ? a : 0.f)) : s.lo_s;
}

// Standalone relu backward.  One wave takes two consecutive rows at a time;
// when both belong to one domain (and alpha is per domain) the relaxation
// of each neuron is computed once for both.  VEC as for k_concretize_wave.
template <bool VEC>
__global__ __launch_bounds__(256) void k_backward_relu(const float* ew, int64_t M, int R, int n,
                                                       const float* lo, const float* hi,
                                                       const float* alpha, int alpha_per_row,
                                                       const float* beta, float* out,
                                                       float* acc) {
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const bool ha = alpha != nullptr, hb = beta != nullptr;
  for (int64_t m0 = w0 * 2; m0 < M; m0 += nw * 2) {
    const int64_t m1 = min(m0 + 1, M - 1);  // past the end: recompute the last row
    const int64_t d0 = m0 / R, d1 = m1 / R;
    const bool shared = d0 == d1 && !alpha_per_row;
    const float* x0 = ew + m0 * n;
    const float* x1 = ew + m1 * n;
    float* o0 = out + m0 * n;
    float* o1 = out + m1 * n;
    const float* l0 = lo + d0 * n;
    const float* h0 = hi + d0 * n;
    const float* l1 = lo + d1 * n;
    const float* h1 = hi + d1 * n;
    const float* a0 = ha ? alpha + (alpha_per_row ? m0 : d0) * n : nullptr;
    const float* a1 = ha ? alpha + (alpha_per_row ? m1 : d1) * n : nullptr;
    const float* b0 = hb ? beta + d0 * n : nullptr;
    const float* b1 = hb ? beta + d1 * n : nullptr;
    double p0 = 0.0, p1 = 0.0;
    if (VEC) {
      const int n4 = n >> 2;
      const v4f zero = {0.f, 0.f, 0.f, 0.f};
      for (int i = lane; i < n4; i += 64) {
        const v4f x = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(x0) + i);
        const v4f y = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(x1) + i);
        const v4f la = reinterpret_cast<const v4f*>(l0)[i];
        const v4f ha4 = reinterpret_cast<const v4f*>(h0)[i];
        const v4f aa = ha ? reinterpret_cast<const v4f*>(a0)[i] : zero;
        const v4f ba = hb ? reinterpret_cast<const v4f*>(b0)[i] : zero;
        v4f e, f;
        if (shared) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const Relax r = relax(la[c], ha4[c]);
            const float ls = lo_slope(r, ha, aa[c]);
            e[c] = relax_apply(x[c], r, ls, hb, ba[c], p0);
            f[c] = relax_apply(y[c], r, ls, hb, ba[c], p1);
          }
        } else {
          const v4f lb4 = reinterpret_cast<const v4f*>(l1)[i];
          const v4f hb4 = reinterpret_cast<const v4f*>(h1)[i];
          const v4f ab = ha ? reinterpret_cast<const v4f*>(a1)[i] : zero;
          const v4f bb = hb ? reinterpret_cast<const v4f*>(b1)[i] : zero;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const Relax r = relax(la[c], ha4[c]);
            e[c] = relax_apply(x[c], r, lo_slope(r, ha, aa[c]), hb, ba[c], p0);
            const Relax q = relax(lb4[c], hb4[c]);
            f[c] = relax_apply(y[c], q, lo_slope(q, ha, ab[c]), hb, bb[c], p1);
          }
        }
        __builtin_nontemporal_store(e, reinterpret_cast<v4f*>(o0) + i);
        __builtin_nontemporal_store(f, reinterpret_cast<v4f*>(o1) + i);
      }
    } else {
      for (int j = lane; j < n; j += 64) {
        const Relax r = relax(l0[j], h0[j]);
        o0[j] = relax_apply(x0[j], r, lo_slope(r, ha, ha ? a0[j] : 0.f), hb, hb ? b0[j] : 0.f,
                            p0);
        const Relax q = shared ? r : relax(l1[j], h1[j]);
        o1[j] = relax_apply(x1[j], q, lo_slope(q, ha, ha ? a1[j] : 0.f), hb, hb ? b1[j] : 0.f,
                            p1);
      }
    }
    p0 = wave_sum_f64(p0);
    p1 = wave_sum_f64(p1);
    if (lane == 0) acc[m0] = (float)((double)acc[m0] + p0);
    if (lane == 1 && m0 + 1 < M) acc[m1] = (float)((double)acc[m1] + p1);
  }
}

// Wide rows (n >= 1024, float4-aligned): one workgroup of 4 waves takes
// RB = 4 consecutive rows, each wave a quarter of the columns (interleaved
// in 256-float4 strides), so the four waves stream neighbouring addresses;
// the per-row acc terms are reduced through LDS.  The relaxation of each
// neuron is computed once for the rows of one domain.
constexpr int RB = 4;

template <bool HA, bool HB>
__global__ __launch_bounds__(256) void k_backward_relu_rows(
    const float* __restrict__ ew, int64_t M, int R, int n, const float* __restrict__ lo,
    const float* __restrict__ hi, const float* __restrict__ alpha, int alpha_per_row,
    const float* __restrict__ beta, float* __restrict__ out, float* __restrict__ acc) {
  __shared__ double red[4][RB];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n4 = n >> 2;
  for (int64_t m0 = (int64_t)blockIdx.x * RB; m0 < M; m0 += (int64_t)gridDim.x * RB) {
    int64_t mr[RB], dr[RB];
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      mr[k] = min(m0 + k, M - 1);  // past the end: recompute the last row
      dr[k] = mr[k] / R;
    }
    const bool shared = dr[0] == dr[RB - 1] && !alpha_per_row;
    double p[RB];
#pragma unroll
    for (int k = 0; k < RB; ++k) p[k] = 0.0;
    for (int i = threadIdx.x; i < n4; i += 256) {
      v4f x[RB], e[RB];
#pragma unroll
      for (int k = 0; k < RB; ++k)
        x[k] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(ew + mr[k] * n) + i);
      if (shared) {
        const v4f l4 = reinterpret_cast<const v4f*>(lo + dr[0] * n)[i];
        const v4f h4 = reinterpret_cast<const v4f*>(hi + dr[0] * n)[i];
        v4f a4 = {0.f, 0.f, 0.f, 0.f}, b4 = {0.f, 0.f, 0.f, 0.f};
        if (HA) a4 = reinterpret_cast<const v4f*>(alpha + dr[0] * n)[i];
        if (HB) b4 = reinterpret_cast<const v4f*>(beta + dr[0] * n)[i];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const Relax r = relax(l4[c], h4[c]);
          const float ls = lo_slope(r, HA, a4[c]);
#pragma unroll
          for (int k = 0; k < RB; ++k) e[k][c] = relax_apply(x[k][c], r, ls, HB, b4[c], p[k]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < RB; ++k) {
          const v4f l4 = reinterpret_cast<const v4f*>(lo + dr[k] * n)[i];
          const v4f h4 = reinterpret_cast<const v4f*>(hi + dr[k] * n)[i];
          v4f a4 = {0.f, 0.f, 0.f, 0.f}, b4 = {0.f, 0.f, 0.f, 0.f};
          if (HA) a4 = reinterpret_cast<const v4f*>(alpha + (alpha_per_row ? mr[k] : dr[k]) * n)[i];
          if (HB) b4 = reinterpret_cast<const v4f*>(beta + dr[k] * n)[i];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const Relax r = relax(l4[c], h4[c]);
            e[k][c] = relax_apply(x[k][c], r, lo_slope(r, HA, a4[c]), HB, b4[c], p[k]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < RB; ++k)
        __builtin_nontemporal_store(e[k], reinterpret_cast<v4f*>(out + mr[k] * n) + i);
    }
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const double t = wave_sum_f64(p[k]);
      if (lane == 0) red[wv][k] = t;
    }
    __syncthreads();
    if (threadIdx.x < RB && m0 + threadIdx.x < M) {
      const int k = threadIdx.x;
      const double t = (red[0][k] + red[1][k]) + (red[2][k] + red[3][k]);
      acc[m0 + k] = (float)((double)acc[m0 + k] + t);
    }
    __syncthreads();
  }
}

__global__ void k_crown_intersect(const float* sl, const int32_t* idx, int k, int64_t B,
                                  int n, float* lo, float* hi) {
  const int64_t total = B * (int64_t)k;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / k;
    const int t = (int)(i % k);
    const int64_t o = b * n + idx[t];
    const float lc = fmaxf(lo[o], sl[b * 2 * k + t]);
    const float hc = fmaxf(fminf(hi[o], -sl[b * 2 * k + k + t]), lc);
    lo[o] = lc;
    hi[o] = hc;
  }
}

__global__ void k_unstable_union(const float* lo, const float* hi, int64_t B, int n,
                                 uint8_t* flag) {
  const int64_t total = B * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (lo[i] < 0.f && hi[i] > 0.f) flag[i % n] = 1;
  }
}

// ---- per-layer batches in one launch (blockIdx.y = layer / array) -------
constexpr int VC_MAXA = 32;

struct LayerPtrs {
  const float* lo[VC_MAXA];
  const float* hi[VC_MAXA];
  int width[VC_MAXA];
  int off[VC_MAXA];
};

__global__ void k_unstable_union_layers(LayerPtrs lp, int64_t B, uint8_t* flag) {
  const int L = blockIdx.y;
  const int n = lp.width[L];
  const int64_t total = B * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (lp.lo[L][i] < 0.f && lp.hi[L][i] > 0.f) flag[lp.off[L] + i % n] = 1;
  }
}

// Compact the union flags of every layer: wave L lists the set flags of
// layer L in increasing order at idx[off[L] ..], with meta = {cnt[0..n),
// off[0..n)}; off is the exclusive prefix sum of the counts.
__global__ void k_union_compact(const uint8_t* flag, LayerPtrs lp, int n_layers, int32_t* idx,
                                int32_t* meta) {
  __shared__ int scnt[VC_MAXA];
  const int L = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool mine = L < n_layers;
  const int w = mine ? lp.width[L] : 0;
  const uint8_t* f = flag + (mine ? lp.off[L] : 0);
  int cnt = 0;
  for (int c0 = 0; c0 < w; c0 += 64) {
    const bool set = c0 + lane < w && f[c0 + lane] != 0;
    cnt += __popcll(__ballot(set));
  }
  if (mine && lane == 0) scnt[L] = cnt;
  __syncthreads();
  if (!mine) return;
  int off = 0;
  for (int k = 0; k < L; ++k) off += scnt[k];
  int run = off;
  for (int c0 = 0; c0 < w; c0 += 64) {
    const bool set = c0 + lane < w && f[c0 + lane] != 0;
    const uint64_t bal = __ballot(set);
    if (set) idx[run + __popcll(bal & ((1ull << lane) - 1ull))] = c0 + lane;
    run += __popcll(bal);
  }
  if (lane == 0) {
    meta[L] = cnt;
    meta[n_layers + L] = off;
  }
}

struct GatherPtrs {
  const float* in[VC_MAXA];
  float* out[VC_MAXA];
  int cols[VC_MAXA];
};

__global__ void k_gather_rows_multi(GatherPtrs gp, const int64_t* idx, int64_t nr) {
  const int a = blockIdx.y;
  const int cols = gp.cols[a];
  const int64_t total = nr * (int64_t)cols;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols;
    const int c = (int)(i % cols);
    gp.out[a][i] = gp.in[a][idx[r] * cols + c];
  }
}

__global__ void k_alpha_grad_reduce(const float* gE, const float* P, int p_bcast, int64_t B,
                                    int R, int n, const float* lo, const float* hi, float* ga,
                                    float* gb) {
  const int64_t total = B * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = i / n;
    const int j = (int)(i % n);
    float sa = 0.f, sb = 0.f;
    for (int q = 0; q < R; ++q) {
      const int64_t o = (d * R + q) * n + j;
      const float ge = gE[o];
      sa += ge * fmaxf(P[p_bcast ? (int64_t)q * n + j : o], 0.f);
      sb += ge;
    }
    Relax s = relax(lo[i], hi[i]);
    if (ga) ga[i] = s.unstable ? sa : 0.f;
    if (gb) gb[i] = sb;
  }
}

// Adam on the loss -lb, then the projection clamp.
__global__ void k_adam(float* p, const float* lbg, float* m, float* v, int64_t n, AdamConst c,
                       float lo_c, float hi_c) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float mi = m[i], vi = v[i];
    float pi = adam_update(p[i], -lbg[i], mi, vi, c);
    pi = fminf(fmaxf(pi, lo_c), hi_c);
    m[i] = mi;
    v[i] = vi;
    p[i] = pi;
  }
}

// Split beta: the backward sees the signed beta (beta * sign), so
// d lb / d beta = sign * d lb / d signed.  Adam on -lb, clamp beta >= 0,
// then write the signed beta for the next evaluation.
__global__ void k_beta_adam(float* beta, const float* sign, const float* gsum, float* m,
                            float* v, int64_t n, AdamConst c, float* signed_out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float s = sign[i];
    float mi = m[i], vi = v[i];
    float pi = adam_update(beta[i], -(gsum[i] * s), mi, vi, c);
    pi = fmaxf(pi, 0.f);
    m[i] = mi;
    v[i] = vi;
    beta[i] = pi;
    signed_out[i] = pi * s;
  }
}

// sign +1 where the upper clamp is 0 (OFF split: z <= 0), -1 where the lower
// clamp is 0 (ON split: z >= 0; it wins when both are 0), else 0.
__device__ __forceinline__ float split_sign(float cl, float ch) {
  return cl == 0.f ? -1.f : (ch == 0.f ? 1.f : 0.f);
}

__global__ void k_split_beta_sign(const float* cl, const float* ch, int64_t n, float* sign) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    sign[i] = split_sign(cl[i], ch[i]);
}

// Dense clamps of one relu layer from per-domain split lists (D, S): entry
// (d, s) clamps neuron `neuron` of layer `layer` (-1 = unused slot) OFF
// (side 0: upper clamp 0) or ON (side 1: lower clamp 0).
__global__ void k_split_clamps(const int64_t* layer, const int64_t* neuron, const int64_t* side,
                               int64_t D, int S, int64_t L, int n, float* cl, float* ch,
                               float* sign) {
  const int64_t total = D * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = i / n;
    const int64_t j = i % n;
    float lo = -INFINITY, hi = INFINITY;
    for (int s = 0; s < S; ++s) {
      const int64_t e = d * S + s;
      if (layer[e] == L && neuron[e] == j) {
        if (side[e] == 0)
          hi = 0.f;
        else
          lo = 0.f;
      }
    }
    cl[i] = lo;
    ch[i] = hi;
    if (sign) sign[i] = split_sign(lo, hi);
  }
}

// One alpha-CROWN iteration's bookkeeping on the device, with the loop
// control of verify_zono_bnb.py:5252-5287: ctl = {previous global max of the
// best bound, stopped flag, evaluated iterations, this iteration's max}.
// Once stopped, later calls (and the fused alpha kernel) do nothing.
// The bookkeeping of n_it consecutive alpha-CROWN iterations it0 ..
// it0 + n_it - 1 whose bounds are lbs[t] (n each), in order, up to the
// first stop (the later ones are discarded): best update, global max, the
// reference's two stop tests.
// stop_host (a pinned host word, nullable) is set to 1 at a stop; progress
// (pinned, nullable) to it0 + n_it once the launch has taken every one of
// its iterations without a stop.
// One sweep over the elements gives every iteration's maximum and sign test
// (each element's running best in registers); one thread then finds the
// first stop, and best is written as it stands after the last iteration
// taken.  Every load, the control word's included, is issued before the
// stopped test, so the launch makes one round trip to memory instead of
// three per iteration (9.2 -> 6.3 us for 4 iterations over 1,644 bounds).
// CACHED: n <= kCtlEpt * kCtlThreads, each thread's elements stay in
// registers for the write; otherwise (1,024 threads) the write pass reads
// them again, and with one iteration per launch (the one-wavefront-per-
// domain alpha kernel's loop) best is written in the sweep itself, eight
// loads per thread in flight (float4 where aligned).
constexpr int kCtlThreads = 512;
constexpr int kCtlThreadsBig = 1024;
constexpr int kCtlEpt = 4;

template <bool CACHED>
__global__ __launch_bounds__(CACHED ? kCtlThreads : kCtlThreadsBig) void k_alpha_control(
    float* best, const float* lbs, int64_t n, int it0, int n_it, double eps, float* ctl,
    int32_t* stop_host, int32_t* progress) {
  constexpr int NTH = CACHED ? kCtlThreads : kCtlThreadsBig;
  constexpr int NW = NTH / 64, E = CACHED ? kCtlEpt : 1;
  __shared__ float smax[VC_ALPHA_CHUNK][NW];
  __shared__ int sneg[VC_ALPHA_CHUNK][NW];
  __shared__ int s_last;
  const float stopped = ctl[1];
  const float prev0 = ctl[0];
  float xv[E][VC_ALPHA_CHUNK], bv[E];
  if (CACHED) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int64_t i = threadIdx.x + (int64_t)e * kCtlThreads;
      const bool in = i < n;
      bv[e] = (in && it0 > 0) ? best[i] : 0.f;
#pragma unroll
      for (int t = 0; t < VC_ALPHA_CHUNK; ++t)
        xv[e][t] = (in && t < n_it) ? lbs[(int64_t)t * n + i] : 0.f;
    }
  }
  if (stopped != 0.f) return;
  float mx[VC_ALPHA_CHUNK];
  int notpos[VC_ALPHA_CHUNK];
#pragma unroll
  for (int t = 0; t < VC_ALPHA_CHUNK; ++t) {
    mx[t] = -INFINITY;
    notpos[t] = 0;
  }
  // iteration it's best: its own bound at it = 0, else max(best, bound)
  const auto run = [&](float b, const float* x, int64_t i) {
#pragma unroll
    for (int t = 0; t < VC_ALPHA_CHUNK; ++t) {
      if (t < n_it) {
        const float v = CACHED ? x[t] : lbs[(int64_t)t * n + i];
        b = it0 + t == 0 ? v : fmaxf(b, v);
        mx[t] = fmaxf(mx[t], b);
        notpos[t] |= !(b > 0.f);
      }
    }
  };
  // one iteration, no cache: best written in the sweep (every iteration a
  // launch takes is written, so the stop test does not gate the write)
  const bool single = !CACHED && n_it == 1;
  if (CACHED) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (threadIdx.x + (int64_t)e * kCtlThreads < n) run(bv[e], xv[e], 0);
  } else if (single) {
    const auto one = [&](float b, float x) {
      b = it0 == 0 ? x : fmaxf(b, x);
      mx[0] = fmaxf(mx[0], b);
      notpos[0] |= !(b > 0.f);
      return b;
    };
    const bool v4 = ((reinterpret_cast<uintptr_t>(best) | reinterpret_cast<uintptr_t>(lbs)) & 15) == 0;
    const int64_t n4 = v4 ? n / 4 : 0;
    float4* b4 = reinterpret_cast<float4*>(best);
    const float4* x4 = reinterpret_cast<const float4*>(lbs);
    for (int64_t i0 = threadIdx.x; i0 < n4; i0 += 8 * NTH) {
      float4 xv8[8], bv8[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t i = i0 + (int64_t)u * NTH;
        const bool in = i < n4;
        xv8[u] = in ? x4[i] : float4{0.f, 0.f, 0.f, 0.f};
        bv8[u] = (in && it0 > 0) ? b4[i] : float4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t i = i0 + (int64_t)u * NTH;
        if (i < n4) {
          float4 o;
          o.x = one(bv8[u].x, xv8[u].x);
          o.y = one(bv8[u].y, xv8[u].y);
          o.z = one(bv8[u].z, xv8[u].z);
          o.w = one(bv8[u].w, xv8[u].w);
          b4[i] = o;
        }
      }
    }
    for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += NTH)
      best[i] = one(it0 > 0 ? best[i] : 0.f, lbs[i]);
  } else {
    for (int64_t i = threadIdx.x; i < n; i += NTH) run(it0 > 0 ? best[i] : 0.f, nullptr, i);
  }
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < VC_ALPHA_CHUNK; ++t) {
    for (int o = 32; o > 0; o >>= 1) {
      mx[t] = fmaxf(mx[t], __shfl_xor(mx[t], o, 64));
      notpos[t] |= __shfl_xor(notpos[t], o, 64);
    }
    if (lane == 0) {
      smax[t][w] = mx[t];
      sneg[t][w] = notpos[t];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float prev = prev0, a = prev0;
    int last = n_it - 1;
    bool stop = false;
    for (int t = 0; t < n_it; ++t) {
      a = smax[t][0];
      int b = sneg[t][0];
      for (int k = 1; k < NW; ++k) {
        a = fmaxf(a, smax[t][k]);
        b |= sneg[t][k];
      }
      const int it = it0 + t;
      stop = b == 0;  // every best bound > 0
      if (!stop && it > 0 && (double)a - (double)prev < eps) stop = true;
      prev = a;
      if (stop) {
        last = t;
        break;
      }
    }
    ctl[0] = a;
    ctl[1] = stop ? 1.f : 0.f;
    ctl[2] = (float)(it0 + last + 1);
    ctl[3] = a;
    // hints for the launching host thread (pinned host memory)
    if (stop && stop_host)
      __hip_atomic_store(stop_host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (!stop && progress)
      __hip_atomic_store(progress, it0 + n_it, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s_last = last;
  }
  __syncthreads();
  if (single) return;
  const int last = s_last;
  const auto upto = [&](float b, const float* x, int64_t i) {
#pragma unroll
    for (int t = 0; t < VC_ALPHA_CHUNK; ++t) {
      if (t <= last) {
        const float v = CACHED ? x[t] : lbs[(int64_t)t * n + i];
        b = it0 + t == 0 ? v : fmaxf(b, v);
      }
    }
    best[i] = b;
  };
  if (CACHED) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int64_t i = threadIdx.x + (int64_t)e * kCtlThreads;
      if (i < n) upto(bv[e], xv[e], i);
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += NTH) upto(it0 > 0 ? best[i] : 0.f, nullptr, i);
  }
}

void alpha_control_launch(float* best, const float* lbs, int64_t n, int it0, int n_it, double eps,
                          float* ctl, int32_t* stop_host, int32_t* progress, hipStream_t st) {
  if (n <= (int64_t)kCtlEpt * kCtlThreads)
    hipLaunchKernelGGL(k_alpha_control<true>, dim3(1), dim3(kCtlThreads), 0, st, best, lbs, n,
                       it0, n_it, eps, ctl, stop_host, progress);
  else
    hipLaunchKernelGGL(k_alpha_control<false>, dim3(1), dim3(kCtlThreadsBig), 0, st, best, lbs,
                       n, it0, n_it, eps, ctl, stop_host, progress);
}

__global__ void k_best_update(float* best, const float* lb, int64_t n, int init, float* out2) {
  __shared__ float smax[16];
  __shared__ int sneg[16];
  float mx = -INFINITY;
  int notpos = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float x = lb[i];
    const float b = init ? x : fmaxf(best[i], x);
    best[i] = b;
    mx = fmaxf(mx, b);
    notpos |= !(b > 0.f);
  }
  for (int o = 32; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    notpos |= __shfl_xor(notpos, o, 64);
  }
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    smax[w] = mx;
    sneg[w] = notpos;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int nw = blockDim.x >> 6;
    float a = smax[0];
    int b = sneg[0];
    for (int i = 1; i < nw; ++i) {
      a = fmaxf(a, smax[i]);
      b |= sneg[i];
    }
    out2[0] = a;
    out2[1] = b ? 0.f : 1.f;
  }
}

__global__ void k_closure(const float* lb, int64_t B, int Q, const int32_t* dptr,
                          const int32_t* qidx, int nd, uint8_t* closed) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < B;
       b += (int64_t)gridDim.x * blockDim.x) {
  bool all = true;
  for (int d = 0; d < nd; ++d) {
    bool any = false;
    for (int t = dptr[d]; t < dptr[d + 1]; ++t) any |= lb[b * Q + qidx[t]] > 0.f;
    all &= any;
  }
  closed[b] = all;
  }
}

// k_closure that also lists the rows left open (in no particular order:
// one atomic per wavefront), counted in *open_cnt, which the caller clears.
__global__ void k_closure_open(const float* lb, int64_t B, int Q, const int32_t* dptr,
                               const int32_t* qidx, int nd, uint8_t* closed, int64_t* open_idx,
                               unsigned long long* open_cnt) {
  const int lane = threadIdx.x & 63;
  for (int64_t b0 = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) & ~(int64_t)63; b0 < B;
       b0 += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = b0 + lane;
    bool all = true;
    if (b < B) {
      for (int d = 0; d < nd; ++d) {
        bool any = false;
        for (int t = dptr[d]; t < dptr[d + 1]; ++t) any |= lb[b * Q + qidx[t]] > 0.f;
        all &= any;
      }
      closed[b] = all;
    }
    const uint64_t open = __ballot(b < B && !all);
    unsigned long long base = 0;
    if (lane == 0 && open) base = atomicAdd(open_cnt, (unsigned long long)__popcll(open));
    base = __shfl(base, 0, 64);
    if ((open >> lane) & 1ull)
      open_idx[base + __popcll(open & ((1ull << lane) - 1ull))] = b;
  }
}

// The open rows' bounds raised to alpha's best (rows[idx[r]] = max(rows,
// src[r]), as k_scatter_max_rows) and their closure recomputed (as
// k_closure; the other rows' bounds, and so their closure, are unchanged).
__global__ void k_scatter_max_close(float* lb, const int64_t* idx, const float* src, int64_t nr,
                                    int Q, const int32_t* dptr, const int32_t* qidx, int nd,
                                    uint8_t* closed) {
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < nr;
       r += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = idx[r];
    float* row = lb + b * Q;
    for (int q = 0; q < Q; ++q) row[q] = fmaxf(row[q], src[r * Q + q]);
    bool all = true;
    for (int d = 0; d < nd; ++d) {
      bool any = false;
      for (int t = dptr[d]; t < dptr[d + 1]; ++t) any |= row[qidx[t]] > 0.f;
      all &= any;
    }
    closed[b] = all;
  }
}

// One thread per domain.  For each disjunct D: total_q = pos(A_q).xl +
// neg(A_q).xh; per dim i the projection threshold
// thr = (-b_q - (total_q - contrib_qi)) / A_qi; xh' = min(xh, min over
// A_qi > 1e-12 of thr), xl' = max(xl, max over A_qi < -1e-12 of thr);
// feasible iff no total_q + b_q > 0 and no xl' > xh'.
__device__ __forceinline__ void clip_dim(const float* A, const float* bq, const float* tot,
                                         const int32_t* qs, int nq, int n, int i, float xl,
                                         float xh, float& lo_o, float& hi_o) {
  float hmin = INFINITY, lmax = -INFINITY;
  for (int t = 0; t < nq; ++t) {
    const int q = qs[t];
    const float a = A[q * n + i];
    const float contrib = fmaxf(a, 0.f) * xl + fminf(a, 0.f) * xh;
    const float other = tot[t] - contrib;
    const float safe = fabsf(a) > 1e-12f ? a : 1.f;
    const float thr = (-bq[q] - other) / safe;
    const float hq = a > 1e-12f ? thr : xh;
    const float lq = a < -1e-12f ? thr : xl;
    hmin = fminf(hmin, hq);
    lmax = fmaxf(lmax, lq);
  }
  hi_o = fminf(hmin, xh);
  lo_o = fmaxf(lmax, xl);
}

constexpr int CLIP_MAXQ = 64;

__global__ void k_clip(const float* xl, const float* xh, const float* A, const float* bv,
                       int64_t B, int Q, int n, const int32_t* dptr, const int32_t* qidx,
                       int nd, float* xlo, float* xho, uint8_t* feas) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < B;
       b += (int64_t)gridDim.x * blockDim.x) {
  const float* Ab = A + b * (int64_t)Q * n;
  const float* bb = bv + b * (int64_t)Q;
  const float* l = xl + b * n;
  const float* h = xh + b * n;
  float* lo_o = xlo + b * n;
  float* hi_o = xho + b * n;
  float tot[CLIP_MAXQ];
  bool any_feas = false, single = false;
  for (int d = 0; d < nd; ++d) {
    const int32_t* qs = qidx + dptr[d];
    const int nq = min(dptr[d + 1] - dptr[d], CLIP_MAXQ);
    bool empty = false;
    for (int t = 0; t < nq; ++t) {
      const int q = qs[t];
      float s1 = 0.f, s2 = 0.f;
      for (int i = 0; i < n; ++i) {
        const float a = Ab[q * n + i];
        s1 += fmaxf(a, 0.f) * l[i];
        s2 += fminf(a, 0.f) * h[i];
      }
      tot[t] = s1 + s2;
      empty |= (tot[t] + bb[q]) > 0.f;
    }
    for (int i = 0; i < n; ++i) {
      float lo, hi;
      clip_dim(Ab, bb, tot, qs, nq, n, i, l[i], h[i], lo, hi);
      empty |= lo > hi;
    }
    const bool fd = !empty;
    if (nd == 1) {
      for (int i = 0; i < n; ++i) clip_dim(Ab, bb, tot, qs, nq, n, i, l[i], h[i], lo_o[i], hi_o[i]);
      feas[b] = fd;
      single = true;
      break;
    }
    if (fd) {
      for (int i = 0; i < n; ++i) {
        float lo, hi;
        clip_dim(Ab, bb, tot, qs, nq, n, i, l[i], h[i], lo, hi);
        if (!any_feas) {
          lo_o[i] = lo;
          hi_o[i] = hi;
        } else {
          lo_o[i] = fminf(lo_o[i], lo);
          hi_o[i] = fmaxf(hi_o[i], hi);
        }
      }
      any_feas = true;
    }
  }
  if (single) continue;
  if (!any_feas) {
    for (int i = 0; i < n; ++i) {
      lo_o[i] = l[i];
      hi_o[i] = h[i];
    }
  }
  feas[b] = any_feas;
  }
}

// Boxes of at most NMAX dims: one thread per box.  The workgroup's rows of
// A and b are copied to LDS with coalesced loads (one record of Q n + Q
// floats per box, odd stride: conflict-free); the box, the per-dimension
// running bounds and the union live in registers (loops over dims fully
// unrolled), and each query's total is formed inside the query loop.  Same
// arithmetic, in the same order per value, as k_clip / clip_dim.
template <int NMAX>
__global__ __launch_bounds__(64) void k_clip_reg(const float* xl, const float* xh,
                                                 const float* A, const float* bv, int64_t B,
                                                 int Q, int n, const int32_t* dptr,
                                                 const int32_t* qidx, int nd, float* xlo,
                                                 float* xho, uint8_t* feas) {
  extern __shared__ float rec[];
  const int qn = Q * n, w = qn + Q, rs = w | 1;
  const float invw = 1.f / (float)w;
  const int t = threadIdx.x;
  const float* Ab = rec + t * rs;
  const float* bb = Ab + qn;
  for (int64_t b0 = (int64_t)blockIdx.x * 64; b0 < B; b0 += (int64_t)gridDim.x * 64) {
    const int nb = (int)min((int64_t)64, B - b0);
    // record r = [A row (Q n) | b row (Q)]; i = r w + c, c < w: the float
    // quotient is at least 0.5 / w from an integer, far above its rounding.
    // Eight loads in flight per thread before their stores (a batch of
    // small domains is otherwise one load latency per element).
    for (int i0 = t; i0 < nb * w; i0 += 64 * 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 64 * k;
        const int r = (int)((i + 0.5f) * invw);
        const int c = i - r * w;
        v[k] = i < nb * w ? (c < qn ? A[(b0 + r) * qn + c] : bv[(b0 + r) * Q + (c - qn)]) : 0.f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 64 * k;
        const int r = (int)((i + 0.5f) * invw);
        if (i < nb * w) rec[r * rs + i - r * w] = v[k];
      }
    }
    __syncthreads();
    if (t < nb) {
      const int64_t b = b0 + t;
      float l[NMAX], h[NMAX], ol[NMAX], oh[NMAX];
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        l[i] = i < n ? xl[b * n + i] : 0.f;
        h[i] = i < n ? xh[b * n + i] : 0.f;
        ol[i] = l[i];
        oh[i] = h[i];
      }
      bool any_feas = false;
      for (int d = 0; d < nd; ++d) {
        const int32_t* qs = qidx + dptr[d];
        const int nq = dptr[d + 1] - dptr[d];
        float hm[NMAX], lm[NMAX];
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          hm[i] = INFINITY;
          lm[i] = -INFINITY;
        }
        bool empty = false;
        for (int k = 0; k < nq; ++k) {
          const int q = qs[k];
          const float* aq = Ab + q * n;
          float s1 = 0.f, s2 = 0.f;
#pragma unroll
          for (int i = 0; i < NMAX; ++i) {
            if (i < n) {
              const float a = aq[i];
              s1 += fmaxf(a, 0.f) * l[i];
              s2 += fminf(a, 0.f) * h[i];
            }
          }
          const float tq = s1 + s2;
          const float bq = bb[q];
          empty |= (tq + bq) > 0.f;
#pragma unroll
          for (int i = 0; i < NMAX; ++i) {
            if (i < n) {
              const float a = aq[i];
              const float contrib = fmaxf(a, 0.f) * l[i] + fminf(a, 0.f) * h[i];
              const float other = tq - contrib;
              const float safe = fabsf(a) > 1e-12f ? a : 1.f;
              const float thr = (-bq - other) / safe;
              hm[i] = fminf(hm[i], a > 1e-12f ? thr : h[i]);
              lm[i] = fmaxf(lm[i], a < -1e-12f ? thr : l[i]);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          hm[i] = fminf(hm[i], h[i]);
          lm[i] = fmaxf(lm[i], l[i]);
          if (i < n) empty |= lm[i] > hm[i];
        }
        if (nd == 1) {
#pragma unroll
          for (int i = 0; i < NMAX; ++i) {
            ol[i] = lm[i];
            oh[i] = hm[i];
          }
          any_feas = !empty;
          break;
        }
        if (!empty) {
#pragma unroll
          for (int i = 0; i < NMAX; ++i) {
            ol[i] = any_feas ? fminf(ol[i], lm[i]) : lm[i];
            oh[i] = any_feas ? fmaxf(oh[i], hm[i]) : hm[i];
          }
          any_feas = true;
        }
      }
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        if (i < n) {
          xlo[b * n + i] = ol[i];
          xho[b * n + i] = oh[i];
        }
      }
      feas[b] = any_feas;
    }
    __syncthreads();
  }
}

// Boxes of n dims with at most QP queries (QP a power of two, QP n <= 64):
// one wavefront per box, lane i QP + q taking query q on dimension i.
// Each lane forms its query's total itself (the same sums in the same
// order as k_clip_reg), its own threshold, and the minimum / maximum over
// a disjunct's queries is a butterfly over the QP lanes of a dimension
// (min and max do not depend on the order).  Same values as k_clip_reg; a
// batch of a few hundred boxes takes one load round trip instead of a
// serial loop per box.
template <int QP>
__global__ __launch_bounds__(256) void k_clip_lanes(const float* __restrict__ xl,
                                                    const float* __restrict__ xh,
                                                    const float* __restrict__ A,
                                                    const float* __restrict__ bv, int64_t B,
                                                    int Q, int n, const int32_t* dptr,
                                                    const int32_t* qidx, int nd, float* xlo,
                                                    float* xho, uint8_t* feas) {
  const int lane = threadIdx.x & 63;
  const int q = lane % QP, i = lane / QP;
  const bool on = q < Q && i < n;
  const int64_t nw = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t b = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); b < B;
       b += nw) {
    const float* aq = A + (b * Q + (on ? q : 0)) * n;
    const float* l = xl + b * n;
    const float* h = xh + b * n;
    const int ii = on ? i : 0;
    const float a = aq[ii], li = l[ii], hi = h[ii];
    const float bq = bv[b * Q + (on ? q : 0)];
    float s1 = 0.f, s2 = 0.f;
    for (int k = 0; k < n; ++k) {
      const float ak = aq[k];
      s1 += fmaxf(ak, 0.f) * l[k];
      s2 += fminf(ak, 0.f) * h[k];
    }
    const float tq = s1 + s2;
    const float contrib = fmaxf(a, 0.f) * li + fminf(a, 0.f) * hi;
    const float other = tq - contrib;
    const float safe = fabsf(a) > 1e-12f ? a : 1.f;
    const float thr = (-bq - other) / safe;
    const float hq = a > 1e-12f ? thr : hi;
    const float lq = a < -1e-12f ? thr : li;
    float ol = li, oh = hi;
    bool any_feas = false;
    for (int d = 0; d < nd; ++d) {
      // this lane's query in disjunct d (listed once or more)
      bool mem = false;
      for (int t = dptr[d]; t < dptr[d + 1]; ++t) mem |= qidx[t] == q;
      mem &= on;
      float hm = mem ? hq : INFINITY, lm = mem ? lq : -INFINITY;
#pragma unroll
      for (int o = 1; o < QP; o <<= 1) {
        hm = fminf(hm, __shfl_xor(hm, o, 64));
        lm = fmaxf(lm, __shfl_xor(lm, o, 64));
      }
      hm = fminf(hm, hi);
      lm = fmaxf(lm, li);
      const bool empty = __ballot((mem && (tq + bq) > 0.f) || (on && lm > hm)) != 0ull;
      if (nd == 1) {
        ol = lm;
        oh = hm;
        any_feas = !empty;
        break;
      }
      if (!empty) {
        ol = any_feas ? fminf(ol, lm) : lm;
        oh = any_feas ? fmaxf(oh, hm) : hm;
        any_feas = true;
      }
    }
    if (on && q == 0) {
      xlo[b * n + i] = ol;
      xho[b * n + i] = oh;
    }
    if (lane == 0) feas[b] = any_feas;
  }
}

// ---- compaction: ascending positions of non-zero flags -------------------
constexpr int CPT = 4;               // flags per thread
constexpr int CCH = NT * CPT;        // flags per block

__device__ __forceinline__ int block_excl_scan(int v, int* total) {
  __shared__ int wsum[NT / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  int off = 0, tot = 0;
  for (int i = 0; i < NT / 64; ++i) {
    if (i < w) off += wsum[i];
    tot += wsum[i];
  }
  __syncthreads();
  *total = tot;
  return off + x - v;
}

__device__ __forceinline__ bool sel_hit(const uint8_t* f, int64_t i, int64_t n, int zero) {
  return i < n && ((f[i] != 0) != (zero != 0));
}

__global__ void k_compact_count(const uint8_t* f, int64_t n, int zero, int64_t* bcnt) {
  const int64_t base = blockIdx.x * (int64_t)CCH + threadIdx.x * CPT;
  int c = 0;
  for (int e = 0; e < CPT; ++e)
    if (sel_hit(f, base + e, n, zero)) ++c;
  int tot;
  block_excl_scan(c, &tot);
  if (threadIdx.x == 0) bcnt[blockIdx.x] = tot;
}

__global__ void k_compact_scan(int64_t* bcnt, int64_t nb, int64_t* count_out) {
  // single block: exclusive scan of nb block counts in chunks of NT
  __shared__ int64_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < nb; c0 += NT) {
    const int64_t i = c0 + threadIdx.x;
    const int64_t v = i < nb ? bcnt[i] : 0;
    __shared__ int64_t buf[NT];
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < NT; o <<= 1) {
      const int64_t y = threadIdx.x >= o ? buf[threadIdx.x - o] : 0;
      __syncthreads();
      buf[threadIdx.x] += y;
      __syncthreads();
    }
    if (i < nb) bcnt[i] = carry + buf[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == NT - 1) carry += buf[NT - 1];
    __syncthreads();
  }
  if (threadIdx.x == 0) count_out[0] = carry;
}

__global__ void k_compact_write(const uint8_t* f, int64_t n, int zero, const int64_t* boff,
                                int64_t* idx) {
  const int64_t base = blockIdx.x * (int64_t)CCH + threadIdx.x * CPT;
  int c = 0;
  for (int e = 0; e < CPT; ++e)
    if (sel_hit(f, base + e, n, zero)) ++c;
  int tot;
  int off = block_excl_scan(c, &tot);
  int64_t o = boff[blockIdx.x] + off;
  for (int e = 0; e < CPT; ++e)
    if (sel_hit(f, base + e, n, zero)) idx[o++] = base + e;
}

// Compaction of up to C1N flags in one launch: one workgroup sweeps the
// flags in passes of C1T x C1P, each thread C1P consecutive flags (one
// 16-byte load when VEC), a workgroup scan per pass and a running carry.
// The same ascending indices as the three-launch form, without its two
// extra launches (the round's compactions are of 65,536 flags or fewer).
constexpr int C1T = 1024, C1P = 16;
constexpr int64_t C1N = (int64_t)1 << 17;

template <bool VEC>
__global__ __launch_bounds__(C1T) void k_compact_single(const uint8_t* __restrict__ f, int64_t n,
                                                         int zero, int64_t* __restrict__ idx,
                                                         int64_t* __restrict__ count_out) {
  __shared__ int wsum[C1T / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t carry = 0;
  for (int64_t c0 = 0; c0 < n; c0 += (int64_t)C1T * C1P) {
    const int64_t base = c0 + (int64_t)threadIdx.x * C1P;
    uint32_t bits = 0;
    if (VEC && base + C1P <= n) {
      const uint4 v = *reinterpret_cast<const uint4*>(f + base);
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < C1P; ++e) {
        const bool set = ((wd[e >> 2] >> (8 * (e & 3))) & 0xffu) != 0;
        if (set != (zero != 0)) bits |= 1u << e;
      }
    } else {
#pragma unroll
      for (int e = 0; e < C1P; ++e)
        if (sel_hit(f, base + e, n, zero)) bits |= 1u << e;
    }
    const int c = __popc(bits);
    int x = c;  // inclusive scan within the wave
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < C1T / 64; ++i) {
      if (i < w) off += wsum[i];
      tot += wsum[i];
    }
    int64_t o = carry + off + x - c;
    for (int e = 0; e < C1P; ++e)
      if ((bits >> e) & 1u) idx[o++] = base + e;
    carry += tot;
    __syncthreads();  // wsum is rewritten by the next pass
  }
  if (threadIdx.x == 0) count_out[0] = carry;
}

__global__ void k_and_flags(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
                            int64_t n, uint8_t* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = (a[i] != 0 && b[i] != 0) ? 1 : 0;
}

// Two compactions of n flags in one launch, one workgroup each (n <= C1N):
// job j selects i where a_j[i] != 0 and (b_j null or b_j[i] != 0), in the
// ascending order of k_compact_single.
struct Compact2 {
  const uint8_t* a[2];
  const uint8_t* b[2];
  int64_t* idx[2];
  int64_t* count[2];
};

__global__ __launch_bounds__(C1T) void k_compact_pair(Compact2 jobs, int64_t n) {
  __shared__ int wsum[C1T / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint8_t* fa = jobs.a[blockIdx.x];
  const uint8_t* fb = jobs.b[blockIdx.x];
  int64_t* idx = jobs.idx[blockIdx.x];
  int64_t carry = 0;
  for (int64_t c0 = 0; c0 < n; c0 += (int64_t)C1T * C1P) {
    const int64_t base = c0 + (int64_t)threadIdx.x * C1P;
    uint32_t bits = 0;
#pragma unroll
    for (int e = 0; e < C1P; ++e) {
      const int64_t i = base + e;
      if (i < n && fa[i] != 0 && (fb == nullptr || fb[i] != 0)) bits |= 1u << e;
    }
    const int c = __popc(bits);
    int x = c;  // inclusive scan within the wave
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < C1T / 64; ++i) {
      if (i < w) off += wsum[i];
      tot += wsum[i];
    }
    int64_t o = carry + off + x - c;
    for (int e = 0; e < C1P; ++e)
      if ((bits >> e) & 1u) idx[o++] = base + e;
    carry += tot;
    __syncthreads();  // wsum is rewritten by the next pass
  }
  if (threadIdx.x == 0) jobs.count[blockIdx.x][0] = carry;
}

// rows[idx[r]] = max(rows[idx[r]], src[r]) over rows of q floats.
__global__ void k_scatter_max_rows(float* rows, const int64_t* idx, const float* src, int64_t nr,
                                   int q) {
  const int64_t total = nr * (int64_t)q;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / q;
    const int c = (int)(i % q);
    float* d = rows + idx[r] * q + c;
    *d = fmaxf(*d, src[i]);
  }
}

__global__ void k_gather_rows(const float* in, const int64_t* idx, int64_t nr, int cols,
                              float* out) {
  const int64_t total = nr * (int64_t)cols;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols;
    const int c = (int)(i % cols);
    out[i] = in[idx[r] * cols + c];
  }
}

__global__ void k_scatter_rows(const float* in, const int64_t* idx, int64_t nr, int cols,
                               float* out) {
  const int64_t total = nr * (int64_t)cols;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols;
    const int c = (int)(i % cols);
    out[idx[r] * cols + c] = in[i];
  }
}

// First index of the maximum width (NaN counts as maximal, like argmax).
__global__ void k_widest(const float* xl, const float* xh, int64_t B, int n, int64_t* ax,
                         uint8_t* usable) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < B;
       b += (int64_t)gridDim.x * blockDim.x) {
  int best = 0;
  float bw = xh[b * n] - xl[b * n];
  if (!isnan(bw)) {
    for (int i = 1; i < n; ++i) {
      const float w = xh[b * n + i] - xl[b * n + i];
      if (isnan(w)) {
        best = i;
        bw = w;
        break;
      }
      if (w > bw) {
        bw = w;
        best = i;
      }
    }
  }
  ax[b] = best;
  if (usable) usable[b] = (xh[b * n + best] - xl[b * n + best]) > 1e-12f;
  }
}

// One workgroup: flag[0] = 1 if any entry of the new box is tighter than the
// old one (xl_new > xl_old or xh_new < xh_old), else 0.  The workgroup owns the
// whole flag, so nothing has to be cleared before the launch.
__global__ __launch_bounds__(1024) void k_box_shrunk(const float* xl_o, const float* xh_o,
                                                     const float* xl_n, const float* xh_n,
                                                     int64_t n, int32_t* flag) {
  __shared__ int any;
  if (threadIdx.x == 0) any = 0;
  __syncthreads();
  int mine = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x)
    mine |= (xl_n[i] > xl_o[i]) | (xh_n[i] < xh_o[i]);
  if (__any(mine) && (threadIdx.x & 63) == 0) any = 1;
  __syncthreads();
  if (threadIdx.x == 0) flag[0] = any;
}

__global__ void k_bisect(const float* xl, const float* xh, const int64_t* ax,
                         const int64_t* uidx, int64_t nu, int n, float* lxl, float* lxh,
                         float* hxl, float* hxh) {
  const int64_t total = nu * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / n;
    const int c = (int)(i % n);
    const int64_t src = uidx[r];
    const int a = (int)ax[src];
    const float l = xl[src * n + c], h = xh[src * n + c];
    const float mid = (xl[src * n + a] + xh[src * n + a]) * 0.5f;
    lxl[i] = l;
    lxh[i] = c == a ? mid : h;
    hxl[i] = c == a ? mid : l;
    hxh[i] = h;
  }
}

__global__ void k_zono_input(const float* xl, const float* xh, int64_t B, int n,
                             const int32_t* vidx, int K, float* c, float* G) {
  const int64_t total = B * (int64_t)n;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    c[i] = (xl[i] + xh[i]) / 2.f;
  }
  const int64_t tg = total * (int64_t)K;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < tg;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t bi = i / K;
    const int k = (int)(i % K);
    const int j = (int)(bi % n);
    G[i] = (vidx[k] == j) ? (xh[bi] - xl[bi]) / 2.f : 0.f;
  }
}

}  // namespace

extern "C" int vc_abi_version(void) { return 1; }

extern "C" int vc_make_slopes(const float* lo, const float* hi, int64_t n, float* lo_s,
                              float* up_s, float* up_t, uint8_t* active, uint8_t* dead,
                              uint8_t* unstable, vc_stream_t stream) {
  if (n < 0 || (n > 0 && (!lo || !hi || !lo_s || !up_s || !up_t))) return VC_ERR_ARG;
  if (n == 0) return VC_OK;
  hipLaunchKernelGGL(k_make_slopes, dim3(vc_blocks(n, NT)), dim3(NT), 0, (hipStream_t)stream,
                     lo, hi, n, lo_s, up_s, up_t, active, dead, unstable);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_alpha_init(const float* lo, const float* hi, int64_t n, float* alpha,
                             vc_stream_t stream) {
  if (n < 0 || (n > 0 && (!lo || !hi || !alpha))) return VC_ERR_ARG;
  if (n == 0) return VC_OK;
  hipLaunchKernelGGL(k_alpha_init, dim3(vc_blocks(n, NT)), dim3(NT), 0, (hipStream_t)stream,
                     lo, hi, n, alpha);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_ibp_relu(const float* l, const float* h, int64_t B, int n,
                           const float* root_lo, const float* root_hi, const float* cl,
                           const float* ch, float* sb_lo, float* sb_hi, float* post_lo,
                           float* post_hi, vc_stream_t stream) {
  if (!sb_lo || !sb_hi || B < 0 || n <= 0) return VC_ERR_ARG;
  if ((l == nullptr) != (h == nullptr) || (!l && !root_lo)) return VC_ERR_ARG;
  if ((root_lo == nullptr) != (root_hi == nullptr) || (cl == nullptr) != (ch == nullptr) ||
      (post_lo == nullptr) != (post_hi == nullptr))
    return VC_ERR_ARG;
  const int64_t total = B * (int64_t)n;
  if (total == 0) return VC_OK;
  hipLaunchKernelGGL(k_ibp_relu, dim3(vc_blocks(total, NT)), dim3(NT), 0, (hipStream_t)stream,
                     l, h, B, n, root_lo, root_hi, cl, ch, sb_lo, sb_hi, post_lo, post_hi);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_concretize(const float* A, const float* acc, const float* xl,
                             const float* xh, int64_t M, int R, int n_in, int a_bcast,
                             float* lb, vc_stream_t stream) {
  if (!A || !acc || !xl || !xh || !lb || R <= 0 || n_in <= 0 || M < 0 || M % R) return VC_ERR_ARG;
  if (M == 0) return VC_OK;
  hipStream_t st = (hipStream_t)stream;
  // the tiled form: RPT x CT rows per workgroup, two up to 16 inputs (at 5
  // inputs, 524,288 domains x 4 rows: 19.6 us against 21.3 for one row
  // per thread and 23.3 for four, whose 31 KB of LDS allow 5 workgroups
  // per CU); LDS for the rows of A and the boxes of at most (TR - 1) / R
  // + 2 domains (a tile's rows straddle domain boundaries), 3 more floats
  // for the aligned start
  const int rpt = n_in <= 16 ? 2 : 1;
  const int64_t tr = (int64_t)rpt * CT;
  const int64_t nd_max = R >= tr ? 2 : std::min<int64_t>(tr, (tr - 1) / R + 2);
  const size_t lds_tile =
      sizeof(float) * ((size_t)tr * n_in + 2 * (((size_t)nd_max * n_in + 3 + 3) & ~(size_t)3));
  if (n_in <= CT_MAXN && !a_bcast && aligned16(A) && lds_tile <= 64 * 1024 &&
      (M + tr - 1) / tr <= 0x7fffffff) {
    const dim3 grid((unsigned)((M + tr - 1) / tr));
    if (rpt == 2)
      hipLaunchKernelGGL(k_concretize_tile<2>, grid, dim3(CT), lds_tile, st, A, acc, xl, xh, M,
                         R, n_in, lb);
    else
      hipLaunchKernelGGL(k_concretize_tile<1>, grid, dim3(CT), lds_tile, st, A, acc, xl, xh, M,
                         R, n_in, lb);
  } else if (n_in <= CT_MAXN) {
    hipLaunchKernelGGL(k_concretize_thread, dim3(vc_blocks(M, CT)), dim3(CT), 0, st, A, a_bcast,
                       acc, xl, xh, M, R, n_in, lb);
  } else if (n_in % 4 == 0 && aligned16(A) && aligned16(xl) && aligned16(xh)) {
    hipLaunchKernelGGL(k_concretize_wave<true>, dim3(vc_blocks((M + CR - 1) / CR * 64, NT)),
                       dim3(NT), 0, st, A, a_bcast, acc, xl, xh, M, R, n_in, lb);
  } else {
    hipLaunchKernelGGL(k_concretize_wave<false>, dim3(vc_blocks((M + CR - 1) / CR * 64, NT)),
                       dim3(NT), 0, st, A, a_bcast, acc, xl, xh, M, R, n_in, lb);
  }
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_backward_relu(const float* ew_in, int64_t M, int R, int n,
                                const float* relu_lo, const float* relu_hi,
                                const float* alpha, int alpha_per_row, const float* beta,
                                float* ew_out, float* acc, vc_stream_t stream) {
  if (!ew_in || !relu_lo || !relu_hi || !ew_out || !acc || R <= 0 || n <= 0 || M < 0 || M % R)
    return VC_ERR_ARG;
  if (M == 0) return VC_OK;
  const bool vec = n % 4 == 0 && aligned16(ew_in) && aligned16(relu_lo) && aligned16(relu_hi) &&
                   aligned16(ew_out) && (!alpha || aligned16(alpha)) && (!beta || aligned16(beta));
  if (vec && n >= 1024) {
    const dim3 grid(vc_blocks((M + RB - 1) / RB, 1));
    hipStream_t st = (hipStream_t)stream;
    if (alpha && beta)
      hipLaunchKernelGGL((k_backward_relu_rows<true, true>), grid, dim3(256), 0, st, ew_in, M, R,
                         n, relu_lo, relu_hi, alpha, alpha_per_row, beta, ew_out, acc);
    else if (alpha)
      hipLaunchKernelGGL((k_backward_relu_rows<true, false>), grid, dim3(256), 0, st, ew_in, M, R,
                         n, relu_lo, relu_hi, alpha, alpha_per_row, beta, ew_out, acc);
    else if (beta)
      hipLaunchKernelGGL((k_backward_relu_rows<false, true>), grid, dim3(256), 0, st, ew_in, M, R,
                         n, relu_lo, relu_hi, alpha, alpha_per_row, beta, ew_out, acc);
    else
      hipLaunchKernelGGL((k_backward_relu_rows<false, false>), grid, dim3(256), 0, st, ew_in, M,
                         R, n, relu_lo, relu_hi, alpha, alpha_per_row, beta, ew_out, acc);
    VC_LAUNCH_CHECK();
    return VC_OK;
  }
  hipLaunchKernelGGL(vec ? k_backward_relu<true> : k_backward_relu<false>,
                     dim3(vc_blocks((M + 1) / 2 * 64, NT)), dim3(NT), 0, (hipStream_t)stream,
                     ew_in, M, R, n, relu_lo, relu_hi, alpha, alpha_per_row, beta, ew_out, acc);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_crown_intersect(const float* sl, const int32_t* idx, int k, int64_t B,
                                  int n, float* lo, float* hi, vc_stream_t stream) {
  if (!sl || !idx || !lo || !hi || k < 0 || B < 0 || n <= 0) return VC_ERR_ARG;
  if ((int64_t)k * B == 0) return VC_OK;
  hipLaunchKernelGGL(k_crown_intersect, dim3(vc_blocks(B * k, NT)), dim3(NT), 0,
                     (hipStream_t)stream, sl, idx, k, B, n, lo, hi);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_unstable_union(const float* lo, const float* hi, int64_t B, int n,
                                 uint8_t* flag, vc_stream_t stream) {
  if (!lo || !hi || !flag || B < 0 || n <= 0) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_fill_u8, dim3(vc_blocks(n, NT)), dim3(NT), 0, st, flag, (int64_t)n,
                     (uint8_t)0);
  if (B > 0)
    hipLaunchKernelGGL(k_unstable_union, dim3(vc_blocks(B * n, NT)), dim3(NT), 0, st, lo, hi,
                       B, n, flag);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_unstable_union_layers(const float* const* lo, const float* const* hi,
                                        const int32_t* widths, int n_layers, int64_t B,
                                        uint8_t* flags, vc_stream_t stream) {
  if (!lo || !hi || !widths || !flags || n_layers < 1 || n_layers > VC_MAXA || B < 0)
    return VC_ERR_ARG;
  LayerPtrs lp{};
  int off = 0, wmax = 0;
  for (int L = 0; L < n_layers; ++L) {
    if (!lo[L] || !hi[L] || widths[L] <= 0) return VC_ERR_ARG;
    lp.lo[L] = lo[L];
    lp.hi[L] = hi[L];
    lp.width[L] = widths[L];
    lp.off[L] = off;
    off += widths[L];
    wmax = widths[L] > wmax ? widths[L] : wmax;
  }
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_fill_u8, dim3(vc_blocks(off, NT)), dim3(NT), 0, st, flags, (int64_t)off,
                     (uint8_t)0);
  if (B > 0)
    hipLaunchKernelGGL(k_unstable_union_layers, dim3(vc_blocks(B * wmax, NT), n_layers),
                       dim3(NT), 0, st, lp, B, flags);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_union_compact(const uint8_t* flags, const int32_t* widths, int n_layers,
                                int32_t* idx, int32_t* meta, vc_stream_t stream) {
  if (!flags || !widths || !idx || !meta || n_layers < 1 || n_layers > 16) return VC_ERR_ARG;
  LayerPtrs lp{};
  int off = 0;
  for (int L = 0; L < n_layers; ++L) {
    if (widths[L] <= 0) return VC_ERR_ARG;
    lp.width[L] = widths[L];
    lp.off[L] = off;
    off += widths[L];
  }
  hipLaunchKernelGGL(k_union_compact, dim3(1), dim3(64 * n_layers), 0, (hipStream_t)stream,
                     flags, lp, n_layers, idx, meta);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_gather_rows_multi(const float* const* in, float* const* out,
                                    const int32_t* cols, int n_arrays, const int64_t* idx,
                                    int64_t n_rows, vc_stream_t stream) {
  if (!in || !out || !cols || !idx || n_arrays < 1 || n_arrays > VC_MAXA || n_rows < 0)
    return VC_ERR_ARG;
  if (n_rows == 0) return VC_OK;
  GatherPtrs gp{};
  int cmax = 0;
  for (int a = 0; a < n_arrays; ++a) {
    if (!in[a] || !out[a] || cols[a] <= 0) return VC_ERR_ARG;
    gp.in[a] = in[a];
    gp.out[a] = out[a];
    gp.cols[a] = cols[a];
    cmax = cols[a] > cmax ? cols[a] : cmax;
  }
  hipLaunchKernelGGL(k_gather_rows_multi, dim3(vc_blocks(n_rows * cmax, NT), n_arrays),
                     dim3(NT), 0, (hipStream_t)stream, gp, idx, n_rows);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_alpha_grad_reduce(const float* gE, const float* P, int p_bcast, int64_t B,
                                    int R, int n, const float* relu_lo, const float* relu_hi,
                                    float* galpha, float* gbeta, vc_stream_t stream) {
  if (!gE || !P || !relu_lo || !relu_hi || R <= 0 || n <= 0 || B < 0) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_alpha_grad_reduce, dim3(vc_blocks(B * n, NT)), dim3(NT), 0,
                     (hipStream_t)stream, gE, P, p_bcast, B, R, n, relu_lo, relu_hi, galpha,
                     gbeta);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_adam_step(float* param, const float* lb_grad, float* exp_avg,
                            float* exp_avg_sq, int64_t n, double b1, double b2, double eps,
                            double step_size, double bc2_sqrt, float lo_clamp, float hi_clamp,
                            vc_stream_t stream) {
  if (!param || !lb_grad || !exp_avg || !exp_avg_sq || n < 0) return VC_ERR_ARG;
  if (n == 0) return VC_OK;
  hipLaunchKernelGGL(k_adam, dim3(vc_blocks(n, NT)), dim3(NT), 0, (hipStream_t)stream, param,
                     lb_grad, exp_avg, exp_avg_sq, n, adam_const(b1, b2, eps, step_size, bc2_sqrt),
                     lo_clamp, hi_clamp);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_beta_adam_step(float* beta, const float* sign, const float* lb_grad_signed,
                                 float* exp_avg, float* exp_avg_sq, int64_t n, double b1,
                                 double b2, double eps, double step_size, double bc2_sqrt,
                                 float* beta_signed, vc_stream_t stream) {
  if (n < 0) return VC_ERR_ARG;
  if (n == 0) return VC_OK;
  if (!beta || !sign || !lb_grad_signed || !exp_avg || !exp_avg_sq || !beta_signed)
    return VC_ERR_ARG;
  hipLaunchKernelGGL(k_beta_adam, dim3(vc_blocks(n, NT)), dim3(NT), 0, (hipStream_t)stream, beta,
                     sign, lb_grad_signed, exp_avg, exp_avg_sq, n,
                     adam_const(b1, b2, eps, step_size, bc2_sqrt), beta_signed);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_split_beta_sign(const float* cl, const float* ch, int64_t n, float* sign,
                                  vc_stream_t stream) {
  if (n < 0) return VC_ERR_ARG;
  if (n == 0) return VC_OK;
  if (!cl || !ch || !sign) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_split_beta_sign, dim3(vc_blocks(n, NT)), dim3(NT), 0, (hipStream_t)stream,
                     cl, ch, n, sign);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_split_clamps(const int64_t* layer, const int64_t* neuron, const int64_t* side,
                               int64_t D, int S, int64_t L, int n, float* cl, float* ch,
                               float* sign, vc_stream_t stream) {
  if (D < 0 || S < 0 || n <= 0 || L < 0) return VC_ERR_ARG;
  if (D == 0) return VC_OK;
  if (!cl || !ch || (S > 0 && (!layer || !neuron || !side))) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_split_clamps, dim3(vc_blocks(D * n, NT)), dim3(NT), 0,
                     (hipStream_t)stream, layer, neuron, side, D, S, L, n, cl, ch, sign);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_best_update(float* best, const float* lb, int64_t n, int init, float* out2,
                              vc_stream_t stream) {
  if (!best || !lb || !out2 || n <= 0) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_best_update, dim3(1), dim3(1024), 0, (hipStream_t)stream, best, lb, n,
                     init, out2);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

int alpha_control_chunk(float* best, const float* lbs, int64_t n, int it0, int n_it, double eps,
                        float* ctl, int32_t* stop_host, hipStream_t stream) {
  if (!best || !lbs || !ctl || n <= 0 || it0 < 0 || n_it < 1) return VC_ERR_ARG;
  if (n_it > VC_ALPHA_CHUNK) return VC_ERR_ARG;
  alpha_control_launch(best, lbs, n, it0, n_it, eps, ctl, stop_host,
                       stop_host ? stop_host + 1 : nullptr, stream);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_alpha_control(float* best, const float* lb, int64_t n, int it, double eps,
                                float* ctl, int32_t* stop_host, vc_stream_t stream) {
  if (!best || !lb || !ctl || n <= 0 || it < 0) return VC_ERR_ARG;
  alpha_control_launch(best, lb, n, it, 1, eps, ctl, stop_host, nullptr, (hipStream_t)stream);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_closure(const float* lb, int64_t B, int Q, const int32_t* d_ptr,
                          const int32_t* q_idx, int n_disj, uint8_t* closed,
                          vc_stream_t stream) {
  if (!lb || !d_ptr || !q_idx || !closed || B < 0 || Q <= 0 || n_disj < 0) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_closure, dim3(vc_blocks(B, NT)), dim3(NT), 0, (hipStream_t)stream, lb,
                     B, Q, d_ptr, q_idx, n_disj, closed);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_clip_box(const float* xl, const float* xh, const float* A, const float* b,
                           int64_t B, int Q, int n, const int32_t* d_ptr,
                           const int32_t* q_idx, int n_disj, float* xl_out, float* xh_out,
                           uint8_t* feasible, vc_stream_t stream) {
  if (!xl || !xh || !A || !b || !d_ptr || !q_idx || !xl_out || !xh_out || !feasible)
    return VC_ERR_ARG;
  if (B < 0 || Q <= 0 || n <= 0 || n_disj <= 0) return VC_ERR_ARG;
  if (Q > CLIP_MAXQ) return VC_ERR_UNSUPPORTED;
  if (B == 0) return VC_OK;
  int qp = 1;
  while (qp < Q) qp <<= 1;
  // one wavefront per box for batches of up to 64 boxes per CU (a few
  // hundred leaves: a load round trip instead of each lane's serial
  // chain); larger batches keep one lane per box, whose throughput is
  // higher (524,288 boxes: 227 us one wavefront per box)
  if (qp * n <= 64 && B <= 64 * (int64_t)vcm::cu_count()) {
    const int64_t nblk = std::min<int64_t>((B + 3) / 4, 65536);
    hipStream_t st = (hipStream_t)stream;
#define VC_CLIP_LANES(QP)                                                                     \
  case QP:                                                                                    \
    hipLaunchKernelGGL(k_clip_lanes<QP>, dim3((unsigned)nblk), dim3(256), 0, st, xl, xh, A, b, \
                       B, Q, n, d_ptr, q_idx, n_disj, xl_out, xh_out, feasible);              \
    break;
    switch (qp) {
      VC_CLIP_LANES(1)
      VC_CLIP_LANES(2)
      VC_CLIP_LANES(4)
      VC_CLIP_LANES(8)
      VC_CLIP_LANES(16)
      VC_CLIP_LANES(32)
      VC_CLIP_LANES(64)
      default: return VC_ERR_UNSUPPORTED;
    }
#undef VC_CLIP_LANES
    VC_LAUNCH_CHECK();
    return VC_OK;
  }
  const size_t rec_bytes = 64 * (size_t)((Q * n + Q) | 1) * sizeof(float);
  if (n <= 8 && rec_bytes <= 32768)
    hipLaunchKernelGGL(k_clip_reg<8>, dim3(vc_blocks(B, 64)), dim3(64), rec_bytes,
                       (hipStream_t)stream, xl, xh, A, b, B, Q, n, d_ptr, q_idx, n_disj, xl_out,
                       xh_out, feasible);
  else if (n <= 16 && rec_bytes <= 32768)
    hipLaunchKernelGGL(k_clip_reg<16>, dim3(vc_blocks(B, 64)), dim3(64), rec_bytes,
                       (hipStream_t)stream, xl, xh, A, b, B, Q, n, d_ptr, q_idx, n_disj, xl_out,
                       xh_out, feasible);
  else
    hipLaunchKernelGGL(k_clip, dim3(vc_blocks(B, 64)), dim3(64), 0, (hipStream_t)stream, xl, xh,
                       A, b, B, Q, n, d_ptr, q_idx, n_disj, xl_out, xh_out, feasible);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int64_t vc_compact_workspace(int64_t n) {
  const int64_t nb = (n + CCH - 1) / CCH;
  return (nb < 1 ? 1 : nb) * (int64_t)sizeof(int64_t);
}

extern "C" int vc_scatter_max_rows(float* rows, const int64_t* idx, const float* src,
                                   int64_t n_rows, int q, vc_stream_t stream) {
  if (!rows || !idx || !src || n_rows < 0 || q <= 0) return VC_ERR_ARG;
  if (n_rows == 0) return VC_OK;
  hipLaunchKernelGGL(k_scatter_max_rows, dim3(vc_blocks(n_rows * q, NT)), dim3(NT), 0,
                     (hipStream_t)stream, rows, idx, src, n_rows, q);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

namespace vcm {
// vc_closure that also lists the open rows (any order) and counts them in
// *open_cnt (cleared by the caller on the stream beforehand).
int closure_open(const float* lb, int64_t B, int Q, const int32_t* d_ptr, const int32_t* q_idx,
                 int n_disj, uint8_t* closed, int64_t* open_idx, int64_t* open_cnt,
                 hipStream_t st) {
  if (!lb || !d_ptr || !q_idx || !closed || !open_idx || !open_cnt || B < 0 || Q <= 0 ||
      n_disj < 0)
    return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_closure_open, dim3(vc_blocks(B, NT)), dim3(NT), 0, st, lb, B, Q, d_ptr,
                     q_idx, n_disj, closed, open_idx,
                     reinterpret_cast<unsigned long long*>(open_cnt));
  VC_LAUNCH_CHECK();
  return VC_OK;
}

// vc_scatter_max_rows followed by vc_closure over all B rows, for distinct
// idx: only the scattered rows change, so only their closure is redone.
int scatter_max_close(float* lb, const int64_t* idx, const float* src, int64_t nr, int Q,
                      const int32_t* d_ptr, const int32_t* q_idx, int n_disj, uint8_t* closed,
                      hipStream_t st) {
  if (!lb || !idx || !src || !d_ptr || !q_idx || !closed || nr < 0 || Q <= 0 || n_disj < 0)
    return VC_ERR_ARG;
  if (nr == 0) return VC_OK;
  hipLaunchKernelGGL(k_scatter_max_close, dim3(vc_blocks(nr, NT)), dim3(NT), 0, st, lb, idx, src,
                     nr, Q, d_ptr, q_idx, n_disj, closed);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

// The feasible rows and the rows that are feasible and splittable, compacted
// together (the input-split round): idx_f / cnt_f over feasible, idx_s /
// cnt_s over feasible AND usable; two vc_compact calls above C1N flags.
int compact_feasible_split(const uint8_t* feasible, const uint8_t* usable, int64_t n,
                           int64_t* idx_f, int64_t* cnt_f, int64_t* idx_s, int64_t* cnt_s,
                           uint8_t* split_tmp, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (!feasible || !usable || !idx_f || !cnt_f || !idx_s || !cnt_s || n < 0) return VC_ERR_ARG;
  if (n <= C1N) {
    Compact2 jobs{{feasible, feasible}, {nullptr, usable}, {idx_f, idx_s}, {cnt_f, cnt_s}};
    hipLaunchKernelGGL(k_compact_pair, dim3(2), dim3(C1T), 0, st, jobs, n);
    VC_LAUNCH_CHECK();
    return VC_OK;
  }
  if (!split_tmp) return VC_ERR_ARG;
  hipLaunchKernelGGL(k_and_flags, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)),
                     dim3(256), 0, st, feasible, usable, n, split_tmp);
  VC_LAUNCH_CHECK();
  int rc = vc_compact(feasible, n, 0, idx_f, cnt_f, ws, ws_bytes, (vc_stream_t)st);
  if (rc != VC_OK) return rc;
  return vc_compact(split_tmp, n, 0, idx_s, cnt_s, ws, ws_bytes, (vc_stream_t)st);
}
}  // namespace vcm

extern "C" int vc_compact(const uint8_t* flags, int64_t n, int select_zero, int64_t* idx_out,
                          int64_t* count_out, void* workspace, int64_t ws_bytes,
                          vc_stream_t stream) {
  if (!flags || !idx_out || !count_out || !workspace || n < 0) return VC_ERR_ARG;
  if (ws_bytes < vc_compact_workspace(n)) return VC_ERR_OOM;
  hipStream_t st = (hipStream_t)stream;
  int64_t nb = (n + CCH - 1) / CCH;
  if (nb < 1) nb = 1;
  if (nb > 2147483647LL) return VC_ERR_ARG;
  if (n <= C1N) {
    if (aligned16(flags))
      hipLaunchKernelGGL(k_compact_single<true>, dim3(1), dim3(C1T), 0, st, flags, n, select_zero,
                         idx_out, count_out);
    else
      hipLaunchKernelGGL(k_compact_single<false>, dim3(1), dim3(C1T), 0, st, flags, n,
                         select_zero, idx_out, count_out);
    VC_LAUNCH_CHECK();
    return VC_OK;
  }
  int64_t* bc = (int64_t*)workspace;
  hipLaunchKernelGGL(k_compact_count, dim3((unsigned)nb), dim3(NT), 0, st, flags, n, select_zero,
                     bc);
  hipLaunchKernelGGL(k_compact_scan, dim3(1), dim3(NT), 0, st, bc, nb, count_out);
  hipLaunchKernelGGL(k_compact_write, dim3((unsigned)nb), dim3(NT), 0, st, flags, n, select_zero,
                     bc, idx_out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_gather_rows(const float* in, const int64_t* idx, int64_t n_rows, int cols,
                              float* out, vc_stream_t stream) {
  if (!in || !idx || !out || n_rows < 0 || cols <= 0) return VC_ERR_ARG;
  if (n_rows == 0) return VC_OK;
  hipLaunchKernelGGL(k_gather_rows, dim3(vc_blocks(n_rows * cols, NT)), dim3(NT), 0,
                     (hipStream_t)stream, in, idx, n_rows, cols, out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_scatter_rows(const float* in, const int64_t* idx, int64_t n_rows, int cols,
                               float* out, vc_stream_t stream) {
  if (!in || !idx || !out || n_rows < 0 || cols <= 0) return VC_ERR_ARG;
  if (n_rows == 0) return VC_OK;
  hipLaunchKernelGGL(k_scatter_rows, dim3(vc_blocks(n_rows * cols, NT)), dim3(NT), 0,
                     (hipStream_t)stream, in, idx, n_rows, cols, out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_widest_axis(const float* xl, const float* xh, int64_t B, int n, int64_t* ax,
                              uint8_t* usable, vc_stream_t stream) {
  if (!xl || !xh || !ax || B < 0 || n <= 0) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_widest, dim3(vc_blocks(B, NT)), dim3(NT), 0, (hipStream_t)stream, xl,
                     xh, B, n, ax, usable);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_box_shrunk(const float* xl_old, const float* xh_old, const float* xl_new,
                             const float* xh_new, int64_t n, int32_t* flag,
                             vc_stream_t stream) {
  if (!flag || n < 0 || (n > 0 && (!xl_old || !xh_old || !xl_new || !xh_new)))
    return VC_ERR_ARG;
  hipLaunchKernelGGL(k_box_shrunk, dim3(1), dim3(1024), 0, (hipStream_t)stream, xl_old, xh_old,
                     xl_new, xh_new, n, flag);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_bisect(const float* xl, const float* xh, const int64_t* ax,
                         const int64_t* u_idx, int64_t n_u, int n, float* low_xl,
                         float* low_xh, float* high_xl, float* high_xh, vc_stream_t stream) {
  if (!xl || !xh || !ax || !u_idx || !low_xl || !low_xh || !high_xl || !high_xh || n_u < 0 ||
      n <= 0)
    return VC_ERR_ARG;
  if (n_u == 0) return VC_OK;
  hipLaunchKernelGGL(k_bisect, dim3(vc_blocks(n_u * n, NT)), dim3(NT), 0, (hipStream_t)stream,
                     xl, xh, ax, u_idx, n_u, n, low_xl, low_xh, high_xl, high_xh);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_zono_input(const float* xl, const float* xh, int64_t B, int n,
                             const int32_t* var_idx, int K, float* c, float* G,
                             vc_stream_t stream) {
  if (!xl || !xh || !c || B < 0 || n <= 0 || K < 0) return VC_ERR_ARG;
  if (K > 0 && (!var_idx || !G)) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  hipLaunchKernelGGL(k_zono_input, dim3(vc_blocks(B * (int64_t)n * (K > 0 ? K : 1), NT)),
                     dim3(NT), 0, (hipStream_t)stream, xl, xh, B, n, var_idx, K, c, G);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
