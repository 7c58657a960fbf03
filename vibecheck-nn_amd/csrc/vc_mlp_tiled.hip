// Whole-network CROWN kernel for narrow fc/ReLU chains with the tile shape
// fixed at compile time (vc_mlp_tiled_crown).
//
// Same computation and register layout as k_mlp_crown in vc_mlp_fused.hip
// (one wavefront per domain; activation rows held like the D operand of
// v_mfma_f32_16x16x4_f32, so a layer's output registers feed the next
// layer's B operand), restructured so that no MFMA sits under a runtime
// condition:
//   - every hidden fc layer uses the same MT M-tiles and KS K-steps (the
//     template parameters; narrower layers are zero-padded), so the MFMA
//     loops unroll completely;
//   - a hidden layer's A fragments are stored [K-step][lane][M-tile], one
//     16-byte LDS read per K-step;
//   - the fc bias rides in the MFMA: row d_l of fc_l's A operand holds the
//     bias (in the zero padding of the last M-tile), so the output row d_l
//     is sum_k bias_k e_k, read out once per layer instead of a VALU dot
//     (BROW; without a free padding row the dot runs on the VALU);
//   - per-row constants (neg(ew) . up_t, bias dots, the concretization)
//     accumulate in fp64: each fp32 product is rounded as torch rounds it,
//     the sum of those products is held to ~1e-16 relative.
//
// fc_0 (M = input width, plus the bias row) is processed one M-tile at a
// time and concretized on the fly.
#include "vc_common.h"
#include "vc_mlp_common.h"
#include "vc_relax.h"

namespace {

using vcm::FW;
using vcm::ks_count;
using vcm::MAXL;

// The work counter of a queue-driven launch, reset on its stream.
__global__ void k_queue_reset(int* q) {
  if (threadIdx.x == 0) *q = 0;
}

// k_queue_reset for the zonotope pass, which also clears the union of
// unstable sets (umask[n], nullable) and the overflow count (nullable) that
// it accumulates.
__global__ void k_zono_init(int* q, unsigned long long* umask, int n, unsigned long long* cnt,
                            unsigned long long* cnt2) {
  if (threadIdx.x == 0 && q) *q = 0;
  if (umask && threadIdx.x < n) umask[threadIdx.x] = 0ull;
  if (threadIdx.x == 0 && cnt) *cnt = 0ull;
  if (threadIdx.x == 0 && cnt2) *cnt2 = 0ull;
}

constexpr int TNW = 12;  // waves per workgroup, one domain each (3 per SIMD)
constexpr int TNP = 1;   // 16-row N-tiles chained together per wave
constexpr int TQMAX = 64;  // spec rows per call (taken 16 at a time)

// LDS slot of lane L's fragment value at K-step ks.  The backward reads
// (lane L, slot L) and the forward reads (lane (g, r) of M-tile mo reads
// slot 16 (r / 4) + 4 g + i of K-step 4 mo + r % 4) both touch 16 distinct
// bank groups per quarter-wave with this XOR swizzle (an involution).
__host__ __device__ __forceinline__ int swz(int L, int ks) {
  return L ^ (((L >> 4) << 2) | (ks & 3));
}

// Kernel instantiations: hidden M-tiles, K-steps, bias row in the A operand.
struct TVariant {
  int MT, KS, brow;
};
constexpr TVariant kVariants[] = {{1, 4, 1},  {2, 8, 1},  {3, 12, 1},
                                  {4, 14, 1}, {4, 16, 1}, {4, 16, 0}};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

struct TGeom {
  int n;               // relu layers (fc_0 .. fc_{n-1}; the last fc is folded into the spec)
  int d[MAXL + 2];     // d[0] = inputs, d[l+1] = width of relu l
  int variant, MT, KS, brow;
  int mt0;             // M-tiles of fc_0 (inputs plus the bias row)
  int offh;            // float offset of the hidden fragments (fc_1 ...)
  int nfloats;         // fragment floats
  int boff[MAXL + 1];  // offset of fc_l's bias in the concatenated biases
};

// Pick the first instantiation that holds every layer.  Returns a VC_ status.
int tiled_geom(const int32_t* dims, int n_relu, TGeom& G) {
  if (!dims || n_relu < 1 || n_relu > MAXL) return VC_ERR_UNSUPPORTED;
  G = TGeom{};
  G.n = n_relu;
  int bo = 0;
  for (int l = 0; l <= n_relu; ++l) {
    if (dims[l] <= 0) return VC_ERR_ARG;
    if (dims[l] > FW) return VC_ERR_UNSUPPORTED;
    G.d[l] = dims[l];
  }
  for (int l = 0; l < n_relu; ++l) {
    G.boff[l] = bo;
    bo += G.d[l + 1];
  }
  int ks_need = 0, mh = 0;
  for (int l = 1; l <= n_relu; ++l) ks_need = ks_count(G.d[l]) > ks_need ? ks_count(G.d[l]) : ks_need;
  for (int l = 1; l < n_relu; ++l) mh = G.d[l] > mh ? G.d[l] : mh;
  G.variant = -1;
  for (int v = 0; v < kNumVariants; ++v) {
    const TVariant& k = kVariants[v];
    if (k.KS >= ks_need && 16 * k.MT >= mh + k.brow) {
      G.variant = v;
      break;
    }
  }
  if (G.variant < 0) return VC_ERR_UNSUPPORTED;
  G.MT = kVariants[G.variant].MT;
  G.KS = kVariants[G.variant].KS;
  G.brow = kVariants[G.variant].brow;
  G.mt0 = (G.d[0] + G.brow + 15) / 16;
  G.offh = G.mt0 * G.KS * 64;
  G.nfloats = G.offh + (n_relu - 1) * G.KS * 64 * 4;
  return VC_OK;
}

// fc_l's backward A operand: A[m][k] = W[k][m] (W: d_out x d_in, m < d_in,
// k < d_out), A[d_in][k] = bias[k] when brow; zero elsewhere.
//   hidden (layout 1): [ks][slot][mt] float4, mt < 4
//   fc_0   (layout 0): [mt][ks][slot]
// with lane L's value of K-step ks at slot swz(L, ks).
__global__ void k_tpack(const float* W, const float* bias, int d_out, int d_in, int KS, int MTt,
                        int layout, int brow, float* frag) {
  const int total = MTt * KS * 64;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    int mt, ks, slot;
    if (layout == 1) {
      mt = e & 3;
      slot = (e >> 2) & 63;
      ks = e >> 8;
    } else {
      slot = e & 63;
      ks = (e >> 6) % KS;
      mt = (e >> 6) / KS;
    }
    const int lane = swz(slot, ks);
    const int t = ks >> 2, i = ks & 3, g = lane >> 4, r = lane & 15;
    const int m = 16 * mt + r, k = 16 * t + 4 * g + i;
    float v = 0.f;
    if (k < d_out) {
      if (m < d_in)
        v = W[k * d_in + m];
      else if (brow && m == d_in)
        v = bias ? bias[k] : 0.f;
    }
    frag[e] = v;
  }
}

struct TCrownArgs {
  const float* lo_in[MAXL];
  const float* hi_in[MAXL];
  float* lo_out[MAXL];
  float* hi_out[MAXL];
};

__device__ __forceinline__ double group_sum4_d(double v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// Relaxation at one relu of the first NP row tiles of F (values of that
// relu's neurons j = 16 t + 4 g + i at K-step 4 t + i):
//   e = pos(x) ls + neg(x) us = x * (x < 0 ? us : ls),  acc += neg(x) ut
// and, without the bias row, acc += e . bias.  sl: ls, us, ut [FW] each,
// zero beyond the layer width; bl: the next fc's bias, zero-padded to FW.
// SGN: the upper slopes carry a flag in their sign bit (alpha's unstable
// neurons); their magnitude is the slope.
template <int KS, int NP, bool BROW, bool SGN = false>
__device__ __forceinline__ void relax_rows(const float* sl, const float* bl, int g,
                                           v4f (&F)[TNP][4], double (&acc)[TNP]) {
  const auto step = [&](int t, int i, float ls, float us, float ut, float bj) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float x = F[p][t][i];
      const bool ng = x < 0.f;
      const float e = x * (ng ? us : ls);
      const float en = ng ? x : 0.f;
      acc[p] += (double)(en * ut);
      if (!BROW) acc[p] += (double)(e * bj);
      F[p][t][i] = e;
    }
  };
  if constexpr (SGN) {
    // one float per load (k_alpha_tiled keeps its third wavefront per SIMD)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int t = ks >> 2, i = ks & 3;
      const int j = 16 * t + 4 * g + i;
      step(t, i, sl[j], fabsf(sl[FW + j]), sl[2 * FW + j], BROW ? 0.f : bl[j]);
    }
  } else {
    // a lane's neurons 16 t + 4 g + i of a tile are consecutive: one
    // float4 per slope array and tile where the arrays are 16-byte aligned
    // (the padding beyond KS holds zeros), else one float each
    const bool al = ((reinterpret_cast<uintptr_t>(sl) | reinterpret_cast<uintptr_t>(bl)) & 15) == 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (4 * t >= KS) break;
      const int j0 = 16 * t + 4 * g;
      float ls[4], us[4], ut[4], bj[4];
      if (al) {
        const float4 l4 = *reinterpret_cast<const float4*>(sl + j0);
        const float4 u4 = *reinterpret_cast<const float4*>(sl + FW + j0);
        const float4 t4 = *reinterpret_cast<const float4*>(sl + 2 * FW + j0);
        const float4 b4 =
            BROW ? float4{0.f, 0.f, 0.f, 0.f} : *reinterpret_cast<const float4*>(bl + j0);
        ls[0] = l4.x; ls[1] = l4.y; ls[2] = l4.z; ls[3] = l4.w;
        us[0] = u4.x; us[1] = u4.y; us[2] = u4.z; us[3] = u4.w;
        ut[0] = t4.x; ut[1] = t4.y; ut[2] = t4.z; ut[3] = t4.w;
        bj[0] = b4.x; bj[1] = b4.y; bj[2] = b4.z; bj[3] = b4.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ls[i] = sl[j0 + i];
          us[i] = sl[FW + j0 + i];
          ut[i] = sl[2 * FW + j0 + i];
          bj[i] = BROW ? 0.f : bl[j0 + i];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * t + i < KS) step(t, i, ls[i], us[i], ut[i], bj[i]);
    }
  }
}

// Backward through hidden fc_l: F (rows at fc_l's output, relaxed) <- A F
// with A = [W_l^T; bias_l]; with the bias row, its output (row mb = d_l,
// held by lane group (mb % 16) / 4) is the bias dot and goes to acc.
// IDX: the bias row's entry (the same M-tile and component in every lane)
// picked by register indexing (s_set_gpr_idx), else by a scalar switch
// (k_alpha_tiled's instance, where the contiguous copy the indexing needs
// costs its third wavefront per SIMD).
template <int MT, int KS, int NP, bool BROW, bool IDX = true>
__device__ __forceinline__ void fc_hidden(const float4* fr, int lane, int g, int mb,
                                          v4f (&F)[TNP][4], double (&acc)[TNP]) {
  v4f o[TNP][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) o[p][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  // the MFMA block at raised wave priority: a wavefront ready to issue its
  // MFMAs wins the arbitration, and the other wavefronts' relaxation VALU
  // work fills the matrix unit's gaps (2% faster on the CROWN rows pass)
  __builtin_amdgcn_s_setprio(1);
  // each K-step's fragments requested one K-step ahead, so that the LDS
  // read overlaps the current K-step's MFMAs instead of preceding them
  float4 a4 = fr[swz(lane, 0)];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const float4 nx = ks + 1 < KS ? fr[(ks + 1) * 64 + swz(lane, ks + 1)] : a4;
    // keep the scheduler from sinking that read below the MFMAs
    __builtin_amdgcn_sched_barrier(0);
    const float a[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int p = 0; p < NP; ++p) o[p][mt] = mfma16x16x4(a[mt], F[p][ks >> 2][ks & 3], o[p][mt]);
    a4 = nx;
  }
  __builtin_amdgcn_s_setprio(0);
  if (BROW) {
    // the bias row's entry: (M-tile, component) is the same for every lane,
    // a scalar index (see IDX)
    const bool mine = g == ((mb & 15) >> 2);
    const int sel = __builtin_amdgcn_readfirstlane(((mb >> 4) << 2) | (mb & 3));
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float v = 0.f;
      if constexpr (IDX) {
        float flat[4 * MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) flat[4 * mt + i] = o[p][mt][i];
        v = sel < 4 * MT ? flat[sel < 4 * MT ? sel : 0] : 0.f;
      } else {
        switch (sel) {
#define VC_BROW_CASE(C)                                               \
  case C:                                                             \
    if ((C >> 2) < MT) v = o[p][(C >> 2) < MT ? (C >> 2) : 0][C & 3]; \
    break;
          VC_BROW_CASE(0) VC_BROW_CASE(1) VC_BROW_CASE(2) VC_BROW_CASE(3)
          VC_BROW_CASE(4) VC_BROW_CASE(5) VC_BROW_CASE(6) VC_BROW_CASE(7)
          VC_BROW_CASE(8) VC_BROW_CASE(9) VC_BROW_CASE(10) VC_BROW_CASE(11)
          VC_BROW_CASE(12) VC_BROW_CASE(13) VC_BROW_CASE(14) VC_BROW_CASE(15)
#undef VC_BROW_CASE
          default: break;
        }
      }
      if (mine) acc[p] += (double)v;
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) F[p][mt] = o[p][mt];
}

// Backward through fc_0 (A = [W_0^T; bias_0], stored per M-tile) and
// concretization: cz += pos(A) xl + neg(A) xh over the d0 inputs, the bias
// row to acc; optionally the input coefficients of live rows to A_rows
// (row-major, d0 per row; row = 16 p + r).
template <int KS, int NP, bool BROW>
__device__ __forceinline__ void fc0_concretize(const float* fr0, int mt0, int d0, int lane, int g,
                                               int r, const float* dxl, const float* dxh,
                                               const v4f (&F)[TNP][4], double (&acc)[TNP],
                                               double (&cz)[TNP], float* A_rows, int n_live) {
  for (int mt = 0; mt < mt0; ++mt) {
    v4f o[TNP];
#pragma unroll
    for (int p = 0; p < NP; ++p) o[p] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const float a = fr0[(mt * KS + ks) * 64 + swz(lane, ks)];
#pragma unroll
      for (int p = 0; p < NP; ++p) o[p] = mfma16x16x4(a, F[p][ks >> 2][ks & 3], o[p]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mt + 4 * g + i;
      const bool in = m < d0;
      const float xlv = in ? dxl[m] : 0.f, xhv = in ? dxh[m] : 0.f;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const float v = o[p][i];
        if (in) {
          cz[p] += (double)(fmaxf(v, 0.f) * xlv);
          cz[p] += (double)(fminf(v, 0.f) * xhv);
          const int row = 16 * p + r;
          if (A_rows && row < n_live) A_rows[(int64_t)row * d0 + m] = v;
        } else if (BROW && m == d0) {
          acc[p] += (double)v;
        }
      }
    }
  }
}

template <int MT, int KS, int NP, bool BROW>
__device__ __forceinline__ void chain_to_input(const TGeom& G, int Ltop, const float* fr0,
                                               const float4* frh, const float* ssl,
                                               const float* sbias, int lane, int g, int r,
                                               const float* dxl, const float* dxh,
                                               v4f (&F)[TNP][4], double (&acc)[TNP],
                                               double (&cz)[TNP], float* A_rows, int n_live) {
  // rows at relu Ltop's output: relax + fc_l for l = Ltop .. 1, then relu 0 + fc_0
  for (int l = Ltop; l >= 1; --l) {
    relax_rows<KS, NP, BROW>(ssl + l * 3 * FW, sbias + l * FW, g, F, acc);
    fc_hidden<MT, KS, NP, BROW>(frh + (l - 1) * KS * 64, lane, g, G.d[l], F, acc);
  }
  relax_rows<KS, NP, BROW>(ssl, sbias, g, F, acc);
  fc0_concretize<KS, NP, BROW>(fr0, G.mt0, G.d[0], lane, g, r, dxl, dxh, F, acc, cz, A_rows,
                               n_live);
}

__device__ __forceinline__ void make_slopes_lds(float* sl, const float* lo, const float* hi, int n,
                                                int lane) {
  for (int j = lane; j < FW; j += 64) {
    float ls = 0.f, us = 0.f, ut = 0.f;
    if (j < n) {
      const Relax s = relax(lo[j], hi[j]);
      ls = s.lo_s;
      us = s.up_s;
      ut = s.up_t;
    }
    sl[j] = ls;
    sl[FW + j] = us;
    sl[2 * FW + j] = ut;
  }
}

// One group of NP seeded row tiles of relu layer L (rows 16 nt0 .. of the
// 2m seeds: row q < m is +W_L[idx[q]], row m + q is -W_L[idx[q]]) through
// fc_L .. fc_0 and the concretization; lb of each row to slb.
template <int MT, int KS, int NP, bool BROW>
__device__ __forceinline__ void seeded_group(const TGeom& G, int L, int nt0, int m,
                                             const int* idx, const float* fr0,
                                             const float4* frh, const float* ssl,
                                             const float* sbias, float* slb, int lane, int g,
                                             int r, const float* dxl, const float* dxh) {
  const int R = 2 * m, d0 = G.d[0];
  v4f F[TNP][4];
  double acc[TNP], cz[TNP];
  // W_L[j][k] = A_L[k][j]: K-step 4 (j / 16) + j % 4, lane group (j % 16) / 4,
  // lane 4 g + i of it, component t for k = 16 t + 4 g + i
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = 16 * (nt0 + p) + r;
    const bool live = row < R;
    const int q = live ? (row < m ? row : row - m) : 0;
    const float sg = row < m ? 1.f : -1.f;
    const int j = live ? idx[q] : 0;
    const int ksj = 4 * (j >> 4) + (j & 3), gj = (j & 15) >> 2;
    acc[p] = (live && g == 0) ? (double)(sg * sbias[L * FW + j]) : 0.0;
    cz[p] = 0.0;
    if (L > 0) {
      const float4* fl = frh + (L - 1) * KS * 64 + ksj * 64;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 w = live ? fl[swz(16 * gj + 4 * g + i, ksj)] : float4{0.f, 0.f, 0.f, 0.f};
        F[p][0][i] = sg * w.x;
        F[p][1][i] = sg * w.y;
        F[p][2][i] = sg * w.z;
        F[p][3][i] = sg * w.w;
      }
    } else if (live) {
      // seeded at relu 0: the row is +-W_0[j] over the inputs
      for (int mt = 0; mt < G.mt0; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mi = 16 * mt + 4 * g + i;
          if (mi < d0) {
            const float v = sg * fr0[(mt * KS + ksj) * 64 + swz(16 * gj + 4 * g + i, ksj)];
            cz[p] += (double)(fmaxf(v, 0.f) * dxl[mi]);
            cz[p] += (double)(fminf(v, 0.f) * dxh[mi]);
          }
        }
    }
  }
  if (L > 0)
    chain_to_input<MT, KS, NP, BROW>(G, L - 1, fr0, frh, ssl, sbias, lane, g, r, dxl, dxh, F, acc,
                                     cz, nullptr, 0);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const double lbd = group_sum4_d(acc[p] + cz[p]);
    const int row = 16 * (nt0 + p) + r;
    if (g == 0 && row < R) slb[row] = (float)lbd;
  }
}

// One group of NP spec row tiles (rows q0 + 16 p + r of the Q shared rows)
// through relu n-1 .. relu 0; lb, acc and the input coefficients out.
template <int MT, int KS, int NP, bool BROW>
__device__ __forceinline__ void spec_group(const TGeom& G, int q0, int Q, const float* spec_rows,
                                           const float* spec_acc, const float* fr0,
                                           const float4* frh, const float* ssl,
                                           const float* sbias, int lane, int g, int r,
                                           const float* dxl, const float* dxh, int64_t dom,
                                           float* lb_out, float* A_out, float* acc_out) {
  const int n = G.n, d0 = G.d[0], dN = G.d[n];
  v4f F[TNP][4];
  double acc[TNP], cz[TNP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = q0 + 16 * p + r;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = 16 * t + 4 * g + i;
        F[p][t][i] = (row < Q && k < dN) ? spec_rows[row * dN + k] : 0.f;
      }
    acc[p] = (row < Q && g == 0) ? (double)spec_acc[row] : 0.0;
    cz[p] = 0.0;
  }
  float* A_rows = A_out ? A_out + (dom * Q + q0) * d0 : nullptr;
  chain_to_input<MT, KS, NP, BROW>(G, n - 1, fr0, frh, ssl, sbias, lane, g, r, dxl, dxh, F, acc,
                                   cz, A_rows, Q - q0);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const double a = group_sum4_d(acc[p]);
    const double lbd = a + group_sum4_d(cz[p]);
    const int row = q0 + 16 * p + r;
    if (g == 0 && row < Q) {
      lb_out[dom * Q + row] = (float)lbd;
      if (acc_out) acc_out[dom * Q + row] = (float)a;
    }
  }
}

template <int MT, int KS, bool BROW>
__global__ __launch_bounds__(TNW * 64) void k_crown_tiled(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, TCrownArgs ca,
    const int32_t* __restrict__ idx_all, const int32_t* __restrict__ idx_meta, int do_crown,
    int per_domain, int Q, const float* __restrict__ spec_rows,
    const float* __restrict__ spec_acc, float* __restrict__ lb_out, float* __restrict__ A_out,
    float* __restrict__ acc_out, unsigned long long* __restrict__ seed_rows, int* queue) {
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;  // [n][FW], zero-padded
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n, d0 = G.d[0];
  // seeded neuron lists: counts idx_meta[L], offsets idx_meta[n + L]
  int nmax = 0;
  for (int l = 1; l <= n; ++l) nmax += G.d[l];
  const int nidx = do_crown ? idx_meta[n + n - 1] + idx_meta[n - 1] : 0;
  int* sidx = reinterpret_cast<int*>(sbias + n * FW);
  float* ssl = sbias + n * FW + nmax + wv * (n * 3 * FW + 7 * FW + MAXL);  // [layer][3][FW]
  float* slb = ssl + n * 3 * FW;                                    // seeded-row bounds
  float* stl = slb + 2 * FW;                                        // current layer lo / hi
  float* sx = stl + 2 * FW;                                         // the box: xl, xh [FW]
  int* sseed = reinterpret_cast<int*>(sx + 2 * FW);                 // this domain's seeds
  int* sscnt = sseed + FW;  // seeded neurons per layer, this wave's domains
  if (lane < MAXL) sscnt[lane] = 0;
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  for (int k = threadIdx.x; k < nidx && k < nmax; k += blockDim.x) sidx[k] = idx_all[k];
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  const float* dxl = sx;
  const float* dxh = sx + FW;

  // the first domain of every wavefront by its index, the rest from the
  // work queue as wavefronts finish (domains differ in cost by their seed
  // counts), else a fixed stride
  const int64_t nwaves = (int64_t)gridDim.x * TNW;
  int64_t dom = (int64_t)blockIdx.x * TNW + wv;
  while (dom < B) {
    const int tnext = (queue && B > nwaves) ? vcm::queue_take(queue, lane) : 0;
    sx[lane] = lane < d0 ? xl[dom * d0 + lane] : 0.f;
    sx[FW + lane] = lane < d0 ? xh[dom * d0 + lane] : 0.f;
    // layer bounds are loaded one layer ahead (lane j holds neuron j)
    float nlo = lane < G.d[1] ? ca.lo_in[0][dom * G.d[1] + lane] : 0.f;
    float nhi = lane < G.d[1] ? ca.hi_in[0][dom * G.d[1] + lane] : 0.f;
    for (int L = 0; L < n; ++L) {
      const int dW = G.d[L + 1];
      stl[lane] = nlo;
      stl[FW + lane] = nhi;
      if (L + 1 < n) {
        const int dn = G.d[L + 2];
        nlo = lane < dn ? ca.lo_in[L + 1][dom * dn + lane] : 0.f;
        nhi = lane < dn ? ca.hi_in[L + 1][dom * dn + lane] : 0.f;
      }
      __threadfence_block();
      int m = do_crown ? min(idx_meta[L], dW) : 0;
      const int* idx = sidx + (do_crown ? idx_meta[n + L] : 0);
      if (per_domain && m > 0) {
        // Seed only the union neurons whose slopes depend on their bounds in
        // this domain: lo < 0 and hi > -1e-7.  An active neuron (lo >= 0)
        // has slopes 1, 1, 0 and a dead one with hi <= -1e-7 has 0, 0, 0
        // whatever the tightening does (lo only rises, hi only falls), so
        // the spec bound and every relaxation are unchanged; only the
        // reported bounds of those neurons stay the zonotope ones.
        const int j = lane < m ? idx[lane] : 0;
        const bool keep = lane < m && stl[j] < 0.f && stl[FW + j] > -1e-7f;
        const uint64_t bal = __ballot(keep);
        if (keep) sseed[__popcll(bal & ((1ull << lane) - 1ull))] = j;
        m = __popcll(bal);
        idx = sseed;
        __threadfence_block();
      }
      const int R = 2 * m;
      const int ntiles = (R + 15) / 16;
      if (lane == 0) sscnt[L] += m;
      for (int nt0 = 0; nt0 < ntiles; nt0 += TNP) {
        if (ntiles - nt0 >= TNP)
          seeded_group<MT, KS, TNP, BROW>(G, L, nt0, m, idx, fr0, frh, ssl, sbias, slb, lane, g,
                                          r, dxl, dxh);
        else
          seeded_group<MT, KS, 1, BROW>(G, L, nt0, m, idx, fr0, frh, ssl, sbias, slb, lane, g, r,
                                        dxl, dxh);
      }
      __threadfence_block();
      // intersect: lo = max(lo, lb+), hi = max(min(hi, -lb-), lo)
      for (int q = lane; q < m; q += 64) {
        const int j = idx[q];
        const float lc = fmaxf(stl[j], slb[q]);
        const float hc = fmaxf(fminf(stl[FW + j], -slb[m + q]), lc);
        stl[j] = lc;
        stl[FW + j] = hc;
      }
      __threadfence_block();
      if (ca.lo_out[L]) {
        for (int j = lane; j < dW; j += 64) {
          ca.lo_out[L][dom * dW + j] = stl[j];
          ca.hi_out[L][dom * dW + j] = stl[FW + j];
        }
      }
      make_slopes_lds(ssl + L * 3 * FW, stl, stl + FW, dW, lane);
      __threadfence_block();
    }
    for (int q0 = 0; q0 < Q; q0 += 16 * TNP) {
      // spec rows (shared, Q x d[n]) through relu n-1 ... relu 0
      if (Q - q0 > 16)
        spec_group<MT, KS, TNP, BROW>(G, q0, Q, spec_rows, spec_acc, fr0, frh, ssl, sbias, lane,
                                      g, r, dxl, dxh, dom, lb_out, A_out, acc_out);
      else
        spec_group<MT, KS, 1, BROW>(G, q0, Q, spec_rows, spec_acc, fr0, frh, ssl, sbias, lane, g,
                                    r, dxl, dxh, dom, lb_out, A_out, acc_out);
    }
    dom = (queue && B > nwaves) ? nwaves + vcm::queue_bcast(tnext) : dom + nwaves;
  }
  __threadfence_block();
  if (seed_rows && lane < n && sscnt[lane] > 0)
    atomicAdd(seed_rows + lane, (unsigned long long)sscnt[lane]);
}

// The same CROWN pass for small batches, where one wavefront per domain
// leaves most of the device idle and each domain's chain of tiles sets the
// time: a workgroup takes D domains with P = waves / D wavefronts each,
// the P wavefronts split every layer's seeded tiles (and the spec tiles),
// and the per-layer steps of each domain (seed filter, intersection,
// slopes) run between workgroup barriers.  Same arithmetic per row as
// k_crown_tiled.
template <int MT, int KS, bool BROW>
__global__ __launch_bounds__(TNW * 64) void k_crown_dom(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, TCrownArgs ca,
    const int32_t* __restrict__ idx_all, const int32_t* __restrict__ idx_meta, int do_crown,
    int per_domain, int Q, const float* __restrict__ spec_rows,
    const float* __restrict__ spec_acc, float* __restrict__ lb_out, float* __restrict__ A_out,
    float* __restrict__ acc_out, unsigned long long* __restrict__ seed_rows, int D) {
  extern __shared__ float smem[];
  __shared__ int s_m[TNW];
  __shared__ int s_cnt[MAXL];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;  // [n][FW], zero-padded
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n, d0 = G.d[0];
  const int P = nw / D, slot = wv / P, pw = wv - slot * P;
  int nmax = 0;
  for (int l = 1; l <= n; ++l) nmax += G.d[l];
  const int nidx = do_crown ? idx_meta[n + n - 1] + idx_meta[n - 1] : 0;
  int* sidx = reinterpret_cast<int*>(sbias + n * FW);
  // domain slot: slopes [n][3][FW], seeded-row bounds [2 FW], layer lo / hi
  // [2 FW], the box [2 FW], the seed list [FW]
  float* ssl = sbias + n * FW + nmax + slot * (n * 3 * FW + 7 * FW);
  float* slb = ssl + n * 3 * FW;
  float* stl = slb + 2 * FW;
  float* sx = stl + 2 * FW;
  int* sseed = reinterpret_cast<int*>(sx + 2 * FW);
  if (threadIdx.x < MAXL) s_cnt[threadIdx.x] = 0;
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  for (int k = threadIdx.x; k < nidx && k < nmax; k += blockDim.x) sidx[k] = idx_all[k];
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  const float* dxl = sx;
  const float* dxh = sx + FW;
  const bool lead = pw == 0;  // the wavefront doing the domain's per-layer steps

  for (int64_t base = (int64_t)blockIdx.x * D; base < B; base += (int64_t)gridDim.x * D) {
    const int64_t dom = base + slot;
    const bool has = slot < D && dom < B;
    if (lead && has) {
      sx[lane] = lane < d0 ? xl[dom * d0 + lane] : 0.f;
      sx[FW + lane] = lane < d0 ? xh[dom * d0 + lane] : 0.f;
    }
    for (int L = 0; L < n; ++L) {
      const int dW = G.d[L + 1];
      const int mu = do_crown ? min(idx_meta[L], dW) : 0;
      const int* uidx = sidx + (do_crown ? idx_meta[n + L] : 0);
      if (lead && has) {
        stl[lane] = lane < dW ? ca.lo_in[L][dom * dW + lane] : 0.f;
        stl[FW + lane] = lane < dW ? ca.hi_in[L][dom * dW + lane] : 0.f;
        __threadfence_block();
        int m = mu;
        if (per_domain && m > 0) {
          // the union neurons whose slopes depend on this domain's bounds
          // (lo < 0, hi > -1e-7); see k_crown_tiled
          const int j = lane < mu ? uidx[lane] : 0;
          const bool keep = lane < mu && stl[j] < 0.f && stl[FW + j] > -1e-7f;
          const uint64_t bal = __ballot(keep);
          if (keep) sseed[__popcll(bal & ((1ull << lane) - 1ull))] = j;
          m = __popcll(bal);
        }
        if (lane == 0) {
          s_m[slot] = m;
          atomicAdd(&s_cnt[L], m);  // LDS: the lead wavefronts of all slots
        }
      }
      __syncthreads();
      const int m = has ? s_m[slot] : 0;
      const int* idx = per_domain ? sseed : uidx;
      const int ntiles = (2 * m + 15) / 16;
      for (int nt = pw; nt < ntiles; nt += P)
        seeded_group<MT, KS, 1, BROW>(G, L, nt, m, idx, fr0, frh, ssl, sbias, slb, lane, g, r,
                                      dxl, dxh);
      __syncthreads();
      if (lead && has) {
        for (int q = lane; q < m; q += 64) {
          const int j = idx[q];
          const float lc = fmaxf(stl[j], slb[q]);
          const float hc = fmaxf(fminf(stl[FW + j], -slb[m + q]), lc);
          stl[j] = lc;
          stl[FW + j] = hc;
        }
        __threadfence_block();
        if (ca.lo_out[L]) {
          for (int j = lane; j < dW; j += 64) {
            ca.lo_out[L][dom * dW + j] = stl[j];
            ca.hi_out[L][dom * dW + j] = stl[FW + j];
          }
        }
        make_slopes_lds(ssl + L * 3 * FW, stl, stl + FW, dW, lane);
      }
      __syncthreads();
    }
    if (has)
      for (int t = pw; 16 * t < Q; t += P)
        spec_group<MT, KS, 1, BROW>(G, 16 * t, Q, spec_rows, spec_acc, fr0, frh, ssl, sbias,
                                    lane, g, r, dxl, dxh, dom, lb_out, A_out, acc_out);
    __syncthreads();
  }
  if (seed_rows && threadIdx.x < n && s_cnt[threadIdx.x] > 0)
    atomicAdd(seed_rows + threadIdx.x, (unsigned long long)s_cnt[threadIdx.x]);
}

// ------------------------------------------------------ alpha-CROWN kernel
// One Adam iteration of batched alpha-CROWN per domain (verify_zono_bnb.py:
// 5248-5287), tile shape fixed at compile time: the spec backward with
// lower slopes active + unstable * alpha, keeping the pre-relaxation rows
// P_l in LDS; fc_0 fused with the concretization and the first gradient
// step gE_0 = W_0 gA + b_0, gA = xl [A >= 0] + xh [A <= 0]; then the
// forward sweep dalpha_l = sum_rows gE_l pos(P_l) (unstable neurons),
// gP_l = gE_l (mpos ls + mneg up_s) + mneg up_t (torch's clamp subgradient),
// gE_{l+1} = W_{l+1} gP_l + b_{l+1}, and torch.optim.Adam on -sum lb with
// the clamp to [0, 1].  Forward products read the backward fragments with a
// lane permutation; with the bias row, the bias enters as a constant-1
// entry of the gradient at index d_{l+1}.
constexpr int ANW = 8;  // waves per workgroup at most (as many as the LDS holds)

struct TAlphaArgs {
  const float* lo[MAXL];
  const float* hi[MAXL];
  float* alpha[MAXL];
  float* m1[MAXL];
  float* m2[MAXL];
  float* grad[MAXL];  // nullable: d(sum lb)/d alpha of the iteration (0 off the unstable set)
};

// Set element j (runtime, < 16 MT) of a D-layout block to v in the lanes of
// its group (the others keep their value).
template <int MT>
__device__ __forceinline__ void set_elem(v4f (&X)[4], int j, int g, float v) {
  const int tb = j >> 4, gb = (j & 15) >> 2, ib = j & 3;
  if (g != gb) return;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) X[t][i] = (t == tb && i == ib) ? v : X[t][i];
}

// Forward product through hidden fc_l (l >= 1) of NX column tiles:
// out = W_l X over the neurons of relu l-1 (K-tiles t < MT), read from
// fc_l's backward fragments ([ks][lane][mt] float4: A[m][k] = W_l[k][m]):
// lane (g, r) of output M-tile mo at K-step (t, i) needs
// W_l[16 mo + r][16 t + 4 g + i], component t of the float4 at K-step
// 4 mo + r % 4, lane 16 (r / 4) + 4 g + i.  The M-tiles of all NX tiles are
// independent accumulators, interleaved.
template <int MT, int KS, int NX, int NT>
__device__ __forceinline__ void fc_forward(const float4* fr, int lane, int g, int r,
                                           const v4f (&X)[NT][4], int x0, v4f (&out)[NX][4],
                                           int kmax = 1 << 30) {
#pragma unroll
  for (int x = 0; x < NX; ++x)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) out[x][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  // the MFMA block at raised wave priority, as in fc_hidden
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a[MT][4];
#pragma unroll
    for (int mo = 0; mo < MT; ++mo) {
      const int ksf = 4 * mo + (r & 3);
      const float4 q = ksf < KS ? fr[ksf * 64 + swz(16 * (r >> 2) + 4 * g + i, ksf)]
                                : float4{0.f, 0.f, 0.f, 0.f};
      a[mo][0] = q.x;
      a[mo][1] = q.y;
      a[mo][2] = q.z;
      a[mo][3] = q.w;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      // K-step (t, i) contracts inputs 16 t + 4 g + i: past the last live
      // one (kmax, the bias row included) every product is zero
      if (t == MT - 1 && 16 * t + i >= kmax) continue;
#pragma unroll
      for (int mo = 0; mo < MT; ++mo)
#pragma unroll
        for (int x = 0; x < NX; ++x)
          out[x][mo] = mfma16x16x4(a[mo][t], X[x0 + x][t][i], out[x][mo]);
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// fc_l's forward product for a uniform hidden width d = 16 (MT - 1) + MR,
// 1 <= MR <= 3, with the bias row in the padding: output rows below
// 16 (MT - 1) by MFMA over the full input tiles t < MT - 1 only; the last
// MR inputs and the bias row (in lanes of group 0 of input tile MT - 1)
// as a rank-(MR + 1) VALU update of those rows; the last MR output rows as
// VALU dot products over every input, reduced across the four lane groups.
// That leaves out one output tile and the input tile's K-steps, which hold
// 2-3 live values of 16 (a 50-wide layer: 36 MFMAs per column tile instead
// of 60).  wk: W_l[o][16 (MT - 1) + kk] for o < 16 (MT - 1), kk <= MR (the
// bias column at kk == MR), 4 per row; wm: W_l[16 (MT - 1) + m][k] for
// m < MR, k < 64 (bias at k = d, zeros past it).
template <int MT, int KS, int NX, int NT, int MR>
__device__ __forceinline__ void fc_forward_rem(const float4* fr, const float* wk, const float* wm,
                                               int lane, int g, int r, const v4f (&X)[NT][4],
                                               int x0, v4f (&out)[NX][4]) {
  static_assert(MR >= 1 && MR <= 3 && MT >= 2, "remainder form");
  constexpr int MF = MT - 1;
#pragma unroll
  for (int x = 0; x < NX; ++x)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) out[x][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a[MF][4];
#pragma unroll
    for (int mo = 0; mo < MF; ++mo) {
      const int ksf = 4 * mo + (r & 3);
      const float4 q = fr[ksf * 64 + swz(16 * (r >> 2) + 4 * g + i, ksf)];
      a[mo][0] = q.x;
      a[mo][1] = q.y;
      a[mo][2] = q.z;
      a[mo][3] = q.w;
    }
#pragma unroll
    for (int t = 0; t < MF; ++t)
#pragma unroll
      for (int mo = 0; mo < MF; ++mo)
#pragma unroll
        for (int x = 0; x < NX; ++x)
          out[x][mo] = mfma16x16x4(a[mo][t], X[x0 + x][t][i], out[x][mo]);
  }
  __builtin_amdgcn_s_setprio(0);
  // the remainder inputs of each column, from its lane in group 0
  float zb[NX][MR + 1];
#pragma unroll
  for (int x = 0; x < NX; ++x)
#pragma unroll
    for (int kk = 0; kk <= MR; ++kk) zb[x][kk] = __shfl(X[x0 + x][MF][kk], r, 64);
#pragma unroll
  for (int mo = 0; mo < MF; ++mo)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 w = *reinterpret_cast<const float4*>(wk + 4 * (16 * mo + 4 * g + i));
      const float w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int x = 0; x < NX; ++x) {
        float acc = out[x][mo][i];
#pragma unroll
        for (int kk = 0; kk <= MR; ++kk) acc = __builtin_fmaf(w4[kk], zb[x][kk], acc);
        out[x][mo][i] = acc;
      }
    }
  // the last MR output rows
  float rem[NX][MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float s[NX];
#pragma unroll
    for (int x = 0; x < NX; ++x) s[x] = 0.f;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float4 w = *reinterpret_cast<const float4*>(wm + 64 * m + 16 * t + 4 * g);
      const float w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int x = 0; x < NX; ++x) s[x] = __builtin_fmaf(w4[i], X[x0 + x][t][i], s[x]);
    }
#pragma unroll
    for (int x = 0; x < NX; ++x) {
      s[x] += __shfl_xor(s[x], 16, 64);
      s[x] += __shfl_xor(s[x], 32, 64);
      rem[x][m] = s[x];
    }
  }
#pragma unroll
  for (int x = 0; x < NX; ++x)
#pragma unroll
    for (int i = 0; i < 4; ++i) out[x][MF][i] = (g == 0 && i < MR) ? rem[x][i < MR ? i : 0] : 0.f;
}

// Per-wave LDS of k_alpha_tiled: slopes [l][ls_eff, us, ut][FW] (us with
// the sign bit set on the unstable neurons: -0.0 for a zero slope), the
// pre-relaxation rows P_l [l][ks][g][r < Q], d lb / d alpha of one layer
// [FW], the box [2 FW].  alpha and its Adam state stay in global memory.
__host__ __device__ inline int alpha_wsz(int n, int KS, int Q) {
  return n * 3 * FW + n * KS * 4 * Q + 3 * FW;
}

struct AlphaLds {
  float *ssl, *sP, *sga, *sx;
};

__device__ __forceinline__ AlphaLds alpha_lds_at(float* w, int n, int KS, int Q) {
  AlphaLds a;
  a.ssl = w;
  a.sP = a.ssl + n * 3 * FW;
  a.sga = a.sP + n * KS * 4 * Q;
  a.sx = a.sga + FW;
  return a;
}

// The box and the slopes of domain dom into the wave's LDS: the relaxation
// of the starting bounds with the lower slope of the unstable neurons
// alpha (init: alpha = (up_s > 0.5) * unstable).
template <int KS>
__device__ __forceinline__ void alpha_load(const TGeom& G, const TAlphaArgs& aa,
                                           const float* xl, const float* xh, int64_t dom,
                                           int init, const AlphaLds& w, int lane) {
  const int n = G.n, d0 = G.d[0];
  w.sx[lane] = lane < d0 ? xl[dom * d0 + lane] : 0.f;
  w.sx[FW + lane] = lane < d0 ? xh[dom * d0 + lane] : 0.f;
#pragma unroll 4
  for (int l = 0; l < n; ++l) {
    const int dW = G.d[l + 1];
    float* sl = w.ssl + l * 3 * FW;
    for (int j = lane; j < FW; j += 64) {
      float ls = 0.f, us = 0.f, ut = 0.f;
      if (j < dW) {
        const int64_t ai = dom * dW + j;
        const Relax s = relax(aa.lo[l][ai], aa.hi[l][ai]);
        // first iteration: alpha = (up_s > 0.5) * unstable
        const float a =
            init ? ((s.unstable && s.up_s > 0.5f) ? 1.f : 0.f) : aa.alpha[l][ai];
        ls = s.active ? 1.f : (s.unstable ? a : 0.f);
        us = s.unstable ? -s.up_s : s.up_s;
        ut = s.up_t;
      }
      sl[j] = ls;
      sl[FW + j] = us;
      sl[2 * FW + j] = ut;
    }
  }
}

// One alpha-CROWN iteration of the wave's domain from its LDS slopes: the
// spec backward keeping P_l, fc_0 with the concretization, the forward
// gradient sweep and the Adam update of alpha (clamped to [0, 1]) on its
// global state, which it writes back for every neuron (init: from alpha =
// (up_s > 0.5) * unstable and a zero state).  Returns the lane's row bound
// (rows r < Q, lanes g == 0).
template <int MT, int KS, bool BROW>
__device__ __forceinline__ double alpha_pass(const TGeom& G, const AlphaLds& w, const float* fr0,
                                             const float4* frh, const float* sbias, int Q,
                                             const float* spec_rows, const float* spec_acc,
                                             const AdamConst& adam, int init, int lane, int g,
                                             int r, const TAlphaArgs& aa, int64_t dom) {
  const int n = G.n, d0 = G.d[0], dN = G.d[n];
  const bool live = r < Q;
  float* ssl = w.ssl;
  float* sP = w.sP;
  float* sga = w.sga;
  const float* dxl = w.sx;
  const float* dxh = w.sx + FW;
  // ---- spec backward with alpha, keeping P_l
  v4f F[TNP][4];
  double acc[TNP], cz[TNP];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = 16 * t + 4 * g + i;
      F[0][t][i] = (live && k < dN) ? spec_rows[r * dN + k] : 0.f;
    }
  acc[0] = (live && g == 0) ? (double)spec_acc[r] : 0.0;
  cz[0] = 0.0;
  for (int l = n - 1; l >= 0; --l) {
    if (live) {
      float* pl = sP + l * KS * 4 * Q;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) pl[(ks * 4 + g) * Q + r] = F[0][ks >> 2][ks & 3];
    }
    relax_rows<KS, 1, BROW, true>(ssl + l * 3 * FW, sbias + l * FW, g, F, acc);
    if (l > 0)
      fc_hidden<MT, KS, 1, BROW, false>(frh + (l - 1) * KS * 64, lane, g, G.d[l], F, acc);
  }
  // ---- fc_0, concretization and gE_0 = W_0 gA + b_0, one input tile at a time
  v4f GE[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) GE[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int mt = 0; mt < G.mt0; ++mt) {
    v4f o = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      o = mfma16x16x4(fr0[(mt * KS + ks) * 64 + swz(lane, ks)], F[0][ks >> 2][ks & 3], o);
    float gA[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mt + 4 * g + i;
      const float v = o[i];
      gA[i] = 0.f;
      if (m < d0) {
        const float xlv = dxl[m], xhv = dxh[m];
        cz[0] += (double)(fmaxf(v, 0.f) * xlv);
        cz[0] += (double)(fminf(v, 0.f) * xhv);
        float gv = 0.f;
        if (v >= 0.f) gv += xlv;
        if (v <= 0.f) gv += xhv;
        gA[i] = live ? gv : 0.f;
      } else if (BROW && m == d0) {
        acc[0] += (double)v;
        gA[i] = live ? 1.f : 0.f;
      }
    }
    // A_fwd0[m'][k'] = A_0[k'][m']: lane (g, r), M-tile mo, K-step (mt, i)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int mo = 0; mo < MT; ++mo) {
        const int ksf = 4 * mo + (r & 3);
        const float a =
            ksf < KS ? fr0[(mt * KS + ksf) * 64 + swz(16 * (r >> 2) + 4 * g + i, ksf)] : 0.f;
        GE[mo] = mfma16x16x4(a, gA[i], GE[mo]);
      }
  }
  const double lbd = group_sum4_d(acc[0] + cz[0]);
  // ---- forward gradient sweep with the Adam update per layer; each
  // layer's alpha and Adam state are requested one layer ahead
  float ca = 0.f, cm = 0.f, cv = 0.f;
  if (!init && lane < G.d[1]) {
    const int64_t ai = dom * G.d[1] + lane;
    ca = aa.alpha[0][ai];
    cm = aa.m1[0][ai];
    cv = aa.m2[0][ai];
  }
  for (int l = 0; l < n; ++l) {
    const int dW = G.d[l + 1];
    float* sl = ssl + l * 3 * FW;
    float na = 0.f, nm = 0.f, nv = 0.f;
    if (!init && l + 1 < n && lane < G.d[l + 2]) {
      const int64_t ai = dom * G.d[l + 2] + lane;
      na = aa.alpha[l + 1][ai];
      nm = aa.m1[l + 1][ai];
      nv = aa.m2[l + 1][ai];
    }
    if (!BROW) {
      // bias of fc_l (l >= 0) added for live rows: gE_l += b_l
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          GE[t][i] = live ? GE[t][i] + sbias[l * FW + 16 * t + 4 * g + i] : 0.f;
    }
    const float* pl = sP + l * KS * 4 * Q;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int t = ks >> 2, i = ks & 3;
      const int j = 16 * t + 4 * g + i;
      const float pv = live ? pl[(ks * 4 + g) * Q + r] : 0.f;
      const float ge = GE[t][i];
      const float s = row_sum16(ge * fmaxf(pv, 0.f));
      if (r == 0) sga[j] = s;
      const bool mp = pv >= 0.f, mn = pv <= 0.f;
      float gp = ge * ((mp ? sl[j] : 0.f) + (mn ? fabsf(sl[FW + j]) : 0.f));
      if (mn) gp = gp + sl[2 * FW + j];
      GE[t][i] = live ? gp : 0.f;
    }
    __threadfence_block();
    {
      const int j = lane;
      if (j < dW) {
        const float usg = sl[FW + j];
        const bool un = signbit(usg);
        float a = init ? ((un && fabsf(usg) > 0.5f) ? 1.f : 0.f) : ca;
        float mi = cm, vi = cv;
        if (un) {
          const float pa = adam_update(a, -sga[j], mi, vi, adam);
          a = fminf(fmaxf(pa, 0.f), 1.f);
        }
        const int64_t ai = dom * dW + j;
        aa.alpha[l][ai] = a;
        aa.m1[l][ai] = mi;
        aa.m2[l][ai] = vi;
        if (aa.grad[l]) aa.grad[l][ai] = un ? sga[j] : 0.f;
      }
      ca = na;
      cm = nm;
      cv = nv;
    }
    __threadfence_block();
    if (l + 1 < n) {
      // the rows at relu l's output (K of fc_{l+1}); with the bias row, a
      // constant 1 at index d_{l+1} picks up b_{l+1}
      if (BROW) set_elem<MT>(GE, dW, g, live ? 1.f : 0.f);
      v4f xin[1][4], nx[1][4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) xin[0][mt] = GE[mt];
      fc_forward<MT, KS, 1, 1>(frh + l * KS * 64, lane, g, r, xin, 0, nx);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) GE[mt] = nx[0][mt];
    }
  }
  return lbd;
}

template <int MT, int KS, bool BROW>
__global__ __launch_bounds__(ANW * 64) void k_alpha_tiled(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, TAlphaArgs aa, int Q,
    const float* __restrict__ spec_rows, const float* __restrict__ spec_acc,
    float* __restrict__ lb_out, AdamConst adam, int init, const float* __restrict__ ctl) {
  if (ctl && ctl[1] != 0.f) return;  // the loop has stopped (vc_alpha_control)
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;  // [n][FW], zero-padded
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n;
  const AlphaLds w = alpha_lds_at(sbias + n * FW + wv * alpha_wsz(n, KS, Q), n, KS, Q);
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  const int nwv = blockDim.x >> 6;
  for (int64_t dom = (int64_t)blockIdx.x * nwv + wv; dom < B; dom += (int64_t)gridDim.x * nwv) {
    alpha_load<KS>(G, aa, xl, xh, dom, init, w, lane);
    __threadfence_block();
    const double lbd = alpha_pass<MT, KS, BROW>(G, w, fr0, frh, sbias, Q, spec_rows, spec_acc,
                                                adam, init, lane, g, r, aa, dom);
    if (g == 0 && r < Q) lb_out[dom * Q + r] = (float)lbd;
    __threadfence_block();
  }
}

// ------------------------------------------- alpha-CROWN, small batches
// The iteration of k_alpha_tiled with every domain's work spread over MT
// wavefronts (a "quad" for MT = 4): wavefront w owns the neurons of M-tile
// w of every layer (16 w .. 16 w + 15).  It keeps their pre-relaxation
// rows, relaxes them, runs only its output M-tile of each fc product (1 /
// MT of the MFMAs), and does the gradient sweep and Adam update of its
// neurons.  The relaxed rows (backward) and the gradient rows (forward)
// are exchanged through LDS once per layer, double-buffered with one
// workgroup barrier each.  A workgroup holds D domains.
constexpr int AQD = 4;  // domains per workgroup at most

__host__ __device__ inline int alpha_quad_floats(int n, int KS, int Q, int MT) {
  // slopes [n][4][FW], Adam state [n][3][FW], P_l [n][KS][4][Q], d lb / d
  // alpha [n][FW], box [2 FW], exchange [2][MT][4][Q][4], row sums
  // [MT + 1][16] doubles
  const int f = n * 8 * FW + n * KS * 4 * Q + 2 * FW + 2 * MT * 16 * Q + 2 * (MT + 1) * 16;
  return (f + 3) & ~3;
}

template <int MT>
__device__ __forceinline__ void quad_exchange(float* xbuf, int w, int g, int r, bool live, int Q,
                                              const v4f& mine, v4f (&all)[4]) {
  if (live)
    *reinterpret_cast<float4*>(xbuf + ((w * 4 + g) * Q + r) * 4) =
        make_float4(mine[0], mine[1], mine[2], mine[3]);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (t < MT && live) {
      const float4 v = *reinterpret_cast<const float4*>(xbuf + ((t * 4 + g) * Q + r) * 4);
      all[t] = v4f{v.x, v.y, v.z, v.w};
    } else {
      all[t] = v4f{0.f, 0.f, 0.f, 0.f};
    }
  }
}

// NL > 0: a net of exactly NL relu layers, every layer loop unrolled (the
// layer widths then come from fixed kernel-argument offsets, read once,
// instead of a scalar load inside each layer's MFMA chain), at most two
// domains per workgroup.
template <int MT, int KS, bool BROW, int NL = 0>
__global__ __launch_bounds__(NL > 0 ? 2 * MT * 64 : AQD * 4 * 64) void k_alpha_quad(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, TAlphaArgs aa, int Q,
    const float* __restrict__ spec_rows, const float* __restrict__ spec_acc,
    float* __restrict__ lb_out, AdamChunk ac, int init, const float* __restrict__ ctl, int D) {
  if (ctl && ctl[1] != 0.f) return;  // the loop has stopped (vc_alpha_control)
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;  // [n][FW], zero-padded
  // the wave index as a scalar: the per-wave tile choices below are then
  // uniform branches, and the loads of an unrolled loop can be issued
  // together instead of one masked block at a time
  const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qd = wid / MT, w = wid - qd * MT;  // domain slot, owned M-tile
  const int g = lane >> 4, r = lane & 15;
  const int n = NL > 0 ? NL : G.n, d0 = G.d[0], dN = G.d[n];
  const bool live = r < Q;
  float* ssl = sbias + n * FW + qd * alpha_quad_floats(n, KS, Q, MT);  // [l][ls, us, ut, un][FW]
  float* sad = ssl + n * 4 * FW;                                        // [l][alpha, m, v][FW]
  float* sP = sad + n * 3 * FW;                                         // [l][ks][g][r < Q]
  float* sga = sP + n * KS * 4 * Q;                                     // [n][FW]
  float* sx = sga + n * FW;                                             // xl, xh [FW]
  float* xch = sx + 2 * FW;                                             // [2][MT][4][Q][4]
  double* sacc = reinterpret_cast<double*>(xch + 2 * MT * 16 * Q);      // [MT + 1][16]
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  const float* dxl = sx;
  const float* dxh = sx + FW;

  for (int64_t b0 = (int64_t)blockIdx.x * D; b0 < B; b0 += (int64_t)gridDim.x * D) {
    const int64_t dom = b0 + qd;
    const bool has = dom < B;
    // ---- the box and the state of the owned neurons
    if (has) {
      if (w == 0) {
        sx[lane] = lane < d0 ? xl[dom * d0 + lane] : 0.f;
        sx[FW + lane] = lane < d0 ? xh[dom * d0 + lane] : 0.f;
      }
      for (int k = lane; k < n * 16; k += 64) {
        const int l = k >> 4, j = 16 * w + (k & 15);
        const int dW = G.d[l + 1];
        float ls = 0.f, us = 0.f, ut = 0.f, un = 0.f, a = 0.f, m1 = 0.f, m2 = 0.f;
        if (j < dW) {
          const int64_t ai = dom * dW + j;
          const Relax s = relax(aa.lo[l][ai], aa.hi[l][ai]);
          if (init) {
            a = (s.unstable && s.up_s > 0.5f) ? 1.f : 0.f;
          } else {
            a = aa.alpha[l][ai];
            m1 = aa.m1[l][ai];
            m2 = aa.m2[l][ai];
          }
          ls = s.active ? 1.f : (s.unstable ? a : 0.f);
          us = s.up_s;
          ut = s.up_t;
          un = s.unstable ? 1.f : 0.f;
        }
        float* sl = ssl + l * 4 * FW;
        float* sa = sad + l * 3 * FW;
        sl[j] = ls;
        sl[FW + j] = us;
        sl[2 * FW + j] = ut;
        sl[3 * FW + j] = un;
        sa[j] = a;
        sa[FW + j] = m1;
        sa[2 * FW + j] = m2;
      }
    }
    __syncthreads();
    // ac.n iterations back to back on the state in LDS; iteration t's
    // bounds go to lb_out + t B Q
    for (int t_it = 0; t_it < ac.n; ++t_it) {
    const AdamConst& adam = ac.c[t_it];
    // ---- spec backward with alpha: the owned slice of the rows
    v4f Fw;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = 16 * w + 4 * g + i;
      Fw[i] = (has && live && k < dN) ? spec_rows[r * dN + k] : 0.f;
    }
    double acc = (has && live && g == 0 && w == 0) ? (double)spec_acc[r] : 0.0;
    double cz = 0.0;
    v4f GEw = v4f{0.f, 0.f, 0.f, 0.f};
    int xb = 0;
#pragma unroll
    for (int l = n - 1; l >= 0; --l) {
      const float* sl = ssl + l * 4 * FW;
      float* pl = sP + l * KS * 4 * Q;
      // the owned neurons' slopes (and bias) first, one float4 each (the
      // padding neurons hold zeros), then the rows and their relaxation
      const int j0 = 16 * w + 4 * g;
      const float4 ls4 = *reinterpret_cast<const float4*>(sl + j0);
      const float4 us4 = *reinterpret_cast<const float4*>(sl + FW + j0);
      const float4 ut4 = *reinterpret_cast<const float4*>(sl + 2 * FW + j0);
      const float4 bb4 = BROW ? float4{0.f, 0.f, 0.f, 0.f}
                              : *reinterpret_cast<const float4*>(sbias + l * FW + j0);
      const float lsa[4] = {ls4.x, ls4.y, ls4.z, ls4.w};
      const float usa[4] = {us4.x, us4.y, us4.z, us4.w};
      const float uta[4] = {ut4.x, ut4.y, ut4.z, ut4.w};
      const float bba[4] = {bb4.x, bb4.y, bb4.z, bb4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * w + i < KS && has && live) pl[((4 * w + i) * 4 + g) * Q + r] = Fw[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (4 * w + i < KS) {
          const float x = Fw[i];
          const bool ng = x < 0.f;
          const float e = x * (ng ? usa[i] : lsa[i]);
          const float en = ng ? x : 0.f;
          acc += (double)(en * uta[i]);
          if (!BROW) acc += (double)(e * bba[i]);
          Fw[i] = e;
        }
      }
      v4f F[4];
      quad_exchange<MT>(xch + xb * MT * 16 * Q, w, g, r, has && live, Q, Fw, F);
      xb ^= 1;
      if (l > 0) {
        // fc_l backward, the owned output M-tile
        v4f o = v4f{0.f, 0.f, 0.f, 0.f};
        const float* fa = reinterpret_cast<const float*>(frh + (l - 1) * KS * 64);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          o = mfma16x16x4(fa[(ks * 64 + swz(lane, ks)) * 4 + w], F[ks >> 2][ks & 3], o);
        if (BROW) {
          const int mb = G.d[l];
          if ((mb >> 4) == w && g == ((mb & 15) >> 2)) acc += (double)o[mb & 3];
        }
        Fw = o;
      } else {
        // fc_0 and the concretization (every wavefront, identical), gA,
        // and the owned slice of gE_0 = W_0 gA + b_0
        for (int mt = 0; mt < G.mt0; ++mt) {
          v4f o = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            o = mfma16x16x4(fr0[(mt * KS + ks) * 64 + swz(lane, ks)], F[ks >> 2][ks & 3], o);
          float gA[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 16 * mt + 4 * g + i;
            const float v = o[i];
            gA[i] = 0.f;
            if (m < d0) {
              const float xlv = dxl[m], xhv = dxh[m];
              cz += (double)(fmaxf(v, 0.f) * xlv);
              cz += (double)(fminf(v, 0.f) * xhv);
              float gv = 0.f;
              if (v >= 0.f) gv += xlv;
              if (v <= 0.f) gv += xhv;
              gA[i] = live ? gv : 0.f;
            } else if (BROW && m == d0) {
              if (w == 0) acc += (double)v;
              gA[i] = live ? 1.f : 0.f;
            }
          }
          const int ksf = 4 * w + (r & 3);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float a =
                ksf < KS ? fr0[(mt * KS + ksf) * 64 + swz(16 * (r >> 2) + 4 * g + i, ksf)] : 0.f;
            GEw = mfma16x16x4(a, gA[i], GEw);
          }
        }
      }
    }
    // ---- lb: the wavefronts' row constants and the concretization, summed
    // in a fixed order
    {
      const double a = group_sum4_d(acc);
      const double c = group_sum4_d(cz);
      if (g == 0) {
        sacc[w * 16 + r] = a;
        if (w == 0) sacc[MT * 16 + r] = c;
      }
    }
    __syncthreads();
    if (has && w == 0 && g == 0 && live) {
      double t = 0.0;
#pragma unroll
      for (int u = 0; u < MT; ++u) t += sacc[u * 16 + r];
      lb_out[(int64_t)t_it * B * Q + dom * Q + r] = (float)(t + sacc[MT * 16 + r]);
    }
    // ---- forward gradient sweep, owned neurons; the Adam update of every
    // layer follows it (it changes only the next iteration's slopes)
#pragma unroll
    for (int l = 0; l < n; ++l) {
      const int dW = G.d[l + 1];
      float* sl = ssl + l * 4 * FW;
      if (!BROW) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          GEw[i] = live ? GEw[i] + sbias[l * FW + 16 * w + 4 * g + i] : 0.f;
      }
      const float* pl = sP + l * KS * 4 * Q;
      // every load of the step first: the rows (a lane past the Q live
      // rows reads row 0 and discards it) and the slopes, one float4 each
      const int j0 = 16 * w + 4 * g;
      const int rq = live ? r : 0;
      float pva[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ks = 4 * w + i;
        pva[i] = ks < KS ? pl[(ks * 4 + g) * Q + rq] : 0.f;
      }
      const float4 ls4 = *reinterpret_cast<const float4*>(sl + j0);
      const float4 us4 = *reinterpret_cast<const float4*>(sl + FW + j0);
      const float4 ut4 = *reinterpret_cast<const float4*>(sl + 2 * FW + j0);
      const float lsa[4] = {ls4.x, ls4.y, ls4.z, ls4.w};
      const float usa[4] = {us4.x, us4.y, us4.z, us4.w};
      const float uta[4] = {ut4.x, ut4.y, ut4.z, ut4.w};
      float sums[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = (has && live) ? pva[i] : 0.f;
        sums[i] = row_sum16(GEw[i] * fmaxf(pv, 0.f));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ks = 4 * w + i;
        if (ks < KS) {
          const float pv = (has && live) ? pva[i] : 0.f;
          const float ge = GEw[i];
          if (r == 0) sga[l * FW + j0 + i] = sums[i];
          const bool mp = pv >= 0.f, mn = pv <= 0.f;
          float gp = ge * ((mp ? lsa[i] : 0.f) + (mn ? usa[i] : 0.f));
          if (mn) gp = gp + uta[i];
          GEw[i] = live ? gp : 0.f;
        }
      }
      if (l + 1 < n) {
        // with the bias row, a constant 1 at index d_{l+1} picks up b_{l+1}
        if (BROW && (dW >> 4) == w && g == ((dW & 15) >> 2)) GEw[dW & 3] = live ? 1.f : 0.f;
        v4f X[4];
        quad_exchange<MT>(xch + xb * MT * 16 * Q, w, g, r, has && live, Q, GEw, X);
        xb ^= 1;
        // fc_{l+1} forward, the owned output M-tile (fragments read
        // transposed: K-step 4 w + r % 4, slot 16 (r / 4) + 4 g + i)
        const float4* fr = frh + l * KS * 64;
        const int ksf = 4 * w + (r & 3);
        v4f o = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 q4 = ksf < KS ? fr[ksf * 64 + swz(16 * (r >> 2) + 4 * g + i, ksf)]
                                     : float4{0.f, 0.f, 0.f, 0.f};
          const float a[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            // inputs 16 t + 4 g + i past the last live one (bias row
            // included) contribute zeros
            if (t == MT - 1 && 16 * t + i >= dW + (BROW ? 1 : 0)) continue;
            o = mfma16x16x4(a[t], X[t][i], o);
          }
        }
        GEw = o;
      }
    }
    // ---- Adam on the owned neurons of every layer, all lanes
    __threadfence_block();
    if (has) {
      if constexpr (NL > 0) {
        // lane k of pass p takes neuron slot 64 p + k (layer slot / 16);
        // every pass's loads are issued before any update (each slot is
        // its own); padding neurons carry no unstable flag
        constexpr int NP = (NL * 16 + 63) / 64;
        float gsv[NP], unv[NP], av[NP], mv[NP], vv[NP];
#pragma unroll
        for (int p2 = 0; p2 < NP; ++p2) {
          const int k = lane + 64 * p2;
          const bool ok = k < NL * 16;
          const int kk = ok ? k : 0;
          const int l = kk >> 4, j = 16 * w + (kk & 15);
          const float* sa = sad + l * 3 * FW;
          gsv[p2] = sga[l * FW + j];
          unv[p2] = ok ? ssl[l * 4 * FW + 3 * FW + j] : 0.f;
          av[p2] = sa[j];
          mv[p2] = sa[FW + j];
          vv[p2] = sa[2 * FW + j];
        }
#pragma unroll
        for (int p2 = 0; p2 < NP; ++p2) {
          const int k = lane + 64 * p2;
          if (k >= NL * 16) continue;
          const int l = k >> 4, j = 16 * w + (k & 15);
          const float gs = gsv[p2];
          const bool un = unv[p2] != 0.f;
          if (un) {
            float* sa = sad + l * 3 * FW;
            float mi = mv[p2], vi = vv[p2];
            float pa = adam_update(av[p2], -gs, mi, vi, adam);
            pa = fminf(fmaxf(pa, 0.f), 1.f);
            sa[FW + j] = mi;
            sa[2 * FW + j] = vi;
            sa[j] = pa;
            ssl[l * 4 * FW + j] = pa;  // unstable: the next iteration's lower slope is alpha
          }
          // the last iteration of the launch leaves its gradient
          if (aa.grad[l] && t_it == ac.n - 1) {
            const int dW = G.d[l + 1];
            if (j < dW) aa.grad[l][dom * dW + j] = un ? gs : 0.f;
          }
        }
      } else {
        for (int k = lane; k < n * 16; k += 64) {
          const int l = k >> 4, j = 16 * w + (k & 15);
          const int dW = G.d[l + 1];
          float* sl = ssl + l * 4 * FW;
          float* sa = sad + l * 3 * FW;
          const float gs = sga[l * FW + j];
          const bool un = j < dW && sl[3 * FW + j] != 0.f;
          if (un) {
            float mi = sa[FW + j], vi = sa[2 * FW + j];
            float pa = adam_update(sa[j], -gs, mi, vi, adam);
            pa = fminf(fmaxf(pa, 0.f), 1.f);
            sa[FW + j] = mi;
            sa[2 * FW + j] = vi;
            sa[j] = pa;
            sl[j] = pa;  // unstable: the next iteration's lower slope is alpha
          }
          // the last iteration of the launch leaves its gradient
          if (aa.grad[l] && j < dW && t_it == ac.n - 1) aa.grad[l][dom * dW + j] = un ? gs : 0.f;
        }
      }
    }
    __threadfence_block();
    }  // iterations
    // ---- the owned neurons' Adam state back (the wave's own LDS writes)
    __threadfence_block();
    if (has) {
      for (int k = lane; k < n * 16; k += 64) {
        const int l = k >> 4, j = 16 * w + (k & 15);
        const int dW = G.d[l + 1];
        if (j < dW) {
          const float* sa = sad + l * 3 * FW;
          const int64_t ai = dom * dW + j;
          aa.alpha[l][ai] = sa[j];
          aa.m1[l][ai] = sa[FW + j];
          aa.m2[l][ai] = sa[2 * FW + j];
        }
      }
    }
    __syncthreads();  // the slot's LDS is rewritten by the next domain
  }
}

// The quad kernel for n relu layers and D domains per workgroup: the
// unrolled instance for the 50-wide variant at the depth of ACAS-Xu's nets
// (6 relu layers), else the general one.
constexpr int kQuadUnrolledV = 3, kQuadUnrolledN = 6;

template <int V>
const void* alpha_quad_fn(int n, int D) {
  constexpr int MT = kVariants[V].MT, KS = kVariants[V].KS;
  constexpr bool BR = kVariants[V].brow != 0;
  if constexpr (V == kQuadUnrolledV) {
    if (n == kQuadUnrolledN && D <= 2)
      return reinterpret_cast<const void*>(&k_alpha_quad<MT, KS, BR, kQuadUnrolledN>);
  }
  return reinterpret_cast<const void*>(&k_alpha_quad<MT, KS, BR>);
}

template <int V>
const void* alpha_fn() {
  return reinterpret_cast<const void*>(
      &k_alpha_tiled<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>);
}

// --------------------------------------------------------- zonotope kernel
// Zonotope pre-activation bounds (verify_zono_bnb.py:3079-3211), one
// wavefront per domain, tile shape fixed at compile time.  The generator
// matrix lives in registers as ZT column tiles in the D layout (rows =
// neurons, column 0 = centre, then the input generators, then one column
// per unstable neuron appended at each relu).  fc products read the tiled
// backward fragments in the forward direction; the bias enters through a
// constant 1 in the centre column at the bias row.
constexpr int ZNW = 8;  // waves per workgroup (fewer when the LDS scratch does not fit)
constexpr int ZT = 8;   // column tiles per wave: 128 columns, centre included
// The |G| partials' rows are ZPS floats apart: lane (g, r) writes row r at
// column 16 t + 4 g, so a row stride of FW would put the 16 rows of a
// quarter-wave on the same four banks; FW + 4 spreads them over all 64.
constexpr int ZPS = FW + 4;
constexpr int ZSCR = 16 * ZPS + 4 * FW;  // relu scratch floats per wave

struct TZonoArgs {
  float* lo[MAXL];
  float* hi[MAXL];
};

// Optional outputs of the zonotope passes for the CROWN passes (the rows
// pass's k_rows_mask, the union of vc_unstable_union_layers, over the same
// bounds): per layer and domain the seed filter lo < 0, hi > -1e-7 as a
// mask ([n][B], masks), and the union of the unstable sets (lo < 0 < hi)
// ORed into umask[n], which the one-wavefront pass's launch clears.
// With ovf_list, the one-wavefront pass also appends every domain it
// leaves to the wide pass to ovf_list (in no particular order: the wide pass
// takes each domain on its own) and counts them in *ovf_count, which the
// caller clears; the wide pass then needs no compaction of the flags.
// clear_count (nullable): a counter of the caller's that the pass's init
// launch also clears (the round's list of open leaves).
struct ZonoMasks {
  uint64_t* masks;
  unsigned long long* umask;
  int64_t* ovf_list;
  unsigned long long* ovf_count;
  unsigned long long* clear_count;
};

// fc_0 on the input block for NP column tiles, tile p starting at column
// base + p * step: column 0 = centre (and the constant 1 of the bias row),
// column 1 + k = radius k.
template <int MT, int KS, int NP, bool BROW>
__device__ __forceinline__ void zono_input_tiles(const TGeom& G, const float* fr0,
                                                 const float* dxl, const float* dxh, int g,
                                                 int r, int base, int step, v4f (&o)[NP][4]) {
  const int d0 = G.d[0];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[p][mt] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int mt = 0; mt < G.mt0; ++mt) {
    float in[NP][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = 16 * mt + 4 * g + i;
      float c = 0.f, rd = 0.f;
      if (k < d0) {
        const float lv = dxl[k], hv = dxh[k];
        c = (lv + hv) / 2.f;
        rd = (hv - lv) / 2.f;
      } else if (BROW && k == d0) {
        c = 1.f;
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const int col = base + p * step + r;
        in[p][i] = col == 0 ? c : (col == 1 + k && k < d0 ? rd : 0.f);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int mo = 0; mo < MT; ++mo) {
        const int ksf = 4 * mo + (r & 3);
        const float a =
            ksf < KS ? fr0[(mt * KS + ksf) * 64 + swz(16 * (r >> 2) + 4 * g + i, ksf)] : 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) o[p][mo] = mfma16x16x4(a, in[p][i], o[p][mo]);
      }
  }
}

// LDS floats of the remainder form's weight tables (fc_forward_rem) for
// n relu layers: wk [n - 1][48][4] and wm [n - 1][MR][64].
__host__ __device__ constexpr int zono_rem_floats(int n, int MT, int MR) {
  return MR > 0 ? (n - 1) * (16 * (MT - 1) * 4 + MR * 64) : 0;
}

// W_l[o][k] (l >= 1; k = d_l is the bias) from fc_l's tiled backward
// fragments: A[m][k'] = W[k'][m] sits at K-step 4 (k' / 16) + k' % 4, lane
// 16 ((k' % 16) / 4) + m % 16, component m / 16.
template <int KS>
__device__ __forceinline__ float frag_weight(const float* frh_l, int o, int k) {
  const int ks = 4 * (o >> 4) + (o & 3);
  const int ln = 16 * ((o & 15) >> 2) + (k & 15);
  return frh_l[(ks * 64 + swz(ln, ks)) * 4 + (k >> 4)];
}

// MR > 0: every hidden layer is 16 (MT - 1) + MR wide and fc_l runs in the
// remainder form (fc_forward_rem); MR = 0: fc_forward over all tiles.
template <int MT, int KS, bool BROW, int MR>
__global__ __launch_bounds__(ZNW * 64) void k_zono_tiled(TGeom G, const float* __restrict__ gfrag,
                                                         const float* __restrict__ gbias,
                                                         int64_t B, const float* __restrict__ xl,
                                                         const float* __restrict__ xh,
                                                         TZonoArgs out, uint8_t* overflow,
                                                         int* queue, ZonoMasks zm) {
  extern __shared__ float smem[];
  // with zm.masks: this wave's unstable sets of the current domain, and the
  // workgroup's union of them over its domains that did not overflow
  __shared__ unsigned long long s_dun[ZNW][MAXL];
  __shared__ unsigned long long s_wun[MAXL];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;  // [n][FW], zero-padded
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n, d0 = G.d[0];
  if (threadIdx.x < MAXL) s_wun[threadIdx.x] = 0ull;
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  // the remainder form's tables, after the fragments they are read from
  float* swk = sbias + n * FW;
  constexpr int MF16 = 16 * (MT - 1);
  float* swm = swk + (n - 1) * MF16 * 4;
  if (MR > 0) {
    __syncthreads();
    const int d = MF16 + MR;
    for (int e = threadIdx.x; e < (n - 1) * MF16 * 4; e += blockDim.x) {
      const int l = 1 + e / (MF16 * 4), o = (e / 4) % MF16, kk = e & 3;
      swk[e] = kk <= MR ? frag_weight<KS>(sfrag + G.offh + (l - 1) * KS * 256, o, MF16 + kk)
                        : 0.f;
    }
    for (int e = threadIdx.x; e < (n - 1) * MR * 64; e += blockDim.x) {
      const int l = 1 + e / (MR * 64), m = (e / 64) % (MR > 0 ? MR : 1), k = e & 63;
      swm[e] = k <= d ? frag_weight<KS>(sfrag + G.offh + (l - 1) * KS * 256, MF16 + m, k) : 0.f;
    }
  }
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  // this wave's relu scratch: |G| partials [16 lanes][ZPS], centre, lambda,
  // mu, new-column index [FW] each
  float* zpart = sbias + n * FW + zono_rem_floats(n, MT, MR) + wv * ZSCR;
  float* zcen = zpart + 16 * ZPS;
  float* zlam = zcen + FW;
  float* zmu = zlam + FW;
  int* zcol = reinterpret_cast<int*>(zmu + FW);

  const int nwv = blockDim.x >> 6;
  // the first domain of every wavefront by its index, the rest from the
  // work queue as wavefronts finish (domains differ in cost by their
  // generator counts), else a fixed stride
  const int64_t nwaves = (int64_t)gridDim.x * nwv;
  int64_t dom = (int64_t)blockIdx.x * nwv + wv;
  while (dom < B) {
    const int tnext = (queue && B > nwaves) ? vcm::queue_take(queue, lane) : 0;
    const float* dxl = xl + dom * d0;
    const float* dxh = xh + dom * d0;
    v4f Z[ZT][4];
    int Kc = 1 + d0;
    bool ovf = Kc > 16 * ZT;
    // ---- fc_0 on the input block, one tile at a time past the last used
#pragma unroll
    for (int nt0 = 0; nt0 < ZT; nt0 += 2) {
      v4f o[2][4];
      if (!ovf && 16 * (nt0 + 1) < Kc) {
        zono_input_tiles<MT, KS, 2, BROW>(G, fr0, dxl, dxh, g, r, 16 * nt0, 16, o);
      } else {
        v4f o1[1][4];
        if (!ovf && 16 * nt0 < Kc) {
          zono_input_tiles<MT, KS, 1, BROW>(G, fr0, dxl, dxh, g, r, 16 * nt0, 16, o1);
        } else {
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) o1[0][mt] = v4f{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          o[0][mt] = o1[0][mt];
          o[1][mt] = v4f{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        Z[nt0][mt] = o[0][mt];
        Z[nt0 + 1][mt] = o[1][mt];
      }
    }
    if (!BROW && r == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) Z[0][t][i] = Z[0][t][i] + sbias[16 * t + 4 * g + i];
    }
    for (int l = 0; l < n && !ovf; ++l) {
      if (l > 0) {
        // fc_l on the used column tiles; the centre column picks up b_l
        if (BROW && r == 0) set_elem<MT>(Z[0], G.d[l], g, 1.f);
        const float4* fr = frh + (l - 1) * KS * 64;
        const float* wk = swk + (l - 1) * MF16 * 4;
        const float* wm = swm + (l - 1) * (MR > 0 ? MR : 1) * 64;
#pragma unroll
        for (int nt0 = 0; nt0 < ZT; nt0 += 2) {
          if (16 * (nt0 + 1) < Kc) {
            v4f o[2][4];
            if constexpr (MR > 0)
              fc_forward_rem<MT, KS, 2, ZT, MR>(fr, wk, wm, lane, g, r, Z, nt0, o);
            else
              fc_forward<MT, KS, 2, ZT>(fr, lane, g, r, Z, nt0, o, G.d[l] + (BROW ? 1 : 0));
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
              Z[nt0][mt] = o[0][mt];
              Z[nt0 + 1][mt] = o[1][mt];
            }
          } else if (16 * nt0 < Kc) {
            // tile nt0 + 1 holds no generator (zeros stay zeros)
            v4f o[1][4];
            if constexpr (MR > 0)
              fc_forward_rem<MT, KS, 1, ZT, MR>(fr, wk, wm, lane, g, r, Z, nt0, o);
            else
              fc_forward<MT, KS, 1, ZT>(fr, lane, g, r, Z, nt0, o, G.d[l] + (BROW ? 1 : 0));
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) Z[nt0][mt] = o[0][mt];
          }
        }
        if (!BROW && r == 0) {
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              Z[0][t][i] = Z[0][t][i] + sbias[l * FW + 16 * t + 4 * g + i];
        }
      }
      // relu_l, transposed through this wave's LDS scratch: lane (g, r)
      // adds |G| over its generator columns (only the tiles below Kc hold
      // any), then lane j owns neuron j -- radius, bounds, lambda, mu and
      // the column of its new generator -- and the rows read lambda, mu
      // and that column back for the scaling and the append.
      const int dM = G.d[l + 1];
      {
        float ps[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) ps[t][i] = 0.f;
#pragma unroll
        for (int nt = 0; nt < ZT; ++nt)
          if (16 * nt < Kc) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                ps[t][i] += (nt > 0 || r > 0) ? fabsf(Z[nt][t][i]) : 0.f;
          }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          *reinterpret_cast<float4*>(zpart + r * ZPS + 16 * t + 4 * g) =
              make_float4(ps[t][0], ps[t][1], ps[t][2], ps[t][3]);
          if (r == 0)
            *reinterpret_cast<float4*>(zcen + 16 * t + 4 * g) =
                make_float4(Z[0][t][0], Z[0][t][1], Z[0][t][2], Z[0][t][3]);
        }
      }
      vcm::wave_lds_fence();
      const int j = lane;
      double sd = 0.0;
#pragma unroll
      for (int q = 0; q < 16; ++q) sd += (double)zpart[q * ZPS + j];
      const float rad = (float)sd;
      const float c = zcen[j];
      const float lo = c - rad, hi = c + rad;
      const bool valid = j < dM;
      const bool ust = valid && lo < 0.f && hi > 0.f;
      const bool dead = hi <= 0.f;
      if (valid) {
        out.lo[l][dom * dM + j] = lo;
        out.hi[l][dom * dM + j] = hi;
      }
      const uint64_t umask = __ballot(ust);
      if (zm.masks) {
        // the neurons the CROWN rows pass seeds for this domain (lo < 0,
        // hi > -1e-7: the filter of k_rows_mask)
        const uint64_t km = __ballot(valid && lo < 0.f && hi > -1e-7f);
        if (lane == 0) zm.masks[(int64_t)l * B + dom] = km;
      }
      if (zm.umask && lane == 0) s_dun[wv][l] = umask;  // its unstable set
      const int cnt = __popcll(umask);
      if (l == n - 1) break;  // the last relu's output is not propagated
      if (Kc + cnt > 16 * ZT) {
        ovf = true;
        break;
      }
      zlam[j] = ust ? hi / (hi - lo) : (dead ? 0.f : 1.f);
      zmu[j] = ust ? (-hi * lo) / (2.f * (hi - lo)) : 0.f;
      zcol[j] = ust ? Kc + __popcll(umask & ((1ull << j) - 1ull)) : -1;
      vcm::wave_lds_fence();
      // scale each row by lambda (centre: lambda c + mu) and put mu in the
      // row's new column; tiles from Kc + cnt on stay zero
#pragma unroll
      for (int nt = 0; nt < ZT; ++nt)
        if (16 * nt < Kc + cnt) {
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const float4 lm = *reinterpret_cast<const float4*>(zlam + 16 * t + 4 * g);
            const float4 mv = *reinterpret_cast<const float4*>(zmu + 16 * t + 4 * g);
            const int4 cv = *reinterpret_cast<const int4*>(zcol + 16 * t + 4 * g);
            const float lam4[4] = {lm.x, lm.y, lm.z, lm.w};
            const float mu4[4] = {mv.x, mv.y, mv.z, mv.w};
            const int col4[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float z = Z[nt][t][i];
              z = (nt == 0 && r == 0) ? lam4[i] * z + mu4[i] : z * lam4[i];
              Z[nt][t][i] = col4[i] == 16 * nt + r ? mu4[i] : z;
            }
          }
        }
      Kc += cnt;
    }
    if (lane == 0) {
      overflow[dom] = ovf ? 1 : 0;
      if (ovf && zm.ovf_list) zm.ovf_list[atomicAdd(zm.ovf_count, 1ull)] = dom;
    }
    // an overflowing domain's sets come from the wide pass, over its bounds
    if (zm.umask && !ovf && lane < n) atomicOr(&s_wun[lane], s_dun[wv][lane]);
    dom = (queue && B > nwaves) ? nwaves + vcm::queue_bcast(tnext) : dom + nwaves;
  }
  if (zm.umask) {
    __syncthreads();
    if (threadIdx.x < n && s_wun[threadIdx.x]) atomicOr(zm.umask + threadIdx.x, s_wun[threadIdx.x]);
  }
}

template <int V, int MR>
const void* zono_fn() {
  return reinterpret_cast<const void*>(
      &k_zono_tiled<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0, MR>);
}

// The remainder form's MR for a geometry, 0 when it does not apply: the
// 49- and 50-wide hidden layers of the (4, 14, bias row) variant, every
// hidden layer the same width.
constexpr int kRemVariant = 3;
static_assert(kVariants[kRemVariant].MT == 4 && kVariants[kRemVariant].KS == 14 &&
                  kVariants[kRemVariant].brow == 1,
              "remainder variant");
int zono_rem(const TGeom& G) {
  if (G.variant != kRemVariant || G.n < 2) return 0;
  const int d = G.d[1];
  for (int l = 2; l <= G.n; ++l)
    if (G.d[l] != d) return 0;
  const int mr = d - 16 * (kVariants[kRemVariant].MT - 1);
  return mr >= 1 && mr <= 2 ? mr : 0;
}

// Second zonotope pass over the domains flagged by the first: one
// workgroup of ZWW waves per domain and up to ZWW * ZWT * 16 generator
// columns.  Column tile T lives in wave T % ZWW as its local tile T / ZWW
// (round robin, so the used tiles spread over the waves); the per-neuron
// |G| sums are reduced across waves through LDS in a fixed order, so every
// wave derives the same bounds, lambda, mu and unstable set.
constexpr int ZWW = 8;  // waves per domain (4: 84 us per launch at the ACAS shape, 8: 64 us)
constexpr int ZWT = 4;  // column tiles per wave: 512 columns
static_assert(ZWW * ZWT * 16 == VC_ZONO_WIDE_COLS, "wide zonotope capacity");

template <int MT, int KS, bool BROW>
__global__ __launch_bounds__(ZWW * 64) void k_zono_wide_tiled(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, TZonoArgs out,
    uint8_t* overflow, const int64_t* __restrict__ list, const int64_t* __restrict__ n_list,
    ZonoMasks zm) {
  extern __shared__ float smem[];
  __shared__ unsigned long long s_wun[MAXL];  // with zm.masks: the union over this workgroup's domains
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;                                // [n][FW]
  double* sred = reinterpret_cast<double*>(sbias + G.n * FW);     // [ZWW][FW]
  float* scen = reinterpret_cast<float*>(sred + ZWW * FW);        // centre column [FW]
  float* slam = scen + FW;                                        // lambda [FW]
  float* smu = slam + FW;                                         // mu [FW]
  unsigned long long* sumask = reinterpret_cast<unsigned long long*>(smu + FW);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n, d0 = G.d[0];
  const int cap = ZWW * ZWT * 16;
  // workgroup k takes list entries k, k + grid, ...: the flagged domains
  // spread evenly whatever their positions; idle workgroups leave at once
  const int64_t nflag = *n_list;
  if ((int64_t)blockIdx.x >= nflag) return;
  if (threadIdx.x < MAXL) s_wun[threadIdx.x] = 0ull;
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);

  {
    for (int64_t q = blockIdx.x; q < nflag; q += gridDim.x) {
      const int64_t dom = list[q];
      if (dom < 0 || dom >= B) continue;
      const float* dxl = xl + dom * d0;
      const float* dxh = xh + dom * d0;
      v4f Z[ZWT][4];
      int Kc = 1 + d0;
      bool ovf = Kc > cap;
      // ---- fc_0 on the input block (local tile q = global tile ZWW q + wv)
#pragma unroll
      for (int q0 = 0; q0 < ZWT; q0 += 2) {
        v4f o[2][4];
        if (!ovf && 16 * (ZWW * (q0 + 1) + wv) < Kc) {
          zono_input_tiles<MT, KS, 2, BROW>(G, fr0, dxl, dxh, g, r, 16 * (ZWW * q0 + wv),
                                            16 * ZWW, o);
        } else {
          v4f o1[1][4];
          if (!ovf && 16 * (ZWW * q0 + wv) < Kc) {
            zono_input_tiles<MT, KS, 1, BROW>(G, fr0, dxl, dxh, g, r, 16 * (ZWW * q0 + wv),
                                              16 * ZWW, o1);
          } else {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) o1[0][mt] = v4f{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            o[0][mt] = o1[0][mt];
            o[1][mt] = v4f{0.f, 0.f, 0.f, 0.f};
          }
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          Z[q0][mt] = o[0][mt];
          Z[q0 + 1][mt] = o[1][mt];
        }
      }
      const bool centre = wv == 0 && r == 0;  // lanes holding column 0
      if (!BROW && centre) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) Z[0][t][i] = Z[0][t][i] + sbias[16 * t + 4 * g + i];
      }
      for (int l = 0; l < n && !ovf; ++l) {
        if (l > 0) {
          if (BROW && centre) set_elem<MT>(Z[0], G.d[l], g, 1.f);
          const float4* fr = frh + (l - 1) * KS * 64;
#pragma unroll
          for (int q0 = 0; q0 < ZWT; q0 += 2) {
            if (16 * (ZWW * (q0 + 1) + wv) < Kc) {
              v4f o[2][4];
              fc_forward<MT, KS, 2, ZWT>(fr, lane, g, r, Z, q0, o, G.d[l] + (BROW ? 1 : 0));
#pragma unroll
              for (int mt = 0; mt < 4; ++mt) {
                Z[q0][mt] = o[0][mt];
                Z[q0 + 1][mt] = o[1][mt];
              }
            } else if (16 * (ZWW * q0 + wv) < Kc) {
              v4f o[1][4];
              fc_forward<MT, KS, 1, ZWT>(fr, lane, g, r, Z, q0, o, G.d[l] + (BROW ? 1 : 0));
#pragma unroll
              for (int mt = 0; mt < 4; ++mt) Z[q0][mt] = o[0][mt];
            }
          }
          if (!BROW && centre) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                Z[0][t][i] = Z[0][t][i] + sbias[l * FW + 16 * t + 4 * g + i];
          }
        }
        // relu_l: partial |G| sums per wave, reduced in a fixed order
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            double sd = 0.0;
#pragma unroll
            for (int q = 0; q < ZWT; ++q)
              if (q > 0 || !centre) sd += (double)fabsf(Z[q][t][i]);
            sd = row_sum16(sd);
            const int j = 16 * t + 4 * g + i;
            if (r == 0) sred[wv * FW + j] = sd;
            if (centre) scen[j] = Z[0][t][i];
          }
        __syncthreads();
        const int dM = G.d[l + 1];
        const bool last = l == n - 1;
        // wave 0, lane j: neuron j's radius (the waves' partials in a fixed
        // order), bounds, lambda and mu, and the unstable set as one mask;
        // the other waves read them back (one reduction, not one per wave)
        if (wv == 0) {
          const int j = lane;
          double sd = sred[j];
#pragma unroll
          for (int w2 = 1; w2 < ZWW; ++w2) sd += sred[w2 * FW + j];
          const float rad = (float)sd;
          const float c = scen[j];
          const float lo = c - rad, hi = c + rad;
          const bool valid = j < dM;
          const bool ust = valid && lo < 0.f && hi > 0.f;
          const bool dead = hi <= 0.f;
          if (valid) {
            out.lo[l][dom * dM + j] = lo;
            out.hi[l][dom * dM + j] = hi;
          }
          slam[j] = ust ? hi / (hi - lo) : (dead ? 0.f : 1.f);
          smu[j] = ust ? (-hi * lo) / (2.f * (hi - lo)) : 0.f;
          const uint64_t um = __ballot(ust);
          if (lane == 0) *sumask = um;
          if (zm.masks) {
            const uint64_t km = __ballot(valid && lo < 0.f && hi > -1e-7f);
            if (lane == 0) zm.masks[(int64_t)l * B + dom] = km;
          }
          if (zm.umask && lane == 0) s_wun[l] |= um;
        }
        __syncthreads();  // sred / scen are rewritten by the next layer after this
        const uint64_t umask = *sumask;
        float mu[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * t + 4 * g + i;
            const float lam = slam[j];
            mu[t][i] = smu[j];
            if (!last) {
#pragma unroll
              for (int q = 0; q < ZWT; ++q)
                Z[q][t][i] = (q == 0 && centre) ? lam * Z[q][t][i] + mu[t][i] : Z[q][t][i] * lam;
            }
          }
        const int cnt = __popcll(umask);
        if (last) break;
        if (Kc + cnt > cap) {
          ovf = true;
          break;
        }
        // append one column per unstable neuron at position Kc + rank
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * t + 4 * g + i;
            if ((umask >> j) & 1ull) {
              const int col = Kc + __popcll(umask & ((1ull << j) - 1ull));
              const int T = col >> 4;
              if ((col & 15) == r && T % ZWW == wv) {
#pragma unroll
                for (int q = 0; q < ZWT; ++q)
                  if (q == T / ZWW) Z[q][t][i] = mu[t][i];
              }
            }
          }
        Kc += cnt;
      }
      if (threadIdx.x == 0) overflow[dom] = ovf ? 1 : 0;
    }
  }
  if (zm.umask) {
    __syncthreads();
    if (threadIdx.x < n && s_wun[threadIdx.x]) atomicOr(zm.umask + threadIdx.x, s_wun[threadIdx.x]);
  }
}

template <int V>
const void* zono_wide_fn() {
  return reinterpret_cast<const void*>(
      &k_zono_wide_tiled<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>);
}

template <int V>
const void* crown_dom_fn() {
  return reinterpret_cast<const void*>(
      &k_crown_dom<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>);
}

template <int V>
const void* crown_fn() {
  return reinterpret_cast<const void*>(
      &k_crown_tiled<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>);
}

}  // namespace

extern "C" int64_t vc_mlp_tiled_floats(const int32_t* dims, int n_relu) {
  TGeom G;
  const int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return -rc;
  return G.nfloats;
}

extern "C" int vc_mlp_tiled_pack(const float* const* W, const float* const* bias,
                                 const int32_t* dims, int n_relu, float* frag,
                                 vc_stream_t stream) {
  TGeom G;
  const int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  if (!W || !frag) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  for (int l = 0; l < n_relu; ++l) {
    if (!W[l] || (G.brow && (!bias || !bias[l]))) return VC_ERR_ARG;
    const float* b = G.brow ? bias[l] : nullptr;
    if (l == 0) {
      const int total = G.mt0 * G.KS * 64;
      hipLaunchKernelGGL(k_tpack, dim3((total + 255) / 256), dim3(256), 0, st, W[0], b, G.d[1],
                         G.d[0], G.KS, G.mt0, 0, G.brow, frag);
    } else {
      const int total = 4 * G.KS * 64;
      hipLaunchKernelGGL(k_tpack, dim3((total + 255) / 256), dim3(256), 0, st, W[l], b,
                         G.d[l + 1], G.d[l], G.KS, 4, 1, G.brow,
                         frag + G.offh + (int64_t)(l - 1) * G.KS * 256);
    }
  }
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_mlp_tiled_crown_mode(int64_t B) {
  return B <= (int64_t)vcm::cu_count() * 4 ? 1 : 0;
}

extern "C" int vc_mlp_tiled_crown(const int32_t* dims, int n_relu, const float* frag,
                                  const float* bias_cat, int64_t B, const float* xl,
                                  const float* xh, const float* const* lo_in,
                                  const float* const* hi_in, float* const* lo_out,
                                  float* const* hi_out, const int32_t* idx_all,
                                  const int32_t* idx_meta, int do_crown, int per_domain, int Q,
                                  const float* spec_rows, const float* spec_acc, float* lb_out,
                                  float* A_out, float* acc_out, uint64_t* seed_rows,
                                  int32_t* queue, vc_stream_t stream) {
  TGeom G;
  int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  if (!frag || !bias_cat || !xl || !xh || !lo_in || !hi_in || B < 0) return VC_ERR_ARG;
  if (Q < 0 || Q > TQMAX) return VC_ERR_UNSUPPORTED;
  if (Q > 0 && (!spec_rows || !spec_acc || !lb_out)) return VC_ERR_ARG;
  if (do_crown && (!idx_all || !idx_meta || !lo_out || !hi_out)) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  TCrownArgs ca;
  int nmax = 0;
  for (int l = 0; l < MAXL; ++l) {
    const bool in = l < n_relu;
    ca.lo_in[l] = in ? lo_in[l] : nullptr;
    ca.hi_in[l] = in ? hi_in[l] : nullptr;
    ca.lo_out[l] = (in && lo_out) ? lo_out[l] : nullptr;
    ca.hi_out[l] = (in && hi_out) ? hi_out[l] : nullptr;
    if (in && (!ca.lo_in[l] || !ca.hi_in[l])) return VC_ERR_ARG;
    if (in) nmax += G.d[l + 1];
  }
  const size_t lds = ((size_t)G.nfloats + (size_t)n_relu * FW + (size_t)nmax +
                      (size_t)TNW * (n_relu * 3 * FW + 7 * FW + MAXL)) *
                     sizeof(float);
  if (lds > 160 * 1024) return VC_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  // small batches: D domains per workgroup, the workgroup's wavefronts
  // shared among them (every domain in flight at once)
  const int cus = vcm::cu_count();
  if (vc_mlp_tiled_crown_mode(B) == 1) {
    const int D = (int)std::min<int64_t>(4, std::max<int64_t>(1, (B + cus - 1) / cus));
    const size_t lds_d = ((size_t)G.nfloats + (size_t)n_relu * FW + (size_t)nmax +
                          (size_t)D * (n_relu * 3 * FW + 7 * FW)) *
                         sizeof(float);
    const void* fd = nullptr;
    switch (G.variant) {
      case 0: fd = crown_dom_fn<0>(); break;
      case 1: fd = crown_dom_fn<1>(); break;
      case 2: fd = crown_dom_fn<2>(); break;
      case 3: fd = crown_dom_fn<3>(); break;
      case 4: fd = crown_dom_fn<4>(); break;
      case 5: fd = crown_dom_fn<5>(); break;
      default: return VC_ERR_UNSUPPORTED;
    }
    if (lds_d + 512 <= 160 * 1024 && vcm::allow_max_lds(fd)) {
      const dim3 gd((unsigned)((B + D - 1) / D)), bd(TNW * 64);
#define VC_TDOM_CASE(V)                                                                       \
  case V:                                                                                     \
    hipLaunchKernelGGL((k_crown_dom<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>), \
                       gd, bd, lds_d, st, G, frag, bias_cat, B, xl, xh, ca, idx_all, idx_meta, \
                       do_crown, per_domain, Q, spec_rows, spec_acc, lb_out, A_out, acc_out,   \
                       reinterpret_cast<unsigned long long*>(seed_rows), D);                   \
    break;
      switch (G.variant) {
        VC_TDOM_CASE(0)
        VC_TDOM_CASE(1)
        VC_TDOM_CASE(2)
        VC_TDOM_CASE(3)
        VC_TDOM_CASE(4)
        VC_TDOM_CASE(5)
        default: return VC_ERR_UNSUPPORTED;
      }
#undef VC_TDOM_CASE
      VC_LAUNCH_CHECK();
      return VC_OK;
    }
  }
  const void* fn = nullptr;
  switch (G.variant) {
    case 0: fn = crown_fn<0>(); break;
    case 1: fn = crown_fn<1>(); break;
    case 2: fn = crown_fn<2>(); break;
    case 3: fn = crown_fn<3>(); break;
    case 4: fn = crown_fn<4>(); break;
    case 5: fn = crown_fn<5>(); break;
    default: return VC_ERR_UNSUPPORTED;
  }
  if (!vcm::allow_max_lds(fn)) return VC_ERR_UNSUPPORTED;
  const dim3 grid(vcm::persistent_grid(B, lds, TNW)), block(TNW * 64);
  if (queue) hipLaunchKernelGGL(k_queue_reset, dim3(1), dim3(64), 0, st, queue);
#define VC_TILED_CASE(V)                                                                     \
  case V:                                                                                    \
    hipLaunchKernelGGL((k_crown_tiled<kVariants[V].MT, kVariants[V].KS,                      \
                                      kVariants[V].brow != 0>),                              \
                       grid, block, lds, st, G, frag, bias_cat, B, xl, xh, ca, idx_all,      \
                       idx_meta, do_crown, per_domain, Q, spec_rows, spec_acc, lb_out, A_out,  \
                       acc_out, reinterpret_cast<unsigned long long*>(seed_rows), queue);    \
    break;
  switch (G.variant) {
    VC_TILED_CASE(0)
    VC_TILED_CASE(1)
    VC_TILED_CASE(2)
    VC_TILED_CASE(3)
    VC_TILED_CASE(4)
    VC_TILED_CASE(5)
    default: return VC_ERR_UNSUPPORTED;
  }
#undef VC_TILED_CASE
  VC_LAUNCH_CHECK();
  return VC_OK;
}

// ------------------------------- layer-synchronous CROWN over packed rows
// vc_mlp_crown_rows computes what vc_mlp_tiled_crown computes, with the
// work laid out by layer instead of by domain.  k_crown_tiled gives each
// domain its own 16-row tiles, so a layer's 2 m seeded rows fill
// ceil(2 m / 16) tiles (about half full at the ACAS-Xu shape) and the Q = 4
// spec rows a quarter of one.  Here the seeded rows of layer L of every
// domain are packed densely into one row list and chained through
// fc_{L-1} .. fc_0 in full tiles; each row reads its own domain's slopes of
// the layers below, which earlier launches left in a per-layer slope buffer,
// and the spec rows of 16 / Q domains share a tile.  Every row is computed
// with the operations of k_crown_tiled in the same order (an MFMA output
// column depends only on its own B column), so the results are the same
// bit for bit.  Launch order per call:
//   k_rows_mask      per domain and layer: the seeded neurons (the union,
//                    per domain filtered as in k_crown_tiled) as a 64-bit mask
//   k_rows_scan1/2   per layer, the rows' offsets (exclusive scan of 2 m)
//   per layer L:
//     k_crown_rows   the rows' bounds: start +-W_L[j], relax and fc down to
//                    the input, concretize over the row's box
//     k_rows_cut     per domain: intersect the bounds, the slopes of layer L,
//                    and layer L + 1's row codes (domain, sign, neuron; layer
//                    0's by k_rows_write)
//   k_spec_rows      the spec rows of every domain, B Q rows in full tiles
namespace {

constexpr int RNW = 8;        // waves per workgroup of the row-chain kernels
constexpr int RSCAN = 1024;   // domains per block of the offset scan
constexpr int SLW = 2 * FW;   // floats per (layer, domain) of the slope buffer

// A row: domain << 7 | negated << 6 | neuron.
__device__ __forceinline__ uint32_t row_code(int64_t d, int neg, int j) {
  return ((uint32_t)d << 7) | ((uint32_t)neg << 6) | (uint32_t)j;
}

// fc0_concretize for rows of different domains: the box values of the
// lane's first-M-tile inputs (m = 4 g + i) come preloaded in registers,
// further M-tiles (more than 16 inputs) read them from dxl / dxh.
template <int KS, bool BROW>
__device__ __forceinline__ void fc0_concretize_pr(const float* fr0, int mt0, int d0, int lane,
                                                  int g, int r, const float (&bxl)[4],
                                                  const float (&bxh)[4], const float* dxl,
                                                  const float* dxh, const v4f (&F)[TNP][4],
                                                  double (&acc)[TNP], double (&cz)[TNP],
                                                  float* A_rows, int n_live) {
  for (int mt = 0; mt < mt0; ++mt) {
    v4f o = v4f{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_s_setprio(1);  // as in fc_hidden
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      o = mfma16x16x4(fr0[(mt * KS + ks) * 64 + swz(lane, ks)], F[0][ks >> 2][ks & 3], o);
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mt + 4 * g + i;
      const bool in = m < d0;
      const float xlv = in ? (mt == 0 ? bxl[i] : dxl[m]) : 0.f;
      const float xhv = in ? (mt == 0 ? bxh[i] : dxh[m]) : 0.f;
      const float v = o[i];
      if (in) {
        cz[0] += (double)(fmaxf(v, 0.f) * xlv);
        cz[0] += (double)(fminf(v, 0.f) * xhv);
        if (A_rows && r < n_live) A_rows[(int64_t)r * d0 + m] = v;
      } else if (BROW && m == d0) {
        acc[0] += (double)v;
      }
    }
  }
}

// The box values a lane's concretization reads first: inputs 4 g + i.
__device__ __forceinline__ void box_load(const float* dxl, const float* dxh, int d0, int g,
                                         float (&bxl)[4], float (&bxh)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * g + i;
    bxl[i] = m < d0 ? dxl[m] : 0.f;
    bxh[i] = m < d0 ? dxh[m] : 0.f;
  }
}

// The slopes of one relu for rows of different domains: each lane's row
// reads those of its own domain from the slope buffer (cb: that domain's
// entry for the layer: [0, FW) lo_s folded into the sign of up_s, [FW, 2 FW)
// up_t), the 4 K-steps of a 16-neuron tile per float4.  lo_s is 0 or 1 and
// up_s > 0 wherever lo_s = 1, so the sign carries it.
struct RowSlopes {
  float4 c[4], u[4];
};

template <int KS>
__device__ __forceinline__ void slopes_load(const float* cb, int g, RowSlopes& s) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (4 * t >= KS) break;
    s.c[t] = *reinterpret_cast<const float4*>(cb + 16 * t + 4 * g);
    s.u[t] = *reinterpret_cast<const float4*>(cb + FW + 16 * t + 4 * g);
  }
}

// The relaxation with per-row slopes: relax_rows with the decoded values
// (equal to make_slopes').
template <int KS, bool BROW>
__device__ __forceinline__ void relax_rows_pr(const RowSlopes& s, const float* bl, int g,
                                              v4f (&F)[TNP][4], double (&acc)[TNP]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (4 * t >= KS) break;
    const float cs[4] = {s.c[t].x, s.c[t].y, s.c[t].z, s.c[t].w};
    const float us4[4] = {s.u[t].x, s.u[t].y, s.u[t].z, s.u[t].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (4 * t + i >= KS) break;
      const int j = 16 * t + 4 * g + i;
      const float us = fabsf(cs[i]);
      const float ls = cs[i] < 0.f ? 1.f : 0.f;
      const float ut = us4[i];
      const float bj = BROW ? 0.f : bl[j];
      const float x = F[0][t][i];
      const bool ng = x < 0.f;
      const float e = x * (ng ? us : ls);
      const float en = ng ? x : 0.f;
      acc[0] += (double)(en * ut);
      if (!BROW) acc[0] += (double)(e * bj);
      F[0][t][i] = e;
    }
  }
}

// Rows at relu Ltop's output through relax + fc_l for l = Ltop .. 1, then
// relu 0 and fc_0 with the concretization (chain_to_input, per-row slopes).
// The slopes of the next relu are requested before each fc's MFMAs.
template <int MT, int KS, bool BROW>
__device__ __forceinline__ void chain_rows(const TGeom& G, int Ltop, const float* fr0,
                                           const float4* frh, const float* slp, int64_t B,
                                           int64_t d, const float* sbias, int lane, int g, int r,
                                           const float* dxl, const float* dxh, v4f (&F)[TNP][4],
                                           double (&acc)[TNP], double (&cz)[TNP], float* A_rows,
                                           int n_live) {
  // the first slopes and the box requested together (one round trip)
  RowSlopes s;
  slopes_load<KS>(slp + ((int64_t)Ltop * B + d) * SLW, g, s);
  float bxl[4], bxh[4];
  box_load(dxl, dxh, G.d[0], g, bxl, bxh);
  for (int l = Ltop; l >= 1; --l) {
    relax_rows_pr<KS, BROW>(s, sbias + l * FW, g, F, acc);
    slopes_load<KS>(slp + ((int64_t)(l - 1) * B + d) * SLW, g, s);
    fc_hidden<MT, KS, 1, BROW>(frh + (l - 1) * KS * 64, lane, g, G.d[l], F, acc);
  }
  relax_rows_pr<KS, BROW>(s, sbias, g, F, acc);
  fc0_concretize_pr<KS, BROW>(fr0, G.mt0, G.d[0], lane, g, r, bxl, bxh, dxl, dxh, F, acc, cz,
                              A_rows, n_live);
}

struct RowsLayers {
  const float* lo[MAXL];
  const float* hi[MAXL];
  float* lo_out[MAXL];
  float* hi_out[MAXL];
};

// The union of unstable neurons per layer as a bit mask, umask[L]: from
// the caller's lists (idx_all, idx_meta of vc_union_compact), or, with no
// lists, cleared here for k_rows_mask to OR into.  One wavefront.
__global__ __launch_bounds__(64) void k_rows_union(TGeom G, const int32_t* __restrict__ idx_all,
                                                   const int32_t* __restrict__ idx_meta,
                                                   unsigned long long* __restrict__ umask) {
  const int lane = threadIdx.x;
  const int n = G.n;
  for (int L = 0; L < n; ++L) {
    unsigned long long v = 0ull;
    if (idx_all) {
      // bit j for every listed neuron j (an OR over the wave)
      const int c = min(idx_meta[L], G.d[L + 1]);
      const int j = lane < c ? idx_all[idx_meta[n + L] + lane] : 0;
      v = (lane < c && j >= 0 && j < FW) ? (1ull << j) : 0ull;
      for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    }
    if (lane == 0) umask[L] = v;
  }
}

// Per domain and layer, the neurons this domain would seed (per_domain:
// lo < 0 and hi > -1e-7, the filter of k_crown_tiled; else every neuron)
// as a bit mask, before the union is applied (k_rows_scan1 does that).
// With want_union, the neurons unstable here (lo < 0 < hi) are ORed into
// umask: per wavefront over its domains, per workgroup through LDS, then
// one atomic per workgroup and layer.  Persistent: each wavefront takes two
// domains at a time, all their loads issued before any is used (NL >= n
// layers' worth of registers).
template <int NL>
__global__ __launch_bounds__(256) void k_rows_mask(TGeom G, int64_t B, RowsLayers rl,
                                                   int per_domain, int want_union,
                                                   uint64_t* __restrict__ masks,
                                                   unsigned long long* __restrict__ umask) {
  __shared__ unsigned long long wu[MAXL];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n = G.n;
  if (threadIdx.x < MAXL) wu[threadIdx.x] = 0ull;
  __syncthreads();
  const bool need = per_domain || want_union;
  uint64_t un[NL];
#pragma unroll
  for (int L = 0; L < NL; ++L) un[L] = 0ull;
  const int64_t stride = (int64_t)gridDim.x * 8;
  for (int64_t d0 = ((int64_t)blockIdx.x * 4 + wv) * 2; d0 < B; d0 += stride) {
    float lo[2][NL], hi[2][NL];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int64_t d = d0 + k;
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        const int dW = L < n ? G.d[L + 1] : 0;
        const bool rd = need && d < B && lane < dW;
        lo[k][L] = rd ? rl.lo[L][d * dW + lane] : 0.f;
        hi[k][L] = rd ? rl.hi[L][d * dW + lane] : 0.f;
      }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int64_t d = d0 + k;
      if (d >= B) break;
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        if (L >= n) break;
        const bool in = lane < G.d[L + 1];
        const bool keep = in && (!per_domain || (lo[k][L] < 0.f && hi[k][L] > -1e-7f));
        const uint64_t m = __ballot(keep);
        un[L] |= __ballot(in && lo[k][L] < 0.f && hi[k][L] > 0.f);
        if (lane == 0) masks[(int64_t)L * B + d] = m;
      }
    }
  }
  if (want_union) {
    if (lane == 0)
      for (int L = 0; L < n; ++L)
        if (un[L]) atomicOr(&wu[L], (unsigned long long)un[L]);
    __syncthreads();
    if (threadIdx.x < n && wu[threadIdx.x]) atomicOr(umask + threadIdx.x, wu[threadIdx.x]);
  }
}

// Per layer (blockIdx.y), within blocks of RSCAN domains: the seeded
// neurons m = mask & umask[L] (written back to masks), and the exclusive
// scan of the row counts 2 |m| (offsets local to the block), block totals
// to bsum.
__global__ __launch_bounds__(RSCAN) void k_rows_scan1(uint64_t* __restrict__ masks,
                                                      const unsigned long long* __restrict__ umask,
                                                      int64_t B, int32_t* __restrict__ off,
                                                      int32_t* __restrict__ bsum, int nblk) {
  __shared__ int wsum[RSCAN / 64];
  const int L = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * RSCAN + threadIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int v = 0;
  if (i < B) {
    const uint64_t m = masks[(int64_t)L * B + i] & (uint64_t)umask[L];
    masks[(int64_t)L * B + i] = m;
    v = 2 * __popcll(m);
  }
  int x = v;  // inclusive scan within the wave
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wv] = x;
  __syncthreads();
  if (wv == 0) {
    int w = lane < RSCAN / 64 ? wsum[lane] : 0;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(w, o, 64);
      if (lane >= o) w += y;
    }
    if (lane < RSCAN / 64) wsum[lane] = w;  // inclusive wave prefix
  }
  __syncthreads();
  const int base = wv > 0 ? wsum[wv - 1] : 0;
  if (i < B) off[(int64_t)L * B + i] = base + x - v;
  if (threadIdx.x == RSCAN - 1) bsum[L * nblk + blockIdx.x] = wsum[RSCAN / 64 - 1];
}

// Per layer (blockIdx.x): exclusive scan of the block totals in place, the
// layer's row total to tot[L] and, when counted, its seeded neurons (half
// the rows) added to seed_rows[L].
__global__ __launch_bounds__(1024) void k_rows_scan2(int32_t* __restrict__ bsum, int nblk,
                                                     int32_t* __restrict__ tot,
                                                     unsigned long long* __restrict__ seed_rows) {
  __shared__ int wsum[16];
  __shared__ int carry;
  const int L = blockIdx.x;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int c0 = 0; c0 < nblk; c0 += 1024) {
    const int k = c0 + threadIdx.x;
    const int v = k < nblk ? bsum[L * nblk + k] : 0;
    int x = v;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    if (wv == 0) {
      int w = lane < 16 ? wsum[lane] : 0;
      for (int o = 1; o < 16; o <<= 1) {
        const int y = __shfl_up(w, o, 64);
        if (lane >= o) w += y;
      }
      if (lane < 16) wsum[lane] = w;
    }
    __syncthreads();
    const int base = carry + (wv > 0 ? wsum[wv - 1] : 0);
    if (k < nblk) bsum[L * nblk + k] = base + x - v;
    __syncthreads();
    if (threadIdx.x == 0) carry += wsum[15];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    tot[L] = carry;
    if (seed_rows) atomicAdd(seed_rows + L, (unsigned long long)(carry / 2));
  }
}

// The row codes of layer L: domain d's rows start at its offset, the m
// "+" rows (neurons in increasing order) then the m "-" rows.
__global__ __launch_bounds__(256) void k_rows_write(int64_t B, int L,
                                                    const uint64_t* __restrict__ masks,
                                                    const int32_t* __restrict__ off,
                                                    const int32_t* __restrict__ bsum, int nblk,
                                                    uint32_t* __restrict__ rows) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int64_t d = (int64_t)blockIdx.x * 4 + wv; d < B; d += (int64_t)gridDim.x * 4) {
    const uint64_t m = masks[(int64_t)L * B + d];
    if (!m) continue;
    const int cnt = __popcll(m);
    const int64_t base = (int64_t)off[(int64_t)L * B + d] + bsum[L * nblk + (int)(d / RSCAN)];
    if ((m >> lane) & 1ull) {
      const int q = __popcll(m & ((1ull << lane) - 1ull));
      rows[base + q] = row_code(d, 0, lane);
      rows[base + cnt + q] = row_code(d, 1, lane);
    }
  }
}

// The bounds of layer L's rows (chains of full 16-row tiles): each
// workgroup takes a contiguous run of tiles, its wavefronts alternate.
template <int MT, int KS, bool BROW>
__global__ __launch_bounds__(RNW * 64, 4) void k_crown_rows(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, int L,
    const uint32_t* __restrict__ rows, const int32_t* __restrict__ tot,
    const float* __restrict__ slp, float* __restrict__ slb) {
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;  // [n][FW], zero-padded
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n, d0 = G.d[0];
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  const int64_t R = tot[L];
  const int64_t ntiles = (R + 15) / 16;
  const int64_t per = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * per;
  const int64_t t1 = t0 + per < ntiles ? t0 + per : ntiles;
  // each tile's row code is requested one tile ahead
  uint32_t code_next = 0u;
  if (t0 + wv < t1 && (t0 + wv) * 16 + r < R) code_next = rows[(t0 + wv) * 16 + r];
  for (int64_t tile = t0 + wv; tile < t1; tile += RNW) {
    const int64_t row = tile * 16 + r;
    const bool live = row < R;
    const uint32_t code = live ? code_next : 0u;
    {
      const int64_t nrow = (tile + RNW) * 16 + r;
      code_next = (tile + RNW < t1 && nrow < R) ? rows[nrow] : 0u;
    }
    const int64_t d = (int64_t)(code >> 7);
    const int j = (int)(code & 63u);
    const float sg = (code >> 6) & 1u ? -1.f : 1.f;
    const float* dxl = xl + d * d0;
    const float* dxh = xh + d * d0;
    const int ksj = 4 * (j >> 4) + (j & 3), gj = (j & 15) >> 2;
    v4f F[TNP][4];
    double acc[TNP], cz[TNP];
    acc[0] = (live && g == 0) ? (double)(sg * sbias[L * FW + j]) : 0.0;
    cz[0] = 0.0;
    if (L > 0) {
      const float4* fl = frh + (L - 1) * KS * 64 + ksj * 64;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 w = live ? fl[swz(16 * gj + 4 * g + i, ksj)] : float4{0.f, 0.f, 0.f, 0.f};
        F[0][0][i] = sg * w.x;
        F[0][1][i] = sg * w.y;
        F[0][2][i] = sg * w.z;
        F[0][3][i] = sg * w.w;
      }
      chain_rows<MT, KS, BROW>(G, L - 1, fr0, frh, slp, B, d, sbias, lane, g, r, dxl, dxh, F,
                               acc, cz, nullptr, 0);
    } else if (live) {
      // seeded at relu 0: the row is +-W_0[j] over the inputs
      for (int mt = 0; mt < G.mt0; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mi = 16 * mt + 4 * g + i;
          if (mi < d0) {
            const float v = sg * fr0[(mt * KS + ksj) * 64 + swz(16 * gj + 4 * g + i, ksj)];
            cz[0] += (double)(fmaxf(v, 0.f) * dxl[mi]);
            cz[0] += (double)(fminf(v, 0.f) * dxh[mi]);
          }
        }
    }
    const double lbd = group_sum4_d(acc[0] + cz[0]);
    if (g == 0 && live) slb[row] = (float)lbd;
  }
}

// Layer L's final bounds of every domain (lane j holds neuron j; two
// domains per wavefront, their loads issued together): lo = max(lo, lb+),
// hi = max(min(hi, -lb-), lo) for the seeded neurons, then the slopes of
// make_slopes into the slope buffer and the bounds to lo_out / hi_out when
// given; and, with wnext, layer L + 1's row codes (k_rows_write's).
// masks null: no seeds (the slopes of the given bounds).
__global__ __launch_bounds__(256) void k_rows_cut(TGeom G, int64_t B, int L, RowsLayers rl,
                                                  const uint64_t* __restrict__ masks,
                                                  const int32_t* __restrict__ off,
                                                  const int32_t* __restrict__ bsum, int nblk,
                                                  const float* __restrict__ slb,
                                                  float* __restrict__ slp, int wnext,
                                                  uint32_t* __restrict__ rows) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int dW = G.d[L + 1];
  const bool in = lane < dW;
  for (int64_t d0 = ((int64_t)blockIdx.x * 4 + wv) * 2; d0 < B; d0 += (int64_t)gridDim.x * 8) {
    float lo[2], hi[2];
    uint64_t m[2], mn[2];
    int64_t base[2], bn[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int64_t d = d0 + k;
      const bool v = d < B;
      lo[k] = (v && in) ? rl.lo[L][d * dW + lane] : 0.f;
      hi[k] = (v && in) ? rl.hi[L][d * dW + lane] : 0.f;
      m[k] = (v && masks) ? masks[(int64_t)L * B + d] : 0ull;
      base[k] = (v && masks)
                    ? (int64_t)off[(int64_t)L * B + d] + bsum[L * nblk + (int)(d / RSCAN)]
                    : 0;
      mn[k] = (v && wnext) ? masks[(int64_t)(L + 1) * B + d] : 0ull;
      bn[k] = (v && wnext) ? (int64_t)off[(int64_t)(L + 1) * B + d] +
                                 bsum[(L + 1) * nblk + (int)(d / RSCAN)]
                           : 0;
    }
    float sp[2], sn[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const bool seeded = in && ((m[k] >> lane) & 1ull);
      const int cnt = __popcll(m[k]);
      const int q = __popcll(m[k] & ((1ull << lane) - 1ull));
      sp[k] = seeded ? slb[base[k] + q] : 0.f;
      sn[k] = seeded ? slb[base[k] + cnt + q] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int64_t d = d0 + k;
      if (d >= B) break;
      float l = lo[k], h = hi[k];
      if (in && ((m[k] >> lane) & 1ull)) {
        const float lc = fmaxf(l, sp[k]);
        const float hc = fmaxf(fminf(h, -sn[k]), lc);
        l = lc;
        h = hc;
      }
      if (in && rl.lo_out[L]) {
        rl.lo_out[L][d * dW + lane] = l;
        rl.hi_out[L][d * dW + lane] = h;
      }
      float code = 0.f, ut = 0.f;
      if (in) {
        const Relax s = relax(l, h);
        code = s.lo_s != 0.f ? -s.up_s : s.up_s;
        ut = s.up_t;
      }
      float* e = slp + ((int64_t)L * B + d) * SLW;
      e[lane] = code;
      e[FW + lane] = ut;
      if (wnext && ((mn[k] >> lane) & 1ull)) {
        const int cnt = __popcll(mn[k]);
        const int q = __popcll(mn[k] & ((1ull << lane) - 1ull));
        rows[bn[k] + q] = row_code(d, 0, lane);
        rows[bn[k] + cnt + q] = row_code(d, 1, lane);
      }
    }
  }
}

// The spec rows of every domain (row d Q + q: domain d, spec row q) through
// relu n-1 .. relu 0 in full tiles; lb, acc and the input coefficients out.
template <int MT, int KS, bool BROW>
__global__ __launch_bounds__(RNW * 64, 4) void k_spec_rows(
    TGeom G, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, int Q,
    const float* __restrict__ spec_rows, const float* __restrict__ spec_acc,
    const float* __restrict__ slp, float* __restrict__ lb_out, float* __restrict__ A_out,
    float* __restrict__ acc_out) {
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + G.nfloats;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n = G.n, d0 = G.d[0], dN = G.d[n];
  vcm::stage_float4(sfrag, gfrag, G.nfloats / 4);
  for (int k = threadIdx.x; k < n * FW; k += blockDim.x) {
    const int l = k / FW, j = k % FW;
    sbias[k] = j < G.d[l + 1] ? gbias[G.boff[l] + j] : 0.f;
  }
  __syncthreads();
  const float* fr0 = sfrag;
  const float4* frh = reinterpret_cast<const float4*>(sfrag + G.offh);
  const int64_t R = B * Q;
  const int64_t ntiles = (R + 15) / 16;
  const int64_t per = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * per;
  const int64_t t1 = t0 + per < ntiles ? t0 + per : ntiles;
  for (int64_t tile = t0 + wv; tile < t1; tile += RNW) {
    const int64_t row = tile * 16 + r;
    const bool live = row < R;
    const int64_t d = live ? row / Q : 0;
    const int q = live ? (int)(row - d * Q) : 0;
    const float* dxl = xl + d * d0;
    const float* dxh = xh + d * d0;
    v4f F[TNP][4];
    double acc[TNP], cz[TNP];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = 16 * t + 4 * g + i;
        F[0][t][i] = (live && k < dN) ? spec_rows[q * dN + k] : 0.f;
      }
    acc[0] = (live && g == 0) ? (double)spec_acc[q] : 0.0;
    cz[0] = 0.0;
    float* A_rows = A_out ? A_out + tile * 16 * d0 : nullptr;
    chain_rows<MT, KS, BROW>(G, n - 1, fr0, frh, slp, B, d, sbias, lane, g, r, dxl, dxh, F, acc,
                             cz, A_rows, (int)(R - tile * 16 < 16 ? R - tile * 16 : 16));
    const double a = group_sum4_d(acc[0]);
    const double lbd = a + group_sum4_d(cz[0]);
    if (g == 0 && live) {
      lb_out[row] = (float)lbd;
      if (acc_out) acc_out[row] = (float)a;
    }
  }
}

template <int V>
const void* crown_rows_fn() {
  return reinterpret_cast<const void*>(
      &k_crown_rows<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>);
}

template <int V>
const void* spec_rows_fn() {
  return reinterpret_cast<const void*>(
      &k_spec_rows<kVariants[V].MT, kVariants[V].KS, kVariants[V].brow != 0>);
}

// The workspace of vc_mlp_crown_rows, carved in order (256-byte aligned).
struct RowsWork {
  uint64_t* masks;  // [n][B]
  unsigned long long* umask;  // [MAXL]
  int32_t* off;     // [n][B]
  int32_t* bsum;    // [n][nblk]
  int32_t* tot;     // [n]
  uint32_t* rows;   // [B * 2 * max width]
  float* slb;       // [B * 2 * max width]
  float* slp;       // [n][B][2 FW]
  size_t bytes;
};

RowsWork rows_carve(char* base, int n, int maxw, int64_t B) {
  RowsWork w{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + o : nullptr;
    o += (bytes + 255) & ~(size_t)255;
    return p;
  };
  const int nblk = (int)((B + RSCAN - 1) / RSCAN);
  w.masks = reinterpret_cast<uint64_t*>(take(sizeof(uint64_t) * n * B));
  w.umask = reinterpret_cast<unsigned long long*>(take(sizeof(unsigned long long) * MAXL));
  w.off = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * n * B));
  w.bsum = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * n * (size_t)nblk));
  w.tot = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * n));
  w.rows = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * B * 2 * (size_t)maxw));
  w.slb = reinterpret_cast<float*>(take(sizeof(float) * B * 2 * (size_t)maxw));
  w.slp = reinterpret_cast<float*>(take(sizeof(float) * n * B * (size_t)SLW));
  w.bytes = o;
  return w;
}

}  // namespace

extern "C" int64_t vc_mlp_crown_rows_workspace(const int32_t* dims, int n_relu, int64_t B) {
  TGeom G;
  const int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return -rc;
  if (B < 0) return -VC_ERR_ARG;
  // the batch limit of crown_rows_run (int32 row offsets, 25-bit domain in
  // the row codes): callers that size a workspace here fall back to the
  // one-wavefront-per-domain CROWN instead
  if (B >= ((int64_t)1 << 24)) return -VC_ERR_UNSUPPORTED;
  int maxw = 1;
  for (int l = 1; l <= n_relu; ++l) maxw = G.d[l] > maxw ? G.d[l] : maxw;
  return (int64_t)rows_carve(nullptr, n_relu, maxw, B).bytes;
}

namespace {
// premasked: the seed masks and the union of the unstable sets are already
// in the workspace (written by the zonotope passes over the same bounds,
// vcm::zono_bounds_masked), so k_rows_union and k_rows_mask are skipped;
// only with do_crown, per_domain and no index lists.
int crown_rows_run(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                   int64_t B, const float* xl, const float* xh, const float* const* lo_in,
                   const float* const* hi_in, float* const* lo_out, float* const* hi_out,
                   const int32_t* idx_all, const int32_t* idx_meta, int do_crown, int per_domain,
                   int Q, const float* spec_rows, const float* spec_acc, float* lb_out,
                   float* A_out, float* acc_out, uint64_t* seed_rows, void* work,
                   int64_t work_bytes, bool premasked, vc_stream_t stream) {
  if (premasked && (!do_crown || !per_domain || idx_all)) return VC_ERR_ARG;
  TGeom G;
  int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  if (!frag || !bias_cat || !xl || !xh || !lo_in || !hi_in || B < 0) return VC_ERR_ARG;
  if (Q < 0 || Q > TQMAX) return VC_ERR_UNSUPPORTED;
  if (Q > 0 && (!spec_rows || !spec_acc || !lb_out)) return VC_ERR_ARG;
  if (idx_all && !idx_meta) return VC_ERR_ARG;
  // row offsets are int32 (up to 2 x 64 rows per domain and layer), and row
  // codes carry the domain in 25 bits
  if (B >= ((int64_t)1 << 24)) return VC_ERR_UNSUPPORTED;
  int maxw = 1;
  for (int l = 1; l <= n_relu; ++l) maxw = G.d[l] > maxw ? G.d[l] : maxw;
  RowsWork w = rows_carve(reinterpret_cast<char*>(work), n_relu, maxw, B);
  if (!work || work_bytes < (int64_t)w.bytes) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  RowsLayers rl{};
  for (int l = 0; l < n_relu; ++l) {
    rl.lo[l] = lo_in[l];
    rl.hi[l] = hi_in[l];
    rl.lo_out[l] = lo_out ? lo_out[l] : nullptr;
    rl.hi_out[l] = hi_out ? hi_out[l] : nullptr;
    if (!rl.lo[l] || !rl.hi[l] || (rl.lo_out[l] == nullptr) != (rl.hi_out[l] == nullptr))
      return VC_ERR_ARG;
  }
  const void* fc = nullptr;
  const void* fs = nullptr;
  switch (G.variant) {
    case 0: fc = crown_rows_fn<0>(); fs = spec_rows_fn<0>(); break;
    case 1: fc = crown_rows_fn<1>(); fs = spec_rows_fn<1>(); break;
    case 2: fc = crown_rows_fn<2>(); fs = spec_rows_fn<2>(); break;
    case 3: fc = crown_rows_fn<3>(); fs = spec_rows_fn<3>(); break;
    case 4: fc = crown_rows_fn<4>(); fs = spec_rows_fn<4>(); break;
    case 5: fc = crown_rows_fn<5>(); fs = spec_rows_fn<5>(); break;
    default: return VC_ERR_UNSUPPORTED;
  }
  const size_t lds = ((size_t)G.nfloats + (size_t)n_relu * FW) * sizeof(float);
  if (lds > 160 * 1024 || !vcm::allow_max_lds(fc) || !vcm::allow_max_lds(fs))
    return VC_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int cus = vcm::cu_count();
  const int per_cu = std::max(1, std::min(2, (int)((160 * 1024) / lds)));
  const dim3 gchain((unsigned)(cus * per_cu)), bchain(RNW * 64);
  const dim3 gdom((unsigned)std::min<int64_t>((B + 3) / 4, 65536)), bdom(256);
  const int nblk = (int)((B + RSCAN - 1) / RSCAN);
  // the mask pass: persistent, 8 domains per workgroup per sweep
  const dim3 gmask((unsigned)std::max<int64_t>(1, std::min<int64_t>((B + 7) / 8, (int64_t)cus * 8)));
  if (do_crown) {
    if (!premasked) {
      hipLaunchKernelGGL(k_rows_union, dim3(1), dim3(64), 0, st, G, idx_all, idx_meta, w.umask);
      if (n_relu <= 8)
        hipLaunchKernelGGL(k_rows_mask<8>, gmask, bdom, 0, st, G, B, rl, per_domain,
                           idx_all ? 0 : 1, w.masks, w.umask);
      else
        hipLaunchKernelGGL(k_rows_mask<MAXL>, gmask, bdom, 0, st, G, B, rl, per_domain,
                           idx_all ? 0 : 1, w.masks, w.umask);
    }
    hipLaunchKernelGGL(k_rows_scan1, dim3((unsigned)nblk, (unsigned)n_relu), dim3(RSCAN), 0, st,
                       w.masks, w.umask, B, w.off, w.bsum, nblk);
    hipLaunchKernelGGL(k_rows_scan2, dim3((unsigned)n_relu), dim3(1024), 0, st, w.bsum, nblk,
                       w.tot, reinterpret_cast<unsigned long long*>(seed_rows));
  }
  // layer 0's rows; every later layer's are written by the previous cut
  if (do_crown)
    hipLaunchKernelGGL(k_rows_write, gdom, bdom, 0, st, B, 0, w.masks, w.off, w.bsum, nblk,
                       w.rows);
  const dim3 gcut((unsigned)std::min<int64_t>((B + 7) / 8, 65536));
  for (int L = 0; L < n_relu; ++L) {
    if (do_crown) {
      void* args[] = {&G, (void*)&frag, (void*)&bias_cat, &B, (void*)&xl, (void*)&xh, &L,
                      (void*)&w.rows, (void*)&w.tot, (void*)&w.slp, (void*)&w.slb};
      if (hipLaunchKernel(fc, gchain, bchain, args, lds, st) != hipSuccess) return VC_ERR_LAUNCH;
    }
    const int wnext = do_crown && L + 1 < n_relu ? 1 : 0;
    hipLaunchKernelGGL(k_rows_cut, gcut, bdom, 0, st, G, B, L, rl,
                       do_crown ? w.masks : (const uint64_t*)nullptr, w.off, w.bsum, nblk,
                       w.slb, w.slp, wnext, w.rows);
  }
  VC_LAUNCH_CHECK();
  if (Q > 0) {
    void* args[] = {&G, (void*)&frag, (void*)&bias_cat, &B, (void*)&xl, (void*)&xh, &Q,
                    (void*)&spec_rows, (void*)&spec_acc, (void*)&w.slp, (void*)&lb_out,
                    (void*)&A_out, (void*)&acc_out};
    if (hipLaunchKernel(fs, gchain, bchain, args, lds, st) != hipSuccess) return VC_ERR_LAUNCH;
  }
  return VC_OK;
}

}  // namespace

extern "C" int vc_mlp_crown_rows(const int32_t* dims, int n_relu, const float* frag,
                                 const float* bias_cat, int64_t B, const float* xl,
                                 const float* xh, const float* const* lo_in,
                                 const float* const* hi_in, float* const* lo_out,
                                 float* const* hi_out, const int32_t* idx_all,
                                 const int32_t* idx_meta, int do_crown, int per_domain, int Q,
                                 const float* spec_rows, const float* spec_acc, float* lb_out,
                                 float* A_out, float* acc_out, uint64_t* seed_rows, void* work,
                                 int64_t work_bytes, vc_stream_t stream) {
  return crown_rows_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_in, hi_in, lo_out, hi_out,
                        idx_all, idx_meta, do_crown, per_domain, Q, spec_rows, spec_acc, lb_out,
                        A_out, acc_out, seed_rows, work, work_bytes, false, stream);
}

// ------------------------------------------- CROWN without allocation
// vc_mlp_tiled_crown_noalloc keeps the union of unstable neurons (flags,
// index lists, counts) and the domain queue's counter in `scratch`, one copy
// per GPU for the life of the process.  Host code never uses the array's
// name as an address: each device's address comes from hipGetSymbolAddress
// with that device current, once, and is kept in g_scratch_dev.
namespace {
constexpr int kScratchNeurons = MAXL * FW;                 // union flags and indices
constexpr size_t kScratchFlags = 0;                        // uint8 [kScratchNeurons]
constexpr size_t kScratchIdx = kScratchNeurons;            // int32 [kScratchNeurons]
constexpr size_t kScratchMeta = kScratchIdx + 4 * kScratchNeurons;  // int32 [2 MAXL]
constexpr size_t kScratchQueue = kScratchMeta + 4 * 2 * MAXL;       // int32 [2]
constexpr size_t kScratchBytes = 8192;
static_assert(kScratchQueue + 8 <= kScratchBytes, "scratch layout");
static_assert(kScratchIdx % 4 == 0 && kScratchMeta % 4 == 0 && kScratchQueue % 4 == 0,
              "scratch alignment");
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
unsigned char* g_scratch_dev[kMaxDevices] = {};

// The device address of `scratch` on the GPU that runs `stream`, looked up
// once per device with that device current.
int scratch_on(hipStream_t stream, unsigned char** out) {
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return VC_ERR_ARG;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return VC_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) return VC_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return VC_ERR_LAUNCH;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return VC_ERR_LAUNCH;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return VC_ERR_LAUNCH;
    if (e != hipSuccess || !p) return VC_ERR_LAUNCH;
    g_scratch_dev[dev] = static_cast<unsigned char*>(p);
  }
  *out = g_scratch_dev[dev];
  return VC_OK;
}
}  // namespace

extern "C" int vc_mlp_tiled_crown_noalloc(const int32_t* dims, int n_relu, const float* frag,
                                          const float* bias_cat, int64_t B, const float* xl,
                                          const float* xh, const float* const* lo_in,
                                          const float* const* hi_in, float* const* lo_out,
                                          float* const* hi_out, int do_crown, int per_domain,
                                          int Q, const float* spec_rows, const float* spec_acc,
                                          float* lb_out, float* A_out, float* acc_out,
                                          vc_stream_t stream) {
  if (!dims || n_relu < 1 || n_relu > MAXL) return VC_ERR_UNSUPPORTED;
  int32_t widths[MAXL];
  int total = 0;
  for (int l = 0; l < n_relu; ++l) {
    widths[l] = dims[l + 1];
    if (widths[l] <= 0) return VC_ERR_ARG;
    total += widths[l];
  }
  // the union lists live in `scratch`: nets beyond its size are refused
  if (total > kScratchNeurons) return VC_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  unsigned char* sp = nullptr;
  int rc = scratch_on(st, &sp);
  if (rc != VC_OK) return rc;
  uint8_t* flags = sp + kScratchFlags;
  int32_t* idx = reinterpret_cast<int32_t*>(sp + kScratchIdx);
  int32_t* meta = reinterpret_cast<int32_t*>(sp + kScratchMeta);
  int32_t* queue = reinterpret_cast<int32_t*>(sp + kScratchQueue);
  if (do_crown && B > 0) {
    // the flags are cleared by a fill kernel inside, the lists written whole
    rc = vc_unstable_union_layers(lo_in, hi_in, widths, n_relu, B, flags, stream);
    if (rc != VC_OK) return rc;
    rc = vc_union_compact(flags, widths, n_relu, idx, meta, stream);
    if (rc != VC_OK) return rc;
  }
  // the queue counter is reset by a kernel before the CROWN launch
  return vc_mlp_tiled_crown(dims, n_relu, frag, bias_cat, B, xl, xh, lo_in, hi_in, lo_out,
                            hi_out, do_crown ? idx : nullptr, do_crown ? meta : nullptr,
                            do_crown, per_domain, Q, spec_rows, spec_acc, lb_out, A_out,
                            acc_out, nullptr, queue, stream);
}

namespace {
// One alpha-CROWN iteration's launch, prepared once per batch: the kernel
// (4 wavefronts per domain for batches that fit at once, else one), its
// shape and the per-layer pointers.
struct AlphaLaunch {
  TGeom G;
  TAlphaArgs aa;
  const void* fn;
  int quad, D;
  dim3 grid, block;
  size_t lds;
};

int alpha_prepare(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                  int64_t B, const float* xl, const float* xh, const float* const* lo,
                  const float* const* hi, float* const* alpha, float* const* exp_avg,
                  float* const* exp_avg_sq, float* const* grad, int Q, const float* spec_rows,
                  const float* spec_acc, const float* lb_out, AlphaLaunch& L,
                  int cu_budget = 0) {
  TGeom& G = L.G;
  int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  if (Q < 1 || Q > 16) return VC_ERR_UNSUPPORTED;
  if (!frag || !bias_cat || !xl || !xh || !lo || !hi || !alpha || !exp_avg || !exp_avg_sq ||
      !spec_rows || !spec_acc || !lb_out || B < 0)
    return VC_ERR_ARG;
  for (int l = 0; l < MAXL; ++l) {
    const bool in = l < n_relu;
    L.aa.lo[l] = in ? lo[l] : nullptr;
    L.aa.hi[l] = in ? hi[l] : nullptr;
    L.aa.alpha[l] = in ? alpha[l] : nullptr;
    L.aa.m1[l] = in ? exp_avg[l] : nullptr;
    L.aa.m2[l] = in ? exp_avg_sq[l] : nullptr;
    L.aa.grad[l] = (in && grad) ? grad[l] : nullptr;
    if (in && (!L.aa.lo[l] || !L.aa.hi[l] || !L.aa.alpha[l] || !L.aa.m1[l] || !L.aa.m2[l]))
      return VC_ERR_ARG;
    if (in && grad && !L.aa.grad[l]) return VC_ERR_ARG;
  }
  const size_t fixed = ((size_t)G.nfloats + (size_t)n_relu * FW) * sizeof(float);
  // small batches: every domain in flight at once, MT wavefronts each, on
  // at most cu_budget compute units' worth of workgroups when given
  const int cus = cu_budget > 0 ? std::min(cu_budget, vcm::cu_count()) : vcm::cu_count();
  const size_t per = (size_t)alpha_quad_floats(n_relu, G.KS, Q, G.MT) * sizeof(float);
  const int fit = fixed + per <= 160 * 1024 ? (int)((160 * 1024 - fixed) / per) : 0;
  const int D = (int)std::min<int64_t>(std::min(AQD, fit), (B + cus - 1) / cus);
  L.quad = 0;
  if (B >= 1 && B <= (int64_t)cus * AQD && D >= 1) {
    const void* fq = nullptr;
    switch (G.variant) {
      case 0: fq = alpha_quad_fn<0>(n_relu, D); break;
      case 1: fq = alpha_quad_fn<1>(n_relu, D); break;
      case 2: fq = alpha_quad_fn<2>(n_relu, D); break;
      case 3: fq = alpha_quad_fn<3>(n_relu, D); break;
      case 4: fq = alpha_quad_fn<4>(n_relu, D); break;
      case 5: fq = alpha_quad_fn<5>(n_relu, D); break;
      default: return VC_ERR_UNSUPPORTED;
    }
    if (vcm::allow_max_lds(fq)) {
      L.fn = fq;
      L.quad = 1;
      L.D = D;
      L.lds = fixed + (size_t)D * per;
      L.grid = dim3((unsigned)((B + D - 1) / D));
      L.block = dim3((unsigned)(D * G.MT * 64));
      return VC_OK;
    }
  }
  const size_t wsz = (size_t)alpha_wsz(n_relu, G.KS, Q) * sizeof(float);
  const int nw = fixed + wsz <= 160 * 1024
                     ? (int)std::min<size_t>(ANW, (160 * 1024 - fixed) / wsz)
                     : 0;
  if (nw < 1) return VC_ERR_UNSUPPORTED;
  L.lds = fixed + nw * wsz;
  switch (G.variant) {
    case 0: L.fn = alpha_fn<0>(); break;
    case 1: L.fn = alpha_fn<1>(); break;
    case 2: L.fn = alpha_fn<2>(); break;
    case 3: L.fn = alpha_fn<3>(); break;
    case 4: L.fn = alpha_fn<4>(); break;
    case 5: L.fn = alpha_fn<5>(); break;
    default: return VC_ERR_UNSUPPORTED;
  }
  if (!vcm::allow_max_lds(L.fn)) return VC_ERR_UNSUPPORTED;
  L.D = 1;
  L.grid = dim3(vcm::persistent_grid(B, L.lds, nw));
  L.block = dim3(nw * 64);
  return VC_OK;
}

// ac.n iterations (the quad kernel; the one-wavefront kernel takes one);
// iteration t's bounds to lb_out + t B Q.
int alpha_launch(const AlphaLaunch& L, const float* frag, const float* bias_cat, int64_t B,
                 const float* xl, const float* xh, int Q, const float* spec_rows,
                 const float* spec_acc, float* lb_out, const AdamChunk& ac, int init,
                 const float* ctl, hipStream_t st) {
  if (ac.n < 1 || ac.n > (L.quad ? VC_ALPHA_CHUNK : 1)) return VC_ERR_ARG;
  TGeom G = L.G;
  TAlphaArgs aa = L.aa;
  int D = L.D;
  AdamChunk acc = ac;
  AdamConst a1 = ac.c[0];
  void* args[] = {&G,
                  (void*)&frag,
                  (void*)&bias_cat,
                  &B,
                  (void*)&xl,
                  (void*)&xh,
                  &aa,
                  &Q,
                  (void*)&spec_rows,
                  (void*)&spec_acc,
                  (void*)&lb_out,
                  L.quad ? (void*)&acc : (void*)&a1,
                  &init,
                  (void*)&ctl,
                  &D};
  if (hipLaunchKernel(L.fn, L.grid, L.block, args, L.lds, st) != hipSuccess) return VC_ERR_LAUNCH;
  return VC_OK;
}
}  // namespace

extern "C" int vc_mlp_tiled_alpha_iter(const int32_t* dims, int n_relu, const float* frag,
                                       const float* bias_cat, int64_t B, const float* xl,
                                       const float* xh, const float* const* lo,
                                       const float* const* hi, float* const* alpha,
                                       float* const* exp_avg, float* const* exp_avg_sq,
                                       float* const* grad, int Q, const float* spec_rows,
                                       const float* spec_acc, float* lb_out, double b1, double b2,
                                       double eps, double step_size, double bc2_sqrt, int init,
                                       const float* ctl, vc_stream_t stream) {
  AlphaLaunch L;
  int rc = alpha_prepare(dims, n_relu, frag, bias_cat, B, xl, xh, lo, hi, alpha, exp_avg,
                         exp_avg_sq, grad, Q, spec_rows, spec_acc, lb_out, L);
  if (rc != VC_OK) return rc;
  if (B == 0) return VC_OK;
  AdamChunk ac;
  ac.n = 1;
  ac.c[0] = adam_const(b1, b2, eps, step_size, bc2_sqrt);
  return alpha_launch(L, frag, bias_cat, B, xl, xh, Q, spec_rows, spec_acc, lb_out, ac, init, ctl,
                      (hipStream_t)stream);
}

namespace {
__global__ void k_alpha_ctl_init(float* ctl) {
  if (threadIdx.x == 0) {
    ctl[0] = -INFINITY;
    ctl[1] = 0.f;
    ctl[2] = 0.f;
    ctl[3] = 0.f;
  }
}
}  // namespace

namespace vcm {
int alpha_run(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
              int64_t B, const float* xl, const float* xh, const float* const* lo,
              const float* const* hi, float* const* alpha, float* const* exp_avg,
              float* const* exp_avg_sq, int Q, const float* spec_rows, const float* spec_acc,
              float* lb_out, float* best, double b1, double b2, double eps, double lr,
              double lr_decay, int n_iters, double early_stop_eps, float* ctl,
              int32_t* stop_host, int cu_budget, vc_stream_t stream) {
  if (!best || !ctl || n_iters < 1) return VC_ERR_ARG;
  if (B < 0) return VC_ERR_ARG;
  AlphaLaunch L;
  int rc = alpha_prepare(dims, n_relu, frag, bias_cat, B, xl, xh, lo, hi, alpha, exp_avg,
                         exp_avg_sq, nullptr, Q, spec_rows, spec_acc, lb_out, L, cu_budget);
  if (rc != VC_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_alpha_ctl_init, dim3(1), dim3(64), 0, st, ctl);
  VC_LAUNCH_CHECK();
  if (B == 0) return VC_OK;
  // the schedule of torch Adam under the reference's loop: step sizes
  // lr_t / (1 - b1^t) and (1 - b2^t)^0.5, lr decayed after every iteration.
  // Once the device has stopped (and said so in *stop_host), the remaining
  // iterations, which would do nothing, are not enqueued.
  // The small-batch kernel runs up to VC_ALPHA_CHUNK iterations per launch
  // on its LDS state; the control replays the stop tests over them in
  // order and discards the ones after a stop.
  // With stop_host, one chunk is kept in flight ahead of the control the
  // host has seen: before chunk k the host waits (bounded) for chunk k - 2's
  // control, so a stop costs at most one enqueued chunk that does nothing.
  volatile int32_t* sh = stop_host;
  const int K = L.quad ? VC_ALPHA_CHUNK : 1;
  double cur_lr = lr;
  for (int it0 = 0, k = 0; it0 < n_iters; it0 += K, ++k) {
    if (sh && k >= 2)
      for (long spin = 0; spin < (1l << 24) && sh[0] == 0 && sh[1] < it0 - K; ++spin) {
      }
    if (sh && sh[0] != 0) break;
    AdamChunk ac;
    ac.n = std::min(K, n_iters - it0);
    for (int t = 0; t < ac.n; ++t) {
      const double step = (double)(it0 + t + 1);
      ac.c[t] = adam_const(b1, b2, eps, cur_lr / (1.0 - pow(b1, step)),
                           pow(1.0 - pow(b2, step), 0.5));
      cur_lr *= lr_decay;
    }
    rc = alpha_launch(L, frag, bias_cat, B, xl, xh, Q, spec_rows, spec_acc, lb_out, ac,
                      it0 == 0 ? 1 : 0, ctl, st);
    if (rc != VC_OK) return rc;
    rc = alpha_control_chunk(best, lb_out, B * (int64_t)Q, it0, ac.n, early_stop_eps, ctl,
                             stop_host, st);
    if (rc != VC_OK) return rc;
  }
  return VC_OK;
}
}  // namespace vcm

extern "C" int vc_mlp_tiled_alpha_run(const int32_t* dims, int n_relu, const float* frag,
                                      const float* bias_cat, int64_t B, const float* xl,
                                      const float* xh, const float* const* lo,
                                      const float* const* hi, float* const* alpha,
                                      float* const* exp_avg, float* const* exp_avg_sq, int Q,
                                      const float* spec_rows, const float* spec_acc,
                                      float* lb_out, float* best, double b1, double b2,
                                      double eps, double lr, double lr_decay, int n_iters,
                                      double early_stop_eps, float* ctl, int32_t* stop_host,
                                      vc_stream_t stream) {
  return vcm::alpha_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo, hi, alpha, exp_avg,
                        exp_avg_sq, Q, spec_rows, spec_acc, lb_out, best, b1, b2, eps, lr,
                        lr_decay, n_iters, early_stop_eps, ctl, stop_host, 0, stream);
}

namespace {
int zono_bounds_run(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                    int64_t B, const float* xl, const float* xh, float* const* lo_out,
                    float* const* hi_out, uint8_t* overflow, int32_t* queue, ZonoMasks zm,
                    vc_stream_t stream) {
  TGeom G;
  int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  if (!frag || !bias_cat || !xl || !xh || !lo_out || !hi_out || !overflow || B < 0)
    return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  TZonoArgs za;
  for (int l = 0; l < MAXL; ++l) {
    za.lo[l] = l < n_relu ? lo_out[l] : nullptr;
    za.hi[l] = l < n_relu ? hi_out[l] : nullptr;
    if (l < n_relu && (!za.lo[l] || !za.hi[l])) return VC_ERR_ARG;
  }
  const int mr = zono_rem(G);
  // the kernel's static LDS (the mask pass's union staging) comes first
  const size_t base =
      ((size_t)G.nfloats + (size_t)n_relu * FW + (size_t)zono_rem_floats(n_relu, G.MT, mr)) *
          sizeof(float) +
      sizeof(unsigned long long) * (ZNW + 1) * MAXL;
  const size_t scr = (size_t)ZSCR * sizeof(float);
  if (base + scr > 160 * 1024) return VC_ERR_UNSUPPORTED;
  // small batches: fewer wavefronts per workgroup, so that the domains
  // spread over every CU (one wavefront per SIMD) instead of sharing the
  // matrix cores of a few (each domain's arithmetic is the same)
  const int64_t per_cu_dom = (B + vcm::cu_count() - 1) / vcm::cu_count();
  const int nw = (int)std::min<int64_t>(std::min<size_t>(ZNW, (160 * 1024 - base) / scr),
                                        std::max<int64_t>(1, per_cu_dom));
  const size_t lds = base + (size_t)nw * scr;
  const void* fn = nullptr;
  switch (G.variant * 4 + mr) {
    case 0: fn = zono_fn<0, 0>(); break;
    case 4: fn = zono_fn<1, 0>(); break;
    case 8: fn = zono_fn<2, 0>(); break;
    case 12: fn = zono_fn<3, 0>(); break;
    case 13: fn = zono_fn<3, 1>(); break;
    case 14: fn = zono_fn<3, 2>(); break;
    case 16: fn = zono_fn<4, 0>(); break;
    case 20: fn = zono_fn<5, 0>(); break;
    default: return VC_ERR_UNSUPPORTED;
  }
  if (!vcm::allow_max_lds(fn)) return VC_ERR_UNSUPPORTED;
  const dim3 grid(vcm::persistent_grid(B, lds, nw)), block(nw * 64);
  hipStream_t st = (hipStream_t)stream;
  if (queue || zm.umask || zm.ovf_count || zm.clear_count)
    hipLaunchKernelGGL(k_zono_init, dim3(1), dim3(64), 0, st, queue, zm.umask, n_relu,
                       zm.ovf_count, zm.clear_count);
#define VC_TZONO_CASE(V, MR)                                                                 \
  case V * 4 + MR:                                                                           \
    hipLaunchKernelGGL((k_zono_tiled<kVariants[V].MT, kVariants[V].KS,                       \
                                     kVariants[V].brow != 0, MR>),                           \
                       grid, block, lds - sizeof(unsigned long long) * (ZNW + 1) * MAXL, st, \
                       G, frag, bias_cat, B, xl, xh, za, overflow, queue, zm);               \
    break;
  switch (G.variant * 4 + mr) {
    VC_TZONO_CASE(0, 0)
    VC_TZONO_CASE(1, 0)
    VC_TZONO_CASE(2, 0)
    VC_TZONO_CASE(3, 0)
    VC_TZONO_CASE(3, 1)
    VC_TZONO_CASE(3, 2)
    VC_TZONO_CASE(4, 0)
    VC_TZONO_CASE(5, 0)
    default: return VC_ERR_UNSUPPORTED;
  }
#undef VC_TZONO_CASE
  VC_LAUNCH_CHECK();
  return VC_OK;
}

int zono_wide_run(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                  int64_t B, const float* xl, const float* xh, float* const* lo_out,
                  float* const* hi_out, uint8_t* overflow, const int64_t* list,
                  const int64_t* n_list, ZonoMasks zm, vc_stream_t stream) {
  TGeom G;
  int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  if (!frag || !bias_cat || !xl || !xh || !lo_out || !hi_out || !overflow || !list ||
      !n_list || B < 0)
    return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  TZonoArgs za;
  for (int l = 0; l < MAXL; ++l) {
    za.lo[l] = l < n_relu ? lo_out[l] : nullptr;
    za.hi[l] = l < n_relu ? hi_out[l] : nullptr;
    if (l < n_relu && (!za.lo[l] || !za.hi[l])) return VC_ERR_ARG;
  }
  const size_t lds = ((size_t)G.nfloats + (size_t)n_relu * FW) * sizeof(float) +
                     (size_t)ZWW * FW * sizeof(double) + (size_t)3 * FW * sizeof(float) +
                     sizeof(unsigned long long);
  if (lds > 160 * 1024 - 2048) return VC_ERR_UNSUPPORTED;
  const void* fn = nullptr;
  switch (G.variant) {
    case 0: fn = zono_wide_fn<0>(); break;
    case 1: fn = zono_wide_fn<1>(); break;
    case 2: fn = zono_wide_fn<2>(); break;
    case 3: fn = zono_wide_fn<3>(); break;
    case 4: fn = zono_wide_fn<4>(); break;
    case 5: fn = zono_wide_fn<5>(); break;
    default: return VC_ERR_UNSUPPORTED;
  }
  if (!vcm::allow_max_lds(fn)) return VC_ERR_UNSUPPORTED;
  int64_t gw = vcm::cu_count();
  if (gw > B) gw = B;
  hipStream_t st = (hipStream_t)stream;
#define VC_TWIDE_CASE(V)                                                                     \
  case V:                                                                                    \
    hipLaunchKernelGGL((k_zono_wide_tiled<kVariants[V].MT, kVariants[V].KS,                  \
                                          kVariants[V].brow != 0>),                          \
                       dim3((unsigned)gw), dim3(ZWW * 64), lds, st, G, frag, bias_cat, B, xl, \
                       xh, za, overflow, list, n_list, zm);                                  \
    break;
  switch (G.variant) {
    VC_TWIDE_CASE(0)
    VC_TWIDE_CASE(1)
    VC_TWIDE_CASE(2)
    VC_TWIDE_CASE(3)
    VC_TWIDE_CASE(4)
    VC_TWIDE_CASE(5)
    default: return VC_ERR_UNSUPPORTED;
  }
#undef VC_TWIDE_CASE
  VC_LAUNCH_CHECK();
  return VC_OK;
}
}  // namespace

extern "C" int vc_mlp_tiled_zono_bounds(const int32_t* dims, int n_relu, const float* frag,
                                        const float* bias_cat, int64_t B, const float* xl,
                                        const float* xh, float* const* lo_out,
                                        float* const* hi_out, uint8_t* overflow,
                                        int32_t* queue, vc_stream_t stream) {
  return zono_bounds_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_out, hi_out, overflow,
                         queue, ZonoMasks{nullptr, nullptr, nullptr, nullptr, nullptr}, stream);
}

extern "C" int vc_mlp_tiled_zono_wide(const int32_t* dims, int n_relu, const float* frag,
                                      const float* bias_cat, int64_t B, const float* xl,
                                      const float* xh, float* const* lo_out,
                                      float* const* hi_out, uint8_t* overflow,
                                      const int64_t* list, const int64_t* n_list,
                                      vc_stream_t stream) {
  return zono_wide_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_out, hi_out, overflow, list,
                       n_list, ZonoMasks{nullptr, nullptr, nullptr, nullptr, nullptr}, stream);
}

// ------------------------------------- the round's masked bound phase
namespace vcm {

namespace {
// The seed masks and the union slots inside a vc_mlp_crown_rows workspace
// for B domains (rows_carve's first two regions).
bool rows_mask_slots(const int32_t* dims, int n_relu, int64_t B, void* rows_work,
                     ZonoMasks& zm) {
  TGeom G;
  if (!rows_work || tiled_geom(dims, n_relu, G) != VC_OK) return false;
  int maxw = 1;
  for (int l = 1; l <= n_relu; ++l) maxw = G.d[l] > maxw ? G.d[l] : maxw;
  const RowsWork w = rows_carve(reinterpret_cast<char*>(rows_work), n_relu, maxw, B);
  zm.masks = w.masks;
  zm.umask = w.umask;
  return true;
}
}  // namespace

int zono_bounds_masked(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                       int64_t B, const float* xl, const float* xh, float* const* lo_out,
                       float* const* hi_out, uint8_t* overflow, int32_t* queue, void* rows_work,
                       int64_t* ovf_list, int64_t* ovf_count, int64_t* clear_count,
                       hipStream_t st) {
  ZonoMasks zm{nullptr, nullptr, nullptr, nullptr,
               reinterpret_cast<unsigned long long*>(clear_count)};
  if (!rows_mask_slots(dims, n_relu, B, rows_work, zm)) return VC_ERR_ARG;
  if ((ovf_list == nullptr) != (ovf_count == nullptr) || n_relu > MAXL) return VC_ERR_ARG;
  zm.ovf_list = ovf_list;
  zm.ovf_count = reinterpret_cast<unsigned long long*>(ovf_count);
  return zono_bounds_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_out, hi_out, overflow,
                         queue, zm, st);
}

int zono_bounds_listed(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                       int64_t B, const float* xl, const float* xh, float* const* lo_out,
                       float* const* hi_out, uint8_t* overflow, int32_t* queue,
                       int64_t* ovf_list, int64_t* ovf_count, unsigned long long* umask,
                       int64_t* clear_count, hipStream_t st) {
  if (!ovf_list || !ovf_count || n_relu > MAXL) return VC_ERR_ARG;
  ZonoMasks zm{nullptr, umask, ovf_list, reinterpret_cast<unsigned long long*>(ovf_count),
               reinterpret_cast<unsigned long long*>(clear_count)};
  return zono_bounds_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_out, hi_out, overflow,
                         queue, zm, st);
}

int zono_wide_union(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                    int64_t B, const float* xl, const float* xh, float* const* lo_out,
                    float* const* hi_out, uint8_t* overflow, const int64_t* list,
                    const int64_t* n_list, unsigned long long* umask, hipStream_t st) {
  return zono_wide_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_out, hi_out, overflow, list,
                       n_list, ZonoMasks{nullptr, umask, nullptr, nullptr, nullptr}, st);
}

namespace {
// vc_union_compact's index lists from the union as bit masks: one
// wavefront per layer, ascending neuron order.
__global__ void k_union_lists(const unsigned long long* __restrict__ umask, TGeom G,
                              int32_t* __restrict__ idx, int32_t* __restrict__ meta) {
  const int L = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = G.n;
  if (L >= n) return;
  int off = 0;
  for (int k = 0; k < L; ++k) off += __popcll(umask[k]);
  const uint64_t m = umask[L];
  if ((m >> lane) & 1ull) idx[off + __popcll(m & ((1ull << lane) - 1ull))] = lane;
  if (lane == 0) {
    meta[L] = __popcll(m);
    meta[n + L] = off;
  }
}
}  // namespace

int union_lists(const int32_t* dims, int n_relu, const unsigned long long* umask, int32_t* idx,
                int32_t* meta, hipStream_t st) {
  TGeom G;
  const int rc = tiled_geom(dims, n_relu, G);
  if (rc != VC_OK) return rc;
  hipLaunchKernelGGL(k_union_lists, dim3(1), dim3(64 * n_relu), 0, st, umask, G, idx, meta);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

int zono_wide_masked(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                     int64_t B, const float* xl, const float* xh, float* const* lo_out,
                     float* const* hi_out, uint8_t* overflow, const int64_t* list,
                     const int64_t* n_list, void* rows_work, hipStream_t st) {
  ZonoMasks zm{nullptr, nullptr, nullptr, nullptr, nullptr};
  if (!rows_mask_slots(dims, n_relu, B, rows_work, zm)) return VC_ERR_ARG;
  return zono_wide_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_out, hi_out, overflow, list,
                       n_list, zm, st);
}

int crown_rows_premasked(const int32_t* dims, int n_relu, const float* frag,
                         const float* bias_cat, int64_t B, const float* xl, const float* xh,
                         const float* const* lo_in, const float* const* hi_in, int Q,
                         const float* spec_rows, const float* spec_acc, float* lb_out,
                         float* A_out, float* acc_out, uint64_t* seed_rows, void* work,
                         int64_t work_bytes, hipStream_t st) {
  return crown_rows_run(dims, n_relu, frag, bias_cat, B, xl, xh, lo_in, hi_in, nullptr, nullptr,
                        nullptr, nullptr, 1, 1, Q, spec_rows, spec_acc, lb_out, A_out, acc_out,
                        seed_rows, work, work_bytes, true, (vc_stream_t)st);
}

}  // namespace vcm
