// Whole-network kernels for narrow fc/ReLU chains (every width <= 64, up to
// 16 ReLU layers; the 5-50x6-5 ACAS-Xu shape): one wavefront per domain,
// persistent workgroups, all weights in LDS.
//
// Register layout.  A 64-wide activation block is held like the D operand
// of v_mfma_f32_16x16x4_f32: lane l = 16 g + r holds, for each 16-row
// M-tile t, the four values of neurons 16 t + 4 g + i (i = 0..3) of column r
// of a 16-column N-tile.  The MFMA B operand takes the lane's value at
// K-index g, so feeding register (t, i) as B contracts neuron 16 t + 4 g + i
// at that K-step: a layer's output registers are the next layer's B
// operand with no data movement, provided the weight (A operand) fragments
// use the same K order.  Fragment (mt, t, i) holds, for lane (g, r),
// A[16 mt + r][16 t + 4 g + i] and is stored as 64 contiguous floats.
//
//   vc_mlp_zono_bounds: zonotope forward (verify_zono_bnb.py:3079-3211):
//     columns of one N-tile set = [centre | input generators | new
//     generators], the centre carried as column 0 through the MFMAs.
//   vc_mlp_crown: CROWN intermediate bounds (verify_zono_bnb.py:4077-4147)
//     and the spec backward + concretization (verify_zono_bnb.py:4270-4453,
//     5117-5134): seeded rows chained through relaxation + fc steps in
//     registers, intersected per domain, slopes kept in LDS.
#include "vc_common.h"
#include "vc_mlp_common.h"
#include "vc_relax.h"

namespace {

using vcm::cu_count;
using vcm::FW;
using vcm::ks_count;
using vcm::MAXL;
constexpr int NWAVE = 8;   // waves (domains in flight) per workgroup
constexpr int NPAR = 4;    // row N-tiles chained together per wave
constexpr int ZNT_NARROW = 8;   // 128 generator columns, 8 waves per workgroup

struct Net {
  int n;                 // relu layers
  int d[MAXL + 2];       // d[0] = inputs, d[l+1] = width of relu l
  int foff[MAXL + 1];    // fragment offset of fc_l (in fragments)
  int boff[MAXL + 1];    // bias offset of fc_l
  int nfrag, nbias;
};

// ----------------------------------------------------------------- packing
// bwd: A[m][k] = W[k][m] (W: d_out x d_in), M = d_in, K = d_out
// fwd: A[m][k] = W[m][k],                 M = d_out, K = d_in
__global__ void k_pack(const float* W, int d_out, int d_in, int bwd, float* frag) {
  const int M = bwd ? d_in : d_out, K = bwd ? d_out : d_in;
  const int MT = (M + 15) / 16, KS = ks_count(K);
  const int total = MT * KS * 64;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const int lane = e & 63, f = e >> 6;
    const int mt = f / KS, ks = f % KS;
    const int t = ks >> 2, i = ks & 3;
    const int g = lane >> 4, r = lane & 15;
    const int m = 16 * mt + r, k = 16 * t + 4 * g + i;
    float v = 0.f;
    if (m < M && k < K) v = bwd ? W[k * d_in + m] : W[m * d_in + k];
    frag[e] = v;
  }
}

// Stage the packed fragments (nfrag * 64 floats, 16-byte aligned) and the
// biases into LDS with 16-byte loads, several in flight per thread.
__device__ __forceinline__ void stage_weights(float* sfrag, float* sbias, const float* gfrag,
                                              const float* gbias, int nfrag, int nbias) {
  vcm::stage_float4(sfrag, gfrag, nfrag * 16);
  for (int k = threadIdx.x; k < nbias; k += blockDim.x) sbias[k] = gbias[k];
  __syncthreads();
}

__device__ __forceinline__ float group_bcast(float v, int lane) {
  return __shfl(v, lane & 48, 64);  // value of lane 16 g (r = 0) of the group
}

// Sum over the 4 lane groups (same r), compensated.
__device__ __forceinline__ float group_sum4(float s, float c) {
  for (int o = 16; o < 64; o <<= 1) {
    const float so = __shfl_xor(s, o, 64), co = __shfl_xor(c, o, 64);
    two_sum_acc(s, c, so);
    c += co;
  }
  return s + c;
}

// --------------------------------------------------------- zonotope kernel
struct ZonoArgs {
  float* lo[MAXL];
  float* hi[MAXL];
};

// ZNT: generator capacity in 16-column tiles (centre included).  NW: waves
// per workgroup.  only_flagged: process only domains whose overflow flag
// is set (the wide second pass); every processed domain gets its flag
// rewritten (1 = still does not fit).
template <int ZNT, int NW>
__global__ __launch_bounds__(NW * 64) void k_mlp_zono(Net net, const float* __restrict__ gfrag,
                                                      const float* __restrict__ gbias, int64_t B,
                                                      const float* __restrict__ xl,
                                                      const float* __restrict__ xh,
                                                      ZonoArgs out, int32_t* overflow,
                                                      int only_flagged) {
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + net.nfrag * 64;
  stage_weights(sfrag, sbias, gfrag, gbias, net.nfrag, net.nbias);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int d0 = net.d[0];

  for (int64_t dom = (int64_t)blockIdx.x * NW + wv; dom < B; dom += (int64_t)gridDim.x * NW) {
    if (only_flagged && overflow[dom] == 0) continue;
    v4f G[ZNT][4];
    // initial block: rows = input dims, col 0 = centre, col 1 + j = radius j
#pragma unroll
    for (int nt = 0; nt < ZNT; ++nt)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * t + 4 * g + i, col = 16 * nt + r;
          float v = 0.f;
          if (row < d0) {
            const float l = xl[dom * d0 + row], h = xh[dom * d0 + row];
            if (col == 0) v = (l + h) / 2.f;
            else if (col == 1 + row) v = (h - l) / 2.f;
          }
          G[nt][t][i] = v;
        }
    int Kc = 1 + d0;
    bool ovf = Kc > ZNT * 16;
    for (int l = 0; l < net.n && !ovf; ++l) {
      const int dK = net.d[l], dM = net.d[l + 1];
      const int KS = ks_count(dK), MT = (dM + 15) / 16;
      const int ntu = (Kc + 15) / 16;
      const float* fr = sfrag + net.foff[l] * 64 + lane;
      // fc_l on every used column tile (two tiles at a time, K-step outer
      // so consecutive MFMAs write independent accumulators); column 0
      // also gets the bias
#pragma unroll
      for (int nt0 = 0; nt0 < ZNT; nt0 += 2) {
        if (nt0 < ntu) {
          const bool two = nt0 + 1 < ntu;
          v4f o[2][4];
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) o[p][mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int ks = 4 * t + i;
              if (ks < KS) {
                float a[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) a[mt] = mt < MT ? fr[(mt * KS + ks) * 64] : 0.f;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
                  if (mt < MT) {
                    o[0][mt] = mfma16x16x4(a[mt], G[nt0][t][i], o[0][mt]);
                    if (two) o[1][mt] = mfma16x16x4(a[mt], G[nt0 + 1][t][i], o[1][mt]);
                  }
              }
            }
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            G[nt0][mt] = o[0][mt];
            if (two) G[nt0 + 1][mt] = o[1][mt];
          }
        }
      }
      if (r == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * t + 4 * g + i;
            if (j < dM) G[0][t][i] = G[0][t][i] + sbias[net.boff[l] + j];
          }
      }
      // relu_l: s_j = sum over generator columns of |G|; lo/hi = c -/+ s
      float lam[4][4], mu[4][4];
      uint64_t umask = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          KSum s;
#pragma unroll
          for (int nt = 0; nt < ZNT; ++nt)
            if (nt < ntu && (nt > 0 || r > 0)) s.add(fabsf(G[nt][t][i]));
          float ss = s.s, sc = s.c;
          for (int o = 8; o > 0; o >>= 1) {
            const float so = __shfl_xor(ss, o, 64), co = __shfl_xor(sc, o, 64);
            two_sum_acc(ss, sc, so);
            sc += co;
          }
          const float rad = ss + sc;
          const float c = group_bcast(G[0][t][i], lane);
          const int j = 16 * t + 4 * g + i;
          const float lo = c - rad, hi = c + rad;
          const bool valid = j < dM;
          const bool ust = valid && lo < 0.f && hi > 0.f;
          const bool dead = hi <= 0.f;
          if (valid && r == 0) {
            out.lo[l][dom * dM + j] = lo;
            out.hi[l][dom * dM + j] = hi;
          }
          lam[t][i] = ust ? hi / (hi - lo) : (dead ? 0.f : 1.f);
          mu[t][i] = ust ? (-hi * lo) / (2.f * (hi - lo)) : 0.f;
          const uint64_t bal = __ballot(ust && r == 0);
#pragma unroll
          for (int gg = 0; gg < 4; ++gg)
            if ((bal >> (16 * gg)) & 1ull) umask |= 1ull << (16 * t + 4 * gg + i);
        }
      const int cnt = __popcll(umask);
      if (l == net.n - 1) break;  // the last relu's output is not propagated
      if (Kc + cnt > ZNT * 16) {
        ovf = true;
        break;
      }
      // scale rows by lam (centre: lam c + mu), append one column per
      // unstable neuron at position Kc + rank
#pragma unroll
      for (int nt = 0; nt < ZNT; ++nt)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (nt == 0 && r == 0) {
              G[nt][t][i] = lam[t][i] * G[nt][t][i] + mu[t][i];
            } else {
              G[nt][t][i] = G[nt][t][i] * lam[t][i];
            }
          }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * t + 4 * g + i;
          if ((umask >> j) & 1ull) {
            const int col = Kc + __popcll(umask & ((1ull << j) - 1ull));
            if ((col & 15) == r) {
#pragma unroll
              for (int nt = 0; nt < ZNT; ++nt)
                if (nt == (col >> 4)) G[nt][t][i] = mu[t][i];
            }
          }
        }
      Kc += cnt;
    }
    if (lane == 0) overflow[dom] = ovf ? 1 : 0;
  }
}

// Zonotope bounds of the domains flagged in `overflow`, one workgroup of
// ZC_W waves per domain: wave w holds generator columns [128 w, 128 w + 128)
// (column 0 = centre), so up to ZC_W * 128 columns.  The per-neuron |G|
// sums are reduced across waves through LDS in a fixed order, so every
// wave derives the same lo/hi, lambda, mu and unstable set.
constexpr int ZC_W = 4;
constexpr int ZC_T = 8;  // tiles per wave

__global__ __launch_bounds__(ZC_W * 64) void k_mlp_zono_coop(
    Net net, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, ZonoArgs out, int32_t* overflow) {
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + net.nfrag * 64;
  float* sred = sbias + ((net.nbias + 63) & ~63);  // [ZC_W][2][FW]: (s, c) partials
  float* scen = sred + ZC_W * 2 * FW;              // centre column [FW]
  stage_weights(sfrag, sbias, gfrag, gbias, net.nfrag, net.nbias);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int d0 = net.d[0];
  const int cap = ZC_W * ZC_T * 16;

  // Each workgroup owns a contiguous range of domains; chunks of the range
  // are scanned in parallel and the flagged domains compacted into LDS.
  __shared__ int s_list[ZC_W * 64];
  __shared__ int s_wcnt[ZC_W];
  const int64_t per = (B + gridDim.x - 1) / gridDim.x;
  const int64_t beg = (int64_t)blockIdx.x * per;
  const int64_t end = beg + per < B ? beg + per : B;
  for (int64_t c0 = beg; c0 < end; c0 += ZC_W * 64) {
    const int64_t dsc = c0 + threadIdx.x;
    const bool flagged = dsc < end && overflow[dsc] != 0;
    const uint64_t bal = __ballot(flagged);
    if (lane == 0) s_wcnt[wv] = __popcll(bal);
    __syncthreads();
    int off = 0, tot = 0;
    for (int w2 = 0; w2 < ZC_W; ++w2) {
      if (w2 < wv) off += s_wcnt[w2];
      tot += s_wcnt[w2];
    }
    if (flagged) s_list[off + __popcll(bal & ((1ull << lane) - 1ull))] = (int)(dsc - c0);
    __syncthreads();
  for (int k = 0; k < tot; ++k) {
    const int64_t dom = c0 + s_list[k];
    v4f G[ZC_T][4];
#pragma unroll
    for (int nt = 0; nt < ZC_T; ++nt)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * t + 4 * g + i, col = 128 * wv + 16 * nt + r;
          float v = 0.f;
          if (row < d0) {
            const float l = xl[dom * d0 + row], h = xh[dom * d0 + row];
            if (col == 0) v = (l + h) / 2.f;
            else if (col == 1 + row) v = (h - l) / 2.f;
          }
          G[nt][t][i] = v;
        }
    int Kc = 1 + d0;
    bool ovf = Kc > cap;
    for (int l = 0; l < net.n && !ovf; ++l) {
      const int dK = net.d[l], dM = net.d[l + 1];
      const int KS = ks_count(dK), MT = (dM + 15) / 16;
      // tiles of this wave in use
      int ntu = (Kc + 15) / 16 - ZC_T * wv;
      ntu = ntu < 0 ? 0 : (ntu > ZC_T ? ZC_T : ntu);
      const float* fr = sfrag + net.foff[l] * 64 + lane;
#pragma unroll
      for (int nt0 = 0; nt0 < ZC_T; nt0 += 2) {
        if (nt0 < ntu) {
          const bool two = nt0 + 1 < ntu;
          v4f o[2][4];
#pragma unroll
          for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) o[p][mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int ks = 4 * t + i;
              if (ks < KS) {
                float a[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) a[mt] = mt < MT ? fr[(mt * KS + ks) * 64] : 0.f;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
                  if (mt < MT) {
                    o[0][mt] = mfma16x16x4(a[mt], G[nt0][t][i], o[0][mt]);
                    if (two) o[1][mt] = mfma16x16x4(a[mt], G[nt0 + 1][t][i], o[1][mt]);
                  }
              }
            }
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            G[nt0][mt] = o[0][mt];
            if (two) G[nt0 + 1][mt] = o[1][mt];
          }
        }
      }
      if (wv == 0 && r == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * t + 4 * g + i;
            if (j < dM) G[0][t][i] = G[0][t][i] + sbias[net.boff[l] + j];
            scen[j] = G[0][t][i];
          }
      }
      // per-wave partial |G| sums over this wave's generator columns
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          KSum s;
#pragma unroll
          for (int nt = 0; nt < ZC_T; ++nt)
            if (nt < ntu && (wv > 0 || nt > 0 || r > 0)) s.add(fabsf(G[nt][t][i]));
          float ss = s.s, sc = s.c;
          for (int o = 8; o > 0; o >>= 1) {
            const float so = __shfl_xor(ss, o, 64), co = __shfl_xor(sc, o, 64);
            two_sum_acc(ss, sc, so);
            sc += co;
          }
          if (r == 0) {
            const int j = 16 * t + 4 * g + i;
            sred[(wv * 2) * FW + j] = ss;
            sred[(wv * 2 + 1) * FW + j] = sc;
          }
        }
      __syncthreads();
      float lam[4][4], mu[4][4];
      uint64_t umask = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * t + 4 * g + i;
          float ss = sred[j], sc = sred[FW + j];
          for (int w2 = 1; w2 < ZC_W; ++w2) {
            two_sum_acc(ss, sc, sred[(w2 * 2) * FW + j]);
            sc += sred[(w2 * 2 + 1) * FW + j];
          }
          const float rad = ss + sc;
          const float c = scen[j];
          const float lo = c - rad, hi = c + rad;
          const bool valid = j < dM;
          const bool ust = valid && lo < 0.f && hi > 0.f;
          const bool dead = hi <= 0.f;
          if (valid && r == 0 && wv == 0) {
            out.lo[l][dom * dM + j] = lo;
            out.hi[l][dom * dM + j] = hi;
          }
          lam[t][i] = ust ? hi / (hi - lo) : (dead ? 0.f : 1.f);
          mu[t][i] = ust ? (-hi * lo) / (2.f * (hi - lo)) : 0.f;
          const uint64_t bal = __ballot(ust && r == 0);
#pragma unroll
          for (int gg = 0; gg < 4; ++gg)
            if ((bal >> (16 * gg)) & 1ull) umask |= 1ull << (16 * t + 4 * gg + i);
        }
      __syncthreads();  // sred / scen are rewritten by the next layer
      const int cnt = __popcll(umask);
      if (l == net.n - 1) break;
      if (Kc + cnt > cap) {
        ovf = true;
        break;
      }
#pragma unroll
      for (int nt = 0; nt < ZC_T; ++nt)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (wv == 0 && nt == 0 && r == 0) G[nt][t][i] = lam[t][i] * G[nt][t][i] + mu[t][i];
            else G[nt][t][i] = G[nt][t][i] * lam[t][i];
          }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * t + 4 * g + i;
          if ((umask >> j) & 1ull) {
            const int col = Kc + __popcll(umask & ((1ull << j) - 1ull));
            if ((col >> 7) == wv && (col & 15) == r) {
              const int tile = (col & 127) >> 4;
#pragma unroll
              for (int nt = 0; nt < ZC_T; ++nt)
                if (nt == tile) G[nt][t][i] = mu[t][i];
            }
          }
        }
      Kc += cnt;
    }
    if (threadIdx.x == 0) overflow[dom] = ovf ? 1 : 0;
  }
    __syncthreads();  // s_list / s_wcnt are rewritten by the next chunk
  }
}

// ------------------------------------------------------------ CROWN kernel
struct CrownArgs {
  const float* lo_in[MAXL];
  const float* hi_in[MAXL];
  float* lo_out[MAXL];
  float* hi_out[MAXL];
  int idx_off[MAXL];
  int idx_cnt[MAXL];
};

// One relaxation + fc backward step through relu layer l and fc_l for the
// first np (<= NPAR) row tiles held in F (values of neurons of relu l),
// leaving in F the rows at fc_l's input.  acc partials collect neg . up_t
// and e . bias.  The MFMAs run K-step outer, (M-tile, row tile) inner, so
// consecutive MFMAs write independent accumulators.
__device__ __forceinline__ void relax_fc(const Net& net, int l, const float* sfrag,
                                         const float* sbias, const float* ssl, int lane, int g,
                                         int np, v4f (&F)[NPAR][4], KSum (&accp)[NPAR]) {
  const int dK = net.d[l + 1], dM = net.d[l];
  const int KS = ks_count(dK), MT = (dM + 15) / 16;
  const float* sl = ssl + l * 3 * FW;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 16 * t + 4 * g + i;
      if (j < dK) {
        const float ls = sl[j], us = sl[FW + j], ut = sl[2 * FW + j];
        const float bj = sbias[net.boff[l] + j];
#pragma unroll
        for (int p = 0; p < NPAR; ++p) {
          if (p < np) {
            const float x = F[p][t][i];
            const float ep = fmaxf(x, 0.f), en = fminf(x, 0.f);
            const float e = ep * ls + en * us;
            accp[p].add(en * ut);
            accp[p].add(e * bj);
            F[p][t][i] = e;
          }
        }
      }
    }
  const float* fr = sfrag + net.foff[l] * 64 + lane;
  v4f o[NPAR][4];
#pragma unroll
  for (int p = 0; p < NPAR; ++p)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[p][mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ks = 4 * t + i;
      if (ks < KS) {
        float a[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) a[mt] = mt < MT ? fr[(mt * KS + ks) * 64] : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          if (mt < MT) {
#pragma unroll
            for (int p = 0; p < NPAR; ++p)
              if (p < np) o[p][mt] = mfma16x16x4(a[mt], F[p][t][i], o[p][mt]);
          }
      }
    }
#pragma unroll
  for (int p = 0; p < NPAR; ++p)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) F[p][mt] = o[p][mt];
}

// lb = acc + sum_i pos(F_i) xl_i + neg(F_i) xh_i over the d0 input dims.
__device__ __forceinline__ void concretize_rows(int d0, const float* xl, const float* xh, int g,
                                                int np, const v4f (&F)[NPAR][4],
                                                KSum (&accp)[NPAR], float (&lb)[NPAR],
                                                float (&accv)[NPAR]) {
#pragma unroll
  for (int p = 0; p < NPAR; ++p) {
    lb[p] = accv[p] = 0.f;
    if (p >= np) continue;
    accv[p] = group_sum4(accp[p].s, accp[p].c);
    KSum c = accp[p];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * t + 4 * g + i;
        if (j < d0) {
          const float a = F[p][t][i];
          c.add(fmaxf(a, 0.f) * xl[j]);
          c.add(fminf(a, 0.f) * xh[j]);
        }
      }
    lb[p] = group_sum4(c.s, c.c);
  }
}

__device__ __forceinline__ void make_layer_slopes(float* sl, const float* lo, const float* hi,
                                                  int n, int lane) {
  for (int j = lane; j < FW; j += 64) {
    float ls = 0.f, us = 0.f, ut = 0.f;
    if (j < n) {
      Relax s = relax(lo[j], hi[j]);
      ls = s.lo_s;
      us = s.up_s;
      ut = s.up_t;
    }
    sl[j] = ls;
    sl[FW + j] = us;
    sl[2 * FW + j] = ut;
  }
}

__global__ __launch_bounds__(NWAVE * 64) void k_mlp_crown(
    Net net, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, CrownArgs ca,
    const int32_t* __restrict__ idx_all, int do_crown, int Q,
    const float* __restrict__ spec_rows, const float* __restrict__ spec_acc,
    float* __restrict__ lb_out, float* __restrict__ A_out, float* __restrict__ acc_out) {
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + net.nfrag * 64;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int nb_pad = (net.nbias + 63) & ~63;
  float* wbase = sbias + nb_pad + wv * (net.n * 3 * FW + 4 * FW);
  float* ssl = wbase;                       // slopes [layer][3][FW]
  float* slb = wbase + net.n * 3 * FW;      // seeded-row bounds (2 * FW)
  float* stl = slb + 2 * FW;                // current layer lo/hi (2 * FW)
  stage_weights(sfrag, sbias, gfrag, gbias, net.nfrag, net.nbias);
  const int d0 = net.d[0];

  for (int64_t dom = (int64_t)blockIdx.x * NWAVE + wv; dom < B; dom += (int64_t)gridDim.x * NWAVE) {
    const float* dxl = xl + dom * d0;
    const float* dxh = xh + dom * d0;
    for (int L = 0; L < net.n; ++L) {
      const int dW = net.d[L + 1];
      const float* lo_in = ca.lo_in[L] + dom * dW;
      const float* hi_in = ca.hi_in[L] + dom * dW;
      for (int j = lane; j < FW; j += 64) {
        stl[j] = j < dW ? lo_in[j] : 0.f;
        stl[FW + j] = j < dW ? hi_in[j] : 0.f;
      }
      __threadfence_block();
      const int m = do_crown ? ca.idx_cnt[L] : 0;
      const int32_t* idx = idx_all + (do_crown ? ca.idx_off[L] : 0);
      const int R = 2 * m;
      const int dS = net.d[L];  // width of the seeded rows after fc_L
      const int ntiles = (R + 15) / 16;
      for (int nt0 = 0; nt0 < ntiles; nt0 += NPAR) {
        const int np = ntiles - nt0 < NPAR ? ntiles - nt0 : NPAR;
        v4f F[NPAR][4];
        KSum accp[NPAR];
        // seed rows: row q < m is +W_L[idx[q]], row m + q is -W_L[idx[q]],
        // read from fc_L's backward fragments (A[k][j] = W_L[j][k] holds
        // W_L[j][16 t + 4 g + i] at fragment (t, 4*(j/16) + j%4), lane
        // 16*((j%16)/4) + 4 g + i)
#pragma unroll
        for (int p = 0; p < NPAR; ++p) {
          const int row = 16 * (nt0 + p) + r;
          const bool live = row < R;
          const int q = live ? (row < m ? row : row - m) : 0;
          const float sg = row < m ? 1.f : -1.f;
          const int j = live ? idx[q] : 0;
          const int KSL = ks_count(net.d[L + 1]);
          const float* fr = sfrag + net.foff[L] * 64;
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int k = 16 * t + 4 * g + i;
              float v = 0.f;
              if (live && k < dS) {
                const int f = t * KSL + 4 * (j >> 4) + (j & 3);
                const int ln = 16 * ((j & 15) >> 2) + 4 * g + i;
                v = sg * fr[f * 64 + ln];
              }
              F[p][t][i] = v;
            }
          if (live && g == 0) accp[p].add(sg * sbias[net.boff[L] + j]);
        }
        for (int l = L - 1; l >= 0; --l)
          relax_fc(net, l, sfrag, sbias, ssl, lane, g, np, F, accp);
        float lb[NPAR], accv[NPAR];
        concretize_rows(d0, dxl, dxh, g, np, F, accp, lb, accv);
#pragma unroll
        for (int p = 0; p < NPAR; ++p) {
          const int row = 16 * (nt0 + p) + r;
          if (g == 0 && row < R) slb[row] = lb[p];
        }
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
      make_layer_slopes(ssl + L * 3 * FW, stl, stl + FW, dW, lane);
      __threadfence_block();
    }
    if (Q > 0) {
      // spec rows (shared, Q x d[n]) through relu n-1 ... relu 0
      const int dN = net.d[net.n];
      v4f F[NPAR][4];
      KSum accp[NPAR];
#pragma unroll
      for (int p = 0; p < NPAR; ++p) {
        const int row = 16 * p + r;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = 16 * t + 4 * g + i;
            F[p][t][i] = (row < Q && k < dN) ? spec_rows[row * dN + k] : 0.f;
          }
        if (row < Q && g == 0) accp[p].add(spec_acc[row]);
      }
      const int np = (Q + 15) / 16;
      for (int l = net.n - 1; l >= 0; --l)
        relax_fc(net, l, sfrag, sbias, ssl, lane, g, np, F, accp);
      float lb[NPAR], accv[NPAR];
      concretize_rows(d0, dxl, dxh, g, np, F, accp, lb, accv);
#pragma unroll
      for (int p = 0; p < NPAR; ++p) {
        const int row = 16 * p + r;
        if (row < Q) {
          if (g == 0) {
            lb_out[dom * Q + row] = lb[p];
            if (acc_out) acc_out[dom * Q + row] = accv[p];
          }
          if (A_out) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int k = 16 * t + 4 * g + i;
                if (k < d0) A_out[(dom * Q + row) * d0 + k] = F[p][t][i];
              }
          }
        }
      }
    }
  }
}

// ------------------------------------------------------ alpha-CROWN kernel
// One Adam iteration of batched alpha-CROWN per domain
// (verify_zono_bnb.py:5248-5287): the spec backward with lower slopes
// active + unstable * alpha (pre-relaxation rows P_l kept in registers),
// concretization, then the gradient of sum_q lb w.r.t. alpha by the
// forward sweep gA = xl [A >= 0] + xh [A <= 0], gE_l = W_l gP_{l-1} + b_l,
// dalpha_l = sum_q gE_l pos(P_l) (unstable only),
// gP_l = gE_l (mpos ls + mneg up_s) + mneg up_t (torch's clamp subgradient),
// and torch.optim.Adam's update of alpha on -sum lb, clamped to [0, 1].
constexpr int AL_MAXL = 7;  // P_l for 8 layers would spill registers
constexpr int NWAVE_A = 4;  // one wave per SIMD: the full register file per wave

struct AlphaArgs {
  const float* lo[MAXL];
  const float* hi[MAXL];
  float* alpha[MAXL];
  float* m1[MAXL];
  float* m2[MAXL];
};

// Forward-direction A operand W_l[16 mt + r][16 t + 4 g + i] read from the
// backward fragments of fc_l (which hold W_l transposed): a lane permutation.
__device__ __forceinline__ float fwd_a(const float* sfrag, const Net& net, int l, int mt, int t,
                                       int i, int lane) {
  const int g = lane >> 4, r = lane & 15;
  const int o = 16 * mt + r;
  if (o >= net.d[l + 1]) return 0.f;
  const int KSb = ks_count(net.d[l + 1]);
  const int f = net.foff[l] + t * KSb + 4 * mt + (r & 3);
  return sfrag[f * 64 + 16 * (r >> 2) + 4 * g + i];
}

// NL: the exact number of ReLU layers (P_l rows live in NL x 16 registers).
template <int NL>
__global__ __launch_bounds__(NWAVE_A * 64) void k_mlp_alpha(
    Net net, const float* __restrict__ gfrag, const float* __restrict__ gbias, int64_t B,
    const float* __restrict__ xl, const float* __restrict__ xh, AlphaArgs aa, int Q,
    const float* __restrict__ spec_rows, const float* __restrict__ spec_acc,
    float* __restrict__ lb_out, AdamConst adam) {
#pragma clang fp contract(off)
  extern __shared__ float smem[];
  float* sfrag = smem;
  float* sbias = smem + net.nfrag * 64;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int nb_pad = (net.nbias + 63) & ~63;
  // per wave: slopes [layer][ls, us, ut, unst][FW], Adam state [layer][alpha, m, v][FW]
  float* ssl = sbias + nb_pad + wv * (net.n * 7 * FW);
  float* sad = ssl + net.n * 4 * FW;
  stage_weights(sfrag, sbias, gfrag, gbias, net.nfrag, net.nbias);
  const int d0 = net.d[0], n = net.n;

  for (int64_t dom = (int64_t)blockIdx.x * NWAVE_A + wv; dom < B;
       dom += (int64_t)gridDim.x * NWAVE_A) {
    const float* dxl = xl + dom * d0;
    const float* dxh = xh + dom * d0;
    for (int l = 0; l < n; ++l) {
      const int dW = net.d[l + 1];
      float* sl = ssl + l * 4 * FW;
      float* sa = sad + l * 3 * FW;
      for (int j = lane; j < FW; j += 64) {
        float ls = 0.f, us = 0.f, ut = 0.f, un = 0.f, a = 0.f, m1 = 0.f, m2 = 0.f;
        if (j < dW) {
          const int64_t ai = dom * dW + j;
          Relax s = relax(aa.lo[l][ai], aa.hi[l][ai]);
          a = aa.alpha[l][ai];
          m1 = aa.m1[l][ai];
          m2 = aa.m2[l][ai];
          ls = s.active ? 1.f : (s.unstable ? a : 0.f);
          us = s.up_s;
          ut = s.up_t;
          un = s.unstable ? 1.f : 0.f;
        }
        sl[j] = ls;
        sl[FW + j] = us;
        sl[2 * FW + j] = ut;
        sl[3 * FW + j] = un;
        sa[j] = a;
        sa[FW + j] = m1;
        sa[2 * FW + j] = m2;
      }
    }
    __threadfence_block();
    const bool live_row = r < Q;
    // ---- spec backward with alpha, keeping P_l
    const int dN = net.d[n];
    v4f F[4];
    KSum accp;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = 16 * t + 4 * g + i;
        F[t][i] = (live_row && k < dN) ? spec_rows[r * dN + k] : 0.f;
      }
    if (live_row && g == 0) accp.add(spec_acc[r]);
    v4f P[NL][4];
#pragma unroll
    for (int ll = NL - 1; ll >= 0; --ll) {
      {
        const int dK = net.d[ll + 1], dM = net.d[ll];
        const float* sl = ssl + ll * 4 * FW;
#pragma unroll
        for (int t = 0; t < 4; ++t) P[ll][t] = F[t];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * t + 4 * g + i;
            if (j < dK) {
              const float x = F[t][i];
              const float ep = fmaxf(x, 0.f), en = fminf(x, 0.f);
              const float e = ep * sl[j] + en * sl[FW + j];
              accp.add(en * sl[2 * FW + j]);
              accp.add(e * sbias[net.boff[ll] + j]);
              F[t][i] = e;
            }
          }
        const int KS = ks_count(dK), MT = (dM + 15) / 16;
        const float* fr = sfrag + net.foff[ll] * 64 + lane;
        v4f o[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) o[mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int ks = 4 * t + i;
            if (ks < KS) {
#pragma unroll
              for (int mt = 0; mt < 4; ++mt)
                if (mt < MT) o[mt] = mfma16x16x4(fr[(mt * KS + ks) * 64], F[t][i], o[mt]);
            }
          }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) F[mt] = o[mt];
      }
    }
    // ---- concretize; gA
    KSum c = accp;
    v4f G[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * t + 4 * g + i;
        float gv = 0.f;
        if (j < d0) {
          const float a = F[t][i];
          c.add(fmaxf(a, 0.f) * dxl[j]);
          c.add(fminf(a, 0.f) * dxh[j]);
          if (live_row) {
            if (a >= 0.f) gv += dxl[j];
            if (a <= 0.f) gv += dxh[j];
          }
        }
        G[t][i] = gv;
      }
    const float lb = group_sum4(c.s, c.c);
    if (g == 0 && live_row) lb_out[dom * Q + r] = lb;
    // ---- gradient sweep toward the output, with the Adam update per layer
    for (int l = 0; l < n; ++l) {
      const int dK = net.d[l], dM = net.d[l + 1];
      const int T = (dK + 15) / 16, MT = (dM + 15) / 16;
      v4f o[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) o[mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (t < T) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
              if (mt < MT) o[mt] = mfma16x16x4(fwd_a(sfrag, net, l, mt, t, i, lane), G[t][i], o[mt]);
        }
      const float* sl = ssl + l * 4 * FW;
      const int dW = dM;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * t + 4 * g + i;
          float ge = o[t][i];
          if (j < dW && live_row) ge = ge + sbias[net.boff[l] + j];
          if (!live_row || j >= dW) ge = 0.f;
          float pv = 0.f;
#pragma unroll
          for (int ll = 0; ll < NL; ++ll)
            if (ll == l) pv = P[ll][t][i];
          // d lb / d alpha_j = sum over rows of gE * pos(P)
          float s = ge * fmaxf(pv, 0.f), cs = 0.f;
          for (int ofs = 8; ofs > 0; ofs >>= 1) {
            const float so = __shfl_xor(s, ofs, 64), co = __shfl_xor(cs, ofs, 64);
            two_sum_acc(s, cs, so);
            cs += co;
          }
          const float ga = s + cs;
          if (r == 0 && j < dW && sl[3 * FW + j] != 0.f) {
            float* sa = sad + l * 3 * FW;
            float mi = sa[FW + j], vi = sa[2 * FW + j];
            float pa = adam_update(sa[j], -ga, mi, vi, adam);
            pa = fminf(fmaxf(pa, 0.f), 1.f);
            sa[FW + j] = mi;
            sa[2 * FW + j] = vi;
            sa[j] = pa;
          }
          const bool mp = pv >= 0.f, mn = pv <= 0.f;
          float gp = ge * ((mp ? sl[j] : 0.f) + (mn ? sl[FW + j] : 0.f));
          if (mn) gp = gp + sl[2 * FW + j];
          G[t][i] = (live_row && j < dW) ? gp : 0.f;
        }
    }
    // write the updated Adam state back (coalesced)
    __threadfence_block();
    for (int l = 0; l < n; ++l) {
      const int dW = net.d[l + 1];
      const float* sa = sad + l * 3 * FW;
      for (int j = lane; j < dW; j += 64) {
        const int64_t ai = dom * dW + j;
        aa.alpha[l][ai] = sa[j];
        aa.m1[l][ai] = sa[FW + j];
        aa.m2[l][ai] = sa[2 * FW + j];
      }
    }
    __threadfence_block();
  }
}

int build_net(const int32_t* dims, int n_relu, Net& net) {
  if (!dims || n_relu < 1 || n_relu > MAXL) return VC_ERR_UNSUPPORTED;
  net.n = n_relu;
  int fo = 0, bo = 0;
  for (int l = 0; l <= n_relu; ++l) {
    net.d[l] = dims[l];
    if (dims[l] <= 0) return VC_ERR_ARG;
    if (dims[l] > FW) return VC_ERR_UNSUPPORTED;
  }
  for (int l = 0; l < n_relu; ++l) {
    net.foff[l] = fo;
    net.boff[l] = bo;
    fo += ((net.d[l] + 15) / 16) * ks_count(net.d[l + 1]);  // bwd: M = d[l], K = d[l+1]
    bo += net.d[l + 1];
  }
  net.nfrag = fo;
  net.nbias = bo;
  return VC_OK;
}

// forward fragment offsets differ (M = d[l+1], K = d[l])
int build_net_fwd(const int32_t* dims, int n_relu, Net& net) {
  int rc = build_net(dims, n_relu, net);
  if (rc != VC_OK) return rc;
  int fo = 0;
  for (int l = 0; l < n_relu; ++l) {
    net.foff[l] = fo;
    fo += ((net.d[l + 1] + 15) / 16) * ks_count(net.d[l]);
  }
  net.nfrag = fo;
  return VC_OK;
}

int persistent_grid(int64_t B, size_t lds_bytes, int nwave = NWAVE) {
  return vcm::persistent_grid(B, lds_bytes, nwave);
}

}  // namespace

extern "C" int64_t vc_mlp_frag_floats(const int32_t* dims, int n_relu, int forward) {
  Net net{};
  const int rc = forward ? build_net_fwd(dims, n_relu, net) : build_net(dims, n_relu, net);
  if (rc != VC_OK) return -rc;
  return (int64_t)net.nfrag * 64;
}

extern "C" int vc_mlp_pack(const float* const* W, const int32_t* dims, int n_relu, int forward,
                           float* frag, vc_stream_t stream) {
  Net net{};
  const int rc = forward ? build_net_fwd(dims, n_relu, net) : build_net(dims, n_relu, net);
  if (rc != VC_OK) return rc;
  if (!W || !frag) return VC_ERR_ARG;
  for (int l = 0; l < n_relu; ++l) {
    if (!W[l]) return VC_ERR_ARG;
    const int d_in = net.d[l], d_out = net.d[l + 1];
    const int M = forward ? d_out : d_in, K = forward ? d_in : d_out;
    const int total = ((M + 15) / 16) * ks_count(K) * 64;
    hipLaunchKernelGGL(k_pack, dim3((total + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       W[l], d_out, d_in, forward ? 0 : 1, frag + (int64_t)net.foff[l] * 64);
  }
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_mlp_zono_bounds(const int32_t* dims, int n_relu, const float* frag_fwd,
                                  const float* bias_cat, int64_t B, const float* xl,
                                  const float* xh, float* const* lo_out, float* const* hi_out,
                                  int32_t* overflow, vc_stream_t stream) {
  Net net{};
  int rc = build_net_fwd(dims, n_relu, net);
  if (rc != VC_OK) return rc;
  if (!frag_fwd || !bias_cat || !xl || !xh || !lo_out || !hi_out || !overflow || B < 0)
    return VC_ERR_ARG;
  if (net.d[0] + 1 > ZNT_NARROW * 16) return VC_ERR_UNSUPPORTED;
  if (B == 0) return VC_OK;
  ZonoArgs za;
  for (int l = 0; l < MAXL; ++l) {
    za.lo[l] = l < n_relu ? lo_out[l] : nullptr;
    za.hi[l] = l < n_relu ? hi_out[l] : nullptr;
    if (l < n_relu && (!za.lo[l] || !za.hi[l])) return VC_ERR_ARG;
  }
  const size_t lds = ((size_t)net.nfrag * 64 + net.nbias) * sizeof(float);
  if (lds > 160 * 1024) return VC_ERR_UNSUPPORTED;
  const size_t lds_c = lds + ((size_t)((net.nbias + 63) & ~63) - net.nbias +
                              (size_t)ZC_W * 2 * FW + FW) * sizeof(float);
  if (lds_c > 160 * 1024) return VC_ERR_UNSUPPORTED;
  const void* fn_n = reinterpret_cast<const void*>(&k_mlp_zono<ZNT_NARROW, NWAVE>);
  const void* fn_c = reinterpret_cast<const void*>(&k_mlp_zono_coop);
  if (hipFuncSetAttribute(fn_n, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
          hipSuccess ||
      hipFuncSetAttribute(fn_c, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_c) !=
          hipSuccess)
    return VC_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL((k_mlp_zono<ZNT_NARROW, NWAVE>), dim3(persistent_grid(B, lds)),
                     dim3(NWAVE * 64), lds, st, net, frag_fwd, bias_cat, B, xl, xh, za,
                     overflow, 0);
  // second pass over the domains that did not fit: one workgroup per
  // flagged domain, each workgroup scanning a strided share of the flags
  int64_t gw = cu_count();
  if (gw > B) gw = B;
  hipLaunchKernelGGL(k_mlp_zono_coop, dim3((unsigned)gw), dim3(ZC_W * 64), lds_c, st, net,
                     frag_fwd, bias_cat, B, xl, xh, za, overflow);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_mlp_zono_wide(const int32_t* dims, int n_relu, const float* frag_fwd,
                                const float* bias_cat, int64_t B, const float* xl,
                                const float* xh, float* const* lo_out, float* const* hi_out,
                                int32_t* overflow, vc_stream_t stream) {
  Net net{};
  int rc = build_net_fwd(dims, n_relu, net);
  if (rc != VC_OK) return rc;
  if (!frag_fwd || !bias_cat || !xl || !xh || !lo_out || !hi_out || !overflow || B < 0)
    return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  ZonoArgs za;
  for (int l = 0; l < MAXL; ++l) {
    za.lo[l] = l < n_relu ? lo_out[l] : nullptr;
    za.hi[l] = l < n_relu ? hi_out[l] : nullptr;
    if (l < n_relu && (!za.lo[l] || !za.hi[l])) return VC_ERR_ARG;
  }
  const size_t lds_c = ((size_t)net.nfrag * 64 + ((net.nbias + 63) & ~63) +
                        (size_t)ZC_W * 2 * FW + FW) * sizeof(float);
  if (lds_c > 160 * 1024) return VC_ERR_UNSUPPORTED;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_mlp_zono_coop),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_c) != hipSuccess)
    return VC_ERR_UNSUPPORTED;
  int64_t gw = cu_count();
  if (gw > B) gw = B;
  hipLaunchKernelGGL(k_mlp_zono_coop, dim3((unsigned)gw), dim3(ZC_W * 64), lds_c,
                     (hipStream_t)stream, net, frag_fwd, bias_cat, B, xl, xh, za, overflow);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_mlp_alpha_iter(const int32_t* dims, int n_relu, const float* frag_bwd,
                                 const float* bias_cat, int64_t B, const float* xl,
                                 const float* xh, const float* const* lo, const float* const* hi,
                                 float* const* alpha, float* const* exp_avg,
                                 float* const* exp_avg_sq, int Q, const float* spec_rows,
                                 const float* spec_acc, float* lb_out, double b1, double b2,
                                 double eps, double step_size, double bc2_sqrt,
                                 vc_stream_t stream) {
  Net net{};
  int rc = build_net(dims, n_relu, net);
  if (rc != VC_OK) return rc;
  if (n_relu > AL_MAXL || Q < 1 || Q > 16) return VC_ERR_UNSUPPORTED;
  if (!frag_bwd || !bias_cat || !xl || !xh || !lo || !hi || !alpha || !exp_avg || !exp_avg_sq ||
      !spec_rows || !spec_acc || !lb_out || B < 0)
    return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  AlphaArgs aa;
  for (int l = 0; l < MAXL; ++l) {
    const bool in = l < n_relu;
    aa.lo[l] = in ? lo[l] : nullptr;
    aa.hi[l] = in ? hi[l] : nullptr;
    aa.alpha[l] = in ? alpha[l] : nullptr;
    aa.m1[l] = in ? exp_avg[l] : nullptr;
    aa.m2[l] = in ? exp_avg_sq[l] : nullptr;
    if (in && (!aa.lo[l] || !aa.hi[l] || !aa.alpha[l] || !aa.m1[l] || !aa.m2[l])) return VC_ERR_ARG;
  }
  const size_t lds = ((size_t)net.nfrag * 64 + ((net.nbias + 63) & ~63) +
                      (size_t)NWAVE_A * net.n * 7 * FW) * sizeof(float);
  if (lds > 160 * 1024) return VC_ERR_UNSUPPORTED;
  const void* fn = nullptr;
  switch (n_relu) {
    case 1: fn = reinterpret_cast<const void*>(&k_mlp_alpha<1>); break;
    case 2: fn = reinterpret_cast<const void*>(&k_mlp_alpha<2>); break;
    case 3: fn = reinterpret_cast<const void*>(&k_mlp_alpha<3>); break;
    case 4: fn = reinterpret_cast<const void*>(&k_mlp_alpha<4>); break;
    case 5: fn = reinterpret_cast<const void*>(&k_mlp_alpha<5>); break;
    case 6: fn = reinterpret_cast<const void*>(&k_mlp_alpha<6>); break;
    default: fn = reinterpret_cast<const void*>(&k_mlp_alpha<7>); break;
  }
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return VC_ERR_UNSUPPORTED;
  const dim3 grid(persistent_grid(B, lds, NWAVE_A)), block(NWAVE_A * 64);
  const AdamConst adam = adam_const(b1, b2, eps, step_size, bc2_sqrt);
  hipStream_t st = (hipStream_t)stream;
#define VC_ALPHA_CASE(NLV)                                                                   \
  case NLV:                                                                                  \
    hipLaunchKernelGGL(k_mlp_alpha<NLV>, grid, block, lds, st, net, frag_bwd, bias_cat, B,   \
                       xl, xh, aa, Q, spec_rows, spec_acc, lb_out, adam);                   \
    break;
  switch (n_relu) {
    VC_ALPHA_CASE(1)
    VC_ALPHA_CASE(2)
    VC_ALPHA_CASE(3)
    VC_ALPHA_CASE(4)
    VC_ALPHA_CASE(5)
    VC_ALPHA_CASE(6)
    VC_ALPHA_CASE(7)
    default: return VC_ERR_UNSUPPORTED;
  }
#undef VC_ALPHA_CASE
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_mlp_crown(const int32_t* dims, int n_relu, const float* frag_bwd,
                            const float* bias_cat, int64_t B, const float* xl, const float* xh,
                            const float* const* lo_in, const float* const* hi_in,
                            float* const* lo_out, float* const* hi_out, const int32_t* idx_all,
                            const int32_t* idx_cnt, int do_crown, int Q, const float* spec_rows,
                            const float* spec_acc, float* lb_out, float* A_out, float* acc_out,
                            vc_stream_t stream) {
  Net net{};
  int rc = build_net(dims, n_relu, net);
  if (rc != VC_OK) return rc;
  if (!frag_bwd || !bias_cat || !xl || !xh || !lo_in || !hi_in || B < 0) return VC_ERR_ARG;
  if (Q < 0 || Q > NPAR * 16) return VC_ERR_UNSUPPORTED;
  if (Q > 0 && (!spec_rows || !spec_acc || !lb_out)) return VC_ERR_ARG;
  if (do_crown && (!idx_all || !idx_cnt || !lo_out || !hi_out)) return VC_ERR_ARG;
  if (B == 0) return VC_OK;
  CrownArgs ca;
  int off = 0;
  for (int l = 0; l < MAXL; ++l) {
    const bool in = l < n_relu;
    ca.lo_in[l] = in ? lo_in[l] : nullptr;
    ca.hi_in[l] = in ? hi_in[l] : nullptr;
    ca.lo_out[l] = (in && lo_out) ? lo_out[l] : nullptr;
    ca.hi_out[l] = (in && hi_out) ? hi_out[l] : nullptr;
    ca.idx_off[l] = off;
    ca.idx_cnt[l] = (in && do_crown) ? idx_cnt[l] : 0;
    if (in && (!ca.lo_in[l] || !ca.hi_in[l])) return VC_ERR_ARG;
    if (in && (ca.idx_cnt[l] < 0 || ca.idx_cnt[l] > net.d[l + 1])) return VC_ERR_ARG;
    off += ca.idx_cnt[l];
  }
  const size_t lds = ((size_t)net.nfrag * 64 + ((net.nbias + 63) & ~63) +
                      (size_t)NWAVE * (net.n * 3 * FW + 4 * FW)) * sizeof(float);
  if (lds > 160 * 1024) return VC_ERR_UNSUPPORTED;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_mlp_crown),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return VC_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(k_mlp_crown, dim3(persistent_grid(B, lds)), dim3(NWAVE * 64), lds,
                     (hipStream_t)stream, net, frag_bwd, bias_cat, B, xl, xh, ca, idx_all,
                     do_crown, Q, spec_rows, spec_acc, lb_out, A_out, acc_out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
