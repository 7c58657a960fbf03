// One input-split BaB round on the narrow-MLP kernels, orchestrated on the
// host in C++ (verify_graph.py:12855-13382 as restated by bab_step in
// vibecheck_amd/verify_graph.py): zonotope bounds, CROWN intermediate bounds
// with the spec bound and its input linearization, closure, alpha-CROWN on
// the open leaves, closure again, one halfspace clip, widest-axis
// bisection.  Every step is one of the library's entry points on the
// caller's stream; the three counts the round needs on the host (open,
// unclosed, feasible + split) are read with a stream synchronisation each,
// with no interpreter between a count and the launches that use it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "vc_common.h"
#include "vc_mlp_common.h"

namespace {

using vcm::MAXL;

// Bump allocation of the round's buffers from the caller's workspace (or,
// with base == nullptr, the size of that layout).
struct Carve {
  char* base;
  size_t used;
  template <class T>
  T* take(int64_t n) {
    const size_t bytes = ((size_t)std::max<int64_t>(n, 1) * sizeof(T) + 255) & ~(size_t)255;
    T* r = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += bytes;
    return r;
  }
};

struct RoundBufs {
  float *sb_lo[MAXL], *sb_hi[MAXL];  // zonotope bounds (B, d_L)
  float *t_lo[MAXL], *t_hi[MAXL];    // CROWN bounds (B, d_L)
  uint8_t* ovf;                      // zonotope overflow flags (B)
  int64_t* idx;                      // compaction output (B)
  int64_t* idx2;                     // second compaction output (B)
  int64_t* cnt;                      // counts [4]
  void* cws;                         // compaction workspace
  int64_t cws_bytes;
  int32_t* uidx;                     // union lists (sum d)
  int32_t* umeta;                    // union counts and offsets (2 n)
  unsigned long long* umask;         // union as bit masks [MAXL]
  int32_t* queue;                    // work counters [2]
  void* rws;                         // layer-synchronous CROWN workspace (large B)
  int64_t rws_bytes;
  // alpha on the open leaves (sized for B)
  float *a_lo[MAXL], *a_hi[MAXL];
  float *a_xl, *a_xh, *a_state, *a_lb, *a_best, *a_ctl;
  // clip on the unclosed leaves
  float *u_xl, *u_xh, *u_A, *u_acc, *c_xl, *c_xh;
  int64_t* ax_u;
  uint8_t *usable, *split;
};

void carve(Carve& c, RoundBufs& r, const int32_t* dims, int n, int64_t B, int Q) {
  const int n_in = dims[0];
  // batches above 4 x CUs take the layer-synchronous CROWN, which needs no
  // buffers for the CROWN bounds
  r.rws_bytes = vc_mlp_tiled_crown_mode(B) == 0 ? vc_mlp_crown_rows_workspace(dims, n, B) : 0;
  if (r.rws_bytes < 0) r.rws_bytes = 0;
  int sumd = 0;
  for (int l = 0; l < n; ++l) {
    const int d = dims[l + 1];
    sumd += d;
    r.sb_lo[l] = c.take<float>(B * d);
    r.sb_hi[l] = c.take<float>(B * d);
    r.t_lo[l] = r.rws_bytes > 0 ? nullptr : c.take<float>(B * d);
    r.t_hi[l] = r.rws_bytes > 0 ? nullptr : c.take<float>(B * d);
    r.a_lo[l] = c.take<float>(B * d);
    r.a_hi[l] = c.take<float>(B * d);
  }
  r.ovf = c.take<uint8_t>(B);
  r.idx = c.take<int64_t>(B);
  r.idx2 = c.take<int64_t>(B);
  r.cnt = c.take<int64_t>(4);
  r.cws_bytes = vc_compact_workspace(B);
  r.cws = c.take<char>(r.cws_bytes);
  r.uidx = c.take<int32_t>(sumd);
  r.umeta = c.take<int32_t>(2 * n);
  r.umask = c.take<unsigned long long>(MAXL);
  r.queue = c.take<int32_t>(2);
  r.rws = r.rws_bytes > 0 ? c.take<char>(r.rws_bytes) : nullptr;
  r.a_xl = c.take<float>(B * n_in);
  r.a_xh = c.take<float>(B * n_in);
  r.a_state = c.take<float>(3 * (int64_t)sumd * B);
  r.a_lb = c.take<float>((int64_t)VC_ALPHA_CHUNK * B * Q);
  r.a_best = c.take<float>(B * Q);
  r.a_ctl = c.take<float>(4);
  r.u_xl = c.take<float>(B * n_in);
  r.u_xh = c.take<float>(B * n_in);
  r.u_A = c.take<float>(B * Q * n_in);
  r.u_acc = c.take<float>(B * Q);
  r.c_xl = c.take<float>(B * n_in);
  r.c_xh = c.take<float>(B * n_in);
  r.ax_u = c.take<int64_t>(B);
  r.usable = c.take<uint8_t>(B);
  r.split = c.take<uint8_t>(B);
}

// alpha's evaluated-iteration count (ctl[2]) as a device count.
__global__ void k_ctl_count(const float* __restrict__ ctl, int64_t* out) {
  if (threadIdx.x == 0) *out = (int64_t)ctl[2];
}

// Device counts to pinned host words, stored by the GPU (system scope);
// with ctl, word k is the alpha loop's evaluated iterations (ctl[2]).
__global__ void k_counts_to_host(const int64_t* __restrict__ dev, int k, int64_t* host,
                                 const float* __restrict__ ctl) {
  if (threadIdx.x < k)
    __hip_atomic_store(host + threadIdx.x, dev[threadIdx.x], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
  if (ctl && threadIdx.x == k)
    __hip_atomic_store(host + k, (int64_t)ctl[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// k counts from the device once every launch before them has run.  With
// pinned host words the GPU stores them there and the host polls (no copy,
// no wake-up latency); the poll is bounded, then the stream is synchronised
// and the counts are read from device memory.
// With ctl, one more count follows the k: the alpha loop's evaluated
// iterations (host[k]; dev[k] is then scratch for the fallback).
int read_counts(const int64_t* dev, int k, int64_t* host, int64_t* pinned, hipStream_t st,
                const float* ctl = nullptr) {
  const int kk = ctl ? k + 1 : k;
  if (pinned) {
    volatile int64_t* pw = pinned;
    for (int i = 0; i < kk; ++i) pw[i] = -1;
    hipLaunchKernelGGL(k_counts_to_host, dim3(1), dim3(64), 0, st, dev, k, pinned, ctl);
    if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
    for (long spin = 0; spin < (1l << 26); ++spin) {
      bool ready = true;
      for (int i = 0; i < kk; ++i) ready = ready && pw[i] >= 0;
      if (ready) {
        for (int i = 0; i < kk; ++i) host[i] = pw[i];
        return VC_OK;
      }
    }
  }
  if (ctl) {
    hipLaunchKernelGGL(k_ctl_count, dim3(1), dim3(64), 0, st, ctl, const_cast<int64_t*>(dev) + k);
    if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
  }
  if (hipMemcpyAsync(host, dev, sizeof(int64_t) * kk, hipMemcpyDeviceToHost, st) != hipSuccess)
    return VC_ERR_LAUNCH;
  return hipStreamSynchronize(st) == hipSuccess ? VC_OK : VC_ERR_LAUNCH;
}

// Clip shrink accounting of the phase timer: w[0] += sum of max(xh - xl, 0)
// over the n values before the clip, w[1] += the same after it.  Double
// atomics per wavefront (any order: a profiling ratio, not a bound).
__global__ void k_clip_widths(const float* __restrict__ xl, const float* __restrict__ xh,
                              const float* __restrict__ cl, const float* __restrict__ ch,
                              int64_t n, double* w) {
  double a = 0.0, b = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    a += (double)fmaxf(xh[i] - xl[i], 0.0f);
    b += (double)fmaxf(ch[i] - cl[i], 0.0f);
  }
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_down(a, o, 64);
    b += __shfl_down(b, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(w, a);
    atomicAdd(w + 1, b);
  }
}

// vc_gather_rows_multi in launches of at most 32 arrays.
int gather(const float* const* in, float* const* out, const int32_t* cols, int n_arrays,
           const int64_t* idx, int64_t n_rows, vc_stream_t stream) {
  for (int a0 = 0; a0 < n_arrays; a0 += 32) {
    const int k = std::min(32, n_arrays - a0);
    const int rc = vc_gather_rows_multi(in + a0, out + a0, cols + a0, k, idx, n_rows, stream);
    if (rc != VC_OK) return rc;
  }
  return VC_OK;
}

}  // namespace

#define VC_TRY(x)                 \
  do {                            \
    const int rc_ = (x);          \
    if (rc_ != VC_OK) return rc_; \
  } while (0)

extern "C" int64_t vc_mlp_bab_round_workspace(const int32_t* dims, int n_relu, int64_t B,
                                              int Q) {
  if (!dims || n_relu < 1 || n_relu > MAXL || B < 0 || Q < 1) return -VC_ERR_ARG;
  Carve c{nullptr, 0};
  RoundBufs r;
  carve(c, r, dims, n_relu, B, Q);
  return (int64_t)c.used;
}

namespace {

// The round's phases, in the order the phase timer's events close them.
enum RoundPhase { PH_BOUND = 0, PH_ALPHA = 1, PH_CLIP = 2, PH_SPLIT = 3 };

// Records phase event k (0: round start; 1..4: end of bound, alpha, clip,
// split) when the caller asked for them.
int mark(void* const* phase_ev, int k, hipStream_t st) {
  if (!phase_ev) return VC_OK;
  return hipEventRecord((hipEvent_t)phase_ev[k], st) == hipSuccess ? VC_OK : VC_ERR_LAUNCH;
}

int bab_round(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat, int Q,
              const float* spec_rows, const float* spec_acc, const int32_t* d_ptr,
              const int32_t* q_idx, int n_disj, int64_t B, const float* xl, const float* xh,
              int alpha_iters, double alpha_lr, double alpha_lr_decay, double alpha_early_stop,
              float* lb, float* A, float* acc, uint8_t* closed, int64_t* unclosed,
              uint8_t* feasible, float* xl_split, float* xh_split, int64_t* ax, float* low_xl,
              float* low_xh, float* high_xl, float* high_xh, uint64_t* seed_rows,
              void* crown_ev0, void* crown_ev1, void* const* phase_ev, double* clip_widths,
              void* work, int64_t work_bytes, int32_t* stop_host, int64_t* pinned,
              int64_t* counts, int& phase, vc_stream_t stream) {
  phase = PH_BOUND;
  if (!dims || !frag || !bias_cat || !spec_rows || !spec_acc || !d_ptr || !q_idx || !xl ||
      !xh || !lb || !A || !acc || !closed || !unclosed || !feasible || !xl_split ||
      !xh_split || !ax || !low_xl || !low_xh || !high_xl || !high_xh || !work || !counts)
    return VC_ERR_ARG;
  if (n_relu < 1 || n_relu > MAXL || B < 0 || Q < 1 || n_disj < 0) return VC_ERR_ARG;
  const int64_t need = vc_mlp_bab_round_workspace(dims, n_relu, B, Q);
  if (need < 0) return (int)-need;
  if (work_bytes < need) return VC_ERR_OOM;
  const int n = n_relu, n_in = dims[0];
  int sumd = 0;
  for (int l = 1; l <= n; ++l) sumd += dims[l];
  // the wide zonotope pass must hold every generator the net can have
  int max_cols = 1;
  for (int l = 0; l < n; ++l) max_cols += dims[l];
  if (max_cols > VC_ZONO_WIDE_COLS) return VC_ERR_UNSUPPORTED;
  for (int k = 0; k < 6; ++k) counts[k] = 0;
  hipStream_t st = (hipStream_t)stream;
  VC_TRY(mark(phase_ev, 0, st));
  if (B == 0) {
    for (int k = 1; k <= 4; ++k) VC_TRY(mark(phase_ev, k, st));
    return VC_OK;
  }
  Carve c{reinterpret_cast<char*>(work), 0};
  RoundBufs r;
  carve(c, r, dims, n, B, Q);

  // ---- bound phase: zonotope, union of the unstable neurons, CROWN + spec.
  // The zonotope passes leave the union of the unstable sets (same bounds,
  // no second pass over them), and for the rows form its per-domain seed
  // masks in its workspace; the one-wavefront pass lists its overflowing
  // domains itself.
  if (r.rws) {
    VC_TRY(vcm::zono_bounds_masked(dims, n, frag, bias_cat, B, xl, xh, r.sb_lo, r.sb_hi, r.ovf,
                                   r.queue + 1, r.rws, r.idx, r.cnt, r.cnt + 3, st));
    VC_TRY(vcm::zono_wide_masked(dims, n, frag, bias_cat, B, xl, xh, r.sb_lo, r.sb_hi, r.ovf,
                                 r.idx, r.cnt, r.rws, st));
  } else {
    VC_TRY(vcm::zono_bounds_listed(dims, n, frag, bias_cat, B, xl, xh, r.sb_lo, r.sb_hi, r.ovf,
                                   r.queue + 1, r.idx, r.cnt, r.umask, r.cnt + 3, st));
    VC_TRY(vcm::zono_wide_union(dims, n, frag, bias_cat, B, xl, xh, r.sb_lo, r.sb_hi, r.ovf,
                                r.idx, r.cnt, r.umask, st));
    VC_TRY(vcm::union_lists(dims, n, r.umask, r.uidx, r.umeta, st));
  }
  if (crown_ev0 && hipEventRecord((hipEvent_t)crown_ev0, st) != hipSuccess) return VC_ERR_LAUNCH;
  // the round reads only the spec bound of the CROWN pass (alpha restarts
  // from the zonotope bounds): the rows form writes no CROWN bounds
  if (r.rws)
    VC_TRY(vcm::crown_rows_premasked(dims, n, frag, bias_cat, B, xl, xh, r.sb_lo, r.sb_hi, Q,
                                     spec_rows, spec_acc, lb, A, acc, seed_rows, r.rws,
                                     r.rws_bytes, st));
  else
    VC_TRY(vc_mlp_tiled_crown(dims, n, frag, bias_cat, B, xl, xh, r.sb_lo, r.sb_hi, r.t_lo,
                              r.t_hi, r.uidx, r.umeta, 1, 1, Q, spec_rows, spec_acc, lb, A,
                              acc, seed_rows, r.queue, stream));
  if (crown_ev1 && hipEventRecord((hipEvent_t)crown_ev1, st) != hipSuccess) return VC_ERR_LAUNCH;
  // with alpha, the closure also lists the open leaves (their order is
  // immaterial: each leaf's alpha is its own, and their bounds go back by
  // index), counted in cnt[3], which the zonotope pass's init cleared
  if (alpha_iters > 0)
    VC_TRY(vcm::closure_open(lb, B, Q, d_ptr, q_idx, n_disj, closed, r.idx, r.cnt + 3, st));
  else
    VC_TRY(vc_closure(lb, B, Q, d_ptr, q_idx, n_disj, closed, stream));
  VC_TRY(mark(phase_ev, 1, st));

  // ---- alpha-CROWN on the open leaves, from their zonotope bounds
  phase = PH_ALPHA;
  int64_t n_open = 0, n_eval = 0;
  if (alpha_iters > 0) {
    VC_TRY(read_counts(r.cnt + 3, 1, &n_open, pinned, st));
    if (n_open > 0) {
      const float* gin[2 * MAXL + 2];
      float* gout[2 * MAXL + 2];
      int32_t gcols[2 * MAXL + 2];
      for (int l = 0; l < n; ++l) {
        gin[2 * l] = r.sb_lo[l];
        gin[2 * l + 1] = r.sb_hi[l];
        gout[2 * l] = r.a_lo[l];
        gout[2 * l + 1] = r.a_hi[l];
        gcols[2 * l] = gcols[2 * l + 1] = dims[l + 1];
      }
      gin[2 * n] = xl;
      gin[2 * n + 1] = xh;
      gout[2 * n] = r.a_xl;
      gout[2 * n + 1] = r.a_xh;
      gcols[2 * n] = gcols[2 * n + 1] = n_in;
      VC_TRY(gather(gin, gout, gcols, 2 * n + 2, r.idx, n_open, stream));
      float *alpha[MAXL], *m1[MAXL], *m2[MAXL];
      int64_t off = 0;
      for (int l = 0; l < n; ++l) {
        const int64_t sz = n_open * dims[l + 1];
        alpha[l] = r.a_state + off;
        m1[l] = r.a_state + (int64_t)sumd * n_open + off;
        m2[l] = r.a_state + 2 * (int64_t)sumd * n_open + off;
        off += sz;
      }
      if (stop_host) {
        reinterpret_cast<volatile int32_t*>(stop_host)[0] = 0;
        reinterpret_cast<volatile int32_t*>(stop_host)[1] = 0;
      }
      VC_TRY(vc_mlp_tiled_alpha_run(dims, n, frag, bias_cat, n_open, r.a_xl, r.a_xh, r.a_lo,
                                    r.a_hi, alpha, m1, m2, Q, spec_rows, spec_acc, r.a_lb,
                                    r.a_best, 0.9, 0.999, 1e-8, alpha_lr, alpha_lr_decay,
                                    alpha_iters, alpha_early_stop, r.a_ctl, stop_host, stream));
      // the open leaves are distinct rows (a compaction's output)
      VC_TRY(vcm::scatter_max_close(lb, r.idx, r.a_best, n_open, Q, d_ptr, q_idx, n_disj, closed,
                                    st));
    }
  }

  VC_TRY(mark(phase_ev, 2, st));

  // ---- the unclosed leaves (and alpha's evaluation count with them)
  phase = PH_CLIP;
  VC_TRY(vc_compact(closed, B, 1, unclosed, r.cnt, r.cws, r.cws_bytes, stream));
  int64_t n_unc = 0;
  if (n_open > 0) {
    int64_t two[2];
    VC_TRY(read_counts(r.cnt, 1, two, pinned, st, r.a_ctl));
    n_unc = two[0];
    n_eval = two[1];
  } else {
    VC_TRY(read_counts(r.cnt, 1, &n_unc, pinned, st));
  }

  // ---- clip, widest axis and bisection of the feasible leaves
  int64_t nf = 0, nu = 0;
  if (n_unc > 0) {
    float* gout[4] = {r.u_xl, r.u_xh, r.u_A, r.u_acc};
    const float* gin[4] = {xl, xh, A, acc};
    const int32_t gcols[4] = {n_in, n_in, Q * n_in, Q};
    VC_TRY(gather(gin, gout, gcols, 4, unclosed, n_unc, stream));
    VC_TRY(vc_clip_box(r.u_xl, r.u_xh, r.u_A, r.u_acc, n_unc, Q, n_in, d_ptr, q_idx, n_disj,
                       r.c_xl, r.c_xh, feasible, stream));
    if (clip_widths) {
      const int64_t nv = n_unc * n_in;
      const int blocks = (int)std::min<int64_t>((nv + 255) / 256, 1024);
      hipLaunchKernelGGL(k_clip_widths, dim3(blocks), dim3(256), 0, st, r.u_xl, r.u_xh, r.c_xl,
                         r.c_xh, nv, clip_widths);
      if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
    }
    VC_TRY(vc_widest_axis(r.c_xl, r.c_xh, n_unc, n_in, r.ax_u, r.usable, stream));
    // the feasible leaves, and the feasible ones with a usable split axis
    VC_TRY(vcm::compact_feasible_split(feasible, r.usable, n_unc, r.idx, r.cnt, r.idx2,
                                       r.cnt + 1, r.split, r.cws, r.cws_bytes, st));
    int64_t two[2];
    VC_TRY(read_counts(r.cnt, 2, two, pinned, st));
    nf = two[0];
    nu = two[1];
    if (nf > 0) {
      // the int64 axes travel as float pairs through the row gather (bit copy)
      const float* fin[3] = {r.c_xl, r.c_xh, reinterpret_cast<const float*>(r.ax_u)};
      float* fout[3] = {xl_split, xh_split, reinterpret_cast<float*>(ax)};
      const int32_t fcols[3] = {n_in, n_in, 2};
      VC_TRY(gather(fin, fout, fcols, 3, r.idx, nf, stream));
    }
  }
  VC_TRY(mark(phase_ev, 3, st));
  phase = PH_SPLIT;
  if (nu > 0)
    VC_TRY(vc_bisect(r.c_xl, r.c_xh, r.ax_u, r.idx2, nu, n_in, low_xl, low_xh, high_xl,
                     high_xh, stream));
  VC_TRY(mark(phase_ev, 4, st));
  counts[0] = n_open;
  counts[1] = n_eval;
  counts[2] = n_unc;
  counts[3] = nf;
  counts[4] = nu;
  counts[5] = nf - nu;
  return VC_OK;
}

}  // namespace

extern "C" int vc_mlp_bab_round(const int32_t* dims, int n_relu, const float* frag,
                                const float* bias_cat, int Q, const float* spec_rows,
                                const float* spec_acc, const int32_t* d_ptr,
                                const int32_t* q_idx, int n_disj, int64_t B, const float* xl,
                                const float* xh, int alpha_iters, double alpha_lr,
                                double alpha_lr_decay, double alpha_early_stop, float* lb,
                                float* A, float* acc, uint8_t* closed, int64_t* unclosed,
                                uint8_t* feasible, float* xl_split, float* xh_split, int64_t* ax,
                                float* low_xl, float* low_xh, float* high_xl, float* high_xh,
                                uint64_t* seed_rows, void* crown_ev0, void* crown_ev1,
                                void* const* phase_ev, double* clip_widths, void* work,
                                int64_t work_bytes, int32_t* stop_host, int64_t* pinned,
                                int64_t* counts, int32_t* fail_phase, vc_stream_t stream) {
  int phase = PH_BOUND;
  const int rc = bab_round(dims, n_relu, frag, bias_cat, Q, spec_rows, spec_acc, d_ptr, q_idx,
                           n_disj, B, xl, xh, alpha_iters, alpha_lr, alpha_lr_decay,
                           alpha_early_stop, lb, A, acc, closed, unclosed, feasible, xl_split,
                           xh_split, ax, low_xl, low_xh, high_xl, high_xh, seed_rows,
                           crown_ev0, crown_ev1, phase_ev, clip_widths, work, work_bytes,
                           stop_host, pinned, counts, phase, stream);
  if (fail_phase) *fail_phase = rc == VC_OK ? -1 : phase;
  return rc;
}
