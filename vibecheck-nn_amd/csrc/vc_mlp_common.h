// Helpers shared by the whole-network MLP kernels (vc_mlp_fused.hip,
// vc_mlp_tiled.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <utility>
#include <vector>

namespace vcm {

constexpr int FW = 64;    // max layer width
constexpr int MAXL = 16;  // max relu layers

// K-steps of a 16x16x4 MFMA chain over dk neurons in the permuted order
// (K-step (t, i) contracts neuron 16 t + 4 g + i in lane group g).
__host__ __device__ inline int ks_count(int dk) {
  const int T = (dk + 15) / 16;
  const int last = dk - 16 * (T - 1);
  return 4 * (T - 1) + (last < 4 ? last : 4);
}

// Copy n4 float4s (16-byte aligned) from global memory into LDS, eight
// loads in flight per thread (no barrier: the caller synchronises).
__device__ __forceinline__ void stage_float4(float* dst_lds, const float* src, int n4) {
  const float4* s = reinterpret_cast<const float4*>(src);
  float4* d = reinterpret_cast<float4*>(dst_lds);
  const int bs = blockDim.x;
  int e = threadIdx.x;
  for (; e + 7 * bs < n4; e += 8 * bs) {
    float4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = s[e + k * bs];
#pragma unroll
    for (int k = 0; k < 8; ++k) d[e + k * bs] = v[k];
  }
  for (; e < n4; e += bs) d[e] = s[e];
}

// Dynamic domain queue: lane 0 of a wavefront takes the next ticket with a
// vector atomic; callers take the following ticket while they process the
// current domain and broadcast it (queue_bcast) only when they need it.
__device__ __forceinline__ int queue_take(int* q, int lane) {
  return lane == 0 ? atomicAdd(q, 1) : 0;
}
__device__ __forceinline__ int64_t queue_bcast(int t) { return (int64_t)__shfl(t, 0, 64); }

// Orders a wavefront's own LDS writes before its later LDS reads of them,
// for LDS that no other wavefront touches: a wavefront's LDS instructions
// execute in issue order, so keeping the compiler from reordering them is
// all that is needed.  A wavefront-scope fence does that and emits no
// wait; __threadfence_block() (workgroup scope) also waits for the wave's
// outstanding global stores (s_waitcnt vmcnt(0)) at every use.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}


// The input-split round's bound phase with the CROWN rows pass's per-domain
// seed masks and union of unstable sets written by the zonotope passes
// (vc_mlp_tiled.hip): rows_work is the vc_mlp_crown_rows workspace of the
// same B that crown_rows_premasked then runs in (per_domain, no index
// lists, no CROWN bounds out), skipping its own pass over the bounds.
// ovf_list / ovf_count (nullable together): the domains the one-wavefront
// pass leaves to the wide pass, appended in no particular order, and their
// count (the wide pass's list, with no compaction of the flags).
// clear_count (nullable): a counter cleared by the pass's init launch.
int zono_bounds_masked(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                       int64_t B, const float* xl, const float* xh, float* const* lo_out,
                       float* const* hi_out, uint8_t* overflow, int32_t* queue, void* rows_work,
                       int64_t* ovf_list, int64_t* ovf_count, int64_t* clear_count,
                       hipStream_t st);
// The zonotope passes with the overflow list and (umask, nullable) the
// union of the unstable sets as bit masks [n_relu], without seed masks; and
// union_lists: vc_union_compact's index lists from that union.
int zono_bounds_listed(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                       int64_t B, const float* xl, const float* xh, float* const* lo_out,
                       float* const* hi_out, uint8_t* overflow, int32_t* queue,
                       int64_t* ovf_list, int64_t* ovf_count, unsigned long long* umask,
                       int64_t* clear_count, hipStream_t st);
int zono_wide_union(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                    int64_t B, const float* xl, const float* xh, float* const* lo_out,
                    float* const* hi_out, uint8_t* overflow, const int64_t* list,
                    const int64_t* n_list, unsigned long long* umask, hipStream_t st);
int union_lists(const int32_t* dims, int n_relu, const unsigned long long* umask, int32_t* idx,
                int32_t* meta, hipStream_t st);
int zono_wide_masked(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
                     int64_t B, const float* xl, const float* xh, float* const* lo_out,
                     float* const* hi_out, uint8_t* overflow, const int64_t* list,
                     const int64_t* n_list, void* rows_work, hipStream_t st);
int crown_rows_premasked(const int32_t* dims, int n_relu, const float* frag,
                         const float* bias_cat, int64_t B, const float* xl, const float* xh,
                         const float* const* lo_in, const float* const* hi_in, int Q,
                         const float* spec_rows, const float* spec_acc, float* lb_out,
                         float* A_out, float* acc_out, uint64_t* seed_rows, void* work,
                         int64_t work_bytes, hipStream_t st);

// vc_closure that also lists the open rows, in no particular order, and
// counts them in *open_cnt, which the caller clears (vc_elementwise.hip).
int closure_open(const float* lb, int64_t B, int Q, const int32_t* d_ptr, const int32_t* q_idx,
                 int n_disj, uint8_t* closed, int64_t* open_idx, int64_t* open_cnt,
                 hipStream_t st);

// vc_scatter_max_rows then vc_closure, for distinct rows idx: one launch
// that redoes the closure of the scattered rows only (vc_elementwise.hip).
int scatter_max_close(float* lb, const int64_t* idx, const float* src, int64_t nr, int Q,
                      const int32_t* d_ptr, const int32_t* q_idx, int n_disj, uint8_t* closed,
                      hipStream_t st);

// The input-split round's two compactions after the clip (vc_elementwise.hip):
// the feasible rows (idx_f, cnt_f) and the feasible rows with a usable split
// axis (idx_s, cnt_s), in one launch up to 2^17 rows; split_tmp (n bytes)
// is used above that.
// vc_mlp_tiled_alpha_run with the small-batch kernel's workgroups held to
// cu_budget compute units' worth (0: the whole device).
int alpha_run(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat,
              int64_t B, const float* xl, const float* xh, const float* const* lo,
              const float* const* hi, float* const* alpha, float* const* exp_avg,
              float* const* exp_avg_sq, int Q, const float* spec_rows, const float* spec_acc,
              float* lb_out, float* best, double b1, double b2, double eps, double lr,
              double lr_decay, int n_iters, double early_stop_eps, float* ctl,
              int32_t* stop_host, int cu_budget, vc_stream_t stream);

int compact_feasible_split(const uint8_t* feasible, const uint8_t* usable, int64_t n,
                           int64_t* idx_f, int64_t* cnt_f, int64_t* idx_s, int64_t* cnt_s,
                           uint8_t* split_tmp, void* ws, int64_t ws_bytes, hipStream_t st);

// Compute units of the current device (read once per device).
inline int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Raise a kernel's dynamic LDS limit to what the CU holds (160 KB less its
// static LDS), once per kernel and device: the attribute call would
// otherwise cost host time on every launch.
inline bool allow_max_lds(const void* fn) {
  static std::mutex mu;
  static std::vector<std::pair<const void*, int>> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& e : done)
    if (e.first == fn && e.second == dev) return true;
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, fn) != hipSuccess) return false;
  const int cap = 160 * 1024 - (int)attr.sharedSizeBytes;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, cap) != hipSuccess)
    return false;
  done.emplace_back(fn, dev);
  return true;
}

// Persistent grid: as many workgroups as fit on the CUs at once given the
// LDS footprint (160 KB per CU, at most two per CU), capped by the work
// (B domains, nwave per workgroup).
inline int persistent_grid(int64_t B, size_t lds_bytes, int nwave) {
  int per_cu = (int)((160 * 1024) / (lds_bytes > 0 ? lds_bytes : 1));
  if (per_cu < 1) per_cu = 1;
  if (per_cu > 2) per_cu = 2;
  int64_t grid = (int64_t)cu_count() * per_cu;
  const int64_t need = (B + nwave - 1) / nwave;
  if (need < grid) grid = need;
  return (int)(grid < 1 ? 1 : grid);
}

}  // namespace vcm
