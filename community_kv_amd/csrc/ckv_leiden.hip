// Batched Leiden over G vertex-disjoint graphs, one level per call, plus the
// two helpers of the multi-level driver (COO aggregation, per-graph label
// densification).  Restates the reference's graph/leiden/_csrc (leiden.cu
// 43-205, local_moving.cu 69-210, refinement.cu 71-300, csr.cu 20-271,
// aggregate.cu 24-184, helpers.cu 9-122) for MI355X:
//
//   * one wave64 per vertex; the vertex's neighbour communities are gathered
//     into a per-wave LDS table by a leader loop (a chunk of 64 row entries at
//     a time, ballot per distinct community, fp64 butterfly sum), so sums are
//     formed in one fixed order and a low-degree vertex touches only its row;
//   * the sweep loops run without host round trips: every sweep's kernels
//     are queued up front and read a device control word (moved count,
//     up/down direction, stall count, done flag) that a one-wave control
//     kernel advances after each sweep, so converged sweeps exit at once;
//   * the symmetric CSR is one stable radix sort of (src, dst) keys, rows
//     ordered by neighbour id.
//
// Move rules follow the reference: synchronous moves on a snapshot, gain
//   dQ = (k_v,new - k_v,old)/m + gamma k_v (Sigma_old - k_v - Sigma_new)/(2 m^2),
// neighbour-community weights rounded to float, the per-vertex jitter and the
// per-sweep rank of the reference's PCG hash (rng.cuh), the up/down gate in
// local moving, the well-connectedness gate and the independent-set commit in
// refinement.  Equal float scores are broken by the order in which the
// reference's 1024-slot table scan prefers a community's home slot, then by
// smaller id.  A vertex keeps at most TABLE_CAP distinct neighbour
// communities (the reference's table size), in order of first appearance.
//
// Launch sequence of ckv_batched_leiden (one stream, no host sync):
//   mirror_kernel, radix sort, row_ptr_kernel, col_kernel, zero_kernel, hub_list_kernel, degree_kernel,
//   graph_sum_kernel (2m), identity_kernel
//   local moving x max_inner_iter: sigma_zero, sigma_scatter, local_moving_kernel (small rows, then
//                                  hubs), local_moving_giant_kernel, lm_control_kernel
//   refine_init_kernel, parent sigma
//   refinement x max_inner_iter: sigma_zero, sigma_scatter, refine_propose_kernel (small, hubs),
//                                refine_propose_giant_kernel,
//                                refine_commit_kernel, refine_control_kernel
//   sigma of the result, modularity_kernel, graph_sum_kernel, finish_kernel (labels, -1 for isolated)
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <stdint.h>

#include "ckv_amd.h"
#include "ckv_error.h"

namespace ckv {
namespace {

constexpr int LWAVES = 4;        // vertices (waves) per workgroup
constexpr int LTHREADS = 64 * LWAVES;
constexpr int TABLE_CAP = 1024;  // distinct neighbour communities per vertex
constexpr int ETHREADS = 256;

enum { CTL_MOVED = 0,  // nonzero once a vertex moved in the current sweep
       CTL_UPDOWN = 1, CTL_STALE = 2, CTL_DONE = 3,
       CTL_OVERFLOW = 4,  // nonzero when a workgroup table overflowed (a broken table bound)
       CTL_WORDS = 8 };

// ----------------------------------------------------------------- hashing (rng.cuh)
__device__ __host__ inline uint32_t pcg_hash(uint32_t x) {
  const uint32_t state = x * 747796405u + 2891336453u;
  const uint32_t word = ((state >> ((state >> 28u) + 4u)) ^ state) * 277803737u;
  return (word >> 22u) ^ word;
}
__device__ inline uint32_t mix4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  uint32_t h = pcg_hash(a);
  h = pcg_hash(h ^ b);
  h = pcg_hash(h ^ c);
  return pcg_hash(h ^ d);
}
__device__ inline float unit_float(uint32_t h) { return (float)(h >> 8) * (1.0f / 16777216.0f); }
__device__ inline float rand_uniform(uint32_t g, uint32_t v, uint32_t level, uint32_t sweep, uint32_t seed) {
  return unit_float(mix4(g, v, (level << 16) | sweep, seed));
}
__device__ inline float rand_uniform_pair(uint32_t g, uint32_t v, uint32_t c, uint32_t level, uint32_t sweep,
                                          uint32_t seed) {
  const uint32_t s = pcg_hash((sweep << 16) ^ c);
  return unit_float(mix4(g, v, (level << 16) | (s & 0xFFFFu), seed));
}
__device__ inline float gumbel(float u) {
  u = fmaxf(u, 1.0e-7f);
  u = fminf(u, 1.0f - 1.0e-7f);
  return -logf(-logf(u));
}

// Tie preference among equal scores (larger wins): the reference scans home
// slot s = pcg_hash(c) & 1023 with thread s & 127 (slice index s >> 7, first
// strict maximum kept) and reduces lanes, then warps, with 32-lane
// shuffle-down trees that keep their own value on ties; then the smaller id.
__device__ inline uint32_t bitrev5(uint32_t x) { return __builtin_bitreverse32(x) >> 27; }
__device__ inline uint32_t cand_pref(int32_t c) {
  const uint32_t s = pcg_hash((uint32_t)c) & 1023u;
  const uint32_t key = (bitrev5((s >> 5) & 3u) << 8) | (bitrev5(s & 31u) << 3) | (s >> 7);
  return ((8191u - key) << 18) | (0x3FFFFu - ((uint32_t)c & 0x3FFFFu));
}
constexpr uint32_t STAY_PREF = 0xFFFFFFFFu;  // staying wins every tie
__device__ inline uint32_t ordered(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline uint64_t pack(float score, uint32_t pref) { return ((uint64_t)ordered(score) << 32) | pref; }

// ----------------------------------------------------------------- wave helpers
__device__ inline int lane() { return (int)__lane_id(); }
__device__ inline double wave_sum_f64(double x) {
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}
__device__ inline uint64_t wave_max_u64(uint64_t x) {
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t y = (uint64_t)__shfl_xor((long long)x, o);
    x = y > x ? y : x;
  }
  return x;
}
__device__ inline int first_lane(uint64_t m) { return __ffsll((long long)m) - 1; }

// The control kernels only test the moved word for zero: set it once per
// sweep (read first, so that later movers do not queue writes to one line).
__device__ inline void mark_moved(int32_t* ctl) {
  if (__hip_atomic_load(ctl + CTL_MOVED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0)
    __hip_atomic_store(ctl + CTL_MOVED, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Neighbour-community table of vertex v over its row [a, b): self loops
// skipped; with `parent`, only neighbours u with parent[u] == pv.  Returns the
// number of table slots to scan (wave-uniform; empty slots hold -1); *e_sum
// gets the summed weight of the admitted entries (every lane).
//
// Rows of at most CAP entries (all rows the per-wave kernels take): every
// lane inserts its neighbour's community into an open-addressing table of
// min(2 x degree, CAP) slots (LDS compare-and-swap) and adds its weight with an
// LDS f64 atomic.  Longer rows (the workgroup kernels' fallback): a leader
// loop over the chunk's distinct communities, entries in order of first
// appearance along the row, later ones dropped once CAP are held.
template <int CAP>
__device__ int build_table(int32_t* tc, double* ts, const int32_t* __restrict__ col,
                           const float* __restrict__ wt, const int32_t* __restrict__ lab,
                           const int32_t* __restrict__ parent, int32_t pv, int32_t v, int32_t a, int32_t b,
                           double* e_sum) {
  const int ln = lane();
  double e_acc = 0.0;
  if (b - a <= CAP) {  // at most CAP distinct communities: no capacity rule to apply
    int size = 64;
    while (size < 2 * (b - a) && size < CAP) size <<= 1;
    for (int j = ln; j < size; j += 64) {
      tc[j] = -1;
      ts[j] = 0.0;
    }
    __builtin_amdgcn_wave_barrier();
    for (int32_t e0 = a; e0 < b; e0 += 64) {
      const int32_t e = e0 + ln;
      bool ok = e < b;
      const int32_t u = ok ? col[e] : v;
      ok = ok && u != v;
      if (parent) ok = ok && parent[u] == pv;
      if (ok) {
        const float w = wt[e];
        const int32_t c = lab[u];
        e_acc += (double)w;
        uint32_t h = pcg_hash((uint32_t)c) & (uint32_t)(size - 1);
        while (true) {
          const int32_t cur = __hip_atomic_load(tc + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          if (cur == c) break;
          if (cur == -1) {
            const int32_t prev = atomicCAS(tc + h, -1, c);
            if (prev == -1 || prev == c) break;
          }
          h = (h + 1) & (uint32_t)(size - 1);
        }
        unsafeAtomicAdd(ts + h, (double)w);
      }
    }
    __builtin_amdgcn_wave_barrier();
    *e_sum = wave_sum_f64(e_acc);
    return size;
  }
  int n = 0;
  for (int32_t e0 = a; e0 < b; e0 += 64) {
    const int32_t e = e0 + ln;
    bool ok = e < b;
    const int32_t u = ok ? col[e] : v;
    ok = ok && u != v;
    const float w = ok ? wt[e] : 0.0f;
    if (parent) ok = ok && parent[u] == pv;
    const int32_t c = ok ? lab[u] : -1;
    if (ok) e_acc += (double)w;
    uint64_t active = __ballot(ok);
    while (active) {
      const int32_t c0 = __shfl(c, first_lane(active));
      const uint64_t m = __ballot(ok && c == c0);
      const double s = wave_sum_f64(((m >> ln) & 1) ? (double)w : 0.0);
      int idx = -1;
      for (int j0 = 0; j0 < n; j0 += 64) {
        const int j = j0 + ln;
        const uint64_t hit = __ballot(j < n && tc[j] == c0);
        if (hit) {
          idx = j0 + first_lane(hit);
          break;
        }
      }
      if (idx < 0 && n < CAP) {
        idx = n++;
        if (ln == 0) {
          tc[idx] = c0;
          ts[idx] = 0.0;
        }
      }
      if (idx >= 0 && ln == 0) ts[idx] += s;
      __builtin_amdgcn_wave_barrier();
      active &= ~m;
    }
  }
  *e_sum = wave_sum_f64(e_acc);
  return n;
}

__device__ float table_lookup(const int32_t* tc, const double* ts, int n, int32_t c) {
  for (int j0 = 0; j0 < n; j0 += 64) {
    const int j = j0 + lane();
    const uint64_t hit = __ballot(j < n && tc[j] == c && c >= 0);
    if (hit) return (float)ts[j0 + first_lane(hit)];
  }
  return 0.0f;
}

// ----------------------------------------------------------------- CSR build
__global__ void mirror_kernel(const int32_t* __restrict__ src, const int32_t* __restrict__ dst,
                              const float* __restrict__ w, int64_t E, int32_t V, int bits,
                              uint64_t* __restrict__ keys, float* __restrict__ vals) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E) return;
  const int32_t u = src[i], t = dst[i];
  const float wi = w[i];
  const uint64_t sentinel = (uint64_t)V << bits;
  const bool ok = u >= 0 && u < V && t >= 0 && t < V;  // out-of-range edges are dropped
  keys[2 * i] = ok ? ((uint64_t)u << bits) | (uint64_t)t : sentinel;
  vals[2 * i] = u == t ? 2.0f * wi : wi;
  keys[2 * i + 1] = (ok && u != t) ? ((uint64_t)t << bits) | (uint64_t)u : sentinel;
  vals[2 * i + 1] = wi;
}

__global__ void row_ptr_kernel(const uint64_t* __restrict__ keys, int64_t n, int32_t V, int bits,
                               int32_t* __restrict__ row_ptr) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v > V) return;
  const uint64_t target = (uint64_t)v << bits;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < target) lo = mid + 1;
    else hi = mid;
  }
  row_ptr[v] = (int32_t)lo;
}

__global__ void col_kernel(const uint64_t* __restrict__ keys, int64_t n, int bits, int32_t* __restrict__ col) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) col[i] = (int32_t)(keys[i] & (((uint64_t)1 << bits) - 1));
}

__global__ void zero_kernel(double* __restrict__ two_m, int32_t G, double* __restrict__ modularity,
                            int32_t* __restrict__ ctl, int32_t* __restrict__ hub_count,
                            int32_t* __restrict__ giant_count) {
  const int i = threadIdx.x;
  for (int g = i; g < G; g += blockDim.x) {
    two_m[g] = 0.0;
    modularity[g] = 0.0;
  }
  if (i < CTL_WORDS) ctl[i] = i == CTL_UPDOWN ? 1 : 0;  // local moving starts with upward moves
  if (i == 0) {
    *hub_count = 0;
    *giant_count = 0;
  }
}

__global__ __launch_bounds__(LTHREADS) void degree_kernel(const int32_t* __restrict__ row_ptr,
                                                          const float* __restrict__ wt, int32_t V, int32_t S,
                                                          double* __restrict__ k_v) {
  const int32_t v = blockIdx.x * LWAVES + (threadIdx.x >> 6);
  if (v >= V) return;
  const int32_t a = row_ptr[v], b = row_ptr[v + 1];
  double s = 0.0;
  for (int32_t e = a + lane(); e < b; e += 64) s += (double)wt[e];
  s = wave_sum_f64(s);
  if (lane() == 0) k_v[v] = s;
}

// out[g] = sum of x over graph g's S vertices (one workgroup per graph, fixed
// order: strided per-thread sums, then a tree over the threads).
__global__ __launch_bounds__(256) void graph_sum_kernel(const double* __restrict__ x, int32_t S,
                                                        double* __restrict__ out) {
  __shared__ double part[256];
  const int32_t g = blockIdx.x;
  double s = 0.0;
  for (int32_t i = threadIdx.x; i < S; i += 256) s += x[(int64_t)g * S + i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[g] = part[0];
}

__global__ void identity_kernel(int32_t V, int32_t* __restrict__ labels) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v < V) labels[v] = v;
}

// ----------------------------------------------------------------- sweeps
__global__ void sigma_zero_kernel(double* __restrict__ sigma, int32_t V, const int32_t* __restrict__ ctl) {
  if (ctl && ctl[CTL_DONE]) return;
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v < V) sigma[v] = 0.0;
}

__global__ void sigma_scatter_kernel(const int32_t* __restrict__ labels, const double* __restrict__ k_v, int32_t V,
                                     double* __restrict__ sigma, const int32_t* __restrict__ ctl) {
  if (ctl && ctl[CTL_DONE]) return;
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= V) return;
  const int32_t c = labels[v];
  const double k = k_v[v];
  if (c >= 0 && k != 0.0) unsafeAtomicAdd(sigma + c, k);
}

struct Graph {
  const int32_t* row_ptr;
  const int32_t* col;
  const float* wt;
  const double* k_v;
  const double* two_m;
  int32_t V;
  int32_t S;
};

template <int CAP>
__device__ void local_moving_vertex(const Graph& gr, const double* __restrict__ sigma, const int32_t* __restrict__ lin,
                                    int32_t* __restrict__ lout, int32_t* __restrict__ ctl, float resolution,
                                    uint32_t level, uint32_t sweep, uint32_t seed, int32_t v, int32_t* tc,
                                    double* ts) {
  const int32_t old = lin[v];
  const bool done = ctl[CTL_DONE] != 0;
  const int32_t a = gr.row_ptr[v], b = gr.row_ptr[v + 1];
  const int32_t g = v / gr.S;
  const double tm = gr.two_m[g];
  if (done || a == b || !(tm > 0.0)) {
    if (lane() == 0) lout[v] = old;
    return;
  }
  const int up_down = ctl[CTL_UPDOWN];
  double e_sum;
  const int n = build_table<CAP>(tc, ts, gr.col, gr.wt, lin, nullptr, 0, v, a, b, &e_sum);
  const float k_old = table_lookup(tc, ts, n, old);
  const double kv = gr.k_v[v];
  const double m_g = 0.5 * tm;
  const double inv_m = 1.0 / m_g;
  const double inv_2m2 = 1.0 / (2.0 * m_g * m_g);
  const double sig_old_excl = sigma[old] - kv;
  const float jitter = (rand_uniform((uint32_t)g, (uint32_t)v, level, sweep, seed) - 0.5f) * 1e-9f;
  uint64_t mine = 0;
  int32_t mine_c = old;
  // every slot's community total is loaded before any is used, so a lane's
  // gathers are in flight together
  constexpr int PER = CAP / 64;
  int32_t cs[PER];
  double sg[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int j = lane() + 64 * k;
    const int32_t c = j < n ? tc[j] : -1;
    cs[k] = (c < 0 || c == old || (c > old ? 1 : 0) != up_down) ? -1 : c;
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) sg[k] = cs[k] >= 0 ? sigma[cs[k]] : 0.0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int32_t c = cs[k];
    if (c < 0) continue;
    const float kn = (float)ts[lane() + 64 * k];
    const double dq = ((double)kn - (double)k_old) * inv_m
                      + (double)resolution * kv * (sig_old_excl - sg[k]) * inv_2m2;
    const float dqf = (float)dq + jitter;
    const uint64_t p = pack(dqf, cand_pref(c));
    if (p > mine) {
      mine = p;
      mine_c = c;
    }
  }
  const uint64_t best = wave_max_u64(mine);
  int32_t choice = old;
  if (best > pack(0.0f, STAY_PREF)) choice = __shfl(mine_c, first_lane(__ballot(mine == best)));
  if (lane() == 0) {
    lout[v] = choice;
    if (choice != old) mark_moved(ctl);
  }
}

// After a local-moving sweep: a stalled sweep flips the direction, two in a
// row end local moving (leiden.cu:113-135).
__global__ void lm_control_kernel(int32_t* __restrict__ ctl) {
  if (threadIdx.x != 0) return;
  if (!ctl[CTL_DONE]) {
    if (ctl[CTL_MOVED] == 0) {
      ctl[CTL_UPDOWN] ^= 1;
      if (++ctl[CTL_STALE] >= 2) ctl[CTL_DONE] = 1;
    } else {
      ctl[CTL_STALE] = 0;
    }
  }
  ctl[CTL_MOVED] = 0;
}

__global__ void refine_init_kernel(const int32_t* __restrict__ lm, int32_t V, int32_t* __restrict__ parent,
                                   int32_t* __restrict__ labels, int32_t* __restrict__ ctl) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v < V) {
    parent[v] = lm[v];
    labels[v] = v;
  }
  if (v < CTL_WORDS && v != CTL_OVERFLOW) ctl[v] = 0;  // an overflow of the local-moving sweeps stays raised
}

// Test hook: raises the overflow word as a broken local-moving table would.
__global__ void raise_overflow_kernel(int32_t* __restrict__ ctl) {
  if (threadIdx.x == 0) ctl[CTL_OVERFLOW] = 1;
}

template <int CAP>
__device__ void refine_propose_vertex(const Graph& gr, const int32_t* __restrict__ parent,
                                      const double* __restrict__ sigma, const double* __restrict__ parent_sigma,
                                      const int32_t* __restrict__ lin, int32_t* __restrict__ prop,
                                      uint32_t* __restrict__ rank, float resolution, float inv_theta, int boltzmann,
                                      uint32_t level, uint32_t sweep, uint32_t seed, int32_t v, int32_t* tc,
                                      double* ts) {
  const int32_t g = v / gr.S;
  if (lane() == 0) rank[v] = mix4((uint32_t)g, (uint32_t)v, (level << 16) | sweep, seed);
  const int32_t old = lin[v];
  const int32_t a = gr.row_ptr[v], b = gr.row_ptr[v + 1];
  const double tm = gr.two_m[g];
  if (a == b || !(tm > 0.0)) {
    if (lane() == 0) prop[v] = old;
    return;
  }
  const int32_t pv = parent[v];
  double e_sum;
  const int n = build_table<CAP>(tc, ts, gr.col, gr.wt, lin, parent, pv, v, a, b, &e_sum);
  const double kv = gr.k_v[v];
  double vol_minus = parent_sigma[pv] - kv;
  if (vol_minus < 0.0) vol_minus = 0.0;
  const double bound = (double)resolution * kv * vol_minus / tm;
  if ((double)(float)e_sum < bound) {  // {v} is not well connected to its parent community
    if (lane() == 0) prop[v] = old;
    return;
  }
  const float k_old = table_lookup(tc, ts, n, old);
  const double m_g = 0.5 * tm;
  const double inv_m = 1.0 / m_g;
  const double inv_2m2 = 1.0 / (2.0 * m_g * m_g);
  const double sig_old_excl = sigma[old] - kv;
  uint64_t mine = 0;
  int32_t mine_c = old;
  constexpr int PER = CAP / 64;  // community totals gathered together, as in local moving
  int32_t cs[PER];
  double sg[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int j = lane() + 64 * k;
    const int32_t c = j < n ? tc[j] : -1;
    cs[k] = (c < 0 || c == old) ? -1 : c;
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) sg[k] = cs[k] >= 0 ? sigma[cs[k]] : 0.0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int32_t c = cs[k];
    if (c < 0) continue;
    const float kn = (float)ts[lane() + 64 * k];
    const double dq = ((double)kn - (double)k_old) * inv_m
                      + (double)resolution * kv * (sig_old_excl - sg[k]) * inv_2m2;
    if (dq < 0.0) continue;
    const float score = boltzmann
        ? (float)(dq * (double)inv_theta)
              + gumbel(rand_uniform_pair((uint32_t)g, (uint32_t)v, (uint32_t)c, level, sweep, seed))
        : (float)dq;
    const uint64_t p = pack(score, cand_pref(c));
    if (p > mine) {
      mine = p;
      mine_c = c;
    }
  }
  const uint64_t best = wave_max_u64(mine);
  const float stay = boltzmann
      ? gumbel(rand_uniform_pair((uint32_t)g, (uint32_t)v, (uint32_t)old, level, sweep, seed))
      : 0.0f;
  int32_t choice = old;
  if (best > pack(stay, STAY_PREF)) choice = __shfl(mine_c, first_lane(__ballot(mine == best)));
  if (lane() == 0) prop[v] = choice;
}

// Vertices with at most SMALL_CAP / 2 row entries (nearly all) run with a
// small LDS table and 8 waves per workgroup; the rest (hubs, listed once per
// call by hub_list_kernel) run with the full TABLE_CAP table, grid-striding
// over the list.
constexpr int SMALL_CAP = 256;
constexpr int SWAVES = 8;
constexpr int HUB_BLOCKS = 768;  // three 48 KB workgroups per CU

constexpr int GIANT_MIN = TABLE_CAP;  // rows longer than this take a whole workgroup
constexpr int GIANT_SLOTS = 4096;
constexpr int GIANT_THREADS = 1024;
constexpr int GIANT_BLOCKS = 512;  // two 65 KB workgroups per CU

__global__ void hub_list_kernel(const int32_t* __restrict__ row_ptr, int32_t V, int32_t* __restrict__ hubs,
                                int32_t* __restrict__ hub_count, int32_t* __restrict__ giants,
                                int32_t* __restrict__ giant_count) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t d = v < V ? row_ptr[v + 1] - row_ptr[v] : 0;
  const bool giant = d > GIANT_MIN, hub = !giant && d > SMALL_CAP / 2;
  const uint64_t mg = __ballot(giant), mh = __ballot(hub);  // one atomic per wave and list
  const uint64_t below = (((uint64_t)1) << lane()) - 1;
  int32_t bg = 0, bh = 0;
  if (lane() == 0) {
    if (mg) bg = atomicAdd(giant_count, __popcll(mg));
    if (mh) bh = atomicAdd(hub_count, __popcll(mh));
  }
  bg = __shfl(bg, 0);
  bh = __shfl(bh, 0);
  if (giant) giants[bg + __popcll(mg & below)] = v;
  if (hub) hubs[bh + __popcll(mh & below)] = v;
}

// Rows longer than GIANT_MIN: one 1024-thread workgroup per vertex.  All
// threads insert the row's neighbour communities into a GIANT_SLOTS-slot LDS
// table (sum of weights in f64, first row position by atomic min); when more
// than TABLE_CAP communities appear, a binary search on the first positions
// keeps exactly the TABLE_CAP that appear first along the row (the rule of
// the per-wave tables).  The row is walked in position order, GIANT_THREADS
// entries at a time, and no community is inserted once TABLE_CAP are held, so
// the table never holds more than 2 x TABLE_CAP - 1.  The candidates are
// scored across the workgroup.  (giant_table reports an overflow only if the
// table bound above were broken; the vertex then stays where it is.)
struct GiantShared {
  int32_t c[GIANT_SLOTS];
  double s[GIANT_SLOTS];
  int32_t first[GIANT_SLOTS];
  uint64_t best[GIANT_THREADS / 64];
  int32_t best_c[GIANT_THREADS / 64];
  double red[GIANT_THREADS / 64];
  int32_t n, overflow, count, k_old_slot;
};

__device__ inline double block_sum_giant(double x, GiantShared& sh) {
  x = wave_sum_f64(x);
  if (lane() == 0) sh.red[threadIdx.x >> 6] = x;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < GIANT_THREADS / 64; ++i) t += sh.red[i];
  __syncthreads();
  return t;
}

// Returns false when the table overflowed (caller falls back); on success
// *thr bounds the kept first positions and *e_sum is the admitted weight.
template <bool REFINE>
__device__ bool giant_table(const Graph& gr, const int32_t* __restrict__ parent, const int32_t* __restrict__ lin,
                            int32_t v, int32_t pv, int32_t a, int32_t b, GiantShared& sh, int32_t* thr,
                            double* e_sum) {
  const int tid = threadIdx.x;
  for (int j = tid; j < GIANT_SLOTS; j += GIANT_THREADS) {
    sh.c[j] = -1;
    sh.s[j] = 0.0;
    sh.first[j] = 0x7FFFFFFF;
  }
  if (tid == 0) {
    sh.n = 0;
    sh.overflow = 0;
  }
  __syncthreads();
  double e_acc = 0.0;
  bool capped = false;  // TABLE_CAP communities held: later ones cannot be among the first TABLE_CAP
  for (int32_t e0 = a; e0 < b; e0 += GIANT_THREADS) {
    const int32_t e = e0 + tid;
    if (e < b) {
      const int32_t u = gr.col[e];
      const bool ok = u != v && (!REFINE || parent[u] == pv);
      if (ok) {
        const float w = gr.wt[e];
        const int32_t c = lin[u];
        e_acc += (double)w;
        uint32_t h = pcg_hash((uint32_t)c) & (GIANT_SLOTS - 1);
        int probes = 0;
        bool placed = false;
        while (probes++ < GIANT_SLOTS) {
          const int32_t cur = __hip_atomic_load(sh.c + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          if (cur == c) {
            placed = true;
            break;
          }
          if (cur == -1) {
            if (capped) break;  // not held: appears after the first TABLE_CAP communities
            const int32_t prev = atomicCAS(sh.c + h, -1, c);
            if (prev == -1) atomicAdd(&sh.n, 1);
            if (prev == -1 || prev == c) {
              placed = true;
              break;
            }
          }
          h = (h + 1) & (GIANT_SLOTS - 1);
        }
        if (placed) {
          unsafeAtomicAdd(sh.s + h, (double)w);
          atomicMin(sh.first + h, e);
        } else if (!capped) {
          sh.overflow = 1;  // unreachable: at most 2 x TABLE_CAP - 1 entries are ever inserted
        }
      }
    }
    __syncthreads();
    capped = sh.n >= TABLE_CAP;
    __syncthreads();
  }
  __syncthreads();
  *e_sum = block_sum_giant(e_acc, sh);
  if (sh.overflow) return false;
  int32_t t = 0x7FFFFFFF;
  if (sh.n > TABLE_CAP) {  // smallest t with TABLE_CAP first positions below it
    int32_t lo = a, hi = b;
    while (lo < hi) {
      const int32_t mid = lo + (hi - lo) / 2;
      if (tid == 0) sh.count = 0;
      __syncthreads();
      int cnt = 0;
      for (int j = tid; j < GIANT_SLOTS; j += GIANT_THREADS) cnt += sh.first[j] < mid + 1;
      if (cnt) atomicAdd(&sh.count, cnt);
      __syncthreads();
      if (sh.count >= TABLE_CAP) hi = mid;
      else lo = mid + 1;
      __syncthreads();
    }
    t = lo + 1;
  }
  *thr = t;
  return true;
}

// Block-wide max of packed candidates; every thread gets the winner.
__device__ inline int32_t giant_pick(uint64_t mine, int32_t mine_c, uint64_t stay, int32_t old, GiantShared& sh) {
  const uint64_t wbest = wave_max_u64(mine);
  const int32_t wc = __shfl(mine_c, first_lane(__ballot(mine == wbest)));
  if (lane() == 0) {
    sh.best[threadIdx.x >> 6] = wbest;
    sh.best_c[threadIdx.x >> 6] = wc;
  }
  __syncthreads();
  uint64_t best = 0;
  int32_t c = old;
  for (int i = 0; i < GIANT_THREADS / 64; ++i)
    if (sh.best[i] > best) {
      best = sh.best[i];
      c = sh.best_c[i];
    }
  __syncthreads();
  return best > stay ? c : old;
}

__device__ float giant_k_old(GiantShared& sh, int32_t old, int32_t thr) {
  if (threadIdx.x == 0) sh.k_old_slot = -1;
  __syncthreads();
  for (int j = threadIdx.x; j < GIANT_SLOTS; j += GIANT_THREADS)
    if (sh.c[j] == old && sh.first[j] < thr) sh.k_old_slot = j;
  __syncthreads();
  const int32_t slot = sh.k_old_slot;
  return slot >= 0 ? (float)sh.s[slot] : 0.0f;
}

template <bool HUB>
__global__ __launch_bounds__(HUB ? LTHREADS : 64 * SWAVES) void local_moving_kernel(
    Graph gr, const double* __restrict__ sigma, const int32_t* __restrict__ lin, int32_t* __restrict__ lout,
    int32_t* __restrict__ ctl, const int32_t* __restrict__ hubs, const int32_t* __restrict__ hub_count,
    float resolution, uint32_t level, uint32_t sweep, uint32_t seed) {
  constexpr int W = HUB ? LWAVES : SWAVES;
  constexpr int CAP = HUB ? TABLE_CAP : SMALL_CAP;
  __shared__ int32_t tab_c[W][CAP];
  __shared__ double tab_s[W][CAP];
  const int wv = threadIdx.x >> 6;
  if (HUB) {
    const int32_t n = *hub_count;
    for (int32_t i = blockIdx.x * W + wv; i < n; i += gridDim.x * W)
      local_moving_vertex<CAP>(gr, sigma, lin, lout, ctl, resolution, level, sweep, seed, hubs[i], tab_c[wv],
                               tab_s[wv]);
  } else {
    const int32_t v = blockIdx.x * W + wv;
    if (v >= gr.V || gr.row_ptr[v + 1] - gr.row_ptr[v] > CAP / 2) return;
    local_moving_vertex<CAP>(gr, sigma, lin, lout, ctl, resolution, level, sweep, seed, v, tab_c[wv], tab_s[wv]);
  }
}

template <bool HUB>
__global__ __launch_bounds__(HUB ? LTHREADS : 64 * SWAVES) void refine_propose_kernel(
    Graph gr, const int32_t* __restrict__ parent, const double* __restrict__ sigma,
    const double* __restrict__ parent_sigma, const int32_t* __restrict__ lin, int32_t* __restrict__ prop,
    uint32_t* __restrict__ rank, const int32_t* __restrict__ ctl, const int32_t* __restrict__ hubs,
    const int32_t* __restrict__ hub_count, float resolution, float inv_theta, int boltzmann, uint32_t level,
    uint32_t sweep, uint32_t seed) {
  constexpr int W = HUB ? LWAVES : SWAVES;
  constexpr int CAP = HUB ? TABLE_CAP : SMALL_CAP;
  __shared__ int32_t tab_c[W][CAP];
  __shared__ double tab_s[W][CAP];
  if (ctl[CTL_DONE]) return;
  const int wv = threadIdx.x >> 6;
  if (HUB) {
    const int32_t n = *hub_count;
    for (int32_t i = blockIdx.x * W + wv; i < n; i += gridDim.x * W)
      refine_propose_vertex<CAP>(gr, parent, sigma, parent_sigma, lin, prop, rank, resolution, inv_theta,
                                 boltzmann, level, sweep, seed, hubs[i], tab_c[wv], tab_s[wv]);
  } else {
    const int32_t v = blockIdx.x * W + wv;
    if (v >= gr.V || gr.row_ptr[v + 1] - gr.row_ptr[v] > CAP / 2) return;
    refine_propose_vertex<CAP>(gr, parent, sigma, parent_sigma, lin, prop, rank, resolution, inv_theta, boltzmann,
                               level, sweep, seed, v, tab_c[wv], tab_s[wv]);
  }
}

__global__ __launch_bounds__(GIANT_THREADS) void local_moving_giant_kernel(
    Graph gr, const double* __restrict__ sigma, const int32_t* __restrict__ lin, int32_t* __restrict__ lout,
    int32_t* __restrict__ ctl, const int32_t* __restrict__ giants, const int32_t* __restrict__ giant_count,
    float resolution, uint32_t level, uint32_t sweep, uint32_t seed) {
  __shared__ GiantShared sh;
  const int32_t count = *giant_count;
  const bool done = ctl[CTL_DONE] != 0;
  const int up_down = ctl[CTL_UPDOWN];
  for (int32_t i = blockIdx.x; i < count; i += gridDim.x) {
    const int32_t v = giants[i];
    const int32_t old = lin[v];
    const int32_t g = v / gr.S;
    const double tm = gr.two_m[g];
    if (done || !(tm > 0.0)) {
      if (threadIdx.x == 0) lout[v] = old;
      continue;
    }
    const int32_t a = gr.row_ptr[v], b = gr.row_ptr[v + 1];
    int32_t thr;
    double e_sum;
    if (!giant_table<false>(gr, nullptr, lin, v, 0, a, b, sh, &thr, &e_sum)) {  // cannot happen: stay, flagged
      if (threadIdx.x == 0) {
        lout[v] = old;
        ctl[CTL_OVERFLOW] = 1;
      }
      __syncthreads();
      continue;
    }
    const float k_old = giant_k_old(sh, old, thr);
    const double kv = gr.k_v[v];
    const double m_g = 0.5 * tm;
    const double inv_m = 1.0 / m_g;
    const double inv_2m2 = 1.0 / (2.0 * m_g * m_g);
    const double sig_old_excl = sigma[old] - kv;
    const float jitter = (rand_uniform((uint32_t)g, (uint32_t)v, level, sweep, seed) - 0.5f) * 1e-9f;
    uint64_t mine = 0;
    int32_t mine_c = old;
    for (int j = threadIdx.x; j < GIANT_SLOTS; j += GIANT_THREADS) {
      const int32_t c = sh.c[j];
      if (c < 0 || sh.first[j] >= thr || c == old || (c > old ? 1 : 0) != up_down) continue;
      const float kn = (float)sh.s[j];
      const double dq = ((double)kn - (double)k_old) * inv_m
                        + (double)resolution * kv * (sig_old_excl - sigma[c]) * inv_2m2;
      const float dqf = (float)dq + jitter;
      const uint64_t p = pack(dqf, cand_pref(c));
      if (p > mine) {
        mine = p;
        mine_c = c;
      }
    }
    const int32_t choice = giant_pick(mine, mine_c, pack(0.0f, STAY_PREF), old, sh);
    if (threadIdx.x == 0) {
      lout[v] = choice;
      if (choice != old) mark_moved(ctl);
    }
  }
}

__global__ __launch_bounds__(GIANT_THREADS) void refine_propose_giant_kernel(
    Graph gr, const int32_t* __restrict__ parent, const double* __restrict__ sigma,
    const double* __restrict__ parent_sigma, const int32_t* __restrict__ lin, int32_t* __restrict__ prop,
    uint32_t* __restrict__ rank, int32_t* __restrict__ ctl, const int32_t* __restrict__ giants,
    const int32_t* __restrict__ giant_count, float resolution, float inv_theta, int boltzmann, uint32_t level,
    uint32_t sweep, uint32_t seed) {
  __shared__ GiantShared sh;
  if (ctl[CTL_DONE]) return;
  const int32_t count = *giant_count;
  for (int32_t i = blockIdx.x; i < count; i += gridDim.x) {
    const int32_t v = giants[i];
    const int32_t g = v / gr.S;
    if (threadIdx.x == 0) rank[v] = mix4((uint32_t)g, (uint32_t)v, (level << 16) | sweep, seed);
    const int32_t old = lin[v];
    const double tm = gr.two_m[g];
    if (!(tm > 0.0)) {
      if (threadIdx.x == 0) prop[v] = old;
      continue;
    }
    const int32_t a = gr.row_ptr[v], b = gr.row_ptr[v + 1];
    const int32_t pv = parent[v];
    int32_t thr;
    double e_sum;
    if (!giant_table<true>(gr, parent, lin, v, pv, a, b, sh, &thr, &e_sum)) {  // cannot happen: stay, flagged
      if (threadIdx.x == 0) {
        prop[v] = old;
        ctl[CTL_OVERFLOW] = 1;
      }
      __syncthreads();
      continue;
    }
    const double kv = gr.k_v[v];
    double vol_minus = parent_sigma[pv] - kv;
    if (vol_minus < 0.0) vol_minus = 0.0;
    const double bound = (double)resolution * kv * vol_minus / tm;
    if ((double)(float)e_sum < bound) {  // {v} is not well connected to its parent community
      if (threadIdx.x == 0) prop[v] = old;
      __syncthreads();
      continue;
    }
    const float k_old = giant_k_old(sh, old, thr);
    const double m_g = 0.5 * tm;
    const double inv_m = 1.0 / m_g;
    const double inv_2m2 = 1.0 / (2.0 * m_g * m_g);
    const double sig_old_excl = sigma[old] - kv;
    uint64_t mine = 0;
    int32_t mine_c = old;
    for (int j = threadIdx.x; j < GIANT_SLOTS; j += GIANT_THREADS) {
      const int32_t c = sh.c[j];
      if (c < 0 || sh.first[j] >= thr || c == old) continue;
      const float kn = (float)sh.s[j];
      const double dq = ((double)kn - (double)k_old) * inv_m
                        + (double)resolution * kv * (sig_old_excl - sigma[c]) * inv_2m2;
      if (dq < 0.0) continue;
      const float score = boltzmann
          ? (float)(dq * (double)inv_theta)
                + gumbel(rand_uniform_pair((uint32_t)g, (uint32_t)v, (uint32_t)c, level, sweep, seed))
          : (float)dq;
      const uint64_t p = pack(score, cand_pref(c));
      if (p > mine) {
        mine = p;
        mine_c = c;
      }
    }
    const float stay = boltzmann
        ? gumbel(rand_uniform_pair((uint32_t)g, (uint32_t)v, (uint32_t)old, level, sweep, seed))
        : 0.0f;
    const int32_t choice = giant_pick(mine, mine_c, pack(stay, STAY_PREF), old, sh);
    if (threadIdx.x == 0) prop[v] = choice;
  }
}

// Commit an independent set of the proposals: a mover commits unless a
// moving neighbour in its parent community outranks it on (rank, id)
// (refinement.cu:263-300).
__global__ __launch_bounds__(LTHREADS) void refine_commit_kernel(
    Graph gr, const int32_t* __restrict__ parent, const int32_t* __restrict__ lin,
    const int32_t* __restrict__ prop, const uint32_t* __restrict__ rank, int32_t* __restrict__ lout,
    int32_t* __restrict__ ctl) {
  const int32_t v = blockIdx.x * LWAVES + (threadIdx.x >> 6);
  if (v >= gr.V) return;
  const int32_t old = lin[v];
  if (ctl[CTL_DONE]) {
    if (lane() == 0) lout[v] = old;
    return;
  }
  const int32_t p = prop[v];
  if (p == old) {
    if (lane() == 0) lout[v] = old;
    return;
  }
  const int32_t pv = parent[v];
  const uint32_t rv = rank[v];
  const int32_t a = gr.row_ptr[v], b = gr.row_ptr[v + 1];
  bool lost = false;
  for (int32_t e = a + lane(); e < b; e += 64) {
    const int32_t u = gr.col[e];
    if (u == v || parent[u] != pv || prop[u] == lin[u]) continue;
    const uint32_t ru = rank[u];
    lost = lost || ru > rv || (ru == rv && u > v);
  }
  const bool any_lost = __ballot(lost) != 0;
  if (lane() == 0) {
    lout[v] = any_lost ? old : p;
    if (!any_lost) mark_moved(ctl);
  }
}

__global__ void refine_control_kernel(int32_t* __restrict__ ctl) {
  if (threadIdx.x != 0) return;
  if (!ctl[CTL_DONE] && ctl[CTL_MOVED] == 0) ctl[CTL_DONE] = 1;
  ctl[CTL_MOVED] = 0;
}

// q_v = in(v) / 2m - gamma k_v Sigma[c_v] / (4 m^2); Q_g is their sum over
// the graph (helpers.cu:41-78).
__global__ __launch_bounds__(LTHREADS) void modularity_kernel(Graph gr, const int32_t* __restrict__ labels,
                                                              const double* __restrict__ sigma, float resolution,
                                                              double* __restrict__ q_v) {
  const int32_t v = blockIdx.x * LWAVES + (threadIdx.x >> 6);
  if (v >= gr.V) return;
  const int32_t g = v / gr.S;
  const double tm = gr.two_m[g];
  if (!(tm > 0.0)) {
    if (lane() == 0) q_v[v] = 0.0;
    return;
  }
  const int32_t cv = labels[v];
  const int32_t a = gr.row_ptr[v], b = gr.row_ptr[v + 1];
  double in_sum = 0.0;
  for (int32_t e = a + lane(); e < b; e += 64)
    if (labels[gr.col[e]] == cv) in_sum += (double)gr.wt[e];
  in_sum = wave_sum_f64(in_sum);
  if (lane() == 0) {
    const double m_g = 0.5 * tm;
    q_v[v] = in_sum / tm - (double)resolution * (gr.k_v[v] * sigma[cv]) / (4.0 * m_g * m_g);
  }
}

// A flagged table overflow turns every graph's modularity into NaN, which the
// host checks: the labels of such a call are not to be trusted.
__global__ void overflow_mark_kernel(const int32_t* __restrict__ ctl, int32_t G, double* __restrict__ modularity) {
  const int32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g < G && ctl[CTL_OVERFLOW] != 0) modularity[g] = __builtin_nan("");
}

__global__ void finish_kernel(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ result, int32_t V,
                              int32_t* __restrict__ labels) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v < V) labels[v] = row_ptr[v] == row_ptr[v + 1] ? -1 : result[v];
}

// ----------------------------------------------------------------- aggregation / densify
__global__ void remap_kernel(const int32_t* __restrict__ src, const int32_t* __restrict__ dst,
                             const float* __restrict__ w, const int32_t* __restrict__ labels, int64_t E,
                             int32_t Vs, int bits, uint64_t* __restrict__ keys, float* __restrict__ vals) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E) return;
  int32_t s = labels[src[i]], t = labels[dst[i]];
  const int32_t lo = s < t ? s : t, hi = s < t ? t : s;
  const bool ok = lo >= 0 && hi < Vs;
  keys[i] = ok ? ((uint64_t)lo << bits) | (uint64_t)hi : ((uint64_t)Vs << bits);
  vals[i] = ok ? w[i] : 0.0f;
}

__global__ void unpack_kernel(const uint64_t* __restrict__ keys, int64_t E, int bits,
                              const int64_t* __restrict__ count, int32_t* __restrict__ out_src,
                              int32_t* __restrict__ out_dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= *count) return;
  const uint64_t k = keys[i];
  out_src[i] = (int32_t)(k >> bits);
  out_dst[i] = (int32_t)(k & (((uint64_t)1 << bits) - 1));
}

// Edges with an endpoint label outside [0, Vs) carry the sentinel key, which
// sorts last: drop that run from the count.
__global__ void count_fix_kernel(const uint64_t* __restrict__ keys, int32_t Vs, int bits, int64_t* __restrict__ count) {
  if (threadIdx.x != 0) return;
  const int64_t n = *count;
  if (n > 0 && (keys[n - 1] >> bits) >= (uint64_t)Vs) *count = n - 1;
}

__global__ void flag_zero_kernel(int32_t* __restrict__ flags, int32_t V) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v < V) flags[v] = 0;
}

// Labels below zero stand for the vertex itself; labels outside the vertex's
// graph are ignored (their vertices get rank -1 in the apply step).
__device__ inline int32_t own_label(const int32_t* labels, int32_t v, int32_t S) {
  const int32_t l = labels[v] < 0 ? v : labels[v];
  return (l / S == v / S) ? l : -1;
}

__global__ void flag_mark_kernel(const int32_t* __restrict__ labels, int32_t V, int32_t S,
                                 int32_t* __restrict__ flags) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= V) return;
  const int32_t l = own_label(labels, v, S);
  if (l >= 0) flags[l] = 1;
}

__global__ void densify_count_kernel(const int32_t* __restrict__ flags, const int32_t* __restrict__ scan, int32_t G,
                                     int32_t S, int32_t* __restrict__ counts) {
  const int32_t g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g < G) {
    const int32_t last = (g + 1) * S - 1;
    counts[g] = scan[last] + flags[last] - scan[g * S];
  }
}

__global__ void densify_apply_kernel(const int32_t* __restrict__ labels, const int32_t* __restrict__ scan, int32_t V,
                                     int32_t S, int32_t new_S, int32_t* __restrict__ dense) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= V) return;
  const int32_t g = v / S;
  const int32_t l = own_label(labels, v, S);
  dense[v] = l < 0 ? -1 : scan[l] - scan[g * S] + g * new_S;
}

// ----------------------------------------------------------------- modularity of a labelled edge list
__device__ inline double block_sum_f64(double x, double* part) {  // 256 threads
  x = wave_sum_f64(x);
  if (lane() == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  return part[0] + part[1] + part[2] + part[3];
}

__global__ void mod_zero_kernel(double* __restrict__ k, double* __restrict__ sig, int32_t V,
                                double* __restrict__ acc) {
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v < V) {
    k[v] = 0.0;
    sig[v] = 0.0;
  }
  if (v < 4) acc[v] = 0.0;
}

__global__ __launch_bounds__(256) void mod_edge_kernel(const int32_t* __restrict__ src,
                                                       const int32_t* __restrict__ dst, const float* __restrict__ w,
                                                       int64_t E, const int32_t* __restrict__ labels, int32_t V,
                                                       double* __restrict__ k, double* __restrict__ acc) {
  __shared__ double part[4];
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  double in = 0.0, xs = 0.0;
  int32_t a = -1;
  if (i < E) {
    const int32_t s0 = src[i], b = dst[i];
    if (s0 >= 0 && s0 < V && b >= 0 && b < V) {
      const double x = (double)w[i];
      a = s0;
      xs = x;
      unsafeAtomicAdd(k + b, x);
      if (labels[s0] == labels[b]) in = x;
    }
  }
  // Source ends: sum runs of equal source within the wave (edge lists come
  // sorted by source, so a hub's edges arrive together), one atomic per run.
  const int ln = lane();
  const int32_t prev_a = __shfl_up(a, 1);
  const int32_t next_a = __shfl_down(a, 1);
  bool h = ln == 0 || prev_a != a;  // a run starts here
  for (int o = 1; o < 64; o <<= 1) {
    const double y = __shfl_up(xs, o);
    const bool hy = __shfl_up(h ? 1 : 0, o) != 0;
    if (ln >= o) {
      if (!h) xs += y;
      h = h || hy;
    }
  }
  if (a >= 0 && (ln == 63 || next_a != a)) unsafeAtomicAdd(k + a, xs);
  in = block_sum_f64(in, part);
  if (threadIdx.x == 0 && in != 0.0) unsafeAtomicAdd(acc, in);
}

__global__ __launch_bounds__(256) void mod_sigma_kernel(const int32_t* __restrict__ labels,
                                                        const double* __restrict__ k, int32_t V,
                                                        double* __restrict__ sig, double* __restrict__ acc) {
  __shared__ double part[4];
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  double kv = 0.0;
  if (v < V) {
    kv = k[v];
    const int32_t l = labels[v];
    if (l >= 0 && l < V && kv != 0.0) unsafeAtomicAdd(sig + l, kv);
  }
  kv = block_sum_f64(kv, part);
  if (threadIdx.x == 0 && kv != 0.0) unsafeAtomicAdd(acc + 1, kv);
}

__global__ __launch_bounds__(256) void mod_square_kernel(const double* __restrict__ sig, int32_t V,
                                                         double* __restrict__ acc) {
  __shared__ double part[4];
  const int32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  double x = v < V ? sig[v] * sig[v] : 0.0;
  x = block_sum_f64(x, part);
  if (threadIdx.x == 0 && x != 0.0) unsafeAtomicAdd(acc + 2, x);
}

__global__ void mod_final_kernel(const double* __restrict__ acc, float resolution, double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  const double two_m = acc[1];
  *out = two_m > 0.0 ? 2.0 * acc[0] / two_m - (double)resolution * acc[2] / (two_m * two_m) : 0.0;
}

// ----------------------------------------------------------------- host side
inline int bits_for(uint64_t x) {  // bits needed to hold values 0..x
  int b = 1;
  while (b < 63 && (x >> b) != 0) ++b;
  return b;
}
inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
inline unsigned blocks(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

int launch_check() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : ckv_internal::set_error(CKV_E_LAUNCH, hipGetErrorString(e));
}

struct LeidenLayout {
  size_t keys_a, keys_b, vals_a, vals_b, temp, temp_bytes, row_ptr, col, k_v, two_m, sigma, psigma, lab_a, lab_b,
      parent, prop, rank, ctl, hubs, hub_count, giants, giant_count, total;
};

LeidenLayout leiden_layout(int64_t E, int32_t G, int32_t S) {
  LeidenLayout L{};
  const int64_t n = 2 * E;
  const int64_t V = (int64_t)G * S;
  size_t temp_bytes = 0;
  if (n > 0)
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, temp_bytes, (uint64_t*)nullptr, (uint64_t*)nullptr,
                                       (float*)nullptr, (float*)nullptr, (int)n, 0, 64, (hipStream_t)0);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  L.keys_a = take(n * 8);
  L.keys_b = take(n * 8);
  L.vals_a = take(n * 4);
  L.vals_b = take(n * 4);
  L.temp_bytes = temp_bytes;
  L.temp = take(temp_bytes);
  L.row_ptr = take((V + 1) * 4);
  L.col = take(n * 4);
  L.k_v = take(V * 8);
  L.two_m = take(G * 8);
  L.sigma = take(V * 8);
  L.psigma = take(V * 8);
  L.lab_a = take(V * 4);
  L.lab_b = take(V * 4);
  L.parent = take(V * 4);
  L.prop = take(V * 4);
  L.rank = take(V * 4);
  L.ctl = take(CTL_WORDS * 4);
  L.hubs = take(V * 4);
  L.hub_count = take(4);
  L.giants = take(V * 4);
  L.giant_count = take(4);
  L.total = off;
  return L;
}

struct AggLayout {
  size_t keys_a, keys_b, vals_a, uniq, temp, temp_bytes, total;
};

AggLayout agg_layout(int64_t E) {
  AggLayout L{};
  size_t sort_bytes = 0, red_bytes = 0;
  if (E > 0) {
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, (uint64_t*)nullptr, (uint64_t*)nullptr, (float*)nullptr,
                                       (float*)nullptr, (int)E, 0, 64, (hipStream_t)0);
    (void)hipcub::DeviceReduce::ReduceByKey(nullptr, red_bytes, (uint64_t*)nullptr, (uint64_t*)nullptr, (float*)nullptr,
                                      (float*)nullptr, (int64_t*)nullptr, hipcub::Sum(), (int)E, (hipStream_t)0);
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  L.keys_a = take(E * 8);
  L.keys_b = take(E * 8);
  L.vals_a = take(E * 4 * 2);  // values in, sorted values
  L.uniq = take(E * 8);
  L.temp_bytes = sort_bytes > red_bytes ? sort_bytes : red_bytes;
  L.temp = take(L.temp_bytes);
  L.total = off;
  return L;
}

size_t densify_temp_bytes(int64_t V) {
  size_t bytes = 0;
  (void)hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, (int32_t*)nullptr, (int32_t*)nullptr, (int)V, (hipStream_t)0);
  return bytes;
}

// Sort the (key, weight) pairs in keys_a / vals_a of an AggLayout, sum equal
// keys, drop the sentinel run and unpack (src, dst).
int coalesce(const AggLayout& L, char* ws, int64_t n, int32_t vertices, int bits, int end_bit, int32_t* out_src,
             int32_t* out_dst, float* out_weight, int64_t* out_count, hipStream_t st) {
  uint64_t* keys_a = (uint64_t*)(ws + L.keys_a);
  uint64_t* keys_b = (uint64_t*)(ws + L.keys_b);
  float* vals_in = (float*)(ws + L.vals_a);
  float* vals_sorted = vals_in + n;
  uint64_t* uniq = (uint64_t*)(ws + L.uniq);
  size_t temp_bytes = L.temp_bytes;
  if (hipcub::DeviceRadixSort::SortPairs(ws + L.temp, temp_bytes, keys_a, keys_b, vals_in, vals_sorted, (int)n, 0,
                                         end_bit, st) != hipSuccess)
    return ckv_internal::set_error(CKV_E_LAUNCH, "edge sort failed");
  temp_bytes = L.temp_bytes;
  if (hipcub::DeviceReduce::ReduceByKey(ws + L.temp, temp_bytes, keys_b, uniq, vals_sorted, out_weight, out_count,
                                        hipcub::Sum(), (int)n, st) != hipSuccess)
    return ckv_internal::set_error(CKV_E_LAUNCH, "edge reduce failed");
  count_fix_kernel<<<1, 64, 0, st>>>(uniq, vertices, bits, out_count);
  unpack_kernel<<<blocks(n, ETHREADS), ETHREADS, 0, st>>>(uniq, n, bits, out_count, out_src, out_dst);
  return launch_check();
}

// Entries of the top-k graph (partition.py:168-249): per row of graph g at
// position p, kappa direct edges (p, col) of weight score * lam / 2 and, when
// lam < 1, kappa (kappa + 1) / 2 co-occurrence pairs (col_i, col_j), i <= j,
// of weight score_i * score_j * (1 - lam); columns outside [0, S) drop the
// entry (sentinel key).  Ends in (min, max) order, global ids g * S + i.
__global__ void adjacency_expand_kernel(const int32_t* __restrict__ idx, const float* __restrict__ sc,
                                        const int64_t* __restrict__ positions, int32_t G, int32_t R, int32_t kappa,
                                        int32_t S, float half_lam, float co_lam, int32_t per_row, int bits,
                                        uint64_t* __restrict__ keys, float* __restrict__ vals) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = (int64_t)G * R * per_row;
  if (i >= n) return;
  const int64_t row = i / per_row;
  int t = (int)(i - row * per_row);
  const int32_t g = (int32_t)(row / R);
  const int32_t* ri = idx + row * kappa;
  const float* rs = sc + row * kappa;
  const uint64_t sentinel = (uint64_t)((int64_t)G * S) << bits;
  const int64_t base = (int64_t)g * S;
  int64_t a, b;
  float w;
  bool ok;
  if (t < kappa) {
    const int32_t c = ri[t];
    const int64_t p = positions[row];
    ok = c >= 0 && c < S && p >= 0 && p < S;
    a = base + p;
    b = base + c;
    w = rs[t] * half_lam;
  } else {
    t -= kappa;  // pair t of the upper triangle (diagonal included), row-major
    int r0 = 0;
    while (t >= kappa - r0) {
      t -= kappa - r0;
      ++r0;
    }
    const int r1 = r0 + t;
    const int32_t c0 = ri[r0], c1 = ri[r1];
    ok = c0 >= 0 && c0 < S && c1 >= 0 && c1 < S;
    a = base + c0;
    b = base + c1;
    w = (rs[r0] * rs[r1]) * co_lam;
  }
  const int64_t lo = a < b ? a : b, hi = a < b ? b : a;
  keys[i] = ok ? ((uint64_t)lo << bits) | (uint64_t)hi : sentinel;
  vals[i] = ok ? w : 0.0f;
}

inline int64_t adjacency_entries(int32_t graphs, int32_t rows, int32_t kappa, float lam) {
  const int per_row = kappa + (lam < 1.0f ? kappa * (kappa + 1) / 2 : 0);
  return (int64_t)graphs * rows * per_row;
}

}  // namespace
}  // namespace ckv

using namespace ckv;

static bool g_test_raise_overflow = false;

extern "C" void ckv_leiden_test_raise_overflow(int32_t enable) { g_test_raise_overflow = enable != 0; }

extern "C" size_t ckv_leiden_workspace_bytes(int64_t edges, int32_t graphs, int32_t seq_len) {
  if (edges < 0 || graphs <= 0 || seq_len <= 0) return 0;
  return leiden_layout(edges, graphs, seq_len).total;
}

extern "C" int ckv_batched_leiden(const int32_t* edge_src, const int32_t* edge_dst, const float* edge_weight,
                                  int64_t edges, int32_t graphs, int32_t seq_len, float resolution, float theta,
                                  int32_t max_inner_iter, int32_t seed, int32_t use_boltzmann, int32_t* labels,
                                  double* modularity, void* workspace, void* stream) {
  if (graphs <= 0 || seq_len <= 0) return ckv_internal::set_error(CKV_E_INVALID, "graphs and seq_len must be positive");
  if (!labels || !modularity) return ckv_internal::set_error(CKV_E_INVALID, "null Leiden output");
  if (edges < 0 || (edges > 0 && (!edge_src || !edge_dst || !edge_weight || !workspace)))
    return ckv_internal::set_error(CKV_E_INVALID, "Leiden edges need src, dst, weight and a workspace");
  const int64_t V64 = (int64_t)graphs * seq_len;
  if (V64 >= (int64_t)1 << 30 || 2 * edges >= ((int64_t)1 << 31) - 1)
    return ckv_internal::set_error(CKV_E_LIMIT, "Leiden graph too large (vertices < 2^30, 2 * edges < 2^31)");
  if (max_inner_iter < 0) return ckv_internal::set_error(CKV_E_INVALID, "max_inner_iter must be nonnegative");
  hipStream_t st = (hipStream_t)stream;
  const int32_t V = (int32_t)V64;
  if (edges == 0) {
    // leiden.cu:68-76: every vertex isolated, modularity 0
    if (hipMemsetAsync(labels, 0xFF, (size_t)V * 4, st) != hipSuccess ||
        hipMemsetAsync(modularity, 0, (size_t)graphs * 8, st) != hipSuccess)
      return launch_check();
    return 0;
  }
  const LeidenLayout L = leiden_layout(edges, graphs, seq_len);
  char* ws = (char*)workspace;
  uint64_t* keys_a = (uint64_t*)(ws + L.keys_a);
  uint64_t* keys_b = (uint64_t*)(ws + L.keys_b);
  float* vals_a = (float*)(ws + L.vals_a);
  float* vals_b = (float*)(ws + L.vals_b);
  int32_t* row_ptr = (int32_t*)(ws + L.row_ptr);
  int32_t* col = (int32_t*)(ws + L.col);
  double* k_v = (double*)(ws + L.k_v);
  double* two_m = (double*)(ws + L.two_m);
  double* sigma = (double*)(ws + L.sigma);
  double* psigma = (double*)(ws + L.psigma);
  int32_t* lab[2] = {(int32_t*)(ws + L.lab_a), (int32_t*)(ws + L.lab_b)};
  int32_t* parent = (int32_t*)(ws + L.parent);
  int32_t* prop = (int32_t*)(ws + L.prop);
  uint32_t* rank = (uint32_t*)(ws + L.rank);
  int32_t* ctl = (int32_t*)(ws + L.ctl);
  int32_t* hubs = (int32_t*)(ws + L.hubs);
  int32_t* hub_count = (int32_t*)(ws + L.hub_count);
  int32_t* giants = (int32_t*)(ws + L.giants);
  int32_t* giant_count = (int32_t*)(ws + L.giant_count);

  const int bits = bits_for((uint64_t)V - 1);
  const int end_bit = bits + bits_for((uint64_t)V);
  const int64_t n = 2 * edges;
  mirror_kernel<<<blocks(edges, ETHREADS), ETHREADS, 0, st>>>(edge_src, edge_dst, edge_weight, edges, V, bits, keys_a,
                                                             vals_a);
  size_t temp_bytes = L.temp_bytes;
  if (hipcub::DeviceRadixSort::SortPairs(ws + L.temp, temp_bytes, keys_a, keys_b, vals_a, vals_b, (int)n, 0, end_bit,
                                         st) != hipSuccess)
    return ckv_internal::set_error(CKV_E_LAUNCH, "Leiden CSR sort failed");
  row_ptr_kernel<<<blocks(V + 1, ETHREADS), ETHREADS, 0, st>>>(keys_b, n, V, bits, row_ptr);
  col_kernel<<<blocks(n, ETHREADS), ETHREADS, 0, st>>>(keys_b, n, bits, col);
  zero_kernel<<<1, 256, 0, st>>>(two_m, graphs, modularity, ctl, hub_count, giant_count);
  hub_list_kernel<<<blocks(V, ETHREADS), ETHREADS, 0, st>>>(row_ptr, V, hubs, hub_count, giants, giant_count);
  const unsigned vgrid = blocks(V, LWAVES);
  degree_kernel<<<vgrid, LTHREADS, 0, st>>>(row_ptr, vals_b, V, seq_len, k_v);
  graph_sum_kernel<<<graphs, 256, 0, st>>>(k_v, seq_len, two_m);
  identity_kernel<<<blocks(V, ETHREADS), ETHREADS, 0, st>>>(V, lab[0]);
  const Graph gr{row_ptr, col, vals_b, k_v, two_m, V, seq_len};

  const unsigned egrid = blocks(V, ETHREADS);
  int cur = 0;
  for (int sweep = 0; sweep < max_inner_iter; ++sweep) {
    sigma_zero_kernel<<<egrid, ETHREADS, 0, st>>>(sigma, V, ctl);
    sigma_scatter_kernel<<<egrid, ETHREADS, 0, st>>>(lab[cur], k_v, V, sigma, ctl);
    local_moving_kernel<false><<<blocks(V, SWAVES), 64 * SWAVES, 0, st>>>(
        gr, sigma, lab[cur], lab[cur ^ 1], ctl, hubs, hub_count, resolution, 0u, (uint32_t)sweep, (uint32_t)seed);
    local_moving_kernel<true><<<HUB_BLOCKS, LTHREADS, 0, st>>>(gr, sigma, lab[cur], lab[cur ^ 1], ctl, hubs,
                                                              hub_count, resolution, 0u, (uint32_t)sweep,
                                                              (uint32_t)seed);
    local_moving_giant_kernel<<<GIANT_BLOCKS, GIANT_THREADS, 0, st>>>(gr, sigma, lab[cur], lab[cur ^ 1], ctl, giants,
                                                                     giant_count, resolution, 0u, (uint32_t)sweep,
                                                                     (uint32_t)seed);
    lm_control_kernel<<<1, 64, 0, st>>>(ctl);
    cur ^= 1;
  }
  if (g_test_raise_overflow) raise_overflow_kernel<<<1, 64, 0, st>>>(ctl);
  // refinement from singletons inside the local-moving communities
  refine_init_kernel<<<egrid, ETHREADS, 0, st>>>(lab[cur], V, parent, lab[cur ^ 1], ctl);
  cur ^= 1;
  sigma_zero_kernel<<<egrid, ETHREADS, 0, st>>>(psigma, V, nullptr);
  sigma_scatter_kernel<<<egrid, ETHREADS, 0, st>>>(parent, k_v, V, psigma, nullptr);
  const float t = theta > 0.0f ? theta : 1.0e-3f;
  const float inv_theta = 1.0f / t;
  for (int sweep = 0; sweep < max_inner_iter; ++sweep) {
    sigma_zero_kernel<<<egrid, ETHREADS, 0, st>>>(sigma, V, ctl);
    sigma_scatter_kernel<<<egrid, ETHREADS, 0, st>>>(lab[cur], k_v, V, sigma, ctl);
    refine_propose_kernel<false><<<blocks(V, SWAVES), 64 * SWAVES, 0, st>>>(
        gr, parent, sigma, psigma, lab[cur], prop, rank, ctl, hubs, hub_count, resolution, inv_theta,
        use_boltzmann ? 1 : 0, 1u, (uint32_t)sweep, (uint32_t)seed);
    refine_propose_kernel<true><<<HUB_BLOCKS, LTHREADS, 0, st>>>(
        gr, parent, sigma, psigma, lab[cur], prop, rank, ctl, hubs, hub_count, resolution, inv_theta,
        use_boltzmann ? 1 : 0, 1u, (uint32_t)sweep, (uint32_t)seed);
    refine_propose_giant_kernel<<<GIANT_BLOCKS, GIANT_THREADS, 0, st>>>(
        gr, parent, sigma, psigma, lab[cur], prop, rank, ctl, giants, giant_count, resolution, inv_theta,
        use_boltzmann ? 1 : 0, 1u, (uint32_t)sweep, (uint32_t)seed);
    refine_commit_kernel<<<vgrid, LTHREADS, 0, st>>>(gr, parent, lab[cur], prop, rank, lab[cur ^ 1], ctl);
    refine_control_kernel<<<1, 64, 0, st>>>(ctl);
    cur ^= 1;
  }
  sigma_zero_kernel<<<egrid, ETHREADS, 0, st>>>(sigma, V, nullptr);
  sigma_scatter_kernel<<<egrid, ETHREADS, 0, st>>>(lab[cur], k_v, V, sigma, nullptr);
  modularity_kernel<<<vgrid, LTHREADS, 0, st>>>(gr, lab[cur], sigma, resolution, psigma);
  graph_sum_kernel<<<graphs, 256, 0, st>>>(psigma, seq_len, modularity);
  overflow_mark_kernel<<<blocks(graphs, ETHREADS), ETHREADS, 0, st>>>(ctl, graphs, modularity);
  finish_kernel<<<egrid, ETHREADS, 0, st>>>(row_ptr, lab[cur], V, labels);
  return launch_check();
}

extern "C" size_t ckv_aggregate_coo_workspace_bytes(int64_t edges) {
  return edges <= 0 ? 0 : agg_layout(edges).total;
}

extern "C" int ckv_aggregate_coo(const int32_t* edge_src, const int32_t* edge_dst, const float* edge_weight,
                                 int64_t edges, const int32_t* labels, int32_t super_vertices, int32_t* out_src,
                                 int32_t* out_dst, float* out_weight, int64_t* out_count, void* workspace,
                                 void* stream) {
  if (edges < 0 || super_vertices <= 0 || !out_count)
    return ckv_internal::set_error(CKV_E_INVALID, "bad aggregation sizes");
  hipStream_t st = (hipStream_t)stream;
  if (edges == 0) {
    if (hipMemsetAsync(out_count, 0, 8, st) != hipSuccess) return launch_check();
    return 0;
  }
  if (!edge_src || !edge_dst || !edge_weight || !labels || !out_src || !out_dst || !out_weight || !workspace)
    return ckv_internal::set_error(CKV_E_INVALID, "null aggregation pointer");
  if (edges >= ((int64_t)1 << 31) - 1 || super_vertices >= (1 << 30))
    return ckv_internal::set_error(CKV_E_LIMIT, "aggregation too large");
  const AggLayout L = agg_layout(edges);
  char* ws = (char*)workspace;
  uint64_t* keys_a = (uint64_t*)(ws + L.keys_a);
  float* vals_in = (float*)(ws + L.vals_a);
  const int bits = bits_for((uint64_t)super_vertices - 1);
  const int end_bit = bits + bits_for((uint64_t)super_vertices);
  remap_kernel<<<blocks(edges, ETHREADS), ETHREADS, 0, st>>>(edge_src, edge_dst, edge_weight, labels, edges,
                                                             super_vertices, bits, keys_a, vals_in);
  return coalesce(L, ws, edges, super_vertices, bits, end_bit, out_src, out_dst, out_weight, out_count, st);
}

extern "C" size_t ckv_densify_workspace_bytes(int32_t graphs, int32_t seq_len) {
  if (graphs <= 0 || seq_len <= 0) return 0;
  const int64_t V = (int64_t)graphs * seq_len;
  return 2 * align256((size_t)V * 4) + align256(densify_temp_bytes(V));
}

extern "C" int ckv_densify_count(const int32_t* labels, int32_t graphs, int32_t seq_len, int32_t* counts,
                                 void* workspace, void* stream) {
  if (!labels || !counts || !workspace || graphs <= 0 || seq_len <= 0)
    return ckv_internal::set_error(CKV_E_INVALID, "bad densify arguments");
  const int64_t V64 = (int64_t)graphs * seq_len;
  if (V64 >= (int64_t)1 << 30) return ckv_internal::set_error(CKV_E_LIMIT, "densify: too many vertices");
  const int32_t V = (int32_t)V64;
  hipStream_t st = (hipStream_t)stream;
  int32_t* flags = (int32_t*)workspace;
  int32_t* scan = (int32_t*)((char*)workspace + align256((size_t)V * 4));
  void* temp = (char*)workspace + 2 * align256((size_t)V * 4);
  size_t temp_bytes = densify_temp_bytes(V);
  flag_zero_kernel<<<blocks(V, ETHREADS), ETHREADS, 0, st>>>(flags, V);
  flag_mark_kernel<<<blocks(V, ETHREADS), ETHREADS, 0, st>>>(labels, V, seq_len, flags);
  if (hipcub::DeviceScan::ExclusiveSum(temp, temp_bytes, flags, scan, V, st) != hipSuccess)
    return ckv_internal::set_error(CKV_E_LAUNCH, "densify scan failed");
  densify_count_kernel<<<blocks(graphs, ETHREADS), ETHREADS, 0, st>>>(flags, scan, graphs, seq_len, counts);
  return launch_check();
}

extern "C" int ckv_densify_apply(const int32_t* labels, int32_t graphs, int32_t seq_len, int32_t new_seq_len,
                                 int32_t* dense, const void* workspace, void* stream) {
  if (!labels || !dense || !workspace || graphs <= 0 || seq_len <= 0 || new_seq_len <= 0)
    return ckv_internal::set_error(CKV_E_INVALID, "bad densify arguments");
  const int64_t V64 = (int64_t)graphs * seq_len;
  if (V64 >= (int64_t)1 << 30 || (int64_t)graphs * new_seq_len >= (int64_t)1 << 30)
    return ckv_internal::set_error(CKV_E_LIMIT, "densify: too many vertices");
  const int32_t V = (int32_t)V64;
  const int32_t* scan = (const int32_t*)((const char*)workspace + align256((size_t)V * 4));
  densify_apply_kernel<<<blocks(V, ETHREADS), ETHREADS, 0, (hipStream_t)stream>>>(labels, scan, V, seq_len,
                                                                                   new_seq_len, dense);
  return launch_check();
}

extern "C" size_t ckv_partition_modularity_workspace_bytes(int32_t vertices) {
  return vertices <= 0 ? 0 : 2 * align256((size_t)vertices * 8) + 256;
}

extern "C" int ckv_partition_modularity(const int32_t* edge_src, const int32_t* edge_dst, const float* edge_weight,
                                        int64_t edges, const int32_t* labels, int32_t vertices, float resolution,
                                        double* modularity, void* workspace, void* stream) {
  if (vertices <= 0 || edges < 0 || !labels || !modularity || !workspace ||
      (edges > 0 && (!edge_src || !edge_dst || !edge_weight)))
    return ckv_internal::set_error(CKV_E_INVALID, "bad modularity arguments");
  hipStream_t st = (hipStream_t)stream;
  double* k = (double*)workspace;
  double* sig = (double*)((char*)workspace + align256((size_t)vertices * 8));
  double* acc = (double*)((char*)workspace + 2 * align256((size_t)vertices * 8));
  mod_zero_kernel<<<blocks(vertices, ETHREADS), ETHREADS, 0, st>>>(k, sig, vertices, acc);
  if (edges > 0)
    mod_edge_kernel<<<blocks(edges, 256), 256, 0, st>>>(edge_src, edge_dst, edge_weight, edges, labels, vertices, k,
                                                        acc);
  mod_sigma_kernel<<<blocks(vertices, 256), 256, 0, st>>>(labels, k, vertices, sig, acc);
  mod_square_kernel<<<blocks(vertices, 256), 256, 0, st>>>(sig, vertices, acc);
  mod_final_kernel<<<1, 64, 0, st>>>(acc, resolution, modularity);
  return launch_check();
}

extern "C" size_t ckv_adjacency_workspace_bytes(int32_t graphs, int32_t rows, int32_t kappa, float lam) {
  if (graphs <= 0 || rows < 0 || kappa <= 0) return 0;
  const int64_t n = adjacency_entries(graphs, rows, kappa, lam);
  return n == 0 ? 0 : agg_layout(n).total;
}

extern "C" int64_t ckv_adjacency_capacity(int32_t graphs, int32_t rows, int32_t kappa, float lam) {
  if (graphs <= 0 || rows < 0 || kappa <= 0) return 0;
  return adjacency_entries(graphs, rows, kappa, lam);
}

extern "C" int ckv_build_adjacency(const int32_t* topk_indices, const float* topk_scores,
                                   const int64_t* query_positions, int32_t graphs, int32_t rows, int32_t kappa,
                                   int32_t seq_len, float lam, int32_t* out_src, int32_t* out_dst, float* out_weight,
                                   int64_t* out_count, void* workspace, void* stream) {
  if (graphs <= 0 || rows < 0 || kappa <= 0 || kappa > 64 || seq_len <= 0 || !out_count || !(lam >= 0.0f && lam <= 1.0f))
    return ckv_internal::set_error(CKV_E_INVALID, "bad adjacency sizes (kappa <= 64, lam in [0, 1])");
  hipStream_t st = (hipStream_t)stream;
  const int64_t n = adjacency_entries(graphs, rows, kappa, lam);
  if (n == 0) {
    if (hipMemsetAsync(out_count, 0, 8, st) != hipSuccess) return launch_check();
    return 0;
  }
  if (!topk_indices || !topk_scores || !query_positions || !out_src || !out_dst || !out_weight || !workspace)
    return ckv_internal::set_error(CKV_E_INVALID, "null adjacency pointer");
  const int64_t V = (int64_t)graphs * seq_len;
  if (n >= ((int64_t)1 << 31) - 1 || V >= (int64_t)1 << 30)
    return ckv_internal::set_error(CKV_E_LIMIT, "adjacency too large");
  const AggLayout L = agg_layout(n);
  char* ws = (char*)workspace;
  const int bits = bits_for((uint64_t)V - 1);
  const int end_bit = bits + bits_for((uint64_t)V);
  const int per_row = (int)(n / ((int64_t)graphs * rows));
  adjacency_expand_kernel<<<blocks(n, ETHREADS), ETHREADS, 0, st>>>(
      topk_indices, topk_scores, query_positions, graphs, rows, kappa, seq_len, lam / 2.0f, 1.0f - lam, per_row, bits,
      (uint64_t*)(ws + L.keys_a), (float*)(ws + L.vals_a));
  return coalesce(L, ws, n, (int32_t)V, bits, end_bit, out_src, out_dst, out_weight, out_count, st);
}
