// Prefill graph state assembled on the GPU from dense community labels: the
// recency-descending membership CSR, FP8 (or f32) centroid tables with their
// community sizes, the modularity weights of the prefill edges and the
// per-token community table.  Restates the reference's state build after
// Leiden (graph/partition.py:382-535, called from build_partitioned_layer
// 538-618).
//
// Every integer output is exact, and the centroid sums follow one fixed order
// (a community's members in ascending position order, in blocks of 64: each
// block summed in order by one wave, lane = two dims, then the block sums
// added in order), so they are reproducible bit for bit; blocks spread a large
// community over many waves.  The modularity weights add edge weights with
// float atomics, like the reference's scatter_add_; their summation order is
// not fixed.
//
// Launch sequence of ckv_build_layer_state (one stream):
//   chunk_hist_kernel     per (graph, position chunk): community histogram
//   csr_scan_kernel       per graph: CSR offsets, each chunk's first slot per
//                         community, and the table of 64-member blocks
//   csr_scatter_kernel    per (graph, chunk): member positions, newest first
//   block_sum_kernel      per (retrieval head, block): in-order key sum of 64 members
//   centroid_kernel       per (retrieval head, community): block sums in order,
//                         mean -> clamp -> E4M3 / f32
//   token_table_kernel    labels -> token_communities (-1 past the prompt)
//   weight_zero_kernel + edge_weight_kernel   modularity weights from an edge list, or
//   weight_zero_kernel + topk_weight_kernel   the same weights from the prefill top-k edges
#include <hip/hip_runtime.h>

#include <algorithm>

#include <stdint.h>

#include "ckv_device.h"
#include "ckv_error.h"

namespace ckv {
namespace {

constexpr int MAX_CHUNKS = 64;           // position chunks per graph (histogram / scatter)
constexpr int MIN_CHUNK = 512;
constexpr int SUM_BLOCK = 64;            // members per centroid partial sum
constexpr int COUNT_THREADS = 1024;
constexpr int SCAN_THREADS = 1024;
constexpr int HIST_THREADS = 256;
constexpr int STATE_LDS_COMMUNITIES = 16384;  // per-community LDS counters of one kernel (64 KB)
constexpr int CENTROID_WAVES = 4;        // community rows per centroid workgroup
constexpr int EDGE_THREADS = 256;

// Positions per chunk: at least MIN_CHUNK, at most MAX_CHUNKS chunks, a multiple of 64.
inline int state_chunk(int seq_len, int num_sink) {
  const int n = seq_len - num_sink;
  int c = (n + MAX_CHUNKS - 1) / MAX_CHUNKS;
  c = (c + 63) / 64 * 64;
  return c < MIN_CHUNK ? MIN_CHUNK : c;
}
inline int state_chunks(int seq_len, int num_sink) {
  const int n = seq_len - num_sink;
  return n <= 0 ? 0 : (n + state_chunk(seq_len, num_sink) - 1) / state_chunk(seq_len, num_sink);
}
// Upper bound of the 64-member blocks of one graph.
inline int64_t state_max_blocks(int seq_len, int num_sink, int maxc) {
  return (int64_t)(seq_len - num_sink + SUM_BLOCK - 1) / SUM_BLOCK + maxc;
}

// Workspace carve-up (int32 units): histograms, block starts, block communities, f32 partial sums.
struct StateWorkspace {
  int32_t* hist;       // [graphs][chunks][maxc]
  int32_t* blk_first;  // [graphs][maxc + 1]
  int32_t* blk_comm;   // [graphs][max_blocks]
  float* partial;      // [retrieval_heads][max_blocks][128]
};

inline size_t state_ws_words(int graphs, int heads, int seq_len, int num_sink, int maxc, StateWorkspace* w,
                             int32_t* base) {
  const int64_t chunks = state_chunks(seq_len, num_sink);
  const int64_t mb = state_max_blocks(seq_len, num_sink, maxc);
  size_t off = 0;
  auto take = [&](int64_t words) {
    const size_t at = off;
    off += (size_t)((words + 63) / 64 * 64);  // 256-byte aligned pieces
    return at;
  };
  const size_t h = take((int64_t)graphs * chunks * maxc);
  const size_t bf = take((int64_t)graphs * (maxc + 1));
  const size_t bc = take((int64_t)graphs * mb);
  const size_t pt = take((int64_t)heads * mb * D);
  if (w && base) {
    w->hist = base + h;
    w->blk_first = base + bf;
    w->blk_comm = base + bc;
    w->partial = reinterpret_cast<float*>(base + pt);
  }
  return off;
}

// community_counts[g] = 1 + the largest label of a non-sink position, 0 when
// there is none, -1 when a non-sink label is negative.
__global__ __launch_bounds__(COUNT_THREADS) void label_count_kernel(const int32_t* __restrict__ labels, int seq_len,
                                                                    int num_sink, int32_t* __restrict__ counts) {
  const int g = blockIdx.x;
  const int32_t* row = labels + (int64_t)g * seq_len;
  int mx = -1, mn = 0;
  for (int p = num_sink + threadIdx.x; p < seq_len; p += COUNT_THREADS) {
    const int v = row[p];
    mx = max(mx, v);
    mn = min(mn, v);
  }
  __shared__ int s_max[COUNT_THREADS / 64], s_min[COUNT_THREADS / 64];
  mx = wave_max_i32(mx);
  mn = -wave_max_i32(-mn);
  if ((threadIdx.x & 63) == 0) {
    s_max[threadIdx.x >> 6] = mx;
    s_min[threadIdx.x >> 6] = mn;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 0; w < COUNT_THREADS / 64; ++w) {
      mx = max(mx, s_max[w]);
      mn = min(mn, s_min[w]);
    }
    counts[g] = mn < 0 ? -1 : mx + 1;
  }
}

// hist[g][chunk][c]: members of community c among the chunk's positions.
// Communities below lds_n are counted in LDS, the others in the output row.
__global__ __launch_bounds__(HIST_THREADS) void chunk_hist_kernel(const int32_t* __restrict__ labels, int seq_len,
                                                                  int num_sink, int maxc, int lds_n, int chunk_len,
                                                                  int chunks, int32_t* __restrict__ hist) {
  extern __shared__ int h_s[];
  const int chunk = blockIdx.x, g = blockIdx.y;
  int32_t* out = hist + ((int64_t)g * chunks + chunk) * maxc;
  for (int c = threadIdx.x; c < lds_n; c += HIST_THREADS) h_s[c] = 0;
  for (int c = lds_n + threadIdx.x; c < maxc; c += HIST_THREADS) out[c] = 0;
  wait_vm();  // the zeroed row is in place before any workgroup thread adds to it
  __syncthreads();
  const int32_t* row = labels + (int64_t)g * seq_len;
  const int p0 = num_sink + chunk * chunk_len;
  const int p1 = min(p0 + chunk_len, seq_len);
  for (int p = p0 + threadIdx.x; p < p1; p += HIST_THREADS) {
    const int c = row[p];
    if (c >= 0 && c < lds_n) atomicAdd(h_s + c, 1);
    else if (c >= lds_n && c < maxc) atomicAdd(out + c, 1);
  }
  __syncthreads();
  for (int c = threadIdx.x; c < lds_n; c += HIST_THREADS) out[c] = h_s[c];
}

// Per graph: offsets[c] = members of communities below c; then every chunk's
// histogram entry becomes the CSR slot of that chunk's newest member of c
// (later chunks first: the CSR is recency descending).
__global__ __launch_bounds__(SCAN_THREADS) void csr_scan_kernel(int maxc, int chunks, int64_t max_blocks,
                                                                int32_t* __restrict__ hist,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ blk_first,
                                                                int32_t* __restrict__ blk_comm) {
  // communities c = k * SCAN_THREADS + tid, one block-wide scan per round k
  const int g = blockIdx.x;
  const int tid = threadIdx.x;
  int32_t* h = hist + (int64_t)g * chunks * maxc;
  int32_t* off = offsets + (int64_t)g * (maxc + 1);
  int32_t* bf = blk_first + (int64_t)g * (maxc + 1);
  int32_t* bc = blk_comm + (int64_t)g * max_blocks;
  __shared__ int s_wave[SCAN_THREADS / 64], s_wblk[SCAN_THREADS / 64];
  int carry = 0, bcarry = 0;
  for (int c0 = 0; c0 < maxc; c0 += SCAN_THREADS) {
    const int c = c0 + tid;
    int t = 0;
    if (c < maxc) {
#pragma unroll 8
      for (int i = 0; i < chunks; ++i) t += h[(int64_t)i * maxc + c];
    }
    const int nb = (t + SUM_BLOCK - 1) / SUM_BLOCK;
    const int inc = wave_inclusive_scan(t);
    const int incb = wave_inclusive_scan(nb);
    if ((tid & 63) == 63) {
      s_wave[tid >> 6] = inc;
      s_wblk[tid >> 6] = incb;
    }
    __syncthreads();
    int base = carry + inc - t, bbase = bcarry + incb - nb;
    int round = 0, bround = 0;
    for (int wv = 0; wv < SCAN_THREADS / 64; ++wv) {
      if (wv < (tid >> 6)) {
        base += s_wave[wv];
        bbase += s_wblk[wv];
      }
      round += s_wave[wv];
      bround += s_wblk[wv];
    }
    __syncthreads();  // s_wave reused next round
    if (c < maxc) {
      off[c] = base;
      bf[c] = bbase;
      for (int j = 0; j < nb; ++j) bc[bbase + j] = c;
      int run = base;
      for (int i0 = chunks - 1; i0 >= 0; i0 -= 8) {  // eight loads in flight, then their stores
        int n[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) n[u] = i0 - u >= 0 ? h[(int64_t)(i0 - u) * maxc + c] : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (i0 - u >= 0) {
            h[(int64_t)(i0 - u) * maxc + c] = run;
            run += n[u];
          }
        }
      }
    }
    carry += round;
    bcarry += bround;
  }
  if (tid == 0) {
    off[maxc] = carry;
    bf[maxc] = bcarry;
  }
}

// One wave per (graph, chunk): walks the chunk's positions from the newest
// down, 64 at a time (lane l takes the l-th newest); lanes with equal labels
// are ranked by lane (newer first) one distinct label per round, and an LDS
// cursor per community advances by each round's members.
// Cursors of communities below lds_n live in LDS, the others in the chunk's
// histogram row (which nothing reads afterwards).
__global__ __launch_bounds__(64) void csr_scatter_kernel(const int32_t* __restrict__ labels, int seq_len, int num_sink,
                                                         int maxc, int lds_n, int chunk_len, int chunks,
                                                         int32_t* __restrict__ hist,
                                                         int32_t* __restrict__ member_positions) {
  extern __shared__ int cur_s[];
  const int chunk = blockIdx.x, g = blockIdx.y;
  const int lane = threadIdx.x;
  int32_t* h = hist + ((int64_t)g * chunks + chunk) * maxc;
  for (int c = lane; c < lds_n; c += 64) cur_s[c] = h[c];
  wave_sync();
  const int32_t* row = labels + (int64_t)g * seq_len;
  int32_t* out = member_positions + (int64_t)g * (seq_len - num_sink);
  const int p0 = num_sink + chunk * chunk_len;
  const int p1 = min(p0 + chunk_len, seq_len);
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int top = p1 - 1; top >= p0; top -= 64) {
    const int p = top - lane;
    const bool ok = p >= p0;
    const int c = ok ? row[p] : -1;
    const bool valid = ok && c >= 0 && c < maxc;
    uint64_t todo = __ballot(valid);
    while (todo) {
      const int leader = __builtin_ctzll(todo);
      const int lc = __builtin_amdgcn_readlane(c, leader);
      const uint64_t m = __ballot(valid && c == lc);
      const int base = lc < lds_n ? cur_s[lc] : h[lc];
      if (valid && c == lc) out[base + __popcll(m & below)] = p;
      wave_sync();
      if (lane == leader) {
        if (lc < lds_n) cur_s[lc] = base + __popcll(m);
        else h[lc] = base + __popcll(m);
      }
      if (lc >= lds_n) wait_vm();  // (wave-uniform) the cursor store lands before a later round reads it
      wave_sync();
      todo &= ~m;
    }
  }
}

// One wave per (retrieval head, 64-member block): members 64k .. 64k+63 of
// community c in ascending position order (the CSR lists them newest first),
// summed in order in f32, lane = dims 2l and 2l+1.  All 64 rows are loaded
// before the sum, so a block costs one gather round.
template <int KT>
__global__ __launch_bounds__(64 * CENTROID_WAVES) void block_sum_kernel(
    const void* __restrict__ keys, int64_t head_stride, int64_t token_stride, const int32_t* __restrict__ to_graph,
    const int32_t* __restrict__ to_kv, const int32_t* __restrict__ offsets, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ blk_first, const int32_t* __restrict__ blk_comm, int64_t max_blocks, int seq_len,
    int num_sink, int maxc, float* __restrict__ partial) {
  const int r = blockIdx.y;
  const int64_t b = (int64_t)blockIdx.x * CENTROID_WAVES + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = to_graph[r];
  const int kvh = to_kv[r];
  if (b >= blk_first[(int64_t)g * (maxc + 1) + maxc]) return;  // past this graph's blocks
  const int c = blk_comm[(int64_t)g * max_blocks + b];
  const int k = (int)(b - blk_first[(int64_t)g * (maxc + 1) + c]);
  const int lo = offsets[(int64_t)g * (maxc + 1) + c];
  const int hi = offsets[(int64_t)g * (maxc + 1) + c + 1];
  const int i0 = SUM_BLOCK * k;  // ascending member index of the block's first member
  const int n = min(SUM_BLOCK, hi - lo - i0);
  const int32_t* mem = positions + (int64_t)g * (seq_len - num_sink);
  const int mine = mem[hi - 1 - (i0 + min(lane, n - 1))];
  const int64_t kb = (int64_t)kvh * head_stride + 2 * lane;
  float x0[SUM_BLOCK], x1[SUM_BLOCK];
#pragma unroll
  for (int u = 0; u < SUM_BLOCK; ++u) {
    const int p = __builtin_amdgcn_readlane(mine, u);  // lanes past n repeat the last member
    if constexpr (KT == CKV_BF16) {
      const uint32_t w = (uint32_t)gload_i32(reinterpret_cast<const int32_t*>(
          reinterpret_cast<const uint16_t*>(keys) + kb + (int64_t)p * token_stride));
      x0[u] = ckv_u2f(w << 16);
      x1[u] = ckv_u2f(w & 0xffff0000u);
    } else {
      const float* kp = reinterpret_cast<const float*>(keys) + kb + (int64_t)p * token_stride;
      x0[u] = gload_f32(kp);
      x1[u] = gload_f32(kp + 1);
    }
  }
  float s0 = 0.0f, s1 = 0.0f;  // (+0 start: an all-negative-zero block sums to +0, as scatter_add_ does)
#pragma unroll
  for (int u = 0; u < SUM_BLOCK; ++u) {
    if (u < n) {
      s0 = s0 + x0[u];
      s1 = s1 + x1[u];
    }
  }
  float* dst = partial + ((int64_t)r * max_blocks + b) * D + 2 * lane;
  dst[0] = s0;
  dst[1] = s1;
}

// One wave per (retrieval head, community row): the community's block sums
// added in order, divided by its size, clamped to +-448, then E4M3 or f32.
// Rows at or past maxc hold zeros.
template <int CT>
__global__ __launch_bounds__(64 * CENTROID_WAVES) void centroid_kernel(
    const int32_t* __restrict__ to_graph, const int32_t* __restrict__ offsets, const int32_t* __restrict__ blk_first,
    const float* __restrict__ partial, int64_t max_blocks, int maxc, int capacity, void* __restrict__ centroids,
    int32_t* __restrict__ sizes) {
  const int r = blockIdx.y;
  const int c = blockIdx.x * CENTROID_WAVES + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (c >= capacity) return;
  const int g = to_graph[r];
  int size = 0, b0 = 0, nb = 0;
  if (c < maxc) {
    size = offsets[(int64_t)g * (maxc + 1) + c + 1] - offsets[(int64_t)g * (maxc + 1) + c];
    b0 = blk_first[(int64_t)g * (maxc + 1) + c];
    nb = blk_first[(int64_t)g * (maxc + 1) + c + 1] - b0;
  }
  const float* src = partial + ((int64_t)r * max_blocks + b0) * D + 2 * lane;
  float s0 = 0.0f, s1 = 0.0f;
  for (int j0 = 0; j0 < nb; j0 += 16) {
    float y0[16], y1[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float* q = src + (int64_t)min(j0 + u, nb - 1) * D;
      y0[u] = gload_f32(q);
      y1[u] = gload_f32(q + 1);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (j0 + u < nb) {
        s0 = s0 + y0[u];
        s1 = s1 + y1[u];
      }
    }
  }
  if (c < maxc) {
    const float den = (float)max(size, 1);
    s0 = s0 / den;
    s1 = s1 / den;
  }
  s0 = fminf(fmaxf(s0, -448.0f), 448.0f);
  s1 = fminf(fmaxf(s1, -448.0f), 448.0f);
  const int64_t row = (int64_t)r * capacity + c;
  if constexpr (CT == CKV_E4M3) {
    const uint16_t pair = (uint16_t)(ckv_f32_to_e4m3(s0) | ((uint16_t)ckv_f32_to_e4m3(s1) << 8));
    reinterpret_cast<uint16_t*>(centroids)[row * (D / 2) + lane] = pair;
  } else {
    float* dst = reinterpret_cast<float*>(centroids) + row * D + 2 * lane;
    dst[0] = s0;
    dst[1] = s1;
  }
  if (lane == 0) sizes[row] = size;
}

__global__ void token_table_kernel(const int32_t* __restrict__ labels, int seq_len, int token_capacity, int graphs,
                                   int32_t* __restrict__ tokens) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)graphs * token_capacity;
  if (i >= total) return;
  const int g = (int)(i / token_capacity);
  const int t = (int)(i % token_capacity);
  tokens[i] = t < seq_len ? labels[(int64_t)g * seq_len + t] : -1;
}

__global__ void weight_zero_kernel(float* __restrict__ weight, int64_t n, float* __restrict__ total, int graphs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) weight[i] = 0.0f;
  if (i < graphs) total[i] = 0.0f;
}

// Community degree weights and 2m: each edge (graph * seq_len + position
// endpoints) adds its weight to both endpoint communities and twice to its
// graph's total.  A workgroup takes EDGES_PER_WG consecutive edges (the list
// is grouped by graph): the weights of the graph of its first edge gather in
// LDS and leave with one global atomic per touched community; edges of other
// graphs (at most a boundary's worth) add straight to global memory.
constexpr int EDGES_PER_WG = 8192;

__global__ __launch_bounds__(EDGE_THREADS) void edge_weight_kernel(
    const int32_t* __restrict__ labels, int seq_len, int graphs, int capacity, int lds_n,
    const int32_t* __restrict__ src, const int32_t* __restrict__ dst, const float* __restrict__ w, int64_t edges,
    float* __restrict__ weight, float* __restrict__ total) {
  extern __shared__ float w_s[];  // communities [0, lds_n) of the first edge's graph
  const int64_t e0 = (int64_t)blockIdx.x * EDGES_PER_WG;
  const int64_t e1 = min(edges, e0 + EDGES_PER_WG);
  const int g0 = src[e0] / seq_len;
  for (int c = threadIdx.x; c < lds_n; c += EDGE_THREADS) w_s[c] = 0.0f;
  __syncthreads();
  float mine = 0.0f;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += EDGE_THREADS) {
    const int s = src[e], d = dst[e];
    const int g = s / seq_len;
    if (g < 0 || g >= graphs || d / seq_len != g) continue;
    const float x = w[e];
    const int sc = labels[(int64_t)g * seq_len + s % seq_len];
    const int dc = labels[(int64_t)g * seq_len + d % seq_len];
    if (g == g0) {
      if (sc >= 0 && sc < lds_n) atomicAdd(w_s + sc, x);
      else if (sc >= lds_n && sc < capacity) atomicAdd(weight + (int64_t)g * capacity + sc, x);
      if (dc >= 0 && dc < lds_n) atomicAdd(w_s + dc, x);
      else if (dc >= lds_n && dc < capacity) atomicAdd(weight + (int64_t)g * capacity + dc, x);
      mine = mine + 2.0f * x;
    } else {
      if (sc >= 0 && sc < capacity) atomicAdd(weight + (int64_t)g * capacity + sc, x);
      if (dc >= 0 && dc < capacity) atomicAdd(weight + (int64_t)g * capacity + dc, x);
      atomicAdd(total + g, 2.0f * x);
    }
  }
  __shared__ float s_part[EDGE_THREADS / 64];
  mine = wave_sum_tree(mine);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = mine;
  __syncthreads();
  if (g0 >= 0 && g0 < graphs) {
    for (int c = threadIdx.x; c < lds_n; c += EDGE_THREADS) {
      const float v = w_s[c];
      if (v != 0.0f) atomicAdd(weight + (int64_t)g0 * capacity + c, v);
    }
    if (threadIdx.x == 0) {
      float t = 0.0f;
      for (int i = 0; i < EDGE_THREADS / 64; ++i) t = t + s_part[i];
      atomicAdd(total + g0, t);
    }
  }
}

// Modularity weights straight from the prefill top-k edges: one thread per
// (query head, row).  With the row's valid columns k (score p_k), S = sum p_k:
// the direct edges (position, column k) weigh lam/2 p_k, the co-occurrence
// edges (k, l), k <= l, weigh (1 - lam) p_k p_l.  Column k's community gains
// lam/2 p_k + (1 - lam) p_k (S + p_k) (its own pair k = k counts at both
// ends), the row position's community gains lam/2 S, and the graph's total
// 2 x (edge weights) = lam S + (1 - lam) (S^2 + sum p_k^2).  A workgroup's
// rows share one head, hence one graph: weights gather in LDS first.
constexpr int TOPK_ROWS_PER_WG = 256;

__global__ __launch_bounds__(TOPK_ROWS_PER_WG) void topk_weight_kernel(
    const int32_t* __restrict__ labels, int seq_len, int capacity, int lds_n, const int32_t* __restrict__ idx,
    const float* __restrict__ sc, int rows, int kappa, int group, int row0, float lam, float* __restrict__ weight,
    float* __restrict__ total) {
  extern __shared__ float w_s[];  // communities [0, lds_n)
  const int h = blockIdx.y;
  const int g = h / group;
  for (int c = threadIdx.x; c < lds_n; c += TOPK_ROWS_PER_WG) w_s[c] = 0.0f;
  __syncthreads();
  const int r = blockIdx.x * TOPK_ROWS_PER_WG + threadIdx.x;
  const int32_t* lab = labels + (int64_t)g * seq_len;
  float mine = 0.0f;
  if (r < rows) {
    const int32_t* ir = idx + ((int64_t)h * rows + r) * kappa;
    const float* sr = sc + ((int64_t)h * rows + r) * kappa;
    int col[16];
    float p[16];
    float s = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      col[k] = k < kappa ? ir[k] : -1;
      p[k] = k < kappa ? sr[k] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (col[k] >= 0 && col[k] < seq_len) {
        s = s + p[k];
        s2 = s2 + p[k] * p[k];
      }
    }
    const float half = 0.5f * lam, co = 1.0f - lam;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (col[k] >= 0 && col[k] < seq_len) {
        const int c = lab[col[k]];
        const float v = half * p[k] + co * (p[k] * (s + p[k]));
        if (c >= 0 && c < lds_n) atomicAdd(w_s + c, v);
        else if (c >= lds_n && c < capacity) atomicAdd(weight + (int64_t)g * capacity + c, v);
      }
    }
    const int pos = row0 + r;
    if (pos >= 0 && pos < seq_len) {
      const int c = lab[pos];
      if (c >= 0 && c < lds_n) atomicAdd(w_s + c, half * s);
      else if (c >= lds_n && c < capacity) atomicAdd(weight + (int64_t)g * capacity + c, half * s);
    }
    mine = lam * s + co * (s * s + s2);
  }
  __shared__ float s_part[TOPK_ROWS_PER_WG / 64];
  mine = wave_sum_tree(mine);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = mine;
  __syncthreads();
  for (int c = threadIdx.x; c < lds_n; c += TOPK_ROWS_PER_WG) {
    const float v = w_s[c];
    if (v != 0.0f) atomicAdd(weight + (int64_t)g * capacity + c, v);
  }
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int i = 0; i < TOPK_ROWS_PER_WG / 64; ++i) t = t + s_part[i];
    atomicAdd(total + g, t);
  }
}

int launch_check() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : ckv_internal::set_error(CKV_E_LAUNCH, hipGetErrorString(e));
}

}  // namespace
}  // namespace ckv

using namespace ckv;

extern "C" size_t ckv_state_workspace_bytes(int32_t graphs, int32_t retrieval_heads, int32_t seq_len,
                                            int32_t num_sink, int32_t max_communities) {
  if (graphs <= 0 || retrieval_heads <= 0 || seq_len <= num_sink || num_sink < 0 || max_communities <= 0) return 0;
  return state_ws_words(graphs, retrieval_heads, seq_len, num_sink, max_communities, nullptr, nullptr) *
         sizeof(int32_t);
}

extern "C" int ckv_label_counts(const int32_t* labels, int32_t graphs, int32_t seq_len, int32_t num_sink,
                                int32_t* community_counts, void* stream) {
  if (!labels || !community_counts) return ckv_internal::set_error(CKV_E_INVALID, "null label-count argument");
  if (graphs <= 0 || seq_len <= 0 || num_sink < 0)
    return ckv_internal::set_error(CKV_E_INVALID, "graphs and seq_len must be positive, num_sink nonnegative");
  hipLaunchKernelGGL(label_count_kernel, dim3(graphs), dim3(COUNT_THREADS), 0, (hipStream_t)stream, labels, seq_len,
                     num_sink, community_counts);
  return launch_check();
}

extern "C" int ckv_build_layer_state(const ckv_state_build_args* a, void* stream) {
  if (!a) return ckv_internal::set_error(CKV_E_INVALID, "null state-build argument");
  if (!a->labels || !a->keys || !a->retrieval_to_graph || !a->retrieval_to_kv || !a->member_offsets ||
      !a->member_positions || !a->centroids || !a->community_sizes || !a->token_communities || !a->workspace)
    return ckv_internal::set_error(CKV_E_INVALID, "null state-build pointer");
  if (a->graphs <= 0 || a->seq_len <= 0 || a->num_sink < 0 || a->num_sink >= a->seq_len ||
      a->retrieval_heads <= 0 || a->kv_heads <= 0)
    return ckv_internal::set_error(CKV_E_INVALID, "bad graph, head or sequence sizes (num_sink < seq_len)");
  if (a->max_communities <= 0 || a->max_communities > CKV_MAX_COMMUNITIES)
    return ckv_internal::set_error(CKV_E_LIMIT, "max_communities must be in [1, 65536]");
  if (a->community_capacity < a->max_communities)
    return ckv_internal::set_error(CKV_E_INVALID, "community_capacity must cover max_communities");
  if (a->token_capacity < a->seq_len) return ckv_internal::set_error(CKV_E_INVALID, "token_capacity < seq_len");
  if (a->key_dtype != CKV_BF16 && a->key_dtype != CKV_F32)
    return ckv_internal::set_error(CKV_E_INVALID, "key dtype must be bf16 or f32");
  if (a->centroid_dtype != CKV_E4M3 && a->centroid_dtype != CKV_F32)
    return ckv_internal::set_error(CKV_E_INVALID, "centroid dtype must be e4m3 or f32");
  if (a->head_stride <= 0 || a->token_stride < CKV_HEAD_DIM)
    return ckv_internal::set_error(CKV_E_INVALID, "bad key strides");
  if (a->edges < 0 || (a->edges > 0 && (!a->edge_src || !a->edge_dst || !a->edge_weight)))
    return ckv_internal::set_error(CKV_E_INVALID, "edges need src, dst and weight");
  if (a->edges > 0 && (!a->community_weight || !a->total_weight))
    return ckv_internal::set_error(CKV_E_INVALID, "edges need community_weight and total_weight outputs");
  if (a->topk_indices) {
    if (a->edges > 0) return ckv_internal::set_error(CKV_E_INVALID, "give either an edge list or top-k edges");
    if (!a->topk_scores || !a->community_weight || !a->total_weight)
      return ckv_internal::set_error(CKV_E_INVALID, "top-k edges need scores and the weight outputs");
    if (a->topk_kappa < 1 || a->topk_kappa > 16 || a->topk_heads <= 0 || a->topk_rows < 0 || a->topk_group <= 0 ||
        a->topk_heads > a->topk_group * a->graphs)
      return ckv_internal::set_error(CKV_E_INVALID, "bad top-k edge shape (kappa 1..16, heads <= group * graphs)");
  }
  const hipStream_t s = (hipStream_t)stream;
  const int maxc = a->max_communities;
  const int chunk_len = state_chunk(a->seq_len, a->num_sink);
  const int chunks = state_chunks(a->seq_len, a->num_sink);
  const int64_t mb = state_max_blocks(a->seq_len, a->num_sink, maxc);
  StateWorkspace w;
  state_ws_words(a->graphs, a->retrieval_heads, a->seq_len, a->num_sink, maxc, &w, a->workspace);
  // communities past lds_n are counted in global memory (64 KB of LDS per kernel)
  const int lds_n = std::min(maxc, STATE_LDS_COMMUNITIES);
  const size_t lds = (size_t)lds_n * sizeof(int);
  hipLaunchKernelGGL(chunk_hist_kernel, dim3(chunks, a->graphs), dim3(HIST_THREADS), lds, s, a->labels, a->seq_len,
                     a->num_sink, maxc, lds_n, chunk_len, chunks, w.hist);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(a->graphs), dim3(SCAN_THREADS), 0, s, maxc, chunks, mb, w.hist,
                     a->member_offsets, w.blk_first, w.blk_comm);
  hipLaunchKernelGGL(csr_scatter_kernel, dim3(chunks, a->graphs), dim3(64), lds, s, a->labels, a->seq_len,
                     a->num_sink, maxc, lds_n, chunk_len, chunks, w.hist, a->member_positions);
  const dim3 bgrid((unsigned)((mb + CENTROID_WAVES - 1) / CENTROID_WAVES), a->retrieval_heads);
  auto sums = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, bgrid, dim3(64 * CENTROID_WAVES), 0, s, a->keys, a->head_stride, a->token_stride,
                       a->retrieval_to_graph, a->retrieval_to_kv, (const int32_t*)a->member_offsets,
                       (const int32_t*)a->member_positions, (const int32_t*)w.blk_first,
                       (const int32_t*)w.blk_comm, mb, a->seq_len, a->num_sink, maxc, w.partial);
  };
  if (a->key_dtype == CKV_BF16) sums(block_sum_kernel<CKV_BF16>); else sums(block_sum_kernel<CKV_F32>);
  const dim3 cgrid((a->community_capacity + CENTROID_WAVES - 1) / CENTROID_WAVES, a->retrieval_heads);
  auto cent = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, cgrid, dim3(64 * CENTROID_WAVES), 0, s, a->retrieval_to_graph,
                       (const int32_t*)a->member_offsets, (const int32_t*)w.blk_first, (const float*)w.partial, mb,
                       maxc, a->community_capacity, a->centroids, a->community_sizes);
  };
  if (a->centroid_dtype == CKV_E4M3) cent(centroid_kernel<CKV_E4M3>); else cent(centroid_kernel<CKV_F32>);
  const int64_t ntok = (int64_t)a->graphs * a->token_capacity;
  hipLaunchKernelGGL(token_table_kernel, dim3((unsigned)((ntok + 255) / 256)), dim3(256), 0, s, a->labels,
                     a->seq_len, a->token_capacity, a->graphs, a->token_communities);
  if (a->community_weight && a->total_weight) {
    const int64_t nw = (int64_t)a->graphs * a->community_capacity;
    const int64_t nz = nw > a->graphs ? nw : a->graphs;
    hipLaunchKernelGGL(weight_zero_kernel, dim3((unsigned)((nz + 255) / 256)), dim3(256), 0, s, a->community_weight,
                       nw, a->total_weight, a->graphs);
    if (a->topk_indices && a->topk_rows > 0) {
      hipLaunchKernelGGL(topk_weight_kernel,
                         dim3((a->topk_rows + TOPK_ROWS_PER_WG - 1) / TOPK_ROWS_PER_WG, a->topk_heads),
                         dim3(TOPK_ROWS_PER_WG), (size_t)lds_n * sizeof(float), s, a->labels,
                         a->seq_len, a->community_capacity, lds_n, a->topk_indices, a->topk_scores, a->topk_rows,
                         a->topk_kappa, a->topk_group, a->topk_row0, a->lam, a->community_weight, a->total_weight);
    }
    if (a->edges > 0) {
      hipLaunchKernelGGL(edge_weight_kernel, dim3((unsigned)((a->edges + EDGES_PER_WG - 1) / EDGES_PER_WG)),
                         dim3(EDGE_THREADS), (size_t)lds_n * sizeof(float), s, a->labels, a->seq_len, a->graphs,
                         a->community_capacity, lds_n, a->edge_src, a->edge_dst, a->edge_weight, a->edges, a->community_weight, a->total_weight);
    }
  }
  return launch_check();
}
