// CommunityKV sparse decode for MI355X (gfx950, wave64).
//
// One decode-layer transition is three stream-ordered launches (four with a
// layer-wise shared graph):
//
//   score_select_kernel     grid (score_blocks, retrieval_heads) x 256
//       Every workgroup scores 64 communities of one retrieval head: 8 lanes
//       per centroid row (16 dims each, 16-byte fp8 loads), pinned fp32
//       summation order, fp16 round-to-nearest-even key.  The last workgroup
//       of each head to finish (agent-scope counter, no spinning) runs the
//       exact weighted threshold selection in LDS (two 8-bit radix passes
//       over order-preserving fp16 keys), emits descriptors in the reference
//       order and materialises the KV position of every attended slot.
//   attend_*_kernel         grid (slot_tiles, retrieval_heads) x 64
//       One wave per 64-slot tile: gathers K/V rows, exact softmax partials
//       (max, sum, P.V) per query head and the tile's top-8 candidates.
//   reduce_update_kernel    grid (retrieval_heads) x 128
//       Merges the split partials, then (graph owners) runs the fused online
//       update: top-8 merge, modularity-gain or nearest-centroid assignment,
//       running-mean FP8 centroid, delta-chunk append, overflow flags.
//   sync_shared_kernel      grid (retrieval_heads) x 128, layer-wise only.
//
// Reference kernels restated: attention/kernels/centroid_selection.py:32-188,
// attention/kernels/_csrc/descriptor_selection.cu:164-487,
// attention/kernels/segmented_attention.py:31-950.
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <string.h>

#include <type_traits>

#include "../../include/ckv_amd.h"
#include "ckv_error.h"
#include "ckv_numerics.h"

namespace {

constexpr int D = CKV_HEAD_DIM;
constexpr int TILE = CKV_TILE;
constexpr int KAPPA = CKV_KAPPA;
constexpr int SCORE_BLOCK = CKV_SCORE_BLOCK;
constexpr int SELECT_THREADS = 256;
constexpr int REDUCE_THREADS = 128;
constexpr float NEG_INF = -__builtin_huge_valf();

thread_local char g_error[512] = "";

int fail(int code, const char* message) {
  snprintf(g_error, sizeof(g_error), "%s", message);
  return code;
}

struct DecodeArgs {
  ckv_kv_cache kv;
  ckv_graph_state st;
  ckv_prefill_csr csr;
  ckv_delta_chunks dl;
  ckv_decode_config cfg;
  ckv_decode_workspace ws;
};

// ---------------------------------------------------------------------------
// Small device helpers
// ---------------------------------------------------------------------------

template <int DT>
__device__ inline float load_elem(const void* base, int64_t index) {
  if constexpr (DT == CKV_BF16) {
    return ckv_bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[index]);
  } else {
    return reinterpret_cast<const float*>(base)[index];
  }
}

// Loads 8 consecutive elements starting at `index` (16- or 32-byte aligned).
template <int DT>
__device__ inline void load8(const void* base, int64_t index, float* out) {
  if constexpr (DT == CKV_BF16) {
    const uint4 raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + index);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = ckv_u2f(w[i] << 16);
      out[2 * i + 1] = ckv_u2f(w[i] & 0xffff0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + index);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + index + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

// Loads 16 centroid values of row `row` starting at dim `d0`.
template <int CT>
__device__ inline void load_centroid16(const void* base, int64_t row, int d0, float* out) {
  if constexpr (CT == CKV_E4M3) {
    const uint4 raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(base) + row * D + d0);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < 4; ++b) out[4 * i + b] = ckv_e4m3_to_f32((uint8_t)((w[i] >> (8 * b)) & 0xffu));
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + row * D + d0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = p[i];
      out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  }
}

template <int CT>
__device__ inline float load_centroid1(const void* base, int64_t index) {
  if constexpr (CT == CKV_E4M3) {
    return ckv_e4m3_to_f32(reinterpret_cast<const uint8_t*>(base)[index]);
  } else {
    return reinterpret_cast<const float*>(base)[index];
  }
}

template <int CT>
__device__ inline void store_centroid1(void* base, int64_t index, float v) {
  if constexpr (CT == CKV_E4M3) {
    reinterpret_cast<uint8_t*>(base)[index] = ckv_f32_to_e4m3(v);
  } else {
    reinterpret_cast<float*>(base)[index] = v;
  }
}

__device__ inline float fmax_exact(float a, float b) { return a > b ? a : b; }

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax_exact(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ inline float wave_sum_tree(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

__device__ inline uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((uint32_t)(v & 0xffffffffu), o, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = shfl_xor_u64(v, o);
    v = w > v ? w : v;
  }
  return v;
}

__device__ inline uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = shfl_xor_u64(v, o);
    v = w < v ? w : v;
  }
  return v;
}

// Order-preserving 32-bit key of an fp32 score (segmented_attention.py:309-314).
__device__ inline uint32_t ordered_f32(float f) {
  const uint32_t b = ckv_f2u(f);
  return (b & 0x80000000u) ? ~b : (b ^ 0x80000000u);
}

__device__ inline float unordered_f32(uint32_t k) {
  return ckv_u2f((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// Top-8 candidate key: score descending, then position ascending.
__device__ inline uint64_t pack_candidate(float score, int32_t position) {
  return ((uint64_t)ordered_f32(score) << 32) | (uint64_t)(0xffffffffu - (uint32_t)position);
}

// Exclusive block scan of two ints over SELECT_THREADS threads; also returns totals.
__device__ inline void block_scan2(int a, int b, int& ea, int& eb, int& ta, int& tb, int* scratch) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int ia = a, ib = b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int xa = __shfl_up(ia, o, 64);
    const int xb = __shfl_up(ib, o, 64);
    if (lane >= o) {
      ia += xa;
      ib += xb;
    }
  }
  if (lane == 63) {
    scratch[2 * wave] = ia;
    scratch[2 * wave + 1] = ib;
  }
  __syncthreads();
  int ba = 0, bb = 0;
  ta = 0;
  tb = 0;
  for (int w = 0; w < SELECT_THREADS / 64; ++w) {
    if (w < wave) {
      ba += scratch[2 * w];
      bb += scratch[2 * w + 1];
    }
    ta += scratch[2 * w];
    tb += scratch[2 * w + 1];
  }
  ea = ba + ia - a;
  eb = bb + ib - b;
  __syncthreads();
}

// Finds, over a 256-bin histogram, the bin where the descending cumulative
// weight first reaches `target`.  Returns the bin (or -1) and the weight
// strictly above it.  Executed by wave 0.
__device__ inline void find_threshold_bin(const int* hist, int target, int* out_bin, int* out_above) {
  const int lane = threadIdx.x & 63;
  const int b0 = 4 * lane;
  const int h0 = hist[b0], h1 = hist[b0 + 1], h2 = hist[b0 + 2], h3 = hist[b0 + 3];
  const int local = h0 + h1 + h2 + h3;
  int suffix = local;  // inclusive suffix over lanes >= lane
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int x = __shfl_down(suffix, o, 64);
    if (lane + o < 64) suffix += x;
  }
  int above = suffix - local;  // weight of bins above this lane's four
  int bin = -1, bin_above = 0;
  const int hs[4] = {h0, h1, h2, h3};
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    if (bin < 0 && above < target && above + hs[i] >= target) {
      bin = b0 + i;
      bin_above = above;
    }
    above += hs[i];
  }
  const uint64_t hit = __ballot(bin >= 0);
  if (hit == 0) {
    if (lane == 0) {
      *out_bin = -1;
      *out_above = 0;
    }
    return;
  }
  const int owner = __ffsll((unsigned long long)hit) - 1;
  if (lane == owner) {
    *out_bin = bin;
    *out_above = bin_above;
  }
}

// ---------------------------------------------------------------------------
// Kernel 1: centroid scoring + (last block per head) exact selection
// ---------------------------------------------------------------------------

template <int CT, int DT>
__global__ __launch_bounds__(SELECT_THREADS) void score_select_kernel(DecodeArgs a) {
  const int rh = blockIdx.y;
  const int blk = blockIdx.x;
  const int tid = threadIdx.x;
  const int G = a.cfg.group_size;
  const int C = a.st.community_capacity;
  int count = a.st.community_counts[rh];
  count = count < 0 ? 0 : (count > C ? C : count);
  const int graph = a.st.retrieval_to_graph[rh];
  const int kvh = a.st.retrieval_to_kv[rh];
  const bool nearest_mode = a.cfg.assignment == CKV_ASSIGN_NEAREST;
  const int cur = a.st.current_position[graph];

  __shared__ float q_s[CKV_MAX_GROUP * D];
  __shared__ float key_s[D];
  __shared__ uint64_t red_u64[SELECT_THREADS / 64];
  __shared__ int last_block;

  for (int i = tid; i < G * D; i += SELECT_THREADS) {
    q_s[i] = load_elem<DT>(a.kv.query, (int64_t)rh * G * D + i);
  }
  if (nearest_mode && tid < D) {
    const bool ok = cur >= 0 && cur < a.kv.capacity;
    key_s[tid] = ok ? load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + (int64_t)cur * a.kv.token_stride + tid) : 0.0f;
  }
  __syncthreads();

  const int lane8 = tid & 7;
  const int sub = tid >> 3;
  uint64_t best_nearest = ~0ull;
  for (int pass = 0; pass < SCORE_BLOCK / (SELECT_THREADS / 8); ++pass) {
    const int c = blk * SCORE_BLOCK + pass * (SELECT_THREADS / 8) + sub;
    const bool active = c < count;
    float cv[16];
    int size = 0;
    if (active) {
      load_centroid16<CT>(a.st.centroids, (int64_t)rh * C + c, 16 * lane8, cv);
      size = a.st.community_sizes[(int64_t)rh * C + c];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) cv[i] = 0.0f;
    }
    float best = NEG_INF;
    for (int g = 0; g < G; ++g) {
      const float* q = q_s + g * D + 16 * lane8;
      float acc = q[0] * cv[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) acc = acc + q[i] * cv[i];
      acc = acc + __shfl_xor(acc, 4, 64);
      acc = acc + __shfl_xor(acc, 2, 64);
      acc = acc + __shfl_xor(acc, 1, 64);
      best = fmax_exact(best, acc);
    }
    const float score = (active && size > 0) ? best : NEG_INF;
    if (lane8 == 0 && c < C) a.ws.scores[(int64_t)rh * C + c] = ckv_f32_to_f16_bits(score);
    if (nearest_mode) {
      float acc;
      {
        const float d0 = key_s[16 * lane8] - cv[0];
        acc = d0 * d0;
      }
#pragma unroll
      for (int i = 1; i < 16; ++i) {
        const float di = key_s[16 * lane8 + i] - cv[i];
        acc = acc + di * di;
      }
      acc = acc + __shfl_xor(acc, 4, 64);
      acc = acc + __shfl_xor(acc, 2, 64);
      acc = acc + __shfl_xor(acc, 1, 64);
      if (active && size > 0) {
        const uint64_t cand = ((uint64_t)ckv_f2u(acc) << 32) | (uint32_t)c;
        best_nearest = cand < best_nearest ? cand : best_nearest;
      }
    }
  }
  if (nearest_mode) {
    const uint64_t w = wave_min_u64(best_nearest);
    if ((tid & 63) == 0) red_u64[tid >> 6] = w;
    __syncthreads();
    if (tid == 0) {
      uint64_t m = red_u64[0];
      for (int i = 1; i < SELECT_THREADS / 64; ++i) m = red_u64[i] < m ? red_u64[i] : m;
      a.ws.nearest_partial[(int64_t)rh * a.ws.score_blocks + blk] = m;
    }
  }

  // Last-arriving workgroup of this head performs the selection.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(a.ws.block_counters + rh, 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_block = (prev == gridDim.x - 1) ? 1 : 0;
    if (last_block) {
      __hip_atomic_store(a.ws.block_counters + rh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!last_block) return;
  __threadfence();

  extern __shared__ __align__(16) unsigned char dyn[];
  const int dcap = a.ws.descriptor_capacity;
  int* desc_comm = reinterpret_cast<int*>(dyn);
  int* desc_end = desc_comm + dcap;
  uint16_t* key16 = reinterpret_cast<uint16_t*>(desc_end + dcap);

  __shared__ int hist[256];
  __shared__ int scan_scratch[2 * (SELECT_THREADS / 64)];
  __shared__ int s_bin, s_above, s_hb, s_mass_above_hb;
  __shared__ int s_high_stored, s_high_count, s_high_mass, s_desc_count, s_sel_count;
  __shared__ int s_last_sel_pos;

  // Only scored communities take part (score_coverage bounds the active count).
  if (count > (int)gridDim.x * SCORE_BLOCK) count = (int)gridDim.x * SCORE_BLOCK;
  const bool budget_mode = a.cfg.selection_mode == CKV_SELECT_BUDGET;
  const int sel_slots = a.cfg.max_selected;
  const int target = budget_mode ? sel_slots : a.cfg.topk_communities;

  for (int c = tid; c < count; c += SELECT_THREADS) {
    key16[c] = ckv_ordered_key16(a.ws.scores[(int64_t)rh * C + c]);
  }
  hist[tid] = 0;
  __syncthreads();
  // Pass 1: weighted histogram of the high key byte.
  for (int c = tid; c < count; c += SELECT_THREADS) {
    const int size = a.st.community_sizes[(int64_t)rh * C + c];
    if (size > 0) atomicAdd(hist + (key16[c] >> 8), budget_mode ? size : 1);
  }
  __syncthreads();
  if (tid < 64) find_threshold_bin(hist, target, &s_bin, &s_above);
  __syncthreads();
  const int hb = s_bin;
  int threshold;  // 16-bit key threshold; -1 selects every non-empty community
  if (hb < 0) {
    threshold = -1;
  } else {
    const int above_hb = s_above;
    hist[tid] = 0;
    __syncthreads();
    for (int c = tid; c < count; c += SELECT_THREADS) {
      const int size = a.st.community_sizes[(int64_t)rh * C + c];
      if (size > 0 && (key16[c] >> 8) == hb) atomicAdd(hist + (key16[c] & 0xff), budget_mode ? size : 1);
    }
    __syncthreads();
    if (tid < 64) find_threshold_bin(hist, target - above_hb, &s_bin, &s_above);
    __syncthreads();
    threshold = (hb << 8) | s_bin;
  }

  // Compaction, high keys first (id order), then threshold keys (id order).
  const int cap_tokens = sel_slots;
  int base_cnt = 0, base_mass = 0, stored = 0;
  for (int start = 0; start < count; start += SELECT_THREADS) {
    const int c = start + tid;
    int size = 0;
    bool high = false;
    if (c < count) {
      size = a.st.community_sizes[(int64_t)rh * C + c];
      high = size > 0 && (int)key16[c] > threshold;
    }
    int ec, em, tc, tm;
    block_scan2(high ? 1 : 0, high ? size : 0, ec, em, tc, tm, scan_scratch);
    if (high) {
      const int idx = base_cnt + ec;
      const int st0 = base_mass + em;
      if (st0 < cap_tokens && idx < dcap) {
        desc_comm[idx] = c;
        desc_end[idx] = min(cap_tokens, st0 + size);
      }
    }
    // number of stored high descriptors: those whose start is below the cap
    int sc_local = (high && base_mass + em < cap_tokens) ? 1 : 0;
    int e2, e3, t2, t3;
    block_scan2(sc_local, 0, e2, e3, t2, t3, scan_scratch);
    stored += t2;
    base_cnt += tc;
    base_mass += tm;
  }
  const int high_count = base_cnt;
  const int high_mass = base_mass;
  const int high_stored = stored;
  int eq_cnt = 0, eq_mass = 0, eq_stored = 0;
  if (threshold >= 0) {
    for (int start = 0; start < count; start += SELECT_THREADS) {
      const int c = start + tid;
      int size = 0;
      bool eq = false;
      if (c < count) {
        size = a.st.community_sizes[(int64_t)rh * C + c];
        eq = size > 0 && (int)key16[c] == threshold;
      }
      int ec, em, tc, tm;
      block_scan2(eq ? 1 : 0, eq ? size : 0, ec, em, tc, tm, scan_scratch);
      bool take = false;
      if (eq) {
        const int st0 = high_mass + eq_mass + em;
        const bool within = budget_mode ? (st0 < sel_slots)
                                        : (eq_cnt + ec < a.cfg.topk_communities - high_count);
        take = within && st0 < cap_tokens;
        const int idx = high_count + eq_cnt + ec;
        if (take && idx < dcap) {
          desc_comm[idx] = c;
          desc_end[idx] = min(cap_tokens, st0 + size);
        }
      }
      int e2, e3, t2, t3;
      block_scan2(take ? 1 : 0, 0, e2, e3, t2, t3, scan_scratch);
      eq_stored += t2;
      eq_cnt += tc;
      eq_mass += tm;
    }
  }
  int desc_count = high_stored + eq_stored;
  if (desc_count > dcap) desc_count = dcap;
  if (tid == 0) {
    const int sel_count = desc_count > 0 ? desc_end[desc_count - 1] : 0;
    s_desc_count = desc_count;
    s_sel_count = sel_count;
    s_high_stored = high_stored < desc_count ? high_stored : desc_count;
    s_high_count = high_count;
    s_high_mass = high_mass;
    s_last_sel_pos = -1;
    a.ws.descriptor_counts[rh] = desc_count;
    a.ws.selected_counts[rh] = sel_count;
  }
  __syncthreads();
  const int n_desc = s_desc_count;
  const int sel_count = s_sel_count;
  for (int i = tid; i < n_desc; i += SELECT_THREADS) {
    a.ws.communities[(int64_t)rh * dcap + i] = desc_comm[i];
    a.ws.cumulative_ends[(int64_t)rh * dcap + i] = desc_end[i];
  }
  const int ns = a.cfg.num_sink;
  for (int t = tid; t < a.ws.budget_tiles; t += SELECT_THREADS) {
    const int off = max(t * TILE - ns, 0);
    int lo = 0, hi = n_desc;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (desc_end[mid] <= off) lo = mid + 1; else hi = mid;
    }
    a.ws.tile_descriptors[(int64_t)rh * a.ws.budget_tiles + t] = max(0, min(lo, n_desc - 1));
  }

  if (nearest_mode && tid == 0) {
    uint64_t m = ~0ull;
    for (int b = 0; b < a.ws.score_blocks; ++b) {
      const uint64_t v = a.ws.nearest_partial[(int64_t)rh * a.ws.score_blocks + b];
      m = v < m ? v : m;
    }
    a.ws.nearest[rh] = (m == ~0ull) ? -1 : (int)(m & 0xffffffffu);
  }
  // Without a membership CSR the call only scores and selects.
  if (a.csr.member_offsets == nullptr) return;

  // Slot materialisation: sinks, selected members (newest first), window, current.
  const int W = a.cfg.local_window;
  const int inc = a.cfg.include_current ? 1 : 0;
  const int slot_cap = a.ws.slot_capacity;
  int32_t* slots = a.ws.slot_positions + (int64_t)rh * slot_cap;
  const int64_t tbl = (int64_t)graph * C;
  for (int s = tid; s < slot_cap; s += SELECT_THREADS) {
    int pos = -1;
    if (s < ns) {
      pos = a.cfg.sink_positions[s];
    } else if (s < ns + sel_count) {
      const int j = s - ns;
      if (j < sel_count) {
        int lo = 0, hi = n_desc;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (desc_end[mid] <= j) lo = mid + 1; else hi = mid;
        }
        const int d = lo;
        const int prev = d > 0 ? desc_end[d - 1] : 0;
        const int m = j - prev;
        const int c = desc_comm[d];
        const int dc = a.dl.community_sizes[tbl + c];
        if (m < dc) {
          int rem = m;
          int ch = a.dl.community_tail[tbl + c];
          const int64_t cb = (int64_t)graph * a.dl.chunks_per_graph;
          for (int guard = 0; guard < 64 && ch >= 0 && ch < a.dl.chunks_per_graph; ++guard) {
            const int cs = a.dl.chunk_size[cb + ch];
            if (rem < cs) {
              const int at = a.dl.chunk_start[cb + ch] + cs - 1 - rem;
              if (at >= 0 && at < a.dl.position_capacity) {
                pos = a.dl.positions[(int64_t)graph * a.dl.position_capacity + at];
              }
              break;
            }
            rem -= cs;
            ch = a.dl.chunk_previous[cb + ch];
          }
        } else {
          const int64_t ob = (int64_t)graph * (C + 1) + c;
          const int at = a.csr.member_offsets[ob] + (m - dc);
          if (at < a.csr.member_offsets[ob + 1] && at < a.csr.member_stride) {
            pos = a.csr.member_positions[(int64_t)graph * a.csr.member_stride + at];
          }
        }
        if (j == sel_count - 1) s_last_sel_pos = pos;
      }
    } else if (s < ns + sel_count + W) {
      continue;  // window slots are resolved after the barrier below
    } else if (inc && s == ns + sel_count + W) {
      pos = cur;
    }
    slots[s] = pos;
  }
  __syncthreads();
  if (W > 0) {
    const int last_pos = s_last_sel_pos;
    const int hs = s_high_stored;
    for (int i = tid; i < W; i += SELECT_THREADS) {
      const int p = cur - W + i;
      int pos = p;
      if (p < 0) pos = -1;
      for (int k = 0; k < ns && pos >= 0; ++k) {
        if (a.cfg.sink_positions[k] == p) pos = -1;
      }
      if (pos >= 0 && p < a.st.token_capacity) {
        const int c = a.st.token_communities[(int64_t)graph * a.st.token_capacity + p];
        if (c >= 0 && c < count) {
          int found = -1;
          int lo = 0, hi = hs;
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (desc_comm[mid] < c) lo = mid + 1; else hi = mid;
          }
          if (lo < hs && desc_comm[lo] == c) found = lo;
          if (found < 0) {
            lo = hs;
            hi = n_desc;
            while (lo < hi) {
              const int mid = (lo + hi) >> 1;
              if (desc_comm[mid] < c) lo = mid + 1; else hi = mid;
            }
            if (lo < n_desc && desc_comm[lo] == c) found = lo;
          }
          if (found >= 0) {
            const int take = desc_end[found] - (found > 0 ? desc_end[found - 1] : 0);
            const int size = a.st.community_sizes[(int64_t)rh * C + c];
            if (take >= size || p >= last_pos) pos = -1;
          }
        }
      }
      slots[ns + sel_count + i] = pos;
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: attention partials (portable wave64 VALU version)
// ---------------------------------------------------------------------------

// One wave per 64-slot tile.  DENSE: rows come from [0, dense_len) and
// blockIdx.y is a KV head; otherwise from the slot table of retrieval head
// blockIdx.y.
template <int DT, bool DENSE>
__global__ __launch_bounds__(64) void attend_generic_kernel(DecodeArgs a, int dense_len, int dense_group) {
  const int tile = blockIdx.x;
  const int head = blockIdx.y;
  const int lane = threadIdx.x;
  const int tiles = gridDim.x;
  const int G = DENSE ? dense_group : a.cfg.group_size;
  const int kvh = DENSE ? head : a.st.retrieval_to_kv[head];
  const float scale = a.cfg.softmax_scale;

  __shared__ float q_s[CKV_MAX_GROUP * D];
  __shared__ float p_s[CKV_MAX_GROUP * TILE];
  __shared__ int pos_s[TILE];

  int pos;
  if (DENSE) {
    const int t = tile * TILE + lane;
    pos = t < dense_len ? t : -1;
  } else {
    pos = a.ws.slot_positions[(int64_t)head * a.ws.slot_capacity + tile * TILE + lane];
  }
  const bool valid = pos >= 0 && pos < a.kv.capacity;
  pos_s[lane] = valid ? pos : -1;
  for (int i = lane; i < G * D; i += 64) q_s[i] = load_elem<DT>(a.kv.query, (int64_t)head * G * D + i);
  __syncthreads();

  float s[CKV_MAX_GROUP];
#pragma unroll
  for (int g = 0; g < CKV_MAX_GROUP; ++g) s[g] = 0.0f;
  if (valid) {
    const int64_t row = kvh * a.kv.head_stride + (int64_t)pos * a.kv.token_stride;
    for (int d0 = 0; d0 < D; d0 += 8) {
      float k[8];
      load8<DT>(a.kv.key, row + d0, k);
#pragma unroll
      for (int g = 0; g < CKV_MAX_GROUP; ++g) {
        if (g < G) {
#pragma unroll
          for (int i = 0; i < 8; ++i) s[g] = s[g] + q_s[g * D + d0 + i] * k[i];
        }
      }
    }
  }
  float m_g[CKV_MAX_GROUP];
#pragma unroll
  for (int g = 0; g < CKV_MAX_GROUP; ++g) {
    if (g < G) {
      const float sc = valid ? s[g] * scale : NEG_INF;
      s[g] = sc;
      const float m = wave_max(sc);
      m_g[g] = m;
      float p = (valid && m != NEG_INF) ? __expf(sc - m) : 0.0f;
      const float l = wave_sum_tree(p);
      if (DT == CKV_BF16) p = ckv_bf16_to_f32(ckv_f32_to_bf16_bits(p));
      p_s[g * TILE + lane] = p;
      if (lane == 0) {
        const int qh = head * G + g;
        a.ws.partial_max[(int64_t)qh * tiles + tile] = m;
        a.ws.partial_sum[(int64_t)qh * tiles + tile] = l;
      }
    }
  }
  __syncthreads();
  // P.V: lane owns dims 2*lane, 2*lane+1.
  float o[CKV_MAX_GROUP][2];
#pragma unroll
  for (int g = 0; g < CKV_MAX_GROUP; ++g) o[g][0] = o[g][1] = 0.0f;
  for (int t = 0; t < TILE; ++t) {
    const int pt = pos_s[t];
    if (pt < 0) continue;
    const int64_t idx = kvh * a.kv.head_stride + (int64_t)pt * a.kv.token_stride + 2 * lane;
    const float v0 = load_elem<DT>(a.kv.value, idx);
    const float v1 = load_elem<DT>(a.kv.value, idx + 1);
#pragma unroll
    for (int g = 0; g < CKV_MAX_GROUP; ++g) {
      if (g < G) {
        const float p = p_s[g * TILE + t];
        o[g][0] = o[g][0] + p * v0;
        o[g][1] = o[g][1] + p * v1;
      }
    }
  }
#pragma unroll
  for (int g = 0; g < CKV_MAX_GROUP; ++g) {
    if (g < G) {
      const int qh = head * G + g;
      float* dst = a.ws.partial_acc + ((int64_t)qh * tiles + tile) * D + 2 * lane;
      dst[0] = o[g][0];
      dst[1] = o[g][1];
    }
  }
  if (!DENSE && a.cfg.assignment != CKV_ASSIGN_NONE) {
    const int slot = tile * TILE + lane;
    uint64_t cand = (valid && slot >= a.cfg.num_sink) ? pack_candidate(s[0], pos) : 0ull;
    for (int r = 0; r < KAPPA; ++r) {
      const uint64_t best = wave_max_u64(cand);
      if (lane == 0) a.ws.partial_topk[((int64_t)head * tiles + tile) * KAPPA + r] = best;
      if (cand == best) cand = 0ull;
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: split merge + fused online update
// ---------------------------------------------------------------------------

template <int DT>
__device__ inline void merge_head(const DecodeArgs& a, int qh, int tiles, void* out, float* lse_out,
                                  float* lse_keep) {
  const int d = threadIdx.x;
  const float* pm = a.ws.partial_max + (int64_t)qh * tiles;
  const float* ps = a.ws.partial_sum + (int64_t)qh * tiles;
  float M = NEG_INF;
  for (int t = 0; t < tiles; ++t) M = fmax_exact(M, pm[t]);
  float denom = 0.0f;
  float acc = 0.0f;
  for (int t = 0; t < tiles; ++t) {
    const float mt = pm[t];
    const float sc = (mt == NEG_INF) ? 0.0f : ckv_expf(mt - M);
    denom = denom + ps[t] * sc;
    acc = acc + a.ws.partial_acc[((int64_t)qh * tiles + t) * D + d] * sc;
  }
  const float r = acc / denom;
  if constexpr (DT == CKV_BF16) {
    reinterpret_cast<uint16_t*>(out)[(int64_t)qh * D + d] = ckv_f32_to_bf16_bits(r);
  } else {
    reinterpret_cast<float*>(out)[(int64_t)qh * D + d] = r;
  }
  const float l = M + ckv_logf(denom);
  if (d == 0) {
    lse_out[qh] = l;
    if (lse_keep) *lse_keep = l;
  }
}

template <int CT, int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void reduce_update_kernel(DecodeArgs a) {
  const int rh = blockIdx.x;
  const int tid = threadIdx.x;
  const int G = a.cfg.group_size;
  const int tiles = a.ws.slot_capacity / TILE;
  __shared__ float s_lse0;
  for (int g = 0; g < G; ++g) {
    merge_head<DT>(a, rh * G + g, tiles, a.ws.output, a.ws.lse, g == 0 ? &s_lse0 : nullptr);
  }
  const int graph = a.st.retrieval_to_graph[rh];
  if (a.cfg.assignment == CKV_ASSIGN_NONE || rh != graph) return;
  __syncthreads();

  const int C = a.st.community_capacity;
  __shared__ uint64_t top[KAPPA];
  __shared__ int s_assigned, s_comm_ov, s_old_size, s_valid_pos, s_cur;

  // Exact top-8 merge over every tile's candidates (wave 0).
  if (tid < 64) {
    const int n = tiles * KAPPA;
    const uint64_t* cand = a.ws.partial_topk + (int64_t)rh * n;
    uint64_t taken_hi = 0ull;  // candidates are unique; exclude by value
    for (int r = 0; r < KAPPA; ++r) {
      uint64_t best = 0ull;
      for (int i = tid; i < n; i += 64) {
        const uint64_t v = cand[i];
        if (v < taken_hi || taken_hi == 0ull) best = v > best ? v : best;
      }
      best = wave_max_u64(best);
      if (tid == 0) top[r] = best;
      taken_hi = best == 0ull ? 1ull : best;  // next round takes values strictly below
      if (best == 0ull) {
        for (int rr = r + 1; rr < KAPPA; ++rr) {
          if (tid == 0) top[rr] = 0ull;
        }
        break;
      }
    }
  }
  __syncthreads();

  if (tid == 0) {
    float sc[KAPPA];
    int ps[KAPPA];
    for (int r = 0; r < KAPPA; ++r) {
      const uint64_t v = top[r];
      if (v == 0ull) {
        sc[r] = NEG_INF;
        ps[r] = -1;
      } else {
        sc[r] = unordered_f32((uint32_t)(v >> 32));
        ps[r] = (int)(0xffffffffu - (uint32_t)(v & 0xffffffffu));
      }
      a.ws.topk_scores[(int64_t)rh * KAPPA + r] = sc[r];
      a.ws.topk_positions[(int64_t)rh * KAPPA + r] = ps[r];
    }
    const int cur = a.st.current_position[graph];
    const int64_t tc_cap = a.st.token_capacity < a.kv.capacity ? a.st.token_capacity : a.kv.capacity;
    const int active = a.st.community_counts[rh];
    const int active_c = active < C ? active : C;
    int assigned;
    bool comm_ov;
    if (a.cfg.assignment == CKV_ASSIGN_DELTA_Q) {
      const float lse0 = s_lse0;
      float p[KAPPA], dw[KAPPA], cw[KAPPA], oldw[KAPPA], dq[KAPPA];
      int comm[KAPPA];
      bool cand[KAPPA], leader[KAPPA];
      const float half_lam = a.cfg.lam * 0.5f;
      float nd = 0.0f, ssum = 0.0f, sq = 0.0f;
      for (int r = 0; r < KAPPA; ++r) {
        const bool valid = ps[r] >= 0 && ps[r] < tc_cap;
        p[r] = valid ? ckv_expf(sc[r] - lse0) : 0.0f;
        dw[r] = p[r] * half_lam;
        nd = nd + dw[r];
        ssum = ssum + p[r];
        sq = sq + p[r] * p[r];
        comm[r] = valid ? a.st.token_communities[(int64_t)graph * a.st.token_capacity + ps[r]] : -1;
        cand[r] = valid && comm[r] >= 0 && comm[r] < active_c;
      }
      const float pair = (ssum * ssum - sq) * (0.5f * (1.0f - a.cfg.lam));
      for (int r = 0; r < KAPPA; ++r) {
        float acc = 0.0f;
        int first = KAPPA;
        for (int j = 0; j < KAPPA; ++j) {
          if (cand[j] && comm[j] == comm[r]) {
            acc = acc + dw[j];
            first = j < first ? j : first;
          }
        }
        cw[r] = acc;
        leader[r] = cand[r] && first == r;
      }
      const float old_total = a.st.total_weight[graph];
      float two_m = 2.0f * old_total;
      two_m = two_m > 1.0f ? two_m : 1.0f;
      float best = NEG_INF;
      for (int r = 0; r < KAPPA; ++r) {
        oldw[r] = cand[r] ? a.st.community_weight[(int64_t)graph * C + comm[r]] : 0.0f;
        dq[r] = (cand[r] && cw[r] > 0.0f) ? (cw[r] - (nd * oldw[r]) / two_m) : NEG_INF;
        best = fmax_exact(best, dq[r]);
      }
      int best_comm = 0x7fffffff;
      for (int r = 0; r < KAPPA; ++r) {
        if (cand[r] && dq[r] == best && comm[r] < best_comm) best_comm = comm[r];
      }
      const bool join = best > 0.0f;
      assigned = join ? best_comm : active;
      comm_ov = assigned >= C;
      if (!comm_ov) {
        for (int r = 0; r < KAPPA; ++r) {
          if (leader[r]) {
            const float inc = cw[r] + ((join && comm[r] == assigned) ? nd : 0.0f);
            a.st.community_weight[(int64_t)graph * C + comm[r]] = oldw[r] + inc;
          }
        }
        if (!join) a.st.community_weight[(int64_t)graph * C + assigned] = nd;
        a.st.community_counts[rh] = active + (join ? 0 : 1);
        a.st.total_weight[graph] = (old_total + nd) + pair;
      }
    } else {
      const int nearest = a.ws.nearest[rh];
      assigned = nearest >= 0 ? nearest : active;
      comm_ov = assigned >= C;
      if (nearest < 0 && !comm_ov) a.st.community_counts[rh] = active + 1;
    }
    a.ws.assigned[graph] = comm_ov ? -1 : assigned;
    const bool valid_pos = cur >= 0 && cur < tc_cap;
    int old_size = 0;
    if (!comm_ov) {
      old_size = a.st.community_sizes[(int64_t)rh * C + assigned];
      a.st.community_sizes[(int64_t)rh * C + assigned] = old_size + 1;
      if (valid_pos) a.st.token_communities[(int64_t)graph * a.st.token_capacity + cur] = assigned;
    }
    s_assigned = assigned;
    s_comm_ov = comm_ov ? 1 : 0;
    s_old_size = old_size;
    s_valid_pos = valid_pos ? 1 : 0;
    s_cur = cur;
  }
  __syncthreads();
  const int kvh = a.st.retrieval_to_kv[rh];
  if (!s_comm_ov && s_valid_pos && tid < D) {
    const int asg = s_assigned;
    const int old_size = s_old_size;
    const int64_t ci = ((int64_t)rh * C + asg) * D + tid;
    const float key = load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + (int64_t)s_cur * a.kv.token_stride + tid);
    float upd;
    if (old_size > 0) {
      const float old = load_centroid1<CT>(a.st.centroids, ci);
      upd = (old * (float)old_size + key) / (float)(old_size + 1);
    } else {
      upd = key;
    }
    store_centroid1<CT>(a.st.centroids, ci, upd);
  }
  if (tid == 0) {
    const int asg = s_assigned;
    const bool comm_ov = s_comm_ov != 0;
    const bool valid_pos = s_valid_pos != 0;
    const int cur = s_cur;
    bool chunk_ov = false, pos_ov = false;
    if (!comm_ov) {
      const int64_t tb = (int64_t)graph * C + asg;
      const int64_t cb = (int64_t)graph * a.dl.chunks_per_graph;
      const int delta_size = a.dl.community_sizes[tb];
      const int old_tail = a.dl.community_tail[tb];
      const int old_cs = old_tail >= 0 ? a.dl.chunk_size[cb + old_tail] : 0;
      const int old_cc = old_tail >= 0 ? a.dl.chunk_capacity[cb + old_tail] : 0;
      const bool allocate = old_tail < 0 || old_cs >= old_cc;
      const int free_chunk = a.dl.next_free_chunk[graph];
      const int free_pos = a.dl.next_free_position[graph];
      const int new_cap = old_tail < 0 ? 1 : old_cc * 2;
      chunk_ov = allocate && free_chunk >= a.dl.chunks_per_graph;
      pos_ov = allocate && free_pos + new_cap > a.dl.position_capacity;
      const bool alloc_ov = chunk_ov || pos_ov;
      const int chunk = allocate ? free_chunk : old_tail;
      const bool valid_chunk = !alloc_ov && chunk >= 0 && chunk < a.dl.chunks_per_graph;
      if (allocate && !alloc_ov) {
        a.dl.next_free_chunk[graph] = free_chunk + 1;
        a.dl.next_free_position[graph] = free_pos + new_cap;
        a.dl.chunk_start[cb + free_chunk] = free_pos;
        a.dl.chunk_capacity[cb + free_chunk] = new_cap;
        a.dl.chunk_previous[cb + free_chunk] = old_tail;
        if (old_tail < 0) {
          a.dl.community_head[tb] = free_chunk;
        } else {
          a.dl.chunk_next[cb + old_tail] = free_chunk;
        }
        a.dl.community_tail[tb] = free_chunk;
      }
      if (valid_chunk && valid_pos) {
        const int start = allocate ? free_pos : a.dl.chunk_start[cb + old_tail];
        const int slot = allocate ? 0 : old_cs;
        a.dl.positions[(int64_t)graph * a.dl.position_capacity + start + slot] = cur;
        a.dl.chunk_size[cb + chunk] = slot + 1;
        a.dl.community_sizes[tb] = delta_size + 1;
      }
    }
    const int overflow = (comm_ov ? 1 : 0) | (chunk_ov ? 2 : 0) | (pos_ov ? 4 : 0) | (valid_pos ? 0 : 8);
    a.ws.overflow[graph] = overflow;
    if (overflow == 0) a.st.current_position[graph] = cur + 1;
  }
}

template <int CT, int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void sync_shared_kernel(DecodeArgs a) {
  const int rh = blockIdx.x;
  const int tid = threadIdx.x;
  const int graph = a.st.retrieval_to_graph[rh];
  if (rh == graph) return;
  const int C = a.st.community_capacity;
  const int community = a.ws.assigned[graph];
  const bool valid = a.ws.overflow[graph] == 0 && community >= 0;
  if (!valid) return;
  const int cur = a.st.current_position[graph] - 1;
  const int64_t tc_cap = a.st.token_capacity < a.kv.capacity ? a.st.token_capacity : a.kv.capacity;
  const bool valid_pos = cur >= 0 && cur < tc_cap;
  const int old_size = a.st.community_sizes[(int64_t)rh * C + community];
  __syncthreads();
  const int kvh = a.st.retrieval_to_kv[rh];
  if (valid_pos && tid < D) {
    const int64_t ci = ((int64_t)rh * C + community) * D + tid;
    const float key = load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + (int64_t)cur * a.kv.token_stride + tid);
    float upd;
    if (old_size > 0) {
      const float old = load_centroid1<CT>(a.st.centroids, ci);
      upd = (old * (float)old_size + key) / (float)(old_size + 1);
    } else {
      upd = key;
    }
    store_centroid1<CT>(a.st.centroids, ci, upd);
  }
  __syncthreads();
  if (tid == 0) {
    a.st.community_sizes[(int64_t)rh * C + community] = old_size + 1;
    a.st.community_counts[rh] = a.st.community_counts[graph];
  }
}

// Merge-only reduce for the dense baseline.
template <int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void dense_reduce_kernel(DecodeArgs a, int tiles) {
  merge_head<DT>(a, blockIdx.x, tiles, a.ws.output, a.ws.lse, nullptr);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

int validate(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
             const ckv_delta_chunks* dl, const ckv_decode_config* cfg, const ckv_decode_workspace* ws) {
  if (!kv || !st || !csr || !dl || !cfg || !ws) return fail(CKV_E_INVALID, "null argument struct");
  if (!kv->query || !kv->key || !kv->value) return fail(CKV_E_INVALID, "null query/key/value");
  if (kv->dtype != CKV_BF16 && kv->dtype != CKV_F32) return fail(CKV_E_INVALID, "kv dtype must be bf16 or f32");
  if (st->centroid_dtype != CKV_E4M3 && st->centroid_dtype != CKV_F32)
    return fail(CKV_E_INVALID, "centroid dtype must be e4m3 or f32");
  if (cfg->group_size < 1 || cfg->group_size > CKV_MAX_GROUP) return fail(CKV_E_INVALID, "group_size must be in [1, 16]");
  if (st->retrieval_heads <= 0 || st->graph_count <= 0 || st->community_capacity <= 0)
    return fail(CKV_E_INVALID, "empty graph state");
  if (st->retrieval_heads * cfg->group_size != kv->query_heads)
    return fail(CKV_E_INVALID, "query heads must equal retrieval heads x group size");
  if (st->community_capacity > CKV_MAX_COMMUNITIES) return fail(CKV_E_LIMIT, "community capacity exceeds 8192");
  if (ws->descriptor_capacity <= 0 || ws->descriptor_capacity > CKV_MAX_DESCRIPTORS)
    return fail(CKV_E_LIMIT, "descriptor capacity must be in [1, 4096]");
  if (ws->slot_capacity <= 0 || ws->slot_capacity % CKV_TILE) return fail(CKV_E_INVALID, "slot capacity must be a positive multiple of 64");
  if (cfg->num_sink < 0 || cfg->max_selected < 0 || cfg->local_window < 0) return fail(CKV_E_INVALID, "negative slot counts");
  if (cfg->num_sink + cfg->max_selected + cfg->local_window + (cfg->include_current ? 1 : 0) > ws->slot_capacity)
    return fail(CKV_E_INVALID, "slot capacity smaller than sinks + selected + window + current");
  if (csr->member_offsets && cfg->num_sink > 0 && !cfg->sink_positions)
    return fail(CKV_E_INVALID, "null sink positions");
  if (csr->member_offsets && (!csr->member_positions || !dl->positions || !dl->chunk_start || !dl->chunk_size ||
                              !dl->chunk_previous || !dl->community_tail || !dl->community_sizes))
    return fail(CKV_E_INVALID, "incomplete membership / delta-chunk state");
  if (cfg->selection_mode != CKV_SELECT_BUDGET && cfg->selection_mode != CKV_SELECT_TOPK)
    return fail(CKV_E_INVALID, "unknown selection mode");
  if (cfg->selection_mode == CKV_SELECT_TOPK && cfg->topk_communities <= 0)
    return fail(CKV_E_INVALID, "topk_communities must be positive");
  if (cfg->assignment < CKV_ASSIGN_NONE || cfg->assignment > CKV_ASSIGN_NEAREST)
    return fail(CKV_E_INVALID, "unknown assignment mode");
  if (cfg->score_coverage <= 0 || cfg->score_coverage > st->community_capacity)
    return fail(CKV_E_INVALID, "score coverage must be in [1, community capacity]");
  if (ws->score_blocks != (cfg->score_coverage + CKV_SCORE_BLOCK - 1) / CKV_SCORE_BLOCK)
    return fail(CKV_E_INVALID, "score_blocks must equal ceil(score_coverage / 64)");
  if (kv->head_stride % 8 || kv->token_stride % 8) return fail(CKV_E_INVALID, "kv strides must be multiples of 8 elements");
  return CKV_OK;
}

template <typename F>
int dispatch(int ct, int dt, F&& f) {
  if (ct == CKV_E4M3 && dt == CKV_BF16) return f(std::integral_constant<int, CKV_E4M3>{}, std::integral_constant<int, CKV_BF16>{});
  if (ct == CKV_E4M3 && dt == CKV_F32) return f(std::integral_constant<int, CKV_E4M3>{}, std::integral_constant<int, CKV_F32>{});
  if (ct == CKV_F32 && dt == CKV_BF16) return f(std::integral_constant<int, CKV_F32>{}, std::integral_constant<int, CKV_BF16>{});
  return f(std::integral_constant<int, CKV_F32>{}, std::integral_constant<int, CKV_F32>{});
}

int launch_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_error, sizeof(g_error), "%s launch failed: %s", what, hipGetErrorString(e));
    return CKV_E_LAUNCH;
  }
  return CKV_OK;
}

DecodeArgs pack(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                const ckv_delta_chunks* dl, const ckv_decode_config* cfg, const ckv_decode_workspace* ws) {
  DecodeArgs a;
  a.kv = *kv;
  a.st = *st;
  a.csr = *csr;
  a.dl = *dl;
  a.cfg = *cfg;
  a.ws = *ws;
  return a;
}

}  // namespace

int ckv_internal::set_error(int code, const char* message) { return fail(code, message); }

extern "C" int ckv_abi_version(void) { return CKV_ABI_VERSION; }

extern "C" int ckv_host_numerics(int op, const float* in, void* out, int64_t n) {
  if (!in || !out || n < 0) return fail(CKV_E_INVALID, "null argument");
  for (int64_t i = 0; i < n; ++i) {
    switch (op) {
      case 0: reinterpret_cast<float*>(out)[i] = ckv_expf(in[i]); break;
      case 1: reinterpret_cast<float*>(out)[i] = ckv_logf(in[i]); break;
      case 2: reinterpret_cast<uint16_t*>(out)[i] = ckv_f32_to_f16_bits(in[i]); break;
      case 3: reinterpret_cast<uint16_t*>(out)[i] = ckv_f32_to_bf16_bits(in[i]); break;
      case 4: reinterpret_cast<uint8_t*>(out)[i] = ckv_f32_to_e4m3(in[i]); break;
      case 5: reinterpret_cast<float*>(out)[i] = ckv_e4m3_to_f32((uint8_t)in[i]); break;
      default: return fail(CKV_E_INVALID, "unknown numerics op");
    }
  }
  return CKV_OK;
}

extern "C" const char* ckv_last_error(void) { return g_error; }

extern "C" int ckv_score_select(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                                const ckv_delta_chunks* dl, const ckv_decode_config* cfg,
                                ckv_decode_workspace* ws, void* stream) {
  int rc = validate(kv, st, csr, dl, cfg, ws);
  if (rc) return rc;
  const DecodeArgs a = pack(kv, st, csr, dl, cfg, ws);
  const size_t lds = (size_t)ws->descriptor_capacity * 8 + (((size_t)st->community_capacity * 2 + 15) & ~(size_t)15);
  const dim3 grid(ws->score_blocks, st->retrieval_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return dispatch(st->centroid_dtype, kv->dtype, [&](auto ct, auto dt) {
    hipLaunchKernelGGL((score_select_kernel<decltype(ct)::value, decltype(dt)::value>), grid, dim3(SELECT_THREADS),
                       lds, s, a);
    return launch_check("score_select");
  });
}

extern "C" int ckv_segmented_attention(const ckv_kv_cache* kv, const ckv_graph_state* st,
                                       const ckv_prefill_csr* csr, const ckv_delta_chunks* dl,
                                       const ckv_decode_config* cfg, ckv_decode_workspace* ws, void* stream) {
  int rc = validate(kv, st, csr, dl, cfg, ws);
  if (rc) return rc;
  if (!ws->slot_positions || !ws->partial_max || !ws->partial_sum || !ws->partial_acc || !ws->output || !ws->lse)
    return fail(CKV_E_INVALID, "attention workspace is incomplete");
  if (cfg->assignment != CKV_ASSIGN_NONE &&
      (!ws->partial_topk || !ws->topk_scores || !ws->topk_positions || !ws->assigned || !ws->overflow ||
       !st->current_position || !st->token_communities || !dl->positions || !dl->chunk_capacity ||
       !dl->chunk_next || !dl->community_head || !dl->next_free_chunk || !dl->next_free_position ||
       (cfg->assignment == CKV_ASSIGN_NEAREST && !ws->nearest)))
    return fail(CKV_E_INVALID, "update state or workspace is incomplete");
  const DecodeArgs a = pack(kv, st, csr, dl, cfg, ws);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int tiles = ws->slot_capacity / TILE;
  return dispatch(st->centroid_dtype, kv->dtype, [&](auto ct, auto dt) {
    constexpr int CT = decltype(ct)::value;
    constexpr int DT = decltype(dt)::value;
    hipLaunchKernelGGL((attend_generic_kernel<DT, false>), dim3(tiles, st->retrieval_heads), dim3(64), 0, s, a, 0, 0);
    int r = launch_check("attend");
    if (r) return r;
    hipLaunchKernelGGL((reduce_update_kernel<CT, DT>), dim3(st->retrieval_heads), dim3(REDUCE_THREADS), 0, s, a);
    r = launch_check("reduce_update");
    if (r) return r;
    if (cfg->assignment != CKV_ASSIGN_NONE && st->retrieval_heads != st->graph_count) {
      hipLaunchKernelGGL((sync_shared_kernel<CT, DT>), dim3(st->retrieval_heads), dim3(REDUCE_THREADS), 0, s, a);
      r = launch_check("sync_shared");
    }
    return r;
  });
}

extern "C" int ckv_decode_layer(const ckv_kv_cache* kv, const ckv_graph_state* st, const ckv_prefill_csr* csr,
                                const ckv_delta_chunks* dl, const ckv_decode_config* cfg,
                                ckv_decode_workspace* ws, void* stream) {
  int rc = ckv_score_select(kv, st, csr, dl, cfg, ws, stream);
  if (rc) return rc;
  return ckv_segmented_attention(kv, st, csr, dl, cfg, ws, stream);
}

extern "C" int ckv_dense_decode(const ckv_kv_cache* kv, int32_t seq_len, float softmax_scale, float* partial_max,
                                float* partial_sum, float* partial_acc, void* output, float* lse, void* stream) {
  if (!kv || !kv->query || !kv->key || !kv->value || !partial_max || !partial_sum || !partial_acc || !output || !lse)
    return fail(CKV_E_INVALID, "null argument");
  if (kv->kv_heads <= 0 || kv->query_heads % kv->kv_heads) return fail(CKV_E_INVALID, "query heads must be a multiple of kv heads");
  const int group = kv->query_heads / kv->kv_heads;
  if (group > CKV_MAX_GROUP) return fail(CKV_E_INVALID, "group size exceeds 16");
  if (seq_len <= 0 || seq_len > kv->capacity) return fail(CKV_E_INVALID, "seq_len out of range");
  if (kv->dtype != CKV_BF16 && kv->dtype != CKV_F32) return fail(CKV_E_INVALID, "kv dtype must be bf16 or f32");
  DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.kv = *kv;
  a.cfg.softmax_scale = softmax_scale;
  a.cfg.group_size = group;
  a.ws.partial_max = partial_max;
  a.ws.partial_sum = partial_sum;
  a.ws.partial_acc = partial_acc;
  a.ws.output = output;
  a.ws.lse = lse;
  const int tiles = (seq_len + TILE - 1) / TILE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kv->dtype == CKV_BF16) {
    hipLaunchKernelGGL((attend_generic_kernel<CKV_BF16, true>), dim3(tiles, kv->kv_heads), dim3(64), 0, s, a, seq_len, group);
    int r = launch_check("dense attend");
    if (r) return r;
    hipLaunchKernelGGL((dense_reduce_kernel<CKV_BF16>), dim3(kv->query_heads), dim3(REDUCE_THREADS), 0, s, a, tiles);
  } else {
    hipLaunchKernelGGL((attend_generic_kernel<CKV_F32, true>), dim3(tiles, kv->kv_heads), dim3(64), 0, s, a, seq_len, group);
    int r = launch_check("dense attend");
    if (r) return r;
    hipLaunchKernelGGL((dense_reduce_kernel<CKV_F32>), dim3(kv->query_heads), dim3(REDUCE_THREADS), 0, s, a, tiles);
  }
  return launch_check("dense reduce");
}
