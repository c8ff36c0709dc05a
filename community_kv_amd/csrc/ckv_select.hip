// Centroid scoring + exact community selection + slot materialisation.
//
// score_select_kernel: grid (score_blocks, retrieval_heads) x 256.  Every
// workgroup scores 64 communities of one retrieval head: 8 lanes per centroid
// row (16 dims each, one 16-byte fp8 load), pinned fp32 summation order (each
// lane sums its 16 products in order, then a butterfly over the 8 lanes), fp16
// round-to-nearest-even key.  The last workgroup of each head to finish
// (agent-scope counter, no spinning) runs the exact weighted threshold
// selection in LDS (two 8-bit radix passes over order-preserving fp16 keys),
// emits descriptors in the reference order and materialises the KV position of
// every attended slot.
//
// Reference: attention/kernels/centroid_selection.py:32-188 (scoring),
// attention/kernels/_csrc/descriptor_selection.cu:164-487 (selection),
// attention/kernels/segmented_attention.py:98-282 (slot -> position mapping).
#include <type_traits>

#include "ckv_device.h"
#include "ckv_error.h"

namespace ckv {

namespace {
int ckv_internal_limit(const char* message) { return ckv_internal::set_error(CKV_E_LIMIT, message); }
}  // namespace

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
  // Per-descriptor membership: decode-delta count and prefill CSR start, one
  // parallel round of loads.
  int* desc_dc = reinterpret_cast<int*>(key16 + ((C + 7) & ~7));
  int* desc_lo = desc_dc + dcap;
  for (int d = tid; d < n_desc; d += SELECT_THREADS) {
    const int c = desc_comm[d];
    desc_dc[d] = a.dl.community_sizes[tbl + c];
    desc_lo[d] = a.csr.member_offsets[(int64_t)graph * (C + 1) + c];
  }
  __syncthreads();
  // Slots in batches of 8 per thread so that the member-position gathers of a
  // batch are in flight together; decode-delta members (newest first) walk
  // their chunk chain afterwards.
  constexpr int BATCH = 8;
  const int32_t* members = a.csr.member_positions + (int64_t)graph * a.csr.member_stride;
  for (int s0 = 0; s0 < slot_cap; s0 += SELECT_THREADS * BATCH) {
    int spos[BATCH];
    int64_t at[BATCH];
    int dm[BATCH];   // member index into the delta chain, or -1
    int dcm[BATCH];  // community of a delta member
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int s = s0 + k * SELECT_THREADS + tid;
      spos[k] = -1;
      at[k] = -1;
      dm[k] = -1;
      dcm[k] = 0;
      if (s >= slot_cap) continue;
      if (s < ns) {
        spos[k] = a.cfg.sink_positions[s];
      } else if (s < ns + sel_count) {
        const int j = s - ns;
        int lo = 0, hi = n_desc;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (desc_end[mid] <= j) lo = mid + 1; else hi = mid;
        }
        const int prev = lo > 0 ? desc_end[lo - 1] : 0;
        const int m = j - prev;
        const int dc = desc_dc[lo];
        if (m < dc) {
          dm[k] = m;
          dcm[k] = desc_comm[lo];
        } else {
          const int64_t idx = (int64_t)desc_lo[lo] + (m - dc);
          if (idx < a.csr.member_stride) at[k] = idx;
        }
      } else if (inc && s == ns + sel_count + W) {
        spos[k] = cur;
      }
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int v = members[at[k] >= 0 ? at[k] : 0];
      if (at[k] >= 0) spos[k] = v;
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      if (dm[k] < 0) continue;
      int rem = dm[k];
      int ch = a.dl.community_tail[tbl + dcm[k]];
      const int64_t cb = (int64_t)graph * a.dl.chunks_per_graph;
      for (int guard = 0; guard < 64 && ch >= 0 && ch < a.dl.chunks_per_graph; ++guard) {
        const int cs = a.dl.chunk_size[cb + ch];
        if (rem < cs) {
          const int p = a.dl.chunk_start[cb + ch] + cs - 1 - rem;
          if (p >= 0 && p < a.dl.position_capacity) spos[k] = a.dl.positions[(int64_t)graph * a.dl.position_capacity + p];
          break;
        }
        rem -= cs;
        ch = a.dl.chunk_previous[cb + ch];
      }
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int s = s0 + k * SELECT_THREADS + tid;
      if (s >= slot_cap) continue;
      if (s >= ns + sel_count && s < ns + sel_count + W) continue;  // window: resolved below
      slots[s] = spos[k];
      if (s == ns + sel_count - 1 && sel_count > 0) s_last_sel_pos = spos[k];
    }
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

int launch_score_select(const DecodeArgs& a, hipStream_t s) {
  // Dynamic LDS: descriptor communities/ends/delta counts/CSR starts + fp16 keys.
  const size_t lds = (size_t)a.ws.descriptor_capacity * 16 + (((size_t)a.st.community_capacity + 7) & ~(size_t)7) * 2;
  const dim3 grid(a.ws.score_blocks, a.st.retrieval_heads);
  const int ct = a.st.centroid_dtype, dt = a.kv.dtype;
  auto launch = [&](auto kernel) {
    if (lds > 48 * 1024) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return ckv_internal_limit("selection LDS exceeds the device limit");
    }
    hipLaunchKernelGGL(kernel, grid, dim3(SELECT_THREADS), lds, s, a);
    return launch_check("score_select");
  };
  if (ct == CKV_E4M3 && dt == CKV_BF16) return launch(score_select_kernel<CKV_E4M3, CKV_BF16>);
  if (ct == CKV_E4M3) return launch(score_select_kernel<CKV_E4M3, CKV_F32>);
  if (dt == CKV_BF16) return launch(score_select_kernel<CKV_F32, CKV_BF16>);
  return launch(score_select_kernel<CKV_F32, CKV_F32>);
}

}  // namespace ckv
