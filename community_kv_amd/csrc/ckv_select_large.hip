// Centroid scoring and exact community selection for heads with more scored
// rows than one workgroup holds in registers (more than 8,192, up to 65,536).
//
//   score_rows_kernel    64 rows of one head per workgroup, on every compute
//                        unit: the fp16 group-maximum score of each row in the
//                        selection's pinned arithmetic (dot16_pair), -inf for
//                        empty rows, into ws.scores; in nearest-centroid mode
//                        also each block's nearest row to the current key.
//   select_large_kernel  one 1,024-thread workgroup per head: weighted
//                        two-pass radix threshold over the stored keys,
//                        id-ordered compaction into descriptors (high keys,
//                        then threshold keys), the selected communities'
//                        membership fields, slot materialisation and every
//                        selection output, as select_body writes them.
//
// The results are those of the single-workgroup selection in ckv_select.hip
// (same keys, threshold, descriptor order, slot layout); only the work is
// spread differently.  Reference: attention/kernels/centroid_selection.py:
// 27, 240-255 (selection above the cluster path's 65,536 communities falls back
// to the multi-kernel selector, attention/kernels/_csrc/descriptor_selection.cu:
// 852-1189).
#include <algorithm>
#include <cstring>

#include "ckv_device.h"
#include "ckv_error.h"
#include "ckv_score.h"
#include "ckv_update.h"

namespace ckv {

namespace {

constexpr int ROWS = SELECT_THREADS / 8;  // rows scored per workgroup (8 lanes per row)
// Scored rows per head above which the separate selection launch scores on
// every compute unit and selects with 1,024 threads per head (one 512-thread
// workgroup scoring and selecting 2,048 rows alone takes ~40 us)
constexpr int LARGE_MIN_ROWS = 1024;
constexpr int LT = 1024;                  // select_large_kernel threads
constexpr int LWAVES = LT / 64;
constexpr int MAT_BATCH_L = 4;            // 64-slot blocks per wave gathered together
#ifndef CKV_LARGE_MAX_PARTS
#define CKV_LARGE_MAX_PARTS 4
#endif
constexpr int LARGE_MAX_PARTS = CKV_LARGE_MAX_PARTS;  // selection workgroups per head at most
constexpr int DEVICE_CUS = 256;                       // compute units one round of workgroups fills

int limit_error(const char* message) { return ckv_internal::set_error(CKV_E_LIMIT, message); }

}  // namespace

// Scores (and, in nearest-centroid mode, block minima of the squared distance
// to the current key: distance bits << 32 | row, into exchange[rh][C + blk])
// of rows [64 * blk, +64) of head rh.
template <int CT, int DT>
__device__ __forceinline__ void score_rows_body(const DecodeArgs& a, const int rh, const int blk) {
  __shared__ float q_s[CKV_MAX_GROUP * D];
  __shared__ float key_s[D];
  __shared__ uint64_t near_s[SELECT_THREADS / 64];
  const int tid = threadIdx.x;
  const int C = a.st.community_capacity;
  const int nscore = min(C, a.ws.score_blocks * SCORE_BLOCK);
  if (blk * ROWS >= nscore) return;  // (batched grids cover the largest item)
  int count = a.st.community_counts[rh];
  count = count < 0 ? 0 : (count > nscore ? nscore : count);
  const int r0 = blk * ROWS;
  const bool nearest_mode = a.cfg.assignment == CKV_ASSIGN_NEAREST;
  if (r0 >= count) {
    if (nearest_mode && tid == 0) a.ws.exchange[(int64_t)rh * ckv_exchange_words(C) + C + blk] = ~0ull;
    return;
  }
  const int G = a.cfg.group_size;
  const int sub = tid >> 3, lane8 = tid & 7;
  const int row = min(r0 + sub, count - 1);
  CentroidFrag<CT> frag;
  load_frag<CT>(a.st.centroids, (int64_t)rh * C + row, 16 * lane8, frag);
  const int size = gload_i32(a.st.community_sizes + (int64_t)rh * C + row);
  for (int e = tid; e < G * D; e += SELECT_THREADS) q_s[e] = load_elem<DT>(a.kv.query, (int64_t)rh * G * D + e);
  if (nearest_mode && tid < D) {
    const int graph = a.st.retrieval_to_graph[rh];
    const int cur = a.st.current_position[graph];
    const int kvh = a.st.retrieval_to_kv[rh];
    const int64_t pc = cur < 0 ? 0 : (cur >= a.kv.capacity ? a.kv.capacity - 1 : cur);
    const float kv = load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + pc * a.kv.token_stride + tid);
    key_s[tid] = (cur >= 0 && cur < a.kv.capacity) ? kv : 0.0f;
  }
  __syncthreads();
  float cv[16];
  decode_frag<CT>(frag, cv);
  float best = NEG_INF;
  for (int g = 0; g < G; g += 2) {
    float qa[16], qb[16];
    load_q_pair(q_s, g, lane8, qa, qb);
    float a0, a1;
    dot16_pair<CT, DT>(qa, qb, cv, a0, a1);
    best = fmax_exact(best, a0);
    if (g + 1 < G) best = fmax_exact(best, a1);
  }
  const int c = r0 + sub;
  if (lane8 == 0 && c < count) a.ws.scores[(int64_t)rh * C + c] = f16_bits_hw(size > 0 ? best : NEG_INF);
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
    acc = add_xor_f32<4>(acc);
    acc = add_xor_f32<2>(acc);
    acc = add_xor_f32<1>(acc);
    const bool live = c < count && size > 0;
    uint64_t cand = live ? (((uint64_t)ckv_f2u(acc) << 32) | (uint32_t)c) : ~0ull;
    cand = wave_min_u64(cand);
    if ((tid & 63) == 0) near_s[tid >> 6] = cand;
    __syncthreads();
    if (tid == 0) {
      uint64_t m = ~0ull;
      for (int w = 0; w < SELECT_THREADS / 64; ++w) m = near_s[w] < m ? near_s[w] : m;
      a.ws.exchange[(int64_t)rh * ckv_exchange_words(C) + C + blk] = m;
    }
  }
}

template <int CT, int DT>
__global__ __launch_bounds__(SELECT_THREADS) void score_rows_kernel(DecodeArgs a) {
  score_rows_body<CT, DT>(a, blockIdx.y, blockIdx.x);
}

// Batched: head blockIdx.y % heads of item blockIdx.y / heads.
template <int CT, int DT>
__global__ __launch_bounds__(SELECT_THREADS) void score_rows_large_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                                int heads) {
  score_rows_body<CT, DT>(table[blockIdx.y / heads], blockIdx.y % heads, blockIdx.x);
}

// LDS of select_large_kernel: seven descriptor arrays and the per-block first
// descriptor of the selection.
__host__ __device__ inline size_t large_lds_bytes(int descriptor_capacity, int max_selected) {
  return (size_t)descriptor_capacity * 7 * 4 + (size_t)((max_selected + 63) / 64 + 2) * 4;
}

// Workgroups past a.st.retrieval_heads run the pending online update of
// another layer `u` (same dtypes), one retrieval head each, on the compute
// units this launch leaves idle (the selection is one workgroup per head).
template <int CT, int DT>
// parts > 1: this workgroup (part `part` of the head's `parts`) repeats the
// selection and resolves every parts-th 64-slot block of the slot table and a
// strided share of the other outputs.
__device__ __forceinline__ void select_large_body(const DecodeArgs& a, const int rh, const int part = 0,
                                                  const int parts = 1) {
  __shared__ __align__(16) int hist[256];
  __shared__ __align__(16) int hist2[256];
  __shared__ int scan_s[4 * LWAVES];
  __shared__ int sink_s[CKV_MAX_SINKS];
  __shared__ int s_max_idx, s_hb, s_above_hb, s_lb, s_last_size, s_last_sel_pos, s_sink_max;
  extern __shared__ __align__(16) int dyn_l[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int C = a.st.community_capacity;
  const int nscore = min(C, a.ws.score_blocks * SCORE_BLOCK);
  const int dcap = a.ws.descriptor_capacity;
  int* desc_comm = dyn_l;
  int* desc_end = desc_comm + dcap;
  int* desc_lo = desc_end + dcap;
  int* desc_dc = desc_lo + dcap;
  int* desc_tl = desc_dc + dcap;
  int* desc_ts = desc_tl + dcap;
  int* desc_tn = desc_ts + dcap;
  int* blk_first = desc_tn + dcap;
  int count = a.st.community_counts[rh];
  count = count < 0 ? 0 : (count > nscore ? nscore : count);
  const int graph = a.st.retrieval_to_graph[rh];
  const int cur = a.st.current_position[graph];
  const bool materialise = a.csr.member_offsets != nullptr;
  const bool nearest_mode = a.cfg.assignment == CKV_ASSIGN_NEAREST;
  const int ns = a.cfg.num_sink;
  const int W = a.cfg.local_window;
  const int cpg = a.dl.chunks_per_graph;
  const int64_t cb = (int64_t)graph * cpg;
  const bool budget_mode = a.cfg.selection_mode == CKV_SELECT_BUDGET;
  const int sel_slots = a.cfg.max_selected;
  const int target = budget_mode ? sel_slots : a.cfg.topk_communities;
  const uint16_t* keys = a.ws.scores + (int64_t)rh * C;
  const int32_t* sizes = a.st.community_sizes + (int64_t)rh * C;

  hist[tid & 255] = 0;
  hist2[tid & 255] = 0;
  if (tid < ns) sink_s[tid] = gload_i32(a.cfg.sink_positions + tid);
  if (tid == 0) s_max_idx = -1;
  __syncthreads();
  if (wave == 0) {  // largest sink position: window tokens beyond it skip the sink test
    int m = -1;
    for (int i = lane; i < ns; i += 64) m = max(m, sink_s[i]);
    m = wave_max_i32(m);
    if (lane == 0) s_sink_max = m;
  }

  // The order-preserving key of row c, or 0 when the row does not compete
  // (past the live communities, or empty: its score is -inf).
  auto row_key = [&](int c, uint16_t bits, int size) -> uint32_t {
    return (c < count && size > 0) ? ckv_ordered_key16(bits) : 0u;
  };
  constexpr int U = 8;  // rows per thread in flight per round of the strided passes
  // ---- pass 1: weight per high byte --------------------------------------------
  for (int c0 = 0; c0 < count; c0 += U * LT) {
    uint16_t kb[U];
    int sz[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + u * LT + tid, nscore - 1);
      kb[u] = keys[c];
      sz[u] = gload_i32(sizes + c);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * LT + tid;
      const uint32_t k = row_key(c, kb[u], sz[u]);
      if (c < count && sz[u] > 0) atomicAdd(hist + (k >> 8), budget_mode ? sz[u] : 1);
    }
  }
  __syncthreads();
  if (wave == 0) {
    int hb, above;
    wave_find_bin(hist, target, hb, above);
    if (lane == 0) {
      s_hb = hb;
      s_above_hb = above;
    }
  }
  __syncthreads();
  const int hb = s_hb;
  int threshold = -1;  // 16-bit key threshold; -1 selects every non-empty community
  if (hb >= 0) {
    // ---- pass 2: weight per low byte within the threshold's high byte ----------
    for (int c0 = 0; c0 < count; c0 += U * LT) {
      uint16_t kb[U];
      int sz[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u * LT + tid, nscore - 1);
        kb[u] = keys[c];
        sz[u] = gload_i32(sizes + c);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * LT + tid;
        const uint32_t k = row_key(c, kb[u], sz[u]);
        if (c < count && sz[u] > 0 && (int)(k >> 8) == hb) atomicAdd(hist2 + (k & 0xff), budget_mode ? sz[u] : 1);
      }
    }
    __syncthreads();
    if (wave == 0) {
      int lb, above;
      wave_find_bin(hist2, target - s_above_hb, lb, above);
      if (lane == 0) s_lb = lb;
    }
    __syncthreads();
    threshold = (hb << 8) | s_lb;
  }

  // ---- compaction in id order: thread t covers rows [t * K, t * K + K) -----------
  const int K = (count + LT - 1) / LT;
  const int cbeg = min(tid * K, count), cend = min(cbeg + K, count);
  int cnt[4] = {0, 0, 0, 0};  // high count, high mass, threshold count, threshold mass
  for (int c0 = cbeg; c0 < cend; c0 += U) {
    uint16_t kb[U];
    int sz[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + u, count - 1);
      kb[u] = keys[c];
      sz[u] = gload_i32(sizes + c);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u;
      const uint32_t k = row_key(c, kb[u], sz[u]);
      const bool ok = c < cend && sz[u] > 0;
      if (ok && (int)k > threshold) {
        cnt[0] += 1;
        cnt[1] += sz[u];
      } else if (ok && threshold >= 0 && (int)k == threshold) {
        cnt[2] += 1;
        cnt[3] += sz[u];
      }
    }
  }
  int base[4], tot[4];
  {
    int inc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) inc[i] = wave_inclusive_scan(cnt[i]);
    if (lane == 63) {
#pragma unroll
      for (int i = 0; i < 4; ++i) scan_s[4 * wave + i] = inc[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      base[i] = inc[i] - cnt[i];
      tot[i] = 0;
    }
    for (int w = 0; w < LWAVES; ++w) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int x = scan_s[4 * w + i];
        if (w < wave) base[i] += x;
        tot[i] += x;
      }
    }
  }
  const int high_count = tot[0], high_mass = tot[1];
  const int cap_sel = sel_slots;
  {
    int hc = base[0], hm = base[1], ec = base[2], em = base[3];
    int my_max = -1;
    for (int c0 = cbeg; c0 < cend; c0 += U) {
      uint16_t kb[U];
      int sz[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u, count - 1);
        kb[u] = keys[c];
        sz[u] = gload_i32(sizes + c);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u;
        const int size = sz[u];
        const uint32_t k = row_key(c, kb[u], size);
        const bool ok = c < cend && size > 0;
        int idx = -1, st = 0, en = 0;
        if (ok && (int)k > threshold) {
          if (hm < cap_sel && hc < dcap) {
            idx = hc;
            st = hm;
            en = min(cap_sel, hm + size);
          }
          hc += 1;
          hm += size;
        } else if (ok && threshold >= 0 && (int)k == threshold) {
          const int st0 = high_mass + em;
          const bool within = budget_mode ? (st0 < sel_slots) : (ec < a.cfg.topk_communities - high_count);
          const int i2 = high_count + ec;
          if (within && st0 < cap_sel && i2 < dcap) {
            idx = i2;
            st = st0;
            en = min(cap_sel, st0 + size);
          }
          ec += 1;
          em += size;
        }
        if (idx >= 0) {
          desc_comm[idx] = c;
          desc_end[idx] = en;
          // first descriptor of every 64-slot block whose first slot lies in [st, en)
          for (int b = (st + 63) >> 6; (b << 6) < en; ++b) blk_first[b] = idx;
          my_max = max(my_max, idx);
          desc_tn[idx] = size;  // (the community size, until the membership fields below)
        }
      }
    }
    my_max = wave_max_i32(my_max);
    if (lane == 0 && my_max >= 0) atomicMax(&s_max_idx, my_max);
  }
  __syncthreads();
  const int n_desc = s_max_idx + 1;
  const int sel_count = n_desc > 0 ? desc_end[n_desc - 1] : 0;
  if (tid == 0) {
    blk_first[(sel_count + 63) / 64] = n_desc;
    s_last_size = n_desc > 0 ? desc_tn[n_desc - 1] : 0;
    s_last_sel_pos = -1;
  }
  // membership fields of the selected communities (two dependent rounds)
  if (materialise) {
    for (int d0 = 0; d0 < n_desc; d0 += LT) {
      const int d = min(d0 + tid, n_desc - 1);
      const int c = desc_comm[d];
      const int lo = gload_i32(a.csr.member_offsets + (int64_t)graph * (C + 1) + c);
      const int dc = gload_i32(a.dl.community_sizes + (int64_t)graph * C + c);
      const int tl = gload_i32(a.dl.community_tail + (int64_t)graph * C + c);
      const bool has = dc > 0 && tl >= 0 && tl < cpg;
      const int t = has ? tl : 0;
      const int ts = cpg > 0 ? gload_i32(a.dl.chunk_start + cb + t) : 0;
      const int tn = cpg > 0 ? gload_i32(a.dl.chunk_size + cb + t) : 0;
      __syncthreads();  // every desc_tn (size) read above is done before the overwrite
      if (d0 + tid < n_desc) {
        desc_lo[d] = lo;
        desc_dc[d] = dc;
        desc_tl[d] = tl;
        desc_ts[d] = has ? ts : 0;
        desc_tn[d] = has ? tn : 0;
      }
    }
  }
  __syncthreads();

  const int slot_cap = a.ws.slot_capacity;
  int32_t* slots = a.ws.slot_positions + (int64_t)rh * slot_cap;
  const int inc = a.cfg.include_current ? 1 : 0;
  const int wbeg = ns + sel_count;
  if (materialise) {
    // ---- slot materialisation: [sinks][selected, newest first][window][current] ----
    const int32_t* members = a.csr.member_positions + (int64_t)graph * a.csr.member_stride;
    const int32_t* dpos = a.dl.positions + (int64_t)graph * a.dl.position_capacity;
    const int nblk_sel = (sel_count + 63) / 64;
    const int nblk_own = nblk_sel > part ? (nblk_sel - part + parts - 1) / parts : 0;
    for (int b0 = wave; b0 < nblk_own; b0 += LWAVES * MAT_BATCH_L) {
      const int32_t* src[MAT_BATCH_L];
      bool gathered[MAT_BATCH_L];
      int slow_d[MAT_BATCH_L], slow_rem[MAT_BATCH_L];
#pragma unroll
      for (int q = 0; q < MAT_BATCH_L; ++q) {
        const int b = part + parts * (b0 + q * LWAVES);
        src[q] = a.st.community_counts + rh;  // in-bounds dummy address when nothing is gathered
        gathered[q] = false;
        slow_d[q] = -1;
        slow_rem[q] = 0;
        if (b < nblk_sel) {
          // a lane's descriptor: the block's first one plus the descriptor ends
          // at or before the lane's slot (a wave-wide mask of ends in the block)
          const int j = 64 * b + lane;
          const int d0 = blk_first[b];
          const int e = d0 + lane < n_desc ? desc_end[d0 + lane] : 0x7fffffff;
          const int off = e - 64 * b;
          const uint64_t mask = wave_or_u64(off >= 1 && off <= 63 ? (1ull << off) : 0ull);
          const uint64_t below = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
          const int d = d0 + __popcll(mask & below);
          if (j < sel_count) {
            const int m = j - (d > 0 ? desc_end[d - 1] : 0);
            const int dc = desc_dc[d];
            if (m < dc) {
              const int tn = desc_tn[d];
              if (m < tn) {
                const int p = desc_ts[d] + tn - 1 - m;
                if (p >= 0 && p < a.dl.position_capacity) {
                  src[q] = dpos + p;
                  gathered[q] = true;
                }
              } else {
                slow_d[q] = d;
                slow_rem[q] = m - tn;
              }
            } else {
              const int64_t idx = (int64_t)desc_lo[d] + (m - dc);
              if (idx >= 0 && idx < a.csr.member_stride) {
                src[q] = members + idx;
                gathered[q] = true;
              }
            }
          }
        }
      }
      int val[MAT_BATCH_L];
#pragma unroll
      for (int q = 0; q < MAT_BATCH_L; ++q) val[q] = gload_i32(src[q]);
#pragma unroll
      for (int q = 0; q < MAT_BATCH_L; ++q) {
        if (!gathered[q]) val[q] = -1;
        if (slow_d[q] >= 0) {  // a delta member older than the tail chunk: walk the chunk chain
          const int tail = desc_tl[slow_d[q]];
          int rem = slow_rem[q];
          if (tail >= 0 && tail < cpg) {
            int ch = a.dl.chunk_previous[cb + tail];
            for (int guard = 0; guard < 64 && ch >= 0 && ch < cpg; ++guard) {
              const int cs = a.dl.chunk_size[cb + ch];
              if (rem < cs) {
                const int p = a.dl.chunk_start[cb + ch] + cs - 1 - rem;
                if (p >= 0 && p < a.dl.position_capacity) val[q] = dpos[p];
                break;
              }
              rem -= cs;
              ch = a.dl.chunk_previous[cb + ch];
            }
          }
        }
        const int j = 64 * (part + parts * (b0 + q * LWAVES)) + lane;
        if (j < sel_count) {
          slots[ns + j] = val[q];
          if (j == sel_count - 1) s_last_sel_pos = val[q];
        }
      }
    }
    if (tid < ns && part == 0) slots[tid] = sink_s[tid];
    __syncthreads();  // s_last_sel_pos
    // the window, the current token and the padding: the part that resolved the last block
    const bool tail_part = part == (nblk_sel > 0 ? (nblk_sel - 1) % parts : 0);
    // Window slot i (position cur - W + i), or -1 when that token is already
    // attended: a sink, or a member of a selected community at or after the
    // selection's oldest attended position.  Selected communities are two
    // id-sorted runs of descriptors: high keys [0, high_count), threshold keys
    // [high_count, n_desc).
    auto find_desc = [&](int c) {
      int lo = 0, hi = min(high_count, n_desc);
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (desc_comm[mid] < c) lo = mid + 1; else hi = mid;
      }
      if (lo < min(high_count, n_desc) && desc_comm[lo] == c) return lo;
      lo = min(high_count, n_desc);
      hi = n_desc;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (desc_comm[mid] < c) lo = mid + 1; else hi = mid;
      }
      return (lo < n_desc && desc_comm[lo] == c) ? lo : -1;
    };
    const int last_pos = s_last_sel_pos;
    const int32_t* tcomm = a.st.token_communities + (int64_t)graph * a.st.token_capacity;
    for (int i = tail_part ? tid : W; i < W; i += LT) {
      const int p = cur - W + i;
      int pos = p < 0 ? -1 : p;
      if (pos >= 0 && p <= s_sink_max) {
        for (int k = 0; k < ns; ++k) {
          if (sink_s[k] == p) pos = -1;
        }
      }
      if (pos >= 0 && p < a.st.token_capacity) {
        const int wc = tcomm[p];
        if (wc >= 0 && wc < count) {
          const int found = find_desc(wc);
          if (found >= 0) {
            const int take = desc_end[found] - (found > 0 ? desc_end[found - 1] : 0);
            const bool full = found < n_desc - 1 || take >= s_last_size;
            if (full || p >= last_pos) pos = -1;
          }
        }
      }
      slots[wbeg + i] = pos;
    }
    if (tail_part) {
      if (inc && tid == 0) slots[wbeg + W] = cur;
      for (int s = wbeg + W + inc + tid; s < slot_cap; s += LT) slots[s] = -1;
    }
  }
  // ---- the other selection outputs (strided over the parts) ------------------------
  if (tid == 0 && part == 0) {
    a.ws.descriptor_counts[rh] = n_desc;
    a.ws.selected_counts[rh] = sel_count;
  }
  const int pt = part + parts * tid, pstride = parts * LT;
  for (int i = pt; i < n_desc; i += pstride) {
    a.ws.communities[(int64_t)rh * dcap + i] = desc_comm[i];
    a.ws.cumulative_ends[(int64_t)rh * dcap + i] = desc_end[i];
  }
  for (int t = pt; t < a.ws.budget_tiles; t += pstride) {
    // first descriptor ending after the tile's first selected slot
    const int off = max(t * TILE - ns, 0);
    int lo = n_desc - 1;
    if (off < sel_count) {
      lo = blk_first[off >> 6];
      int hi = min(blk_first[(off >> 6) + 1], n_desc - 1);
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (desc_end[mid] <= off) lo = mid + 1; else hi = mid;
      }
    }
    a.ws.tile_descriptors[(int64_t)rh * a.ws.budget_tiles + t] = max(0, min(lo, n_desc - 1));
  }
  for (int c = count + pt; c < nscore; c += pstride) a.ws.scores[(int64_t)rh * C + c] = (uint16_t)0xfc00u;
  if (nearest_mode && wave == 0 && part == 0) {
    const uint64_t* bm = a.ws.exchange + (int64_t)rh * ckv_exchange_words(C) + C;
    const int nb = (count + ROWS - 1) / ROWS;
    uint64_t m = ~0ull;
    for (int b = lane; b < nb; b += 64) m = bm[b] < m ? bm[b] : m;
    m = wave_min_u64(m);
    if (lane == 0) a.ws.nearest[rh] = (m == ~0ull) ? -1 : (int)(m & 0xffffffffu);
  }
}

// Workgroups past a.st.retrieval_heads run the pending online update of
// another layer `u` (same dtypes), one retrieval head each, on the compute
// units this launch leaves idle (the selection is one workgroup per head).
template <int CT, int DT>
__global__ __launch_bounds__(LT) void select_large_kernel(DecodeArgs a, DecodeArgs u, int parts) {
  const int nsel = a.st.retrieval_heads * parts;
  if ((int)blockIdx.x >= nsel) {
    const int urh = (int)blockIdx.x - nsel;
    owner_update<CT, DT>(u, urh, u.ws.lse[(int64_t)urh * u.cfg.group_size]);
    return;
  }
  select_large_body<CT, DT>(a, blockIdx.x % a.st.retrieval_heads, blockIdx.x / a.st.retrieval_heads, parts);
}

// Batched: head blockIdx.x % heads of item blockIdx.x / heads.
template <int CT, int DT>
__global__ __launch_bounds__(LT) void select_large_batch_kernel(const DecodeArgs* __restrict__ table, int heads,
                                                                 int parts) {
  const int per_item = heads * parts;
  const int r = blockIdx.x % per_item;
  select_large_body<CT, DT>(table[blockIdx.x / per_item], r % heads, r / heads, parts);
}

bool large_selection(const DecodeArgs& a) {
  return std::min(a.st.community_capacity, a.ws.score_blocks * SCORE_BLOCK) > LARGE_MIN_ROWS;
}

int launch_select_large(const DecodeArgs& a, hipStream_t s, const DecodeArgs* pending) {
  const int nscore = std::min(a.st.community_capacity, a.ws.score_blocks * SCORE_BLOCK);
  if (nscore > CKV_MAX_COMMUNITIES) return limit_error("more than 65536 scored communities per head");
  if (a.cfg.assignment == CKV_ASSIGN_NEAREST && a.ws.exchange == nullptr)
    return limit_error("nearest-centroid assignment above 8192 scored communities needs the exchange workspace");
  const size_t lds = large_lds_bytes(a.ws.descriptor_capacity, a.cfg.max_selected);
  DecodeArgs u;
  memset(&u, 0, sizeof(u));
  const bool upd = pending != nullptr && pending->cfg.assignment != CKV_ASSIGN_NONE;
  if (upd) u = *pending;
  const dim3 sg((nscore + ROWS - 1) / ROWS, a.st.retrieval_heads);
  // The pending update rides in the selection launch (one workgroup per head
  // beside the selection's one per head), not in the scoring launch: the
  // update's dependent chain is longer than the scoring but shorter than the
  // selection.
  // parts per head: the selection repeats side by side on otherwise idle
  // compute units and splits the (instruction-bound) slot resolution
  const int ublocks = upd ? u.st.retrieval_heads : 0;
  const int parts = std::max(1, std::min(LARGE_MAX_PARTS, (DEVICE_CUS - ublocks) / std::max(1, a.st.retrieval_heads)));
  const int select_blocks = a.st.retrieval_heads * parts + ublocks;
  auto go = [&](auto score, auto select) {
    hipLaunchKernelGGL(score, sg, dim3(SELECT_THREADS), 0, s, a);
    int rc = launch_check("score_rows");
    if (rc) return rc;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(select),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return limit_error("large selection LDS (descriptors x 28 + selected / 16 bytes) exceeds the device limit");
    }
    hipLaunchKernelGGL(select, dim3(select_blocks), dim3(LT), lds, s, a, u, parts);
    return launch_check("select_large");
  };
  const bool e4m3 = a.st.centroid_dtype == CKV_E4M3, bf16 = a.kv.dtype == CKV_BF16;
  if (e4m3 && bf16) return go(score_rows_kernel<CKV_E4M3, CKV_BF16>, select_large_kernel<CKV_E4M3, CKV_BF16>);
  if (e4m3) return go(score_rows_kernel<CKV_E4M3, CKV_F32>, select_large_kernel<CKV_E4M3, CKV_F32>);
  if (bf16) return go(score_rows_kernel<CKV_F32, CKV_BF16>, select_large_kernel<CKV_F32, CKV_BF16>);
  return go(score_rows_kernel<CKV_F32, CKV_F32>, select_large_kernel<CKV_F32, CKV_F32>);
}

// The large selection for every item of a batch (bf16 KV): scoring of every
// item's rows on all compute units, then one 1,024-thread workgroup per
// (item, head).  h is the first item (dtypes, heads); max_nscore and max_lds
// the largest item's scored rows and selection LDS.
int launch_batch_select_large(const DecodeArgs& h, const DecodeArgs* table, int count, int max_nscore,
                              size_t max_lds, hipStream_t s) {
  if (max_nscore > CKV_MAX_COMMUNITIES) return limit_error("more than 65536 scored communities per head");
  const int heads = h.st.retrieval_heads;
  const dim3 sg((max_nscore + ROWS - 1) / ROWS, count * heads);
  auto go = [&](auto score, auto select) {
    hipLaunchKernelGGL(score, sg, dim3(SELECT_THREADS), 0, s, table, heads);
    int rc = launch_check("score_rows_large_batch");
    if (rc) return rc;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(select),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return limit_error("large selection LDS (descriptors x 28 + selected / 16 bytes) exceeds the device limit");
    }
    const int parts = std::max(1, std::min(LARGE_MAX_PARTS, DEVICE_CUS / std::max(1, count * heads)));
    hipLaunchKernelGGL(select, dim3(count * heads * parts), dim3(LT), max_lds, s, table, heads, parts);
    return launch_check("select_large_batch");
  };
  if (h.st.centroid_dtype == CKV_E4M3)
    return go(score_rows_large_batch_kernel<CKV_E4M3, CKV_BF16>, select_large_batch_kernel<CKV_E4M3, CKV_BF16>);
  return go(score_rows_large_batch_kernel<CKV_F32, CKV_BF16>, select_large_batch_kernel<CKV_F32, CKV_BF16>);
}

size_t select_large_lds_bytes(const DecodeArgs& a) {
  return large_lds_bytes(a.ws.descriptor_capacity, a.cfg.max_selected);
}

}  // namespace ckv
